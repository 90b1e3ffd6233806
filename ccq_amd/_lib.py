"""ctypes binding of libccq_hip.so (the C ABI declared in include/ccq_hip.h).

The shared library is built in-tree by ``ccq_amd/build.py``.  Loading fails
loudly when it is missing: there is no CPU or PyTorch fallback for any op.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libccq_hip.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); must match include/ccq_hip.h
SIGNATURES = {
    "ccq_abi_version": (_I, []),
    "ccq_last_error": (ctypes.c_char_p, []),
    "ccq_clean_saved_bytes": (_SZ, [_I64, _I, _I, _I, _I, _I, _I]),
    "ccq_clean_fwd": (_I, [_P] * 14 + [_I] * 7 + [_P]),
    "ccq_clean_bwd_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I, _I, _I, _I]),
    "ccq_clean_bwd": (_I, [_P] * 24 + [_I] * 7 + [_P]),
    "ccq_chunk_index": (_I, [_P, _I, _P, _P, _I, _P]),
    "ccq_gdn_saved_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "ccq_gdn_bwd_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "ccq_gdn_fwd": (_I, [_P] * 10 + [_I] + [_P] * 3 + [_I] * 6 + [_F, _P]),
    "ccq_gdn_bwd": (_I, [_P] * 9 + [_I] + [_P] * 10 + [_I] * 6 + [_F, _P]),
    "ccq_gla_saved_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "ccq_gla_bwd_workspace_bytes": (_SZ, [_I64, _I, _I, _I, _I]),
    "ccq_gla_fwd": (_I, [_P] * 9 + [_I] + [_P] * 3 + [_I] * 6 + [_F, _P]),
    "ccq_gla_bwd": (_I, [_P] * 8 + [_I] + [_P] * 11 + [_I] * 6 + [_F, _P]),
    "ccq_decode_workspace_bytes": (_SZ, [_I64, _I, _I]),
    "ccq_gdn_decode": (_I, [_P] * 19 + [_I] * 10 + [_F, _P]),
    "ccq_gla_decode": (_I, [_P] * 17 + [_I] * 10 + [_F, _P]),
    "ccq_gdn_decode_noalloc": (_I, [_P] * 18 + [_I] * 10 + [_F, _P]),
    "ccq_decode_step_workspace_bytes": (_SZ, [_I] * 4),
    "ccq_gdn_decode_in_proj": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _I, _P, _F] + [_I] * 9 + [_P] * 13 + [_I, _P]),
    "ccq_gdn_layer_decode_step": (_I, [_P, _I64, _I, _I, _I] + [_P] * 10 + [_I] * 7 + [_F, _F, _P]),
    "ccq_gdn_decode_step": (_I, [_P] * 14 + [_I] * 8 + [_F, _P]),
    "ccq_gla_decode_step": (_I, [_P] * 13 + [_I] * 7 + [_F, _P]),
    "ccq_clean_z_saved_bytes": (_SZ, [_I, _I, _I]),
    "ccq_clean_z_bwd_workspace_bytes": (_SZ, [_I, _I, _I]),
    "ccq_clean_z_fwd": (_I, [_P] * 8 + [_I] + [_P] * 3 + [_I] * 7 + [_P]),
    "ccq_clean_z_bwd": (_I, [_P] * 7 + [_I] + [_P] * 10 + [_I] * 7 + [_P]),
    "ccq_conv_bwd_workspace_bytes": (_SZ, [_I64, _I, _I]),
    "ccq_conv_fwd": (_I, [_P] * 9 + [_I] * 7 + [_F, _P]),
    "ccq_conv_bwd": (_I, [_P] * 12 + [_I] * 7 + [_P]),
    "ccq_gated_rmsnorm_bwd_workspace_bytes": (_SZ, [_I64, _I]),
    "ccq_gated_rmsnorm_fwd": (_I, [_P] * 5 + [_I64, _I, _F, _P]),
    "ccq_gated_rmsnorm_bwd": (_I, [_P] * 9 + [_I64, _I, _P]),
    "ccq_gated_rmsnorm_fwd_strided": (_I, [_P, _P, _I64, _I, _P, _P, _P, _I64, _I, _F, _P]),
    "ccq_narrow_linear_bwd_workspace_bytes": (_SZ, [_I64, _I, _I]),
    "ccq_narrow_linear_fwd": (_I, [_P, _I64, _P, _P, _P, _I64, _I, _I, _P]),
    "ccq_narrow_linear_bwd": (_I, [_P, _I64] + [_P] * 6 + [_I64, _I, _I, _P]),
    "ccq_l2norm_fwd": (_I, [_P, _P, _P, _I64, _I, _F, _P]),
    "ccq_l2norm_bwd": (_I, [_P, _P, _P, _P, _P, _I64, _I, _P]),
    "ccq_gdn_decode_prologue": (_I, [_P] * 5 + [_I64] + [_P] * 19 + [_I] * 7 + [_F, _P]),
    "ccq_decode_linear": (_I, [_P, _I64, _P, _P, _I64, _P, _I64, _I, _I, _I, _P, _F, _P]),
    "ccq_decode_linear_glu": (_I, [_P, _I64, _P, _P, _I64, _I, _I, _I, _P, _F, _P]),
    "ccq_decode_linear_split": (_I, [_P, _I64, _P, _P, _I64, _P, _I64, _I, _I, _I, _I, _P, _P]),
    "ccq_decode_linear_split_workspace_bytes": (_SZ, [_I, _I]),
    "ccq_decode_linear_gnorm": (_I, [_P, _I64, _P, _I64, _P, _I, _F, _P, _P, _I64, _P, _I64, _I, _I, _I, _P, _P]),
    "ccq_greedy_embed": (_I, [_P, _I64, _I, _I, _P, _I64, _I, _P, _I64, _P, _I64, _P]),
    "ccq_timing_enable": (_I, [_I]),
    "ccq_timing_reset": (_I, []),
    "ccq_timing_select": (_I, [ctypes.c_char_p]),
    "ccq_timing_read": (_I, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64)]),
}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m ccq_amd.build` "
                "(or __graft_entry__.build()); the CCQ ops have no fallback")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def ptr(t: Optional[torch.Tensor]):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().ccq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


KERNELS = ("conv_fwd", "conv_bwd", "gnorm_fwd", "gnorm_bwd",
           "clean_fwd_sum", "clean_fwd", "clean_bwd_rows", "clean_bwd_dq", "clean_bwd_gsum", "clean_bwd_dk",
           "clean_bwd_gate",
           "gdn_prep", "gdn_fwd_state", "gdn_fwd_o", "gdn_bwd_state", "gdn_bwd_dqkw", "gdn_bwd_wy",
           "gla_intra", "gla_fwd_state", "gla_fwd_o", "gla_bwd_state", "gla_bwd_dv", "gla_bwd_dqk", "gla_bwd_gk",
           "clean_z_fwd", "clean_z_bwd", "narrow_fwd", "narrow_bwd")


def timing_enable(on: bool) -> None:
    call("ccq_timing_enable", int(bool(on)))


def timing_select(kernel) -> None:
    """Record timing events for `kernel` only (None: every kernel)."""
    call("ccq_timing_select", None if kernel is None else kernel.encode())


def timing_reset() -> None:
    call("ccq_timing_reset")


def timing_read(kernel: str):
    """(total milliseconds, launches) recorded for `kernel` since the last reset."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    call("ccq_timing_read", kernel.encode(), ctypes.byref(ms), ctypes.byref(n))
    return ms.value, n.value
