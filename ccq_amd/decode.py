"""Recurrent (decode) step of CCQ-GDN and CCQ-GLA: a few tokens per sequence against the cached
states (S, C = sum k k^T, m = sum k), on the gfx950 decode kernels (``ccq_gdn_decode`` /
``ccq_gla_decode`` of ``libccq_hip.so``).  Inference only: the ``fused_recurrent_*`` operators
route calls that need gradients through the chunk kernels instead.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import call, ptr, stream_of
from .clean import _check_qk, _f32, check_device, norm_cu_seqlens, reshape_lambda_3d, seq_count

__all__ = ["gdn_decode", "gla_decode", "needs_grad"]


def needs_grad(*xs) -> bool:
    """True when autograd would record a graph through any of the tensors."""
    return torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in xs)


def _prep(q, k, v, lambda_h, gate_w, gate_b, cu_seqlens, enable_ccq, **others):
    _check_qk(q, k)
    if v.dtype != torch.bfloat16 or v.ndim != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError("v must be bf16 [B, T, H, V] matching q")
    check_device(q.device, v=v, lambda_h=lambda_h, gate_w=gate_w, gate_b=gate_b, **others)
    cu_seqlens = norm_cu_seqlens(cu_seqlens, q)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    gw, gb = _f32(gate_w), _f32(gate_b)
    lam = None
    if enable_ccq and gw is None:
        lam = reshape_lambda_3d(lambda_h, q)
    B, T, H, K = q.shape
    N = seq_count(B, cu_seqlens)
    ws = torch.empty(_lib.load().ccq_decode_workspace_bytes(B * T, H, K), device=q.device, dtype=torch.uint8)
    return q, k, v, lam, gw, gb, N, ws, cu_seqlens


def _states(N, H, K, V, dev, want, enable_ccq, subtract_mean):
    S = torch.empty(N, H, K, V, device=dev, dtype=torch.float32) if want else None
    C = torch.empty(N, H, K, K, device=dev, dtype=torch.float32) if (want and enable_ccq) else None
    m = torch.empty(N, H, K, device=dev, dtype=torch.float32) if (want and enable_ccq and subtract_mean) else None
    return S, C, m


def gdn_decode(q, k, v, lambda_h, g, beta, scale, initial_state=None, initial_cov_state=None,
               initial_mean_state=None, output_final_state=True, use_l2norm=True, cu_seqlens=None,
               position_offset=0, subtract_mean=True, enable_ccq=True, gate_w=None, gate_b=None, gk=None, gv=None):
    """One recurrent CCQ-GDN call; ``gk`` ``[B, T, H, K]`` / ``gv`` ``[B, T, H, V]`` optionally decay
    the state's rows / columns besides the scalar ``g``.  Returns ``(o, S, C, m)`` (states None
    unless requested)."""
    q, k, v, lam, gw, gb, N, ws, cu_seqlens = _prep(
        q, k, v, lambda_h, gate_w, gate_b, cu_seqlens, enable_ccq, g=g, beta=beta, gk=gk, gv=gv,
        initial_state=initial_state, initial_cov_state=initial_cov_state, initial_mean_state=initial_mean_state)
    if gk is not None and gk.shape != q.shape:
        raise ValueError(f"gk must have q's shape {tuple(q.shape)} (got {tuple(gk.shape)})")
    if gv is not None and gv.shape != v.shape:
        raise ValueError(f"gv must have v's shape {tuple(v.shape)} (got {tuple(gv.shape)})")
    B, T, H, K = q.shape
    V = v.shape[-1]
    if beta is None:
        beta = torch.ones(B, T, H, device=q.device, dtype=torch.float32)
    o = torch.empty(B, T, H, V, device=q.device, dtype=v.dtype)
    S, C, m = _states(N, H, K, V, q.device, output_final_state, enable_ccq, subtract_mean)
    # every converted copy is bound to a name so that its buffer outlives the launch
    g32, b32, gk32, gv32, s0, c0, m0 = (_f32(x) for x in (g, beta, gk, gv, initial_state, initial_cov_state,
                                                           initial_mean_state))
    call("ccq_gdn_decode", ptr(q), ptr(k), ptr(v), ptr(lam), ptr(gw), ptr(gb), ptr(g32), ptr(b32), ptr(gk32),
         ptr(gv32), ptr(s0), ptr(c0), ptr(m0), ptr(cu_seqlens),
         ptr(o), ptr(S), ptr(C), ptr(m), ptr(ws), B, T, H, K, V, N, int(position_offset), int(bool(subtract_mean)),
         int(bool(use_l2norm)), int(bool(enable_ccq)), float(scale), stream_of(q))
    return o, S, C, m


def gla_decode(q, k, v, lambda_h, gk, scale, initial_state=None, initial_cov_state=None, initial_mean_state=None,
               output_final_state=True, cu_seqlens=None, position_offset=0, subtract_mean=True, gate_w=None,
               gate_b=None, gv=None, reverse=False):
    """One recurrent CCQ-GLA call (l2norm of q and k always on, as the reference).  ``gk`` / ``gv``:
    log decays of the state's rows ``[B, T, H, K]`` and columns ``[B, T, H, V]``; ``reverse`` runs
    the backbone recurrence from the last token to the first.  Returns ``(o, S, C, m)``."""
    q, k, v, lam, gw, gb, N, ws, cu_seqlens = _prep(
        q, k, v, lambda_h, gate_w, gate_b, cu_seqlens, True, gk=gk, gv=gv, initial_state=initial_state,
        initial_cov_state=initial_cov_state, initial_mean_state=initial_mean_state)
    B, T, H, K = q.shape
    V = v.shape[-1]
    if gk is not None and gk.shape != q.shape:
        raise ValueError(f"gk must have q's shape {tuple(q.shape)} (got {tuple(gk.shape)})")
    if gv is not None and gv.shape != v.shape:
        raise ValueError(f"gv must have v's shape {tuple(v.shape)} (got {tuple(gv.shape)})")
    o = torch.empty(B, T, H, V, device=q.device, dtype=v.dtype)
    S, C, m = _states(N, H, K, V, q.device, output_final_state, True, subtract_mean)
    gk32, gv32, s0, c0, m0 = (_f32(x) for x in (gk, gv, initial_state, initial_cov_state, initial_mean_state))
    call("ccq_gla_decode", ptr(q), ptr(k), ptr(v), ptr(lam), ptr(gw), ptr(gb), ptr(gk32), ptr(gv32),
         ptr(s0), ptr(c0), ptr(m0), ptr(cu_seqlens),
         ptr(o), ptr(S), ptr(C), ptr(m), ptr(ws), B, T, H, K, V, N, int(position_offset), int(bool(subtract_mean)),
         1, int(bool(reverse)), float(scale), stream_of(q))
    return o, S, C, m
