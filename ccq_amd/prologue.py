"""The layers' prologue and epilogue on the GPU: the short causal convolution (+ SiLU, + the per-head
L2 normalisation of q and k) and the gated RMSNorm of the output, as single HIP passes
(``ccq_conv_fwd`` / ``ccq_conv_bwd``, ``ccq_gated_rmsnorm_fwd`` / ``_bwd`` of ``libccq_hip.so``).

The reference layers run projection -> fla ``ShortConvolution`` (SiLU) -> the operators' l2norm
(``ccq/gdn/layer.py:266-296``, ``ccq/ops/ccq_gdn/fused_chunk.py:43-44``) and fla
``FusedRMSNormGated`` (``ccq/gdn/layer.py:402-404``).  Here one pass over the projected q reads it
once and writes both the activation (for the lambda gate) and its per-head normalised copy (for
the operator, which then skips its own l2norm); k needs only the normalised copy.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import call, ptr, stream_of
from .clean import check_device

__all__ = ["short_conv", "gated_rmsnorm", "narrow_linear", "narrow_ok"]


def last_inputs(cache: Optional[torch.Tensor], W: int) -> Optional[torch.Tensor]:
    """A convolution cache as this library keeps it, ``[N, D, W-1]`` (each sequence's previous W-1
    inputs, oldest first).  A cache of width W -- the last W inputs, the form fla's ShortConvolution is
    understood to keep (not pinned: fla is not available here) -- is accepted and its last W-1 columns
    used; other widths raise."""
    if cache is None:
        return None
    if cache.shape[-1] == W:
        return cache[..., 1:]
    if cache.shape[-1] != W - 1:
        raise ValueError(f"convolution cache of width {cache.shape[-1]} for a kernel of {W} taps "
                         f"(expected {W - 1}, or {W})")
    return cache


def _seqs(x: torch.Tensor, cu_seqlens: Optional[torch.Tensor]):
    B, T = x.shape[:2]
    if cu_seqlens is None:
        return B, T, B, None
    if B != 1:
        raise ValueError("varlen inputs (cu_seqlens) need batch size 1")
    cu = cu_seqlens.to(device=x.device, dtype=torch.int64).contiguous()
    return 1, T, cu.numel() - 1, cu


class ShortConvFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, cache, cu_seqlens, activation, head_dim, want_y, want_norm,
                output_final_state, eps):
        if x.dtype != torch.bfloat16 or not x.is_cuda:
            raise TypeError("short_conv runs on bf16 CUDA activations")
        x = x.contiguous()
        B, T, N, cu = _seqs(x, cu_seqlens)
        D = x.shape[-1]
        W = weight.shape[-1]
        w32 = weight.detach().float().reshape(D, W).contiguous()
        b32 = bias.detach().float().contiguous() if bias is not None else None
        c32 = cache.detach().float().contiguous() if cache is not None else None
        y = torch.empty_like(x) if want_y else None
        yn = torch.empty_like(x) if want_norm else None
        rstd = torch.empty(B * T, D // head_dim, device=x.device, dtype=torch.float32) if want_norm else None
        cout = torch.empty(N, D, W - 1, device=x.device, dtype=torch.float32) if (output_final_state and W > 1) else None
        call("ccq_conv_fwd", ptr(x), ptr(w32), ptr(b32), ptr(c32), ptr(cu), ptr(y), ptr(yn), ptr(rstd), ptr(cout),
             B, T, N, D, W, int(head_dim if want_norm else 0), int(activation), float(eps), stream_of(x))
        ctx.save_for_backward(x, w32, b32, c32, cu, rstd)
        ctx.meta = (B, T, N, D, W, head_dim, activation, weight.shape, weight.dtype,
                    None if bias is None else bias.dtype)
        if cout is not None and cache is not None:
            cout = cout.to(cache.dtype)
        elif cout is not None:
            cout = cout.to(x.dtype)
        return y, yn, cout

    @staticmethod
    def backward(ctx, dy, dyn, dcache):
        x, w32, b32, c32, cu, rstd = ctx.saved_tensors
        B, T, N, D, W, head_dim, activation, wshape, wdtype, bdtype = ctx.meta
        dx = torch.empty_like(x)
        dw = torch.empty(D, W, device=x.device, dtype=torch.float32)
        db = torch.empty(D, device=x.device, dtype=torch.float32) if b32 is not None else None
        ws = torch.empty(_lib.load().ccq_conv_bwd_workspace_bytes(B * T, D, W), device=x.device, dtype=torch.uint8)
        d16 = dy.to(torch.bfloat16).contiguous() if dy is not None else None
        n16 = dyn.to(torch.bfloat16).contiguous() if dyn is not None else None
        call("ccq_conv_bwd", ptr(x), ptr(w32), ptr(b32), ptr(c32), ptr(cu), ptr(d16), ptr(n16), ptr(rstd), ptr(dx),
             ptr(dw), ptr(db), ptr(ws), B, T, N, D, W, int(head_dim if n16 is not None else 0), int(activation),
             stream_of(x))
        dwo = dw.view(wshape).to(wdtype)
        dbo = db.to(bdtype) if db is not None else None
        return dx, dwo, dbo, None, None, None, None, None, None, None, None


def short_conv(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
               cache: Optional[torch.Tensor] = None, cu_seqlens: Optional[torch.Tensor] = None,
               activation: bool = True, head_dim: Optional[int] = None, want_y: bool = True,
               output_final_state: bool = False, eps: float = 1e-6):
    """Causal depthwise convolution over time of ``x [B, T, D]`` (bf16, CUDA) with ``weight``
    ``[D, 1, W]`` (or ``[D, W]``), optional ``bias [D]``, SiLU when ``activation``; ``cache``
    ``[N, D, W-1]`` holds each sequence's previous W-1 inputs (``[N, D, W]`` is accepted:
    ``last_inputs``); the returned cache is ``[N, D, W-1]``.  With ``head_dim`` it also returns the
    per-head L2-normalised output.  Returns ``(y, y_norm, final_cache)`` (None where not asked)."""
    check_device(x.device, weight=weight, bias=bias, cache=cache)
    cache = last_inputs(cache, weight.shape[-1])
    want_norm = head_dim is not None
    return ShortConvFunction.apply(x, weight, bias, cache, cu_seqlens, bool(activation),
                                   int(head_dim) if want_norm else 8, bool(want_y), want_norm,
                                   bool(output_final_state), float(eps))


class GatedRMSNormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, g, weight, eps):
        if x.dtype != torch.bfloat16 or g.dtype != torch.bfloat16 or not x.is_cuda:
            raise TypeError("gated_rmsnorm runs on bf16 CUDA activations")
        dv = x.shape[-1]
        x2, g2 = x.contiguous().view(-1, dv), g.contiguous().view(-1, dv)
        w32 = weight.detach().float().contiguous() if weight is not None else None
        y = torch.empty_like(x2)
        rstd = torch.empty(x2.shape[0], device=x.device, dtype=torch.float32)
        call("ccq_gated_rmsnorm_fwd", ptr(x2), ptr(g2), ptr(w32), ptr(y), ptr(rstd), x2.shape[0], dv, float(eps),
             stream_of(x))
        ctx.save_for_backward(x2, g2, w32, rstd)
        ctx.meta = (x.shape, None if weight is None else weight.dtype)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        x2, g2, w32, rstd = ctx.saved_tensors
        shape, wdtype = ctx.meta
        dv = x2.shape[-1]
        d2 = dy.to(torch.bfloat16).contiguous().view(-1, dv)
        dx, dg = torch.empty_like(x2), torch.empty_like(g2)
        dw = torch.empty(dv, device=x2.device, dtype=torch.float32) if w32 is not None else None
        ws = None
        if dw is not None:
            ws = torch.empty(_lib.load().ccq_gated_rmsnorm_bwd_workspace_bytes(x2.shape[0], dv), device=x2.device,
                             dtype=torch.uint8)
        call("ccq_gated_rmsnorm_bwd", ptr(x2), ptr(g2), ptr(w32), ptr(rstd), ptr(d2), ptr(dx), ptr(dg), ptr(dw),
             ptr(ws), x2.shape[0], dv, stream_of(x2))
        return dx.view(shape), dg.view(shape), (dw.to(wdtype) if dw is not None else None), None


def gated_rmsnorm(x: torch.Tensor, g: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-5):
    """``x / sqrt(mean(x^2) + eps) * weight * silu(g)`` over the last dimension (bf16, CUDA,
    <= 512 wide)."""
    check_device(x.device, g=g, weight=weight)
    return GatedRMSNormFunction.apply(x, g, weight, float(eps))


class NarrowLinearFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias):
        K, N = x.shape[-1], weight.shape[0]
        x2 = x.reshape(-1, K)
        if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        w16 = weight.detach().to(torch.bfloat16).contiguous()
        b32 = bias.detach().float().contiguous() if bias is not None else None
        y = torch.empty(x2.shape[0], N, device=x.device, dtype=torch.bfloat16)
        call("ccq_narrow_linear_fwd", ptr(x2), x2.stride(0), ptr(w16), ptr(b32), ptr(y), x2.shape[0], K, N,
             stream_of(x))
        ctx.save_for_backward(x2, w16)
        ctx.meta = (x.shape, weight.dtype, None if bias is None else bias.dtype)
        return y.view(*x.shape[:-1], N)

    @staticmethod
    def backward(ctx, dy):
        x2, w16 = ctx.saved_tensors
        shape, wdtype, bdtype = ctx.meta
        M, K = x2.shape
        N = w16.shape[0]
        d2 = dy.to(torch.bfloat16).reshape(M, N).contiguous()
        dx = torch.empty(M, K, device=x2.device, dtype=torch.bfloat16) if ctx.needs_input_grad[0] else None
        dw = torch.empty(N, K, device=x2.device, dtype=torch.float32)
        db = torch.empty(N, device=x2.device, dtype=torch.float32) if bdtype is not None else None
        ws = torch.empty(_lib.load().ccq_narrow_linear_bwd_workspace_bytes(M, K, N), device=x2.device,
                         dtype=torch.uint8)
        call("ccq_narrow_linear_bwd", ptr(x2), x2.stride(0), ptr(w16), ptr(d2), ptr(dx), ptr(dw), ptr(db), ptr(ws),
             M, K, N, stream_of(x2))
        return (dx.view(shape) if dx is not None else None, dw.to(wdtype),
                db.to(bdtype) if db is not None else None)


def narrow_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``narrow_linear`` takes this call: bf16 activations and weights on the GPU, at most 16
    outputs, an input width that is a multiple of 32 in [32, 2016]."""
    K = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and weight.dim() == 2
            and weight.shape[0] <= 16 and weight.shape[1] == K and K % 32 == 0 and 32 <= K <= 2016)


def narrow_linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x @ weight.T + bias`` for a weight of at most 16 rows (bf16, CUDA; fp32 accumulation, one
    bf16 rounding, as a bf16 GEMM): one MFMA pass over x forward, one pass over x and dy backward
    (``ccq_narrow_linear_fwd`` / ``_bwd``).  See ``narrow_ok`` for the shapes it takes."""
    if not narrow_ok(x, weight):
        raise ValueError(f"narrow_linear: x {tuple(x.shape)} {x.dtype} on {x.device}, weight "
                         f"{tuple(weight.shape)} {weight.dtype}: needs bf16 on the GPU, <= 16 outputs and an input "
                         f"width that is a multiple of 32 in [32, 2016]")
    check_device(x.device, weight=weight, bias=bias)
    return NarrowLinearFunction.apply(x, weight, bias)
