"""CCQ-GLA operators on MI355X: mirror of the reference's ``ccq/ops/ccq_gla`` package
(``chunk_ccq_gla``, ``fused_chunk_ccq_gla``, ``fused_recurrent_ccq_gla``) and of fla's
``chunk_gla`` backbone as the reference calls it, built on the gfx950 kernels of
``libccq_hip.so``.

One autograd function runs the whole path: l2norm of q and k (unconditional in the
reference, ``ccq/ops/ccq_gla/fused_chunk.py:31-32``), the cleaning forward (the cleaned
query stays fp32 in HBM), and the GLA chunk forward on it; the backward runs the GLA
backward, the cleaning backward (which adds the backbone's dk before rounding) and the
l2norm backward.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import call, ptr, stream_of
from ._pad import CHUNK_K, STEP_K, cut_tail, pad_tail, padded_sizes
from .ccq_gdn import _Chunks, _default_scale, _stock_mean
from .clean import as_kernel_dtype, in_dtype
from .clean import _check_qk, _f32, check_device, clean_backward, clean_forward, l2norm_bwd, l2norm_fwd, \
    norm_cu_seqlens, reduce_dlambda, reshape_lambda_3d

__all__ = ["chunk_ccq_gla", "fused_chunk_ccq_gla", "fused_recurrent_ccq_gla", "chunk_gla", "ChunkCCQGLAFunction"]


def _gla_forward(q16, q32, k, v, gk32, s0, ch: _Chunks, scale, want_final):
    B, T, H, K = k.shape
    V = v.shape[-1]
    dev = k.device
    saved = torch.empty(_lib.load().ccq_gla_saved_bytes(B * T, ch.count, H, K, V), device=dev, dtype=torch.uint8)
    o = torch.empty(B, T, H, V, device=dev, dtype=v.dtype)
    sfin = torch.empty(ch.N, H, K, V, device=dev, dtype=torch.float32) if want_final else None
    call("ccq_gla_fwd", ptr(q16), ptr(q32), ptr(k), ptr(v), ptr(gk32), ptr(s0), ptr(ch.cu), ptr(ch.index),
         ptr(ch.offsets), ch.count, ptr(o), ptr(sfin), ptr(saved), B, T, H, K, V, ch.N, float(scale), stream_of(k))
    return o, sfin, saved


def _gla_backward(q16, q32, k, v, gk32, ch: _Chunks, saved, do, dsfin, sfin, scale, want_dgk, want_ds0,
                  dv_f32=False):
    B, T, H, K = k.shape
    V = v.shape[-1]
    dev = k.device
    ws = torch.empty(_lib.load().ccq_gla_bwd_workspace_bytes(B * T, ch.count, H, K, V), device=dev,
                     dtype=torch.uint8)
    dq32 = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
    dk32 = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
    dv = torch.empty(v.shape, device=dev, dtype=torch.float32 if dv_f32 else v.dtype)
    dgk = torch.empty(B, T, H, K, device=dev, dtype=torch.float32) if want_dgk else None
    ds0 = torch.empty(ch.N, H, K, V, device=dev, dtype=torch.float32) if want_ds0 else None
    do = do.contiguous().to(torch.bfloat16)
    if do.data_ptr() % 16:  # read with 16-byte loads: a view at an odd offset gets its own buffer
        do = do.clone()
    dsfin = _f32(dsfin)  # bound to a name: the buffer must outlive the launch
    call("ccq_gla_bwd", ptr(q16), ptr(q32), ptr(k), ptr(v), ptr(gk32), ptr(ch.cu), ptr(ch.index), ptr(ch.offsets),
         ch.count, ptr(saved), ptr(do), ptr(dsfin), ptr(sfin), ptr(ws), ptr(dq32), ptr(dk32), None if dv_f32 else ptr(dv),
         ptr(dv) if dv_f32 else None, ptr(dgk), ptr(ds0), B, T, H, K, V, ch.N, float(scale), stream_of(k))
    return dq32, dk32, dv, dgk, ds0


class ChunkCCQGLAFunction(torch.autograd.Function):
    """l2norm -> CCQ cleaning -> gated linear attention (chunk form), forward and backward on the GPU.

    With ``enable_ccq`` False the cleaning is skipped (the backbone alone, fla's ``chunk_gla``)."""

    @staticmethod
    def forward(ctx, q, k, v, lambda_h, gk, scale, initial_state, initial_cov_state, initial_mean_state,
                output_final_state, use_l2norm, cu_seqlens, position_offset, subtract_mean, enable_ccq, gate_w,
                gate_b):
        _check_qk(q, k)
        if v.dtype != torch.bfloat16 or v.ndim != 4 or v.shape[:3] != q.shape[:3]:
            raise ValueError("v must be bf16 [B, T, H, V] matching q")
        if gk is not None and gk.shape != q.shape:
            raise ValueError(f"gk must have q's shape {tuple(q.shape)} (got {tuple(gk.shape)})")
        check_device(q.device, v=v, lambda_h=lambda_h, gk=gk, initial_state=initial_state,
                     initial_cov_state=initial_cov_state, initial_mean_state=initial_mean_state, gate_w=gate_w,
                     gate_b=gate_b)
        cu_seqlens = norm_cu_seqlens(cu_seqlens, q)
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
        B, T, H, K = q.shape
        ch = _Chunks(B, T, cu_seqlens, q.device)
        rq = rk = None
        qn, kn = q, k
        if use_l2norm:
            qn, rq = l2norm_fwd(q)
            kn, rk = l2norm_fwd(k)
        gk32 = _f32(gk)   # any log decay <= 0: the kernels never form a factor above e^80
        s0 = _f32(initial_state)
        gw, gb = _f32(gate_w), _f32(gate_b)
        h0 = _f32(initial_cov_state)
        m0 = _f32(initial_mean_state) if subtract_mean else None
        hfin = mfin = lam_used = qc32 = csaved = None
        want = bool(output_final_state)
        if enable_ccq:
            lam3 = None if gw is not None else reshape_lambda_3d(lambda_h, q)
            _, qc32, hfin, mfin, lam_used, csaved = clean_forward(qn, kn, lam3, gw, gb, h0, m0, cu_seqlens,
                                                                  position_offset, subtract_mean, want_bf16=False,
                                                                  want_f32=True, want_hfin=want, want_mfin=want)
            o, sfin, saved = _gla_forward(None, qc32, kn, v, gk32, s0, ch, scale, want)
        else:
            o, sfin, saved = _gla_forward(qn, None, kn, v, gk32, s0, ch, scale, want)
        ctx.save_for_backward(q, k, qn, kn, v, gk32, qc32, saved, rq, rk, lam_used, h0, m0, csaved, gw, gb,
                              cu_seqlens, s0, sfin)
        ctx.ch = ch
        ctx.scale = scale
        ctx.use_l2norm = bool(use_l2norm)
        ctx.enable_ccq = bool(enable_ccq)
        ctx.position_offset = int(position_offset)
        ctx.subtract_mean = bool(subtract_mean)
        ctx.lambda_h = lambda_h if isinstance(lambda_h, torch.Tensor) else None
        ctx.gk_dtype = gk.dtype if gk is not None else None
        return o, sfin, hfin, mfin

    @staticmethod
    def backward(ctx, do, dsfin, dhfin, dmfin):
        (q, k, qn, kn, v, gk32, qc32, saved, rq, rk, lam_used, h0, m0, csaved, gw, gb, cu_seqlens, s0,
         sfin) = ctx.saved_tensors
        ch = ctx.ch
        want_dgk = gk32 is not None and ctx.needs_input_grad[4]
        dq32g, dk32g, dv, dgk, ds0 = _gla_backward(
            None if ctx.enable_ccq else qn, qc32, kn, v, gk32, ch, saved, do, dsfin, sfin, ctx.scale, want_dgk,
            s0 is not None)
        dlam = dgw = dgb = dh0 = dm0 = None
        if ctx.enable_ccq:
            want_dlam = ctx.lambda_h is not None and ctx.lambda_h.requires_grad
            dqn, dkn, dlam3, dgw, dgb, dh0, dm0 = clean_backward(
                qn, kn, lam_used, gw, gb, dq32g, dk32g, h0, m0, cu_seqlens, csaved, dhfin, dmfin, ctx.position_offset,
                ctx.subtract_mean, want_dlam=want_dlam, dq_f32=ctx.use_l2norm, dk_f32=ctx.use_l2norm)
            dlam = reduce_dlambda(dlam3, ctx.lambda_h) if dlam3 is not None else None
        else:
            dqn, dkn = dq32g, dk32g
        if ctx.use_l2norm:
            dq = l2norm_bwd(q, rq, dqn)
            dk = l2norm_bwd(k, rk, dkn)
        else:
            dq = dqn.to(q.dtype)
            dk = dkn.to(k.dtype)
        dgk_out = dgk.to(ctx.gk_dtype) if dgk is not None else None
        return (dq, dk, dv, dlam, dgk_out, None, ds0, dh0, dm0, None, None, None, None, None, None, dgw, dgb)


def fused_chunk_ccq_gla(q, k, v, lambda_h, g=None, scale=None, initial_state=None, initial_cov_state=None,
                        initial_mean_state=None, output_final_state=False, cu_seqlens=None, position_offset=0,
                        subtract_mean=True, gate_w=None, gate_b=None):
    """CCQ-GLA, fused path (reference ``ccq/ops/ccq_gla/fused_chunk.py:16-46``): l2norm, cleaning, then
    the GLA chunk recurrence with per-channel log decay ``g`` ``[B, T, H, K]``.

    Returns ``(o, final_state, final_cov_state, final_mean_state)``; the last three are None unless
    ``output_final_state``.  ``gate_w``/``gate_b`` (optional) select the fused per-head gate.
    """
    dt = q.dtype
    q, k, v = as_kernel_dtype(q, k, v)
    K, V = q.shape[-1], v.shape[-1]
    scale = _default_scale(scale, K)
    # head sizes between the kernels' run zero-padded (ccq_amd/_pad.py)
    Kp, Vp = padded_sizes(K, V, CHUNK_K)
    if (Kp, Vp) != (K, V):
        q, k, v, g = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(v, Vp), pad_tail(g, Kp)
        initial_state = pad_tail(initial_state, Kp, Vp)
        initial_cov_state = pad_tail(initial_cov_state, Kp, Kp)
        initial_mean_state = pad_tail(initial_mean_state, Kp)
        gate_w = pad_tail(gate_w, Kp)
    o, sfin, hfin, mfin = ChunkCCQGLAFunction.apply(
        q, k, v, lambda_h, g, scale, initial_state, initial_cov_state,
        initial_mean_state if subtract_mean else None, bool(output_final_state), True, cu_seqlens,
        int(position_offset), bool(subtract_mean), True, gate_w, gate_b)
    o = in_dtype(cut_tail(o, V), dt)
    if not output_final_state:
        return o, None, None, None
    return o, cut_tail(sfin, K, V), cut_tail(hfin, K, K), cut_tail(mfin, K)


def chunk_ccq_gla(q, k, v, lambda_h, g=None, scale=None, initial_state=None, initial_cov_state=None,
                  initial_mean_state=None, output_final_state=False, cu_seqlens=None, position_offset=0,
                  subtract_mean=True):
    """CCQ-GLA, stock ``chunk`` mode (reference ``ccq/ops/ccq_gla/chunk.py:17-59``).  Same mathematics as
    ``fused_chunk_ccq_gla`` (z-read, cleaning, backbone); computed by the same kernels, with the stock
    path's key-sum gradients (``_stock_mean``: the reference cleans through ``_CCQCleanQ`` here)."""
    o, s, c, m = fused_chunk_ccq_gla(q, k, v, lambda_h, g, scale, initial_state, initial_cov_state,
                                     _stock_mean(initial_mean_state), output_final_state, cu_seqlens, position_offset,
                                     subtract_mean)
    return o, s, c, _stock_mean(m)


def fused_recurrent_ccq_gla(q, k, v, lambda_h, gk=None, gv=None, scale=None, initial_state=None,
                            initial_cov_state=None, initial_mean_state=None, output_final_state=False,
                            reverse=False, cu_seqlens=None, position_offset=0, subtract_mean=True):
    """CCQ-GLA, recurrent mode (reference ``ccq/ops/ccq_gla/fused_recurrent.py:9-51``), used for
    decode and (in the reference layer, also in training) for sequences of at most 64 tokens.
    ``gk`` / ``gv`` decay the backbone state's rows / columns; ``reverse`` runs the backbone
    recurrence from the last token to the first (the cleaning runs forwards, as in the reference).
    Without autograd it runs the decode kernels; when a gradient is needed it runs the chunk
    kernels (same recurrence, with a backward): with ``reverse``, the cleaning followed by the GLA
    backbone on the time-reversed sequences, with the reference's key-sum gradients for this path
    (``_stock_mean``).  Gradients with ``gv`` are not supported."""
    from .decode import gla_decode, needs_grad
    if not needs_grad(q, k, v, lambda_h, gk, gv, initial_state, initial_cov_state, initial_mean_state):
        dt = q.dtype
        q, k, v = as_kernel_dtype(q, k, v)
        K, V = q.shape[-1], v.shape[-1]
        scale = _default_scale(scale, K)
        s0, cov0, m0 = initial_state, initial_cov_state, initial_mean_state if subtract_mean else None
        Kp, Vp = padded_sizes(K, V, STEP_K)
        if (Kp, Vp) != (K, V):
            q, k, v, gk, gv = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(v, Vp), pad_tail(gk, Kp), pad_tail(gv, Vp)
            s0, cov0, m0 = pad_tail(s0, Kp, Vp), pad_tail(cov0, Kp, Kp), pad_tail(m0, Kp)
        o, s, c, m = gla_decode(q, k, v, lambda_h, gk, scale, s0, cov0, m0, bool(output_final_state), cu_seqlens,
                                position_offset, subtract_mean, gv=gv, reverse=bool(reverse))
        o = in_dtype(cut_tail(o, V), dt)
        if not output_final_state:
            return o, None, None, None
        return o, cut_tail(s, K, V), cut_tail(c, K, K), cut_tail(m, K)
    if gv is not None:
        raise NotImplementedError("fused_recurrent_ccq_gla: gradients through the per-value decay gv are not "
                                  "supported (inference with gv runs on the decode kernels)")
    if reverse:
        return _reverse_gla(q, k, v, lambda_h, gk, scale, initial_state, initial_cov_state, initial_mean_state,
                            output_final_state, cu_seqlens, position_offset, subtract_mean)
    return chunk_ccq_gla(q, k, v, lambda_h, gk, scale, initial_state, initial_cov_state, initial_mean_state,
                         output_final_state, cu_seqlens, position_offset, subtract_mean)


def _time_flip(x):
    """Each sequence reversed in time: dense [B, T, ...] along T; a packed batch [1, total, ...]
    along its whole length, which also reverses the order of its sequences."""
    return None if x is None else x.flip(1)


def _reverse_gla(q, k, v, lambda_h, gk, scale, initial_state, initial_cov_state, initial_mean_state,
                 output_final_state, cu_seqlens, position_offset, subtract_mean):
    """Differentiable CCQ-GLA with the backbone run backwards in time: the forward cleaning
    (l2norm, covariance read, cleaning), then the GLA backbone on the time-reversed cleaned
    queries, keys, values and decays, whose outputs are reversed back.  Reversing a packed batch
    also reverses the order of its sequences: the cu_seqlens of the reversed batch are the mirrored
    offsets, and the backbone's initial / final states are taken and returned in the reversed
    order."""
    from .clean import fused_ccq_clean_read
    from .l2norm import l2norm
    qn, kn = l2norm(q), l2norm(k)
    qc, hf, mf = fused_ccq_clean_read(qn, kn, lambda_h, position_offset=position_offset,
                                      initial_cov_state=initial_cov_state,
                                      initial_mean_state=_stock_mean(initial_mean_state) if subtract_mean else None,
                                      output_final_state=output_final_state, subtract_mean=subtract_mean,
                                      cu_seqlens=cu_seqlens)
    cu_r, s0 = None, initial_state
    if cu_seqlens is not None:
        cu_r = (cu_seqlens[-1] - cu_seqlens.flip(0)).contiguous()
        if s0 is not None:
            s0 = s0.flip(0)
    o_r, s = chunk_gla(_time_flip(qc), _time_flip(kn), _time_flip(v), _time_flip(gk), scale=scale, initial_state=s0,
                       output_final_state=output_final_state, cu_seqlens=cu_r)
    o = o_r.flip(1)
    if not output_final_state:
        return o, None, None, None
    if cu_seqlens is not None:
        s = s.flip(0)
    return o, s, hf, _stock_mean(mf)


def chunk_gla(q, k, v, g=None, scale=None, initial_state=None, output_final_state=False, cu_seqlens=None, **kwargs):
    """The GLA backbone alone (fla's ``chunk_gla`` signature as the reference calls it,
    ``ccq/ops/ccq_gla/fused_chunk.py:42-45``).  q, k, v bf16, fp16 or fp32 (computed on bf16
    operands, returned in the input dtype); g the per-channel log decay."""
    if kwargs:
        unknown = ", ".join(sorted(kwargs))
        raise TypeError(f"chunk_gla: unsupported keyword arguments: {unknown}")
    dt = q.dtype
    q, k, v = as_kernel_dtype(q, k, v)
    K, V = q.shape[-1], v.shape[-1]
    scale = _default_scale(scale, K)
    Kp, Vp = padded_sizes(K, V, CHUNK_K)
    if (Kp, Vp) != (K, V):
        q, k, v, g = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(v, Vp), pad_tail(g, Kp)
        initial_state = pad_tail(initial_state, Kp, Vp)
    o, sfin, _, _ = ChunkCCQGLAFunction.apply(
        q, k, v, None, g, scale, initial_state, None, None, bool(output_final_state),
        False, cu_seqlens, 0, True, False, None, None)
    return in_dtype(cut_tail(o, V), dt), (cut_tail(sfin, K, V) if output_final_state else None)
