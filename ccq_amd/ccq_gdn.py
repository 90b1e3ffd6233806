"""CCQ-GDN operators on MI355X: mirror of the reference's ``ccq/ops/ccq_gdn``
package (``chunk_ccq_gdn``, ``fused_chunk_ccq_gdn``, ``fused_recurrent_ccq_gdn``,
``fused_ccq_clean``), built on the gfx950 kernels of ``libccq_hip.so``.

One autograd function runs the whole path: optional l2norm of q and k, the
cleaning forward (the cleaned query stays fp32 in HBM), the gated-delta-rule
chunk forward on it; the backward runs the gated-delta-rule backward, then the
cleaning backward (which adds the backbone's dk before rounding), then the
l2norm backward.  The stock ``chunk`` mode and the ``fused_chunk`` mode of the
reference compute the same mathematics and share this implementation.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._lib import call, ptr, stream_of
from ._pad import CHUNK_K, STEP_K, cut_tail, pad_tail, padded_sizes
from .clean import as_kernel_dtype, in_dtype
from .clean import (_check_qk, _f32, check_device, clean_backward, clean_forward, l2norm_bwd, l2norm_fwd,
                    norm_cu_seqlens, reduce_dlambda, reshape_lambda_3d, seq_count)

__all__ = ["chunk_ccq_gdn", "fused_chunk_ccq_gdn", "fused_recurrent_ccq_gdn", "fused_ccq_clean",
           "chunk_gated_delta_rule", "ChunkCCQGDNFunction"]

BT = 64


class _Chunks:
    """Chunk bookkeeping for dense or varlen inputs."""

    def __init__(self, B: int, T: int, cu_seqlens: Optional[torch.Tensor], device):
        self.cu = cu_seqlens
        if cu_seqlens is None:
            self.N = B
            self.count = B * ((T + BT - 1) // BT)
            self.index = None
            self.offsets = None
        else:
            self.N = cu_seqlens.numel() - 1
            cap = (B * T) // BT + self.N + 1
            self.count = cap
            self.index = torch.empty(cap, 2, device=device, dtype=torch.int32)
            self.offsets = torch.empty(self.N + 1, device=device, dtype=torch.int32)
            call("ccq_chunk_index", ptr(cu_seqlens), self.N, ptr(self.offsets), ptr(self.index), cap,
                 stream_of(cu_seqlens))


def _gdn_forward(q16, q32, k, v, g32, beta32, s0, ch: _Chunks, scale, want_final):
    B, T, H, K = k.shape
    V = v.shape[-1]
    dev = k.device
    saved = torch.empty(_lib.load().ccq_gdn_saved_bytes(B * T, ch.count, H, K, V), device=dev, dtype=torch.uint8)
    o = torch.empty(B, T, H, V, device=dev, dtype=v.dtype)
    sfin = torch.empty(ch.N, H, K, V, device=dev, dtype=torch.float32) if want_final else None
    call("ccq_gdn_fwd", ptr(q16), ptr(q32), ptr(k), ptr(v), ptr(g32), ptr(beta32), ptr(s0), ptr(ch.cu),
         ptr(ch.index), ptr(ch.offsets), ch.count, ptr(o), ptr(sfin), ptr(saved), B, T, H, K, V, ch.N, float(scale),
         stream_of(k))
    return o, sfin, saved


def _gdn_backward(q16, q32, k, v, g32, beta32, ch: _Chunks, saved, do, dsfin, scale, want_ds0):
    B, T, H, K = k.shape
    V = v.shape[-1]
    dev = k.device
    ws = torch.empty(_lib.load().ccq_gdn_bwd_workspace_bytes(B * T, ch.count, H, K, V), device=dev,
                     dtype=torch.uint8)
    dq32 = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
    dk32 = torch.empty(B, T, H, K, device=dev, dtype=torch.float32)
    dv = torch.empty_like(v)
    dbeta = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    dg = torch.empty(B, T, H, device=dev, dtype=torch.float32)
    ds0 = torch.empty(ch.N, H, K, V, device=dev, dtype=torch.float32) if want_ds0 else None
    do = do.contiguous().to(torch.bfloat16)
    if do.data_ptr() % 16:  # read with 16-byte loads: a view at an odd offset gets its own buffer
        do = do.clone()
    dsfin = _f32(dsfin)  # bound to a name: the buffer must outlive the launch
    call("ccq_gdn_bwd", ptr(q16), ptr(q32), ptr(k), ptr(v), ptr(g32), ptr(beta32), ptr(ch.cu), ptr(ch.index),
         ptr(ch.offsets), ch.count, ptr(saved), ptr(do), ptr(dsfin), ptr(ws), ptr(dq32), ptr(dk32), ptr(dv),
         ptr(dbeta), ptr(dg), ptr(ds0), B, T, H, K, V, ch.N, float(scale), stream_of(k))
    return dq32, dk32, dv, dbeta, dg, ds0


class ChunkCCQGDNFunction(torch.autograd.Function):
    """l2norm -> CCQ cleaning -> gated delta rule (chunk form), forward and backward on the GPU."""

    @staticmethod
    def forward(ctx, q, k, v, lambda_h, g, beta, scale, initial_state, initial_cov_state, initial_mean_state,
                output_final_state, use_l2norm, cu_seqlens, position_offset, subtract_mean, enable_ccq, gate_w,
                gate_b):
        _check_qk(q, k)
        if v.dtype != torch.bfloat16 or v.ndim != 4 or v.shape[:3] != q.shape[:3]:
            raise ValueError("v must be bf16 [B, T, H, V] matching q")
        check_device(q.device, v=v, lambda_h=lambda_h, g=g, beta=beta, initial_state=initial_state,
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
        g32 = _f32(g)
        beta32 = _f32(beta)
        s0 = _f32(initial_state)
        gw, gb = _f32(gate_w), _f32(gate_b)
        h0 = _f32(initial_cov_state)
        m0 = _f32(initial_mean_state) if subtract_mean else None
        hfin = mfin = None
        lam_used = None
        if enable_ccq:
            lam3 = None if gw is not None else reshape_lambda_3d(lambda_h, q)
            want = bool(output_final_state)
            _, qc32, hfin, mfin, lam_used, csaved = clean_forward(qn, kn, lam3, gw, gb, h0, m0, cu_seqlens,
                                                                  position_offset, subtract_mean, want_bf16=False,
                                                                  want_f32=True, want_hfin=want, want_mfin=want)
            o, sfin, saved = _gdn_forward(None, qc32, kn, v, g32, beta32, s0, ch, scale, bool(output_final_state))
        else:
            qc32 = csaved = None
            o, sfin, saved = _gdn_forward(qn, None, kn, v, g32, beta32, s0, ch, scale, bool(output_final_state))
        ctx.save_for_backward(q, k, qn, kn, v, g32, beta32, qc32, saved, rq, rk, lam_used, h0, m0, csaved, gw, gb,
                              cu_seqlens, s0)
        ctx.ch = ch
        ctx.scale = scale
        ctx.use_l2norm = bool(use_l2norm)
        ctx.enable_ccq = bool(enable_ccq)
        ctx.position_offset = int(position_offset)
        ctx.subtract_mean = bool(subtract_mean)
        ctx.lambda_h = lambda_h if isinstance(lambda_h, torch.Tensor) else None
        ctx.g_dtype = g.dtype if g is not None else None
        ctx.beta_dtype = beta.dtype
        ctx.has_g = g is not None
        return o, sfin, hfin, mfin

    @staticmethod
    def backward(ctx, do, dsfin, dhfin, dmfin):
        (q, k, qn, kn, v, g32, beta32, qc32, saved, rq, rk, lam_used, h0, m0, csaved, gw, gb, cu_seqlens,
         s0) = ctx.saved_tensors
        ch = ctx.ch
        dq32g, dk32g, dv, dbeta, dg, ds0 = _gdn_backward(
            None if ctx.enable_ccq else qn, qc32, kn, v, g32, beta32, ch, saved, do, dsfin, ctx.scale,
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
        dg_out = dg.to(ctx.g_dtype) if ctx.has_g else None
        return (dq, dk, dv, dlam, dg_out, dbeta.to(ctx.beta_dtype), None, ds0, dh0, dm0, None, None, None, None,
                None, None, dgw, dgb)


def _stock_mean(x):
    """Key-sum gradients of the reference's stock cleaning path: ``chunk`` mode, the recurrent ops and
    ``fused_ccq_clean`` clean through ``_CCQCleanQ`` (``ccq/ops/common/clean.py:691-748``), whose
    backward returns no gradient for the initial key sum and ignores the one arriving at the final key
    sum.  Detaching the initial key sum going in and the final one coming out of the fused operator
    gives those gradients; the covariance states keep theirs (the reference reads z through fla's
    GLA kernels, which differentiate the initial and the final covariance state)."""
    return None if x is None else x.detach()


def _default_scale(scale, K):
    return K ** -0.5 if scale is None else float(scale)


def fused_chunk_ccq_gdn(q, k, v, lambda_h, g, beta, scale=None, initial_state=None, initial_cov_state=None,
                        initial_mean_state=None, output_final_state=False, use_qk_l2norm_in_kernel=False,
                        cu_seqlens=None, position_offset=0, subtract_mean=True, enable_ccq=True, gate_w=None,
                        gate_b=None, **kwargs):
    """CCQ-GDN, fused path (reference ``ccq/ops/ccq_gdn/fused_chunk.py:16-59``).

    Returns ``(o, final_state, final_cov_state, final_mean_state)``; the last three are None unless
    ``output_final_state`` (the CCQ states are None when ``enable_ccq`` is False).
    ``gate_w``/``gate_b`` (optional) select the fused per-head gate instead of ``lambda_h``.
    """
    if kwargs:
        unknown = ", ".join(sorted(kwargs))
        raise TypeError(f"fused_chunk_ccq_gdn: unsupported keyword arguments: {unknown}")
    dt = q.dtype
    q, k, v = as_kernel_dtype(q, k, v)
    K, V = q.shape[-1], v.shape[-1]
    scale = _default_scale(scale, K)
    # head sizes between the kernels' run zero-padded (ccq_amd/_pad.py)
    Kp, Vp = padded_sizes(K, V, CHUNK_K)
    if (Kp, Vp) != (K, V):
        q, k, v = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(v, Vp)
        initial_state = pad_tail(initial_state, Kp, Vp)
        initial_cov_state = pad_tail(initial_cov_state, Kp, Kp)
        initial_mean_state = pad_tail(initial_mean_state, Kp)
        gate_w = pad_tail(gate_w, Kp)
    o, sfin, hfin, mfin = ChunkCCQGDNFunction.apply(
        q, k, v, lambda_h, g, beta, scale, initial_state, initial_cov_state,
        initial_mean_state if subtract_mean else None, bool(output_final_state), bool(use_qk_l2norm_in_kernel),
        cu_seqlens, int(position_offset), bool(subtract_mean), bool(enable_ccq), gate_w, gate_b)
    o = in_dtype(cut_tail(o, V), dt)
    if not output_final_state:
        return o, None, None, None
    return o, cut_tail(sfin, K, V), cut_tail(hfin, K, K), cut_tail(mfin, K)


def chunk_ccq_gdn(q, k, v, lambda_h, g, beta, scale=None, initial_state=None, initial_cov_state=None,
                  initial_mean_state=None, output_final_state=False, use_qk_l2norm_in_kernel=False, cu_seqlens=None,
                  cp_context=None, transpose_state_layout=False, position_offset=0, subtract_mean=True,
                  enable_ccq=True, **kwargs):
    """CCQ-GDN, stock ``chunk`` mode (reference ``ccq/ops/ccq_gdn/chunk.py:12-84``).

    Same mathematics as ``fused_chunk_ccq_gdn``; the reference's z-read + clean + backbone
    pipeline is computed by the same kernels here, with that pipeline's key-sum gradients
    (``_stock_mean``: none for ``initial_mean_state``, none taken from the final key sum).
    ``transpose_state_layout`` selects ``[N, H, V, K]`` backbone states (fla's option);
    ``cp_context`` (context parallelism) is not supported on one GPU.
    """
    if cp_context is not None:
        raise NotImplementedError("chunk_ccq_gdn: context parallelism (cp_context) is not supported")
    if transpose_state_layout and initial_state is not None:
        initial_state = initial_state.transpose(-1, -2)
    o, s, c, m = fused_chunk_ccq_gdn(q, k, v, lambda_h, g, beta, scale, initial_state, initial_cov_state,
                                     _stock_mean(initial_mean_state), output_final_state, use_qk_l2norm_in_kernel,
                                     cu_seqlens, position_offset, subtract_mean, enable_ccq, **kwargs)
    if transpose_state_layout and s is not None:
        s = s.transpose(-1, -2).contiguous()
    return o, s, c, _stock_mean(m)


def fused_recurrent_ccq_gdn(q, k, v, lambda_h, g=None, gk=None, gv=None, beta=None, scale=None, initial_state=None,
                            initial_cov_state=None, initial_mean_state=None, output_final_state=False,
                            use_qk_l2norm_in_kernel=False, cu_seqlens=None, transpose_state_layout=False,
                            position_offset=0, subtract_mean=True, enable_ccq=True):
    """CCQ-GDN, recurrent (decode) mode (reference ``ccq/ops/ccq_gdn/fused_recurrent.py:18-75``).

    Without autograd (decode, generation) this runs the decode kernels: rank-1 updates of the
    cached S, C and m per token, with the optional per-key / per-value decays ``gk`` / ``gv`` of
    fla's recurrent gated delta rule.  When a gradient is needed it runs the chunk kernels, which
    compute the same recurrence (without gk / gv) and have a backward, with the reference's
    key-sum gradients for this path (``_stock_mean``).
    """
    from .decode import gdn_decode, needs_grad
    if beta is None:
        beta = torch.ones(q.shape[:3], device=q.device, dtype=torch.float32)
    if not needs_grad(q, k, v, lambda_h, g, gk, gv, beta, initial_state, initial_cov_state, initial_mean_state):
        s0 = initial_state
        if transpose_state_layout and s0 is not None:
            s0 = s0.transpose(-1, -2)
        dt = q.dtype
        q, k, v = as_kernel_dtype(q, k, v)
        K, V = q.shape[-1], v.shape[-1]
        scale = _default_scale(scale, K)
        cov0, m0 = initial_cov_state, initial_mean_state if subtract_mean else None
        Kp, Vp = padded_sizes(K, V, STEP_K)
        if (Kp, Vp) != (K, V):
            q, k, v, gk, gv = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(v, Vp), pad_tail(gk, Kp), pad_tail(gv, Vp)
            s0, cov0, m0 = pad_tail(s0, Kp, Vp), pad_tail(cov0, Kp, Kp), pad_tail(m0, Kp)
        o, s, c, m = gdn_decode(q, k, v, lambda_h, g, beta, scale, s0, cov0, m0, bool(output_final_state),
                                bool(use_qk_l2norm_in_kernel), cu_seqlens, position_offset, subtract_mean, enable_ccq,
                                gk=gk, gv=gv)
        o = in_dtype(cut_tail(o, V), dt)
        if not output_final_state:
            return o, None, None, None
        s, c, m = cut_tail(s, K, V), cut_tail(c, K, K), cut_tail(m, K)
        if transpose_state_layout:
            s = s.transpose(-1, -2).contiguous()
        return o, s, c, m
    if gk is not None or gv is not None:
        raise NotImplementedError("fused_recurrent_ccq_gdn: gradients through the per-key / per-value decays "
                                  "(gk, gv) are not supported (inference with them runs on the decode kernels)")
    return chunk_ccq_gdn(q, k, v, lambda_h, g, beta, scale, initial_state, initial_cov_state, initial_mean_state,
                         output_final_state, use_qk_l2norm_in_kernel, cu_seqlens, None, transpose_state_layout,
                         position_offset, subtract_mean, enable_ccq)


def chunk_gated_delta_rule(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                           use_qk_l2norm_in_kernel=False, cu_seqlens=None, **kwargs):
    """The backbone alone (fla's ``chunk_gated_delta_rule`` signature), on the same kernels."""
    o, s, _, _ = fused_chunk_ccq_gdn(q, k, v, None, g, beta, scale, initial_state, None, None, output_final_state,
                                     use_qk_l2norm_in_kernel, cu_seqlens, enable_ccq=False, **kwargs)
    return o, s


def fused_ccq_clean(q, k, lambda_h, *, initial_cov_state=None, initial_mean_state=None, output_final_state=False,
                    cu_seqlens=None, use_qk_l2norm_in_kernel=False, position_offset=0, subtract_mean=True,
                    use_chunk=True, chunk_size=64):
    """Cleaning for the decode / short-sequence path (reference ``ccq/ops/ccq_gdn/fused_clean.py:34-83``).

    Returns ``(q_clean, k, final_cov_state, final_mean_state, use_qk_l2norm_in_kernel)``; the key-sum
    gradients are those of the reference's ``_CCQCleanQ`` (``_stock_mean``).
    """
    from .clean import fused_ccq_clean_read
    from .l2norm import l2norm
    if use_qk_l2norm_in_kernel:
        q = l2norm(q, eps=1e-6)
        k = l2norm(k, eps=1e-6)
        use_qk_l2norm_in_kernel = False
    qc, hf, mf = fused_ccq_clean_read(q, k, lambda_h, position_offset=position_offset,
                                      initial_cov_state=initial_cov_state,
                                      initial_mean_state=_stock_mean(initial_mean_state),
                                      output_final_state=output_final_state, subtract_mean=subtract_mean,
                                      cu_seqlens=cu_seqlens)
    return qc, k, hf, _stock_mean(mf), use_qk_l2norm_in_kernel
