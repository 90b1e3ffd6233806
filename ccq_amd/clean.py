"""CCQ cleaning operator on MI355X (mirror of the reference's
``ccq/ops/common/fused_read.py`` public surface: ``fused_ccq_clean_read`` and
``FusedCCQCleanRead``; the lambda coercion of ``clean.py:314-325``).

Forward and backward each run hand-written gfx950 kernels through the C ABI
of ``libccq_hip.so``; nothing here computes on the CPU or falls back to
PyTorch math.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from ._lib import call, ptr, stream_of

__all__ = ["fused_ccq_clean_read", "FusedCCQCleanRead", "reshape_lambda_3d", "reduce_dlambda", "seq_count",
           "norm_cu_seqlens", "check_device",
           "l2norm_fwd", "l2norm_bwd", "_CCQCleanQ", "_ccq_compute_z_and_sum_kk"]


def seq_count(B: int, cu_seqlens: Optional[torch.Tensor]) -> int:
    return B if cu_seqlens is None else cu_seqlens.numel() - 1


def reshape_lambda_3d(lam, q: torch.Tensor) -> torch.Tensor:
    """lambda (python scalar, 0-d, ``(H,)``, ``(B,T,H,1)`` or ``(B,T,H)``) -> ``(B,T,H)`` in q's dtype,
    as the reference's ``_reshape_lambda_3d`` (``clean.py:314-325``); returned as contiguous fp32
    for the kernels (the q-dtype rounding is kept)."""
    B, T, H = q.shape[:3]
    if not isinstance(lam, torch.Tensor):
        out = torch.full((B, T, H), float(lam), device=q.device, dtype=q.dtype)
    elif lam.ndim == 0:
        out = lam.expand(B, T, H).to(q.dtype)
    elif lam.ndim == 1 and lam.shape[0] == H:
        out = lam.view(1, 1, H).expand(B, T, H).to(q.dtype)
    elif lam.ndim == 4 and lam.shape[-1] == 1:
        out = lam.squeeze(-1).to(q.dtype)
    else:
        out = lam.to(q.dtype)
    return out.float().contiguous()


def reduce_dlambda(dlam3: torch.Tensor, lam) -> Optional[torch.Tensor]:
    """Gradient for lambda in its original shape (``fused_read.py:502-513``)."""
    if not isinstance(lam, torch.Tensor) or not lam.requires_grad:
        return None
    if lam.ndim == 0:
        dl = dlam3.sum()
    elif lam.ndim == 1:
        dl = dlam3.sum(dim=(0, 1))
    elif lam.ndim == 4 and lam.shape[-1] == 1:
        dl = dlam3.unsqueeze(-1)
    else:
        dl = dlam3
    return dl.to(lam.dtype)


def norm_cu_seqlens(cu_seqlens: Optional[torch.Tensor], q: torch.Tensor) -> Optional[torch.Tensor]:
    """``cu_seqlens`` as the kernels read it: int64, contiguous, on q's device.  The reference takes
    int32 as well (fla's ``get_unpad_data`` and HF packing produce it; ``fused_read.py:115-116, 468``
    widen it to int64), and varlen inputs are a single packed row (B == 1)."""
    if cu_seqlens is None:
        return None
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.ndim != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor [N + 1] of sequence boundaries")
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"cu_seqlens must be int32 or int64 (got {cu_seqlens.dtype})")
    if q.shape[0] != 1:
        raise ValueError(f"varlen inputs (cu_seqlens) are one packed row: batch size 1, not {q.shape[0]}")
    return cu_seqlens.to(device=q.device, dtype=torch.int64).contiguous()


def check_device(device: torch.device, **tensors) -> None:
    """Every tensor argument must live on the inputs' GPU: the kernels dereference raw pointers."""
    for name, t in tensors.items():
        if isinstance(t, torch.Tensor) and t.device != device:
            raise ValueError(f"{name} must be on {device} like q (got {t.device})")


def _check_qk(q: torch.Tensor, k: torch.Tensor):
    if not (q.is_cuda and k.is_cuda):
        raise RuntimeError("ccq_amd ops run on the GPU only (inputs are on the CPU)")
    if q.device != k.device:
        raise ValueError(f"q and k must be on one device (got {q.device}, {k.device})")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise TypeError(f"ccq_amd kernels take bf16 q/k (got {q.dtype}, {k.dtype})")
    if q.shape != k.shape or q.ndim != 4:
        raise ValueError(f"q and k must both be [B, T, H, K] (got {tuple(q.shape)}, {tuple(k.shape)})")


ACCEPTED_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def as_kernel_dtype(*xs):
    """The activations (q, k, v) as the kernels take them, bf16: the operands of every product
    enter the matrix cores as bf16, with fp32 accumulation and fp32 states.  The reference runs
    its kernels in the input dtype; here fp16 and fp32 inputs are rounded to bf16 on the way in
    (a differentiable cast, so gradients return in the input dtype) and the callers return their
    outputs in the input dtype.  Other dtypes raise."""
    out = []
    for x in xs:
        if x is not None and x.dtype not in ACCEPTED_DTYPES:
            raise TypeError(f"ccq_amd ops take bf16, fp16 or fp32 activations (got {x.dtype})")
        out.append(x if x is None or x.dtype == torch.bfloat16 else x.to(torch.bfloat16))
    return tuple(out)


def in_dtype(x: Optional[torch.Tensor], dtype: torch.dtype) -> Optional[torch.Tensor]:
    """An output back in the caller's input dtype (no-op for bf16 inputs)."""
    return x if x is None or x.dtype == dtype else x.to(dtype)


def _f32(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.float().contiguous()


def l2norm_fwd(x: torch.Tensor, eps: float = 1e-6):
    """Row L2 normalisation (fla ``l2norm``, called at ``ccq/ops/ccq_gdn/fused_chunk.py:43-44``)."""
    x = x.contiguous()
    D = x.shape[-1]
    rows = x.numel() // D
    y = torch.empty_like(x)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    call("ccq_l2norm_fwd", ptr(x), ptr(y), ptr(rstd), rows, D, float(eps), stream_of(x))
    return y, rstd


def l2norm_bwd(x: torch.Tensor, rstd: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    D = x.shape[-1]
    rows = x.numel() // D
    dy = dy.contiguous()
    dx = torch.empty_like(x)
    is32 = dy.dtype == torch.float32
    if not is32:
        dy = dy.to(torch.bfloat16)
    call("ccq_l2norm_bwd", ptr(x), ptr(rstd), ptr(dy) if is32 else None, None if is32 else ptr(dy), ptr(dx), rows, D,
         stream_of(x))
    return dx


def clean_forward(q, k, lam3, gate_w, gate_b, h0, m0, cu_seqlens, position_offset, subtract_mean, *,
                  want_bf16=True, want_f32=False, want_hfin=False, want_mfin=False):
    """Launch the cleaning forward.  Returns (q_clean bf16|None, q_clean fp32|None, h_final|None,
    m_final|None, lambda used (gate output or lam3), saved buffer for the backward)."""
    B, T, H, K = q.shape
    N = seq_count(B, cu_seqlens)
    dev = q.device
    varlen = cu_seqlens is not None
    saved = torch.empty(_lib.load().ccq_clean_saved_bytes(B * T, B, T, N, H, K, int(varlen)), device=dev,
                        dtype=torch.uint8)
    qc = torch.empty_like(q) if want_bf16 else None
    qc32 = torch.empty(q.shape, device=dev, dtype=torch.float32) if want_f32 else None
    hfin = torch.empty(N, H, K, K, device=dev, dtype=torch.float32) if want_hfin else None
    mfin = torch.empty(N, H, K, device=dev, dtype=torch.float32) if (want_mfin and subtract_mean) else None
    lam_out = torch.empty(B, T, H, device=dev, dtype=torch.float32) if gate_w is not None else None
    call("ccq_clean_fwd", ptr(q), ptr(k), ptr(lam3), ptr(gate_w), ptr(gate_b), ptr(lam_out), ptr(h0), ptr(m0),
         ptr(cu_seqlens), ptr(saved), ptr(qc), ptr(qc32), ptr(hfin), ptr(mfin), B, T, H, K, N, int(position_offset),
         int(bool(subtract_mean)), stream_of(q))
    return qc, qc32, hfin, mfin, (lam_out if gate_w is not None else lam3), saved


def clean_backward(q, k, lam_used, gate_w, gate_b, dqc, dk_extra, h0, m0, cu_seqlens, saved, dh_fin, dm_fin,
                   position_offset, subtract_mean, *, want_dlam=True, dq_f32=False, dk_f32=False):
    """Launch the cleaning backward.  Returns (dq, dk, dlam3|None, dgate_w|None, dgate_b|None, dh0|None, dm0|None)."""
    B, T, H, K = q.shape
    N = seq_count(B, cu_seqlens)
    dev = q.device
    gate = gate_w is not None
    varlen = cu_seqlens is not None
    ws = torch.empty(_lib.load().ccq_clean_bwd_workspace_bytes(B * T, B, T, N, H, K, int(varlen), int(gate)),
                     device=dev, dtype=torch.uint8)
    dqc = dqc.contiguous()
    d32 = dqc if dqc.dtype == torch.float32 else None
    d16 = None if d32 is not None else dqc.to(torch.bfloat16)
    # the kernels read the upstream gradient in 16-byte vectors
    if d32 is not None and d32.data_ptr() % 16:
        d32 = d32.clone()
    if d16 is not None and d16.data_ptr() % 16:
        d16 = d16.clone()
    dq = torch.empty(q.shape, device=dev, dtype=torch.float32 if dq_f32 else q.dtype)
    dk = torch.empty(k.shape, device=dev, dtype=torch.float32 if dk_f32 else k.dtype)
    dlam = torch.empty(B, T, H, device=dev, dtype=torch.float32) if (want_dlam and not gate) else None
    dgw = torch.empty_like(gate_w) if gate else None
    dgb = torch.empty_like(gate_b) if gate else None
    dh0 = torch.empty(N, H, K, K, device=dev, dtype=torch.float32) if h0 is not None else None
    dm0 = torch.empty(N, H, K, device=dev, dtype=torch.float32) if (m0 is not None and subtract_mean) else None
    # converted copies are bound to names so that each buffer outlives the launch (a temporary
    # freed inside the argument list could be handed to the next conversion)
    dh_fin, dm_fin = _f32(dh_fin), _f32(dm_fin)
    call("ccq_clean_bwd", ptr(q), ptr(k), ptr(lam_used), ptr(gate_w), ptr(gate_b), ptr(d32), ptr(d16),
         ptr(dk_extra), ptr(h0), ptr(m0), ptr(cu_seqlens), ptr(saved), ptr(dh_fin), ptr(dm_fin),
         None if dq_f32 else ptr(dq), ptr(dq) if dq_f32 else None, None if dk_f32 else ptr(dk),
         ptr(dk) if dk_f32 else None, ptr(dlam), ptr(dgw), ptr(dgb), ptr(dh0), ptr(dm0), ptr(ws), B, T, H, K, N,
         int(position_offset), int(bool(subtract_mean)), stream_of(q))
    return dq, dk, dlam, dgw, dgb, dh0, dm0


class FusedCCQCleanRead(torch.autograd.Function):
    """q_clean, final covariance and final key-sum states from (q, k, lambda): one forward kernel
    and one backward kernel pair (reference ``FusedCCQCleanRead``, ``fused_read.py:474-514``).

    ``gate_w`` / ``gate_b`` (optional, fp32 ``[H, K]`` / ``[H]``) switch to the fused per-head gate
    ``lambda = sigmoid(gate_w[h]·q + gate_b[h])``; ``lambda_h`` is then ignored."""

    @staticmethod
    def forward(ctx, q, k, lambda_h, position_offset, initial_cov_state, initial_mean_state, output_final_state,
                subtract_mean, cu_seqlens, gate_w=None, gate_b=None):
        _check_qk(q, k)
        check_device(q.device, lambda_h=lambda_h, initial_cov_state=initial_cov_state,
                     initial_mean_state=initial_mean_state, gate_w=gate_w, gate_b=gate_b)
        cu_seqlens = norm_cu_seqlens(cu_seqlens, q)
        q, k = q.contiguous(), k.contiguous()
        gw, gb = _f32(gate_w), _f32(gate_b)
        lam3 = None if gw is not None else reshape_lambda_3d(lambda_h, q)
        h0 = _f32(initial_cov_state)
        m0 = _f32(initial_mean_state) if subtract_mean else None
        want = bool(output_final_state)
        qc, _, hfin, mfin, lam_used, saved = clean_forward(q, k, lam3, gw, gb, h0, m0, cu_seqlens, position_offset,
                                                           subtract_mean, want_hfin=want, want_mfin=want)
        ctx.save_for_backward(q, k, lam_used, h0, m0, saved, cu_seqlens, gw, gb)
        ctx.lambda_h = lambda_h if isinstance(lambda_h, torch.Tensor) else None
        ctx.position_offset = int(position_offset)
        ctx.subtract_mean = bool(subtract_mean)
        ctx.has_h0 = initial_cov_state is not None
        ctx.has_m0 = initial_mean_state is not None and subtract_mean
        ctx.gate = gw is not None
        return qc, hfin, mfin

    @staticmethod
    def backward(ctx, dqc, dfinal_cov, dfinal_mean):
        q, k, lam_used, h0, m0, saved, cu_seqlens, gw, gb = ctx.saved_tensors
        want_dlam = ctx.lambda_h is not None and ctx.lambda_h.requires_grad
        dq, dk, dlam, dgw, dgb, dh0, dm0 = clean_backward(
            q, k, lam_used, gw, gb, dqc, None, h0, m0, cu_seqlens, saved, dfinal_cov, dfinal_mean,
            ctx.position_offset, ctx.subtract_mean, want_dlam=want_dlam)
        dl = reduce_dlambda(dlam, ctx.lambda_h) if (dlam is not None) else None
        return dq, dk, dl, None, dh0, dm0, None, None, None, dgw, dgb


def fused_ccq_clean_read(q, k, lambda_h, *, position_offset=0, initial_cov_state=None, initial_mean_state=None,
                         output_final_state=False, subtract_mean=True, cu_seqlens=None, gate_w=None, gate_b=None):
    """Fused covariance read + cleaning (reference ``fused_read.py:517-531``).

    Returns ``(q_clean, final_cov_state, final_mean_state)``; the states are None unless requested.
    """
    from ._pad import STEP_K, cut_tail, pad_tail, padded_sizes
    dt = q.dtype
    q, k = as_kernel_dtype(q, k)
    # head sizes between the kernels' run zero-padded (ccq_amd/_pad.py)
    K = q.shape[-1]
    Kp, _ = padded_sizes(K, None, STEP_K)
    if Kp != K:
        q, k, gate_w = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(gate_w, Kp)
        initial_cov_state, initial_mean_state = pad_tail(initial_cov_state, Kp, Kp), pad_tail(initial_mean_state, Kp)
    qc, hf, mf = FusedCCQCleanRead.apply(q, k, lambda_h, int(position_offset), initial_cov_state, initial_mean_state,
                                         bool(output_final_state), bool(subtract_mean), cu_seqlens, gate_w, gate_b)
    if not output_final_state:
        hf, mf = None, None
    return in_dtype(cut_tail(qc, K), dt), cut_tail(hf, K, K), cut_tail(mf, K)


# ---------------------------------------------------------------------------
# the reference's stock `chunk` building blocks (ccq/ops/common/__init__.py):
# the covariance read z and the cleaning given z
# ---------------------------------------------------------------------------

class _CCQCleanQ(torch.autograd.Function):
    """Cleaning given a precomputed covariance read ``z`` (reference ``_CCQCleanQ``,
    ``ccq/ops/common/clean.py:691-748``): ``q_clean = q - λ (z/pos - (m·q) m/pos²)`` with the running
    key sum ``m`` (initial ``initial_state_K``).  Returns ``(q_clean, final_state_K | None)``.

    Gradients are the reference's (``clean.py:720-748``): dq, dk, dz and dλ; the gradient arriving
    at ``final_state_K`` is not propagated and ``initial_state_K`` gets none."""

    @staticmethod
    def forward(ctx, q, k, z, lambda_h, position_offset, initial_state_K, output_final_state, subtract_mean,
                cu_seqlens):
        from .ccq_gdn import _Chunks
        _check_qk(q, k)
        if z.shape != q.shape:
            raise ValueError(f"z must have q's shape {tuple(q.shape)} (got {tuple(z.shape)})")
        check_device(q.device, z=z, lambda_h=lambda_h, initial_state_K=initial_state_K)
        from ._pad import STEP_K, pad_tail, padded_sizes
        cu_seqlens = norm_cu_seqlens(cu_seqlens, q)
        q, k = q.contiguous(), k.contiguous()
        z16 = z.contiguous().to(torch.bfloat16)
        lam3 = reshape_lambda_3d(lambda_h, q)
        m0 = _f32(initial_state_K)
        # head sizes between the kernels' run zero-padded (ccq_amd/_pad.py); results sliced back here
        # and in the backward
        ctx.k0 = K0 = q.shape[-1]
        Kp, _ = padded_sizes(K0, None, STEP_K)
        if Kp != K0:
            q, k, z16, m0 = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(z16, Kp), pad_tail(m0, Kp)
        B, T, H, K = q.shape
        ch = _Chunks(B, T, cu_seqlens, q.device)
        saved = torch.empty(_lib.load().ccq_clean_z_saved_bytes(ch.count, H, K), device=q.device, dtype=torch.uint8)
        qc = torch.empty_like(q)
        mfin = torch.empty(ch.N, H, K, device=q.device, dtype=torch.float32) if output_final_state else None
        call("ccq_clean_z_fwd", ptr(q), ptr(k), ptr(z16), ptr(lam3), ptr(m0), ptr(cu_seqlens), ptr(ch.index),
             ptr(ch.offsets), ch.count, ptr(saved), ptr(qc), ptr(mfin), B, T, H, K, ch.N, int(position_offset),
             int(bool(subtract_mean)), stream_of(q))
        ctx.save_for_backward(q, k, z16, lam3, saved, cu_seqlens)
        ctx.ch = ch
        ctx.lambda_h = lambda_h if isinstance(lambda_h, torch.Tensor) else None
        ctx.z_dtype = z.dtype
        ctx.position_offset = int(position_offset)
        ctx.subtract_mean = bool(subtract_mean)
        if K != K0:
            qc, mfin = qc[..., :K0].contiguous(), (mfin[..., :K0].contiguous() if mfin is not None else None)
        return qc, mfin

    @staticmethod
    def backward(ctx, dqc, dmfin):
        from ._pad import cut_tail, pad_tail
        q, k, z16, lam3, saved, cu_seqlens = ctx.saved_tensors
        ch = ctx.ch
        B, T, H, K = q.shape
        K0 = ctx.k0
        dqc = pad_tail(dqc, K)
        ws = torch.empty(_lib.load().ccq_clean_z_bwd_workspace_bytes(ch.count, H, K), device=q.device,
                         dtype=torch.uint8)
        dqc = dqc.contiguous()
        d32 = dqc if dqc.dtype == torch.float32 else None
        d16 = None if d32 is not None else dqc.to(torch.bfloat16)
        dq, dk, dz = torch.empty_like(q), torch.empty_like(k), torch.empty_like(q)
        want_dlam = ctx.lambda_h is not None and ctx.lambda_h.requires_grad
        dlam = torch.empty(B, T, H, device=q.device, dtype=torch.float32) if want_dlam else None
        # dm_final / dm0 (the ABI's extension) stay off: the reference drops both
        call("ccq_clean_z_bwd", ptr(q), ptr(k), ptr(z16), ptr(lam3), ptr(cu_seqlens), ptr(ch.index), ptr(ch.offsets),
             ch.count, ptr(saved), ptr(d16), ptr(d32), None, ptr(dq), ptr(dk), ptr(dz), ptr(dlam), None,
             ptr(ws), B, T, H, K, ch.N, ctx.position_offset, int(ctx.subtract_mean), stream_of(q))
        dl = reduce_dlambda(dlam, ctx.lambda_h) if dlam is not None else None
        return (cut_tail(dq, K0), cut_tail(dk, K0), cut_tail(dz, K0).to(ctx.z_dtype), dl, None, None, None, None,
                None)


class _CovarianceRead(torch.autograd.Function):
    """``z = C_tᵀ q_t`` through the GLA chunk kernels with ``v = k`` (no decay, scale 1).  The two
    roles of k (key and value) are summed in fp32 before the gradient is rounded to k's dtype."""

    @staticmethod
    def forward(ctx, q, k, initial_state, output_final_state, cu_seqlens):
        from .ccq_gdn import _Chunks
        from .ccq_gla import _gla_forward
        _check_qk(q, k)
        check_device(q.device, initial_state=initial_state)
        cu_seqlens = norm_cu_seqlens(cu_seqlens, q)
        q, k = q.contiguous(), k.contiguous()
        B, T, H, K = q.shape
        ch = _Chunks(B, T, cu_seqlens, q.device)
        h0 = _f32(initial_state)
        want = bool(output_final_state)
        z, hfin, saved = _gla_forward(q, None, k, k, None, h0, ch, 1.0, want)
        ctx.save_for_backward(q, k, saved, h0, hfin)
        ctx.ch = ch
        return z, hfin

    @staticmethod
    def backward(ctx, dz, dhfin):
        from .ccq_gla import _gla_backward
        q, k, saved, h0, hfin = ctx.saved_tensors
        dq32, dk32, dv32, _, dh0 = _gla_backward(q, None, k, k, None, ctx.ch, saved, dz, dhfin, hfin, 1.0, False,
                                                 h0 is not None, dv_f32=True)
        return dq32.to(q.dtype), (dk32 + dv32).to(k.dtype), dh0, None, None


def _ccq_compute_z_and_sum_kk(q, k, output_final_state, cu_seqlens, initial_state=None, use_chunk=True,
                              chunk_size=64):
    """Covariance read ``z_t = C_tᵀ q_t`` with ``C_t = C_0 + Σ_{j≤t} k_j k_jᵀ`` and the final ``C``
    (reference ``clean.py:751-771``: fla ``chunk_simple_gla(q, k, v=k, scale=1)``, or the recurrent
    form for short inputs; both are the same recurrence).  Evaluated by the GLA chunk kernels with
    ``v = k``, no decay and ``scale = 1``; differentiable in q, k and ``initial_state``.
    Returns ``(z, final_state | None)`` with z in q's dtype."""
    from ._pad import CHUNK_K, cut_tail, pad_tail, padded_sizes
    # head sizes between the kernels' run zero-padded (ccq_amd/_pad.py)
    K = q.shape[-1]
    Kp, _ = padded_sizes(K, None, CHUNK_K)
    if Kp != K:
        q, k, initial_state = pad_tail(q, Kp), pad_tail(k, Kp), pad_tail(initial_state, Kp, Kp)
    z, hfin = _CovarianceRead.apply(q, k, initial_state, bool(output_final_state), cu_seqlens)
    return cut_tail(z, K), (cut_tail(hfin, K, K) if output_final_state else None)
