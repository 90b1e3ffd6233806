"""CPU oracle for the CCQ cleaning operator and the chunked linear-attention
backbones (gated delta rule, GLA) that consume the cleaned query.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``ccq_amd``) may import
this module; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or the
timed CPU baseline.

Everything here is plain PyTorch on the CPU, written for clarity, and runs in
whatever floating dtype it is handed (float64 for the oracle, float32 for the
CPU baseline).  Layouts follow the reference: q, k ``[B, T, H, K]``, v
``[B, T, H, V]``, per-token scalars ``[B, T, H]``; varlen inputs have ``B == 1``
plus ``cu_seqlens`` ``[N + 1]``; states are indexed by sequence ``[N, H, ...]``.

State conventions (fla's, which the reference relies on; ``fused_read.py:161-166``):

* covariance state ``h`` is ``[K, K]`` with the read ``z_t = h_tᵀ q_t``
  (the running sum ``h_t = h_0 + Σ_{j≤t} k_j k_jᵀ`` is symmetric when h_0 is);
* backbone state ``S`` is ``[K, V]`` with ``o_t = S_tᵀ (scale · q_t)``.

Pinning of each function (what checks it, besides agreeing with the others) is
listed in the test module ``tests/test_oracle.py``.  The backbone recurrences
(``gdn_recurrent``, ``gla_recurrent``) restate the published algorithms of the
third-party ``flash-linear-attention`` package (fla >= 0.4.2, pinned by the
reference's ``pyproject.toml:17``; not vendored, not installed): their exact
rounding is **parity unpinned** -- they are pinned only by closed forms and
special cases.
"""

from __future__ import annotations

import math
from typing import Iterator, Optional

import torch

__all__ = [
    "positions",
    "reshape_lambda",
    "l2norm",
    "lambda_gate",
    "clean_fwd_bruteforce",
    "clean_fwd_chunked",
    "clean_bwd_closed",
    "covariance_read",
    "clean_given_z",
    "gdn_recurrent",
    "gdn_chunked",
    "gla_recurrent",
    "gla_chunked",
    "ccq_gdn_forward",
    "ccq_gla_forward",
    "ccq_decode_gdn",
    "ccq_decode_gla",
    "round_through",
]


# ---------------------------------------------------------------------------
# small helpers
# ---------------------------------------------------------------------------

def _segments(B: int, T: int, cu_seqlens) -> Iterator[tuple]:
    """Yield (sequence index n, batch row b, start, end) for dense or varlen inputs."""
    if cu_seqlens is None:
        for b in range(B):
            yield b, b, 0, T
    else:
        cu = [int(x) for x in cu_seqlens.tolist()]
        assert B == 1, "varlen inputs must have batch size 1"
        for n in range(len(cu) - 1):
            yield n, 0, cu[n], cu[n + 1]


def _num_seqs(B, cu_seqlens):
    return B if cu_seqlens is None else len(cu_seqlens) - 1


def positions(T: int, cu_seqlens=None, position_offset: int = 0, dtype=torch.float64) -> torch.Tensor:
    """Segment-relative 1-based positions plus offset, clamped at 1 -> ``[T]``.

    Follows ``fused_read.py:463-471`` (and the in-kernel copies at
    ``fused_read.py:130-132``, ``clean.py:293-295``).
    """
    if cu_seqlens is None:
        pos = torch.arange(1, T + 1, dtype=dtype) + position_offset
    else:
        pos = torch.empty(T, dtype=dtype)
        cu = [int(x) for x in cu_seqlens.tolist()]
        for n in range(len(cu) - 1):
            pos[cu[n]:cu[n + 1]] = torch.arange(1, cu[n + 1] - cu[n] + 1, dtype=dtype) + position_offset
    return pos.clamp_min(1.0)


def reshape_lambda(lam, B: int, T: int, H: int, dtype=torch.float64) -> torch.Tensor:
    """Coerce lambda (python scalar, 0-d, ``(H,)``, ``(B,T,H,1)`` or ``(B,T,H)``) to ``(B,T,H)``.

    Follows ``clean.py:314-325`` (without the cast to q's dtype).
    """
    if not isinstance(lam, torch.Tensor):
        return torch.full((B, T, H), float(lam), dtype=dtype)
    lam = lam.to(dtype)
    if lam.ndim == 0:
        return lam.expand(B, T, H).clone()
    if lam.ndim == 1 and lam.shape[0] == H:
        return lam.view(1, 1, H).expand(B, T, H).clone()
    if lam.ndim == 4 and lam.shape[-1] == 1:
        return lam.squeeze(-1).clone()
    return lam.clone()


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Row L2 normalisation ``x / sqrt(Σx² + eps)`` over the last dim.

    The reference calls fla's ``l2norm(x, eps=1e-6)`` (e.g.
    ``ccq/ops/ccq_gdn/fused_chunk.py:43-44``); the eps placement inside the
    square root is fla's published kernel and is an assumption here.
    """
    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + eps)


def lambda_gate(q: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per-head gate ``λ = σ(W[h]·q_t + b[h])`` -> ``[B, T, H]``.

    The reference's layer uses a dense ``Linear(H·K -> H)`` followed by a
    sigmoid (``ccq/gdn/layer.py:174, 292``); the per-head ``[H, K]`` weight is
    its block-diagonal special case, the form the benchmark configs specify.
    """
    return torch.sigmoid(torch.einsum("bthk,hk->bth", q, w) + b)


# ---------------------------------------------------------------------------
# CCQ cleaning operator
# ---------------------------------------------------------------------------

def clean_fwd_bruteforce(q, k, lam, *, position_offset=0, h0=None, m0=None,
                         subtract_mean=True, cu_seqlens=None):
    """Per-token loop of the closed-form cleaning operator.

    ``fused_read.py:11-16``::

        h_t = h_0 + Σ_{j≤t} k_j k_jᵀ,  m_t = m_0 + Σ_{j≤t} k_j
        z_t = h_tᵀ q_t,  s_t = m_t·q_t
        corr_t = z_t/pos_t − s_t m_t/pos_t²   (mean term only if subtract_mean)
        q_clean_t = q_t − λ_t corr_t

    Returns ``(q_clean, h_final [N,H,K,K], m_final [N,H,K] or None)``.
    Differentiable (no in-place ops on tracked tensors).  Use on small T only.
    """
    B, T, H, K = q.shape
    lam = reshape_lambda(lam, B, T, H, q.dtype)
    pos = positions(T, cu_seqlens, position_offset, q.dtype)
    rows = [[None] * T for _ in range(B)]
    hf, mf = [], []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        C = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, K, dtype=q.dtype)
        m = m0[n].to(q.dtype) if (m0 is not None and subtract_mean) else torch.zeros(H, K, dtype=q.dtype)
        for t in range(s0, s1):
            kt, qt = k[b, t], q[b, t]
            C = C + kt[:, :, None] * kt[:, None, :]
            m = m + kt
            p = pos[t]
            z = torch.einsum("hab,ha->hb", C, qt)
            corr = z / p
            if subtract_mean:
                s = (m * qt).sum(-1)
                corr = corr - (s / (p * p))[:, None] * m
            rows[b][t] = qt - lam[b, t][:, None] * corr
        hf.append(C)
        mf.append(m)
    out = torch.stack([torch.stack(r, 0) for r in rows], 0)
    return out, torch.stack(hf, 0), (torch.stack(mf, 0) if subtract_mean else None)


def clean_fwd_chunked(q, k, lam, *, position_offset=0, h0=None, m0=None,
                      subtract_mean=True, cu_seqlens=None, BT=64, return_states=False):
    """Chunked form of the cleaning forward, ``fused_read.py:128-174`` with the
    chunk-start states of ``fused_read.py:385-391``::

        A_n = (Q_n K_nᵀ) ∘ M_causal(incl. diag)
        Z_n = Q_n H_n + A_n K_n
        cum = prefix_n + cumsum(K_n)
        q_clean = Q_n − λ (Z_n/pos − (s/pos²) cum),  s = rowsum(cum ∘ Q_n)

    Differentiable.  With ``return_states`` also returns the per-sequence list
    of chunk-start states (used by the closed-form backward).
    """
    B, T, H, K = q.shape
    lam = reshape_lambda(lam, B, T, H, q.dtype)
    pos = positions(T, cu_seqlens, position_offset, q.dtype)
    pieces = [[] for _ in range(B)]
    hf, mf, states = [], [], []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        Hs = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, K, dtype=q.dtype)
        pre = m0[n].to(q.dtype) if (m0 is not None and subtract_mean) else torch.zeros(H, K, dtype=q.dtype)
        seq_states = []
        for c0 in range(s0, s1, BT):
            c1 = min(c0 + BT, s1)
            L = c1 - c0
            Q, Kc = q[b, c0:c1], k[b, c0:c1]                      # [L,H,K]
            mask = torch.tril(torch.ones(L, L, dtype=torch.bool))
            A = torch.einsum("thk,shk->hts", Q, Kc) * mask        # [H,L,L]
            Z = torch.einsum("thk,hkv->thv", Q, Hs) + torch.einsum("hts,shv->thv", A, Kc)
            p = pos[c0:c1][:, None]                               # [L,1]
            corr = Z / p[..., None]
            cum = pre[None] + torch.cumsum(Kc, 0)                 # [L,H,K]
            if subtract_mean:
                s = (cum * Q).sum(-1)                              # [L,H]
                corr = corr - (s / (p * p))[..., None] * cum
            pieces[b].append(Q - lam[b, c0:c1][..., None] * corr)
            seq_states.append((Hs, pre))
            Hs = Hs + torch.einsum("thk,thv->hkv", Kc, Kc)
            pre = cum[-1]
        hf.append(Hs)
        mf.append(pre)
        states.append(seq_states)
    out = torch.stack([torch.cat(p, 0) for p in pieces], 0) if cu_seqlens is None else \
        torch.cat(pieces[0], 0)[None]
    res = (out, torch.stack(hf, 0), torch.stack(mf, 0) if subtract_mean else None)
    if return_states:
        return res + (states,)
    return res


def clean_bwd_closed(q, k, lam, dqc, *, position_offset=0, h0=None, m0=None,
                     subtract_mean=True, cu_seqlens=None, dh_final=None, dm_final=None, BT=64):
    """Closed-form backward of the cleaning operator, ``fused_read.py:18-25``::

        dλ_t = −dqc_t·corr_t          dz_t = −λ_t dqc_t / pos_t
        ds_t =  λ_t (dqc_t·m_t)/pos_t²
        dm_t =  λ_t s_t dqc_t/pos_t² + ds_t q_t
        dq_t =  dqc_t + ds_t m_t + h_t dz_t
        dk_j =  Σ_{t≥j} [q_t (k_j·dz_t) + dz_t (k_j·q_t) + dm_t]

    in the chunked arrangement of ``fused_read.py:241-307`` (intra-chunk terms
    ``Aᵀ dZ + Bᵀ Q`` with ``B = dZ Kᵀ ∘ M``, state term ``k (G + Gᵀ)`` with
    ``G`` the suffix of ``Σ q dzᵀ`` plus ``dh_final``) and the chunk carry of
    ``fused_read.py:355-376``.  Gradient into the initial states:
    ``dh0 = Σ_t q_t dz_tᵀ + dh_final`` (fla's ``chunk_bwd_dh`` layout),
    ``dm0 = Σ_t dm_t + dm_final``.

    Returns ``(dq, dk, dlam [B,T,H], dh0 or None, dm0 or None)``.
    """
    B, T, H, K = q.shape
    dt = q.dtype
    lam = reshape_lambda(lam, B, T, H, dt)
    pos = positions(T, cu_seqlens, position_offset, dt)
    _, _, _, states = clean_fwd_chunked(q, k, lam, position_offset=position_offset, h0=h0, m0=m0,
                                        subtract_mean=subtract_mean, cu_seqlens=cu_seqlens, BT=BT,
                                        return_states=True)
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dlam = torch.zeros(B, T, H, dtype=dt)
    dh0s, dm0s = [], []
    for si, (n, b, s0, s1) in enumerate(_segments(B, T, cu_seqlens)):
        G = dh_final[n].to(dt).clone() if dh_final is not None else torch.zeros(H, K, K, dtype=dt)
        dmc = dm_final[n].to(dt).clone() if dm_final is not None else torch.zeros(H, K, dtype=dt)
        starts = list(range(s0, s1, BT))
        for ci in reversed(range(len(starts))):
            c0 = starts[ci]
            c1 = min(c0 + BT, s1)
            L = c1 - c0
            Hs, pre = states[si][ci]
            Q, Kc, Dq = q[b, c0:c1], k[b, c0:c1], dqc[b, c0:c1].to(dt)
            lm = lam[b, c0:c1]                                   # [L,H]
            p = pos[c0:c1][:, None]                              # [L,1]
            mask = torch.tril(torch.ones(L, L, dtype=torch.bool))
            dZ = -(lm / p)[..., None] * Dq                       # [L,H,K]
            A = torch.einsum("thk,shk->hts", Q, Kc) * mask
            Bm = torch.einsum("thk,shk->hts", dZ, Kc) * mask
            Z = torch.einsum("thk,hkv->thv", Q, Hs) + torch.einsum("hts,shv->thv", A, Kc)
            corr = Z / p[..., None]
            cum = pre[None] + torch.cumsum(Kc, 0)
            dqt = Dq + torch.einsum("hab,thb->tha", Hs, dZ) + torch.einsum("hts,shk->thk", Bm, Kc)
            dkt = torch.einsum("hts,thk->shk", A, dZ) + torch.einsum("hts,thk->shk", Bm, Q) \
                + torch.einsum("shk,hkv->shv", Kc, G + G.transpose(-1, -2))
            if subtract_mean:
                s = (cum * Q).sum(-1)
                w = (cum * Dq).sum(-1)
                corr = corr - (s / (p * p))[..., None] * cum
                ds = lm * w / (p * p)
                dm = (lm * s / (p * p))[..., None] * Dq + ds[..., None] * Q
                dqt = dqt + ds[..., None] * cum
                suffix = torch.flip(torch.cumsum(torch.flip(dm, [0]), 0), [0])
                dkt = dkt + suffix + dmc[None]
                dmc = dmc + dm.sum(0)
            dlam[b, c0:c1] = -(Dq * corr).sum(-1)
            dq[b, c0:c1] = dqt
            dk[b, c0:c1] = dkt
            G = G + torch.einsum("thk,thv->hkv", Q, dZ)
        dh0s.append(G)
        dm0s.append(dmc)
    dh0 = torch.stack(dh0s, 0) if h0 is not None else None
    dm0 = torch.stack(dm0s, 0) if (m0 is not None and subtract_mean) else None
    return dq, dk, dlam, dh0, dm0


def covariance_read(q, k, *, h0=None, cu_seqlens=None):
    """``z_t = h_tᵀ q_t`` with ``h_t = h_0 + Σ_{j≤t} k_j k_jᵀ`` and the final ``h`` (the reference's
    ``_ccq_compute_z_and_sum_kk``, ``clean.py:751-771``: ``chunk_simple_gla(q, k, v=k, scale=1)``).
    Per-token loop; returns ``(z, h_final [N,H,K,K])``.  Differentiable."""
    B, T, H, K = q.shape
    rows = [[None] * T for _ in range(B)]
    hf = []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        C = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, K, dtype=q.dtype)
        for t in range(s0, s1):
            kt = k[b, t]
            C = C + kt[:, :, None] * kt[:, None, :]
            rows[b][t] = torch.einsum("hab,ha->hb", C, q[b, t])
        hf.append(C)
    return torch.stack([torch.stack(r, 0) for r in rows], 0), torch.stack(hf, 0)


def clean_given_z(q, k, z, lam, *, position_offset=0, m0=None, subtract_mean=True, cu_seqlens=None):
    """Cleaning with a precomputed read ``z`` (the reference's ``_CCQCleanQ`` forward,
    ``clean.py:286-311``)::

        m_t = m_0 + Σ_{j≤t} k_j,   q_clean_t = q_t − λ_t (z_t/pos_t − (m_t·q_t) m_t/pos_t²)

    Returns ``(q_clean, m_final or None)``.  Differentiable.  With ``z`` from
    ``covariance_read`` it is ``clean_fwd_bruteforce`` (checked in tests).
    """
    B, T, H, K = q.shape
    lam = reshape_lambda(lam, B, T, H, q.dtype)
    pos = positions(T, cu_seqlens, position_offset, q.dtype)
    rows = [[None] * T for _ in range(B)]
    mf = []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        m = m0[n].to(q.dtype) if (m0 is not None and subtract_mean) else torch.zeros(H, K, dtype=q.dtype)
        for t in range(s0, s1):
            qt = q[b, t]
            m = m + k[b, t]
            p = pos[t]
            corr = z[b, t] / p
            if subtract_mean:
                corr = corr - ((m * qt).sum(-1) / (p * p))[:, None] * m
            rows[b][t] = qt - lam[b, t][:, None] * corr
        mf.append(m)
    out = torch.stack([torch.stack(r, 0) for r in rows], 0)
    return out, (torch.stack(mf, 0) if subtract_mean else None)


# ---------------------------------------------------------------------------
# backbones
# ---------------------------------------------------------------------------

def gdn_recurrent(q, k, v, g, beta, *, scale=None, h0=None, cu_seqlens=None, gk=None, gv=None):
    """Gated delta rule, one token at a time (arXiv:2412.06464; fla's naive
    recurrence that ``chunk_gated_delta_rule`` implements)::

        S ← exp(g_t) S;   u = β_t (v_t − Sᵀ k_t);   S ← S + k_t uᵀ;   o_t = Sᵀ (scale q_t)

    ``gk`` ``[B,T,H,K]`` / ``gv`` ``[B,T,H,V]`` (optional) also decay the state's rows / columns
    before the delta step, ``S ← exp(g_t) diag(exp(gk_t)) S diag(exp(gv_t))``: the per-key /
    per-value gates that the reference hands to fla's ``fused_recurrent_gated_delta_rule``
    (``ccq/ops/ccq_gdn/fused_recurrent.py:66-74``); fla is not available here, so these two
    follow its published recurrence and are pinned by closed forms only.
    ``scale`` defaults to ``K**-0.5``.  Returns ``(o, S_final [N,H,K,V])``.
    Differentiable.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    rows = [[None] * T for _ in range(B)]
    finals = []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        S = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, V, dtype=q.dtype)
        for t in range(s0, s1):
            S = S * torch.exp(g[b, t])[:, None, None]
            if gk is not None:
                S = S * torch.exp(gk[b, t])[:, :, None]
            if gv is not None:
                S = S * torch.exp(gv[b, t])[:, None, :]
            u = beta[b, t][:, None] * (v[b, t] - torch.einsum("hkv,hk->hv", S, k[b, t]))
            S = S + k[b, t][:, :, None] * u[:, None, :]
            rows[b][t] = torch.einsum("hkv,hk->hv", S, q[b, t] * scale)
        finals.append(S)
    o = torch.stack([torch.stack(r, 0) for r in rows], 0)
    return o, torch.stack(finals, 0)


def gdn_chunked(q, k, v, g, beta, *, scale=None, h0=None, cu_seqlens=None, BT=64):
    """Chunked (WY) form of the gated delta rule.  Per chunk, with ``G`` the
    in-chunk cumulative sum of g, ``γ = exp(G)``, ``Γ_ij = exp(G_i − G_j)``::

        A = strict_lower(diag(β) (K Kᵀ ∘ Γ)),   T = (I + A)⁻¹
        w = T diag(βγ) K,   u = T diag(β) V,   U = u − w S
        O = scale [diag(γ) Q S + (Q Kᵀ ∘ Γ ∘ M) U]
        S ← γ_L S + (diag(γ_L/γ) K)ᵀ U

    Equal to ``gdn_recurrent`` (checked in tests).  Differentiable.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    pieces = [[] for _ in range(B)]
    finals = []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        S = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, V, dtype=q.dtype)
        for c0 in range(s0, s1, BT):
            c1 = min(c0 + BT, s1)
            L = c1 - c0
            Q, Kc, Vc = q[b, c0:c1], k[b, c0:c1], v[b, c0:c1]
            G = torch.cumsum(g[b, c0:c1].to(q.dtype), 0)         # [L,H]
            bt = beta[b, c0:c1].to(q.dtype)                      # [L,H]
            Gh = G.transpose(0, 1)                               # [H,L]
            incl = torch.tril(torch.ones(L, L, dtype=torch.bool))
            strict = torch.tril(torch.ones(L, L, dtype=torch.bool), -1)
            diff = Gh[:, :, None] - Gh[:, None, :]               # [H,L,L]  G_i - G_j
            Gam_incl = torch.exp(torch.where(incl, diff, torch.full_like(diff, -math.inf)))
            Gam_strict = torch.exp(torch.where(strict, diff, torch.full_like(diff, -math.inf)))
            KK = torch.einsum("thk,shk->hts", Kc, Kc)
            A = bt.transpose(0, 1)[:, :, None] * KK * Gam_strict
            Tm = torch.linalg.solve_triangular(torch.eye(L, dtype=q.dtype) + A,
                                               torch.eye(L, dtype=q.dtype).expand(H, L, L),
                                               upper=False, unitriangular=True)
            gam = torch.exp(Gh)                                  # [H,L]
            w = Tm @ ((bt.transpose(0, 1) * gam)[..., None] * Kc.transpose(0, 1))   # [H,L,K]
            u = Tm @ (bt.transpose(0, 1)[..., None] * Vc.transpose(0, 1))           # [H,L,V]
            U = u - w @ S
            P = torch.einsum("thk,shk->hts", Q, Kc) * Gam_incl
            O = (gam[..., None] * Q.transpose(0, 1)) @ S + P @ U                      # [H,L,V]
            pieces[b].append(scale * O.transpose(0, 1))
            gL = gam[:, -1]                                                          # [H]
            Kt = (torch.exp(Gh[:, -1:] - Gh))[..., None] * Kc.transpose(0, 1)       # [H,L,K]
            S = gL[:, None, None] * S + Kt.transpose(-1, -2) @ U
        finals.append(S)
    o = torch.stack([torch.cat(p, 0) for p in pieces], 0) if cu_seqlens is None else \
        torch.cat(pieces[0], 0)[None]
    return o, torch.stack(finals, 0)


def gla_recurrent(q, k, v, gk, *, scale=None, h0=None, cu_seqlens=None, gv=None, reverse=False):
    """Gated linear attention, one token at a time (arXiv:2312.06635; fla's
    naive recurrence for ``chunk_gla`` / ``fused_recurrent_gla``)::

        S ← diag(exp(gk_t)) S diag(exp(gv_t)) + k_t v_tᵀ;   o_t = Sᵀ (scale q_t)

    ``gk`` is the per-channel log decay of the state's rows ``[B,T,H,K]``, ``gv`` that of its
    columns ``[B,T,H,V]`` (``None`` means no decay); ``reverse`` visits each sequence from its
    last token to its first (``fused_recurrent_gla(reverse=True)``, as the reference forwards it,
    ``ccq/ops/ccq_gla/fused_recurrent.py:41-49``).  Returns ``(o, S_final [N,H,K,V])``.
    Differentiable.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    rows = [[None] * T for _ in range(B)]
    finals = []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        S = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, V, dtype=q.dtype)
        for t in (range(s1 - 1, s0 - 1, -1) if reverse else range(s0, s1)):
            if gk is not None:
                S = S * torch.exp(gk[b, t])[:, :, None]
            if gv is not None:
                S = S * torch.exp(gv[b, t])[:, None, :]
            S = S + k[b, t][:, :, None] * v[b, t][:, None, :]
            rows[b][t] = torch.einsum("hkv,hk->hv", S, q[b, t] * scale)
        finals.append(S)
    o = torch.stack([torch.stack(r, 0) for r in rows], 0)
    return o, torch.stack(finals, 0)


def gla_chunked(q, k, v, gk, *, scale=None, h0=None, cu_seqlens=None, BT=64):
    """Chunked GLA.  With ``Gk`` the in-chunk cumulative log decay per channel::

        O = scale [(Q∘e^{Gk}) S + ((Q∘e^{Gk}) (K∘e^{−Gk})ᵀ ∘ M) V]
        S ← diag(e^{Gk_L}) S + (K∘e^{Gk_L − Gk})ᵀ V

    (pairwise exponents are formed as differences, so nothing overflows).
    Equal to ``gla_recurrent`` (checked in tests).  Differentiable.
    """
    B, T, H, K = q.shape
    V = v.shape[-1]
    scale = K ** -0.5 if scale is None else scale
    pieces = [[] for _ in range(B)]
    finals = []
    for n, b, s0, s1 in _segments(B, T, cu_seqlens):
        S = h0[n].to(q.dtype) if h0 is not None else torch.zeros(H, K, V, dtype=q.dtype)
        for c0 in range(s0, s1, BT):
            c1 = min(c0 + BT, s1)
            L = c1 - c0
            Q, Kc, Vc = q[b, c0:c1], k[b, c0:c1], v[b, c0:c1]
            if gk is not None:
                G = torch.cumsum(gk[b, c0:c1].to(q.dtype), 0)     # [L,H,K]
            else:
                G = torch.zeros(L, H, K, dtype=q.dtype)
            incl = torch.tril(torch.ones(L, L, dtype=torch.bool))
            diff = G[:, None] - G[None, :]                          # [L,L,H,K]  G_t - G_s
            diff = torch.where(incl[:, :, None, None], diff, torch.full_like(diff, -math.inf))
            P = torch.einsum("thk,shk,tshk->hts", Q, Kc, torch.exp(diff))
            Qg = Q * torch.exp(G)
            O = torch.einsum("thk,hkv->thv", Qg, S) + torch.einsum("hts,shv->thv", P, Vc)
            pieces[b].append(scale * O)
            GL = G[-1]                                              # [H,K]
            S = torch.exp(GL)[:, :, None] * S + torch.einsum("thk,thv->hkv", Kc * torch.exp(GL[None] - G), Vc)
        finals.append(S)
    o = torch.stack([torch.cat(p, 0) for p in pieces], 0) if cu_seqlens is None else \
        torch.cat(pieces[0], 0)[None]
    return o, torch.stack(finals, 0)


# ---------------------------------------------------------------------------
# composed operators (what the reference's orchestrators compute)
# ---------------------------------------------------------------------------

def round_through(x, dtype):
    """Forward value rounded through ``dtype``; the gradient passes unrounded (straight through),
    so the oracle's gradients stay in the working precision."""
    if dtype is None:
        return x
    return x + (x.to(dtype).to(x.dtype) - x).detach()


def _l2norm_io(q, k, io_dtype):
    """l2norm of q and k; ``io_dtype`` rounds the forward results through that dtype, as fla's
    l2norm returns its input's dtype (bf16 in the reference's training runs)."""
    return round_through(l2norm(q), io_dtype), round_through(l2norm(k), io_dtype)


def ccq_gdn_forward(q, k, v, lam, g, beta, *, scale=None, h0=None, h0_cov=None, m0=None,
                    position_offset=0, subtract_mean=True, cu_seqlens=None,
                    use_qk_l2norm=False, enable_ccq=True, qc_dtype=None, chunked=True, l2norm_dtype=None):
    """``fused_chunk_ccq_gdn`` / ``chunk_ccq_gdn`` (``ccq/ops/ccq_gdn/fused_chunk.py:35-59``,
    ``chunk.py:93-143``): optional l2norm, cleaning, then the gated delta rule on
    the cleaned query.  ``qc_dtype`` rounds q_clean through that dtype, as the
    reference does when it hands q_clean (in q's dtype) to the backbone;
    ``l2norm_dtype`` does the same for the l2norm outputs.

    Returns ``(o, S_final, h_final, m_final)``.
    """
    if use_qk_l2norm:   # with enable_ccq off the backbone normalises (use_qk_l2norm_in_kernel, :35-40)
        q, k = _l2norm_io(q, k, l2norm_dtype)
    if not enable_ccq:
        fn = gdn_chunked if chunked else gdn_recurrent
        o, S = fn(q, k, v, g, beta, scale=scale, h0=h0, cu_seqlens=cu_seqlens)
        return o, S, None, None
    cl = clean_fwd_chunked if chunked else clean_fwd_bruteforce
    qc, hf, mf = cl(q, k, lam, position_offset=position_offset, h0=h0_cov,
                    m0=m0 if subtract_mean else None, subtract_mean=subtract_mean, cu_seqlens=cu_seqlens)
    qc = round_through(qc, qc_dtype)
    fn = gdn_chunked if chunked else gdn_recurrent
    o, S = fn(qc, k, v, g, beta, scale=scale, h0=h0, cu_seqlens=cu_seqlens)
    return o, S, hf, mf


def ccq_gla_forward(q, k, v, lam, gk, *, scale=None, h0=None, h0_cov=None, m0=None,
                    position_offset=0, subtract_mean=True, cu_seqlens=None, qc_dtype=None,
                    chunked=True, l2norm_dtype=None):
    """``fused_chunk_ccq_gla`` / ``chunk_ccq_gla`` (``ccq/ops/ccq_gla/fused_chunk.py:31-46``):
    unconditional l2norm, cleaning, then GLA on the cleaned query."""
    q, k = _l2norm_io(q, k, l2norm_dtype)
    cl = clean_fwd_chunked if chunked else clean_fwd_bruteforce
    qc, hf, mf = cl(q, k, lam, position_offset=position_offset, h0=h0_cov,
                    m0=m0 if subtract_mean else None, subtract_mean=subtract_mean, cu_seqlens=cu_seqlens)
    qc = round_through(qc, qc_dtype)
    fn = gla_chunked if chunked else gla_recurrent
    o, S = fn(qc, k, v, gk, scale=scale, h0=h0, cu_seqlens=cu_seqlens)
    return o, S, hf, mf


def ccq_decode_gdn(q, k, v, lam, g, beta, S, C, m, pos, *, scale=None, subtract_mean=True,
                   use_qk_l2norm=True, gk=None, gv=None):
    """Recurrent CCQ-GDN over a few tokens from a cache ``(S, C, m, pos)``.

    ``fused_recurrent_ccq_gdn`` (``ccq/ops/ccq_gdn/fused_recurrent.py:18-75``) ->
    ``fused_ccq_clean(use_chunk=False)`` (``fused_clean.py:34-83``): rank-1
    updates of C and m per token, the cleaning with positions
    ``pos + t + 1``, then the gated delta rule from S.  Returns
    ``(o, S', C', m', pos + q_len)`` -- the cache tuple of ``gdn/layer.py:394-400``.
    """
    if use_qk_l2norm:
        q, k = l2norm(q), l2norm(k)
    qc, C2, m2 = clean_fwd_bruteforce(q, k, lam, position_offset=pos, h0=C,
                                      m0=m if subtract_mean else None, subtract_mean=subtract_mean)
    o, S2 = gdn_recurrent(qc, k, v, g, beta, scale=scale, h0=S, gk=gk, gv=gv)
    return o, S2, C2, m2, pos + q.shape[1]


def ccq_decode_gla(q, k, v, lam, gk, S, C, m, pos, *, scale=None, subtract_mean=True, gv=None, reverse=False,
                   cu_seqlens=None):
    """Recurrent CCQ-GLA (``ccq/ops/ccq_gla/fused_recurrent.py:9-51``): l2norm, the cleaning
    (forwards in time), then the GLA recurrence with the row / column decays gk / gv, backwards
    in time with ``reverse`` (``:41-49``)."""
    q, k = l2norm(q), l2norm(k)
    qc, C2, m2 = clean_fwd_bruteforce(q, k, lam, position_offset=pos, h0=C,
                                      m0=m if subtract_mean else None, subtract_mean=subtract_mean,
                                      cu_seqlens=cu_seqlens)
    o, S2 = gla_recurrent(qc, k, v, gk, scale=scale, h0=S, gv=gv, reverse=reverse, cu_seqlens=cu_seqlens)
    return o, S2, C2, m2, pos + q.shape[1]
