"""GPU parity of the recurrent (decode) kernels: one call over a few tokens against the cached
states (S, C = sum k k^T, m = sum k, position) versus the CPU oracle, and the state hand-off from a
chunked prefill to single-token decode steps versus one chunked pass over all tokens.

Tolerance: relative L2 <= 2e-3 for the bf16 output; the fp32 states, computed in fp32 end to end,
are held to 2e-4."""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ccq_oracle as O
from tests._util import bf, l2n, rel

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-3
TOL_STATE = 2e-4


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


def _cache(N, H, K, V, gen, pos):
    S = torch.randn(N, H, K, V, generator=gen) * 0.1
    kk = l2n(torch.randn(N, H, pos, K, generator=gen))
    C = kk.transpose(-1, -2) @ kk                 # sum of k k^T over `pos` earlier tokens
    m = kk.sum(-2)
    return S.float(), C.float(), m.float()


DECODE_CASES = [
    # B, T, H, K, V, pos, subtract_mean, backbone
    (3, 1, 2, 64, 64, 37, True, "gdn"),
    (2, 3, 2, 128, 128, 100, True, "gdn"),
    (2, 1, 4, 256, 512, 500, True, "gdn"),
    (2, 2, 2, 128, 64, 9, False, "gdn"),
    (3, 1, 2, 128, 256, 37, True, "gla"),
    (2, 3, 2, 256, 128, 70, True, "gla"),
    # head sizes between the kernels' (zero-padded to K = 64 / 128, V = 128, results sliced back)
    (2, 2, 2, 40, 72, 11, True, "gdn"),
    (2, 1, 2, 96, 100, 30, True, "gla"),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=[str(i) for i in range(len(DECODE_CASES))])
def test_decode_step(case):
    dev = _cuda()
    from ccq_amd import fused_recurrent_ccq_gdn, fused_recurrent_ccq_gla
    B, T, H, K, V, pos, sub, bb = case
    gen = torch.Generator().manual_seed(7)
    # q, k already l2-normalised and bf16 (the kernel's normalisation is checked by the hand-off test)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    v = bf(torch.randn(B, T, H, V, generator=gen))
    lam = bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen)))
    S, C, m = _cache(B, H, K, V, gen, pos)
    d = torch.float64
    print(f"test_decode_step {case}", flush=True)
    if bb == "gdn":
        a_log = torch.empty(H).uniform_(0.0, math.log(16.0), generator=gen)
        g = (-F.softplus(torch.randn(B, T, H, generator=gen)) * a_log.exp() * 0.1).float()
        beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float()
        o_r, S_r, C_r, m_r, _ = O.ccq_decode_gdn(q.to(d), k.to(d), v.to(d), lam.to(d).squeeze(-1), g.to(d),
                                                 beta.to(d), S.to(d), C.to(d), m.to(d), pos, subtract_mean=sub,
                                                 use_qk_l2norm=False)
        with torch.no_grad():
            o, S2, C2, m2 = fused_recurrent_ccq_gdn(
                q.to(dev), k.to(dev), v.to(dev), lam.to(dev), g=g.to(dev), beta=beta.to(dev),
                initial_state=S.to(dev), initial_cov_state=C.to(dev), initial_mean_state=m.to(dev),
                output_final_state=True, use_qk_l2norm_in_kernel=False, position_offset=pos, subtract_mean=sub)
    else:
        gk = (F.logsigmoid(torch.randn(B, T, H, K, generator=gen)) / 16).float()
        # the GLA op always l2-normalises; q and k are unit rows already, so this is a rounding no-op
        o_r, S_r, C_r, m_r, _ = O.ccq_decode_gla(q.to(d), k.to(d), v.to(d), lam.to(d).squeeze(-1), gk.to(d),
                                                 S.to(d), C.to(d), m.to(d), pos, subtract_mean=sub)
        with torch.no_grad():
            o, S2, C2, m2 = fused_recurrent_ccq_gla(
                q.to(dev), k.to(dev), v.to(dev), lam.to(dev), gk=gk.to(dev), initial_state=S.to(dev),
                initial_cov_state=C.to(dev), initial_mean_state=m.to(dev), output_final_state=True,
                position_offset=pos, subtract_mean=sub)
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "S": rel(S2, S_r), "C": rel(C2, C_r)}
    if sub:
        errs["m"] = rel(m2, m_r)
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    assert errs["o"] <= TOL_BF16
    tol = TOL_STATE if bb == "gdn" else 1e-3  # GLA: q, k pass through the op's own l2norm (bf16 rounding)
    for n in ("S", "C", "m"):
        if n in errs:
            assert errs[n] <= tol, n


@pytest.mark.parametrize("bb", ["gdn", "gla"])
def test_prefill_then_decode_matches_one_pass(bb):
    """Chunked prefill of T0 tokens with final states, then T1 single-token decode calls carrying
    (S, C, m, position_offset) equal one chunked pass over T0 + T1 tokens (reference cache
    contract, ccq/gdn/layer.py:318-336, :394-400)."""
    dev = _cuda()
    from ccq_amd import fused_chunk_ccq_gdn, fused_chunk_ccq_gla, fused_recurrent_ccq_gdn, fused_recurrent_ccq_gla
    B, T0, T1, H, K, V = 2, 100, 3, 2, 128, 128
    T = T0 + T1
    gen = torch.Generator().manual_seed(11)
    q = bf(torch.randn(B, T, H, K, generator=gen)).to(dev)
    k = bf(torch.randn(B, T, H, K, generator=gen)).to(dev)
    v = bf(torch.randn(B, T, H, V, generator=gen)).to(dev)
    lam = bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen))).to(dev)
    print(f"test_prefill_then_decode_matches_one_pass {bb}", flush=True)
    with torch.no_grad():
        if bb == "gdn":
            g = (-F.softplus(torch.randn(B, T, H, generator=gen)) * 0.3).float().to(dev)
            beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float().to(dev)
            o_full, *_ = fused_chunk_ccq_gdn(q, k, v, lam, g, beta, use_qk_l2norm_in_kernel=True)
            o, S, C, m = fused_chunk_ccq_gdn(q[:, :T0], k[:, :T0], v[:, :T0], lam[:, :T0], g[:, :T0], beta[:, :T0],
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
            outs = [o]
            for t in range(T0, T):
                sl = slice(t, t + 1)
                o, S, C, m = fused_recurrent_ccq_gdn(q[:, sl], k[:, sl], v[:, sl], lam[:, sl], g=g[:, sl],
                                                     beta=beta[:, sl], initial_state=S, initial_cov_state=C,
                                                     initial_mean_state=m, output_final_state=True,
                                                     use_qk_l2norm_in_kernel=True, position_offset=t)
                outs.append(o)
        else:
            gk = (F.logsigmoid(torch.randn(B, T, H, K, generator=gen)) / 16).float().to(dev)
            o_full, *_ = fused_chunk_ccq_gla(q, k, v, lam, gk)
            o, S, C, m = fused_chunk_ccq_gla(q[:, :T0], k[:, :T0], v[:, :T0], lam[:, :T0], gk[:, :T0],
                                             output_final_state=True)
            outs = [o]
            for t in range(T0, T):
                sl = slice(t, t + 1)
                o, S, C, m = fused_recurrent_ccq_gla(q[:, sl], k[:, sl], v[:, sl], lam[:, sl], gk=gk[:, sl],
                                                     initial_state=S, initial_cov_state=C, initial_mean_state=m,
                                                     output_final_state=True, position_offset=t)
                outs.append(o)
    torch.cuda.synchronize()
    o_split = torch.cat(outs, 1)
    err_dec = rel(o_split[:, T0:], o_full[:, T0:].float())
    err_pre = rel(o_split[:, :T0], o_full[:, :T0].float())
    print(bb, f"prefill {err_pre:.2e} decode {err_dec:.2e}", flush=True)
    # the first T0 outputs do not depend on later tokens; GLA's split of the in-chunk decay at a
    # reference row inside the last (partial) chunk moves with its length, so only fp32 rounding differs
    assert err_pre <= 2e-4
    assert err_dec <= TOL_BF16


GLA_OPTION_CASES = [
    # B, T, H, K, V, gv, reverse, cu
    (2, 40, 2, 64, 128, True, False, None),
    (2, 40, 2, 64, 128, True, True, None),
    (1, 70, 2, 128, 64, False, True, [0, 30, 31, 70]),
]


@pytest.mark.parametrize("case", GLA_OPTION_CASES, ids=[str(i) for i in range(len(GLA_OPTION_CASES))])
def test_gla_recurrent_value_decay_and_reverse(case):
    """fused_recurrent_ccq_gla with the per-value decay gv and reverse=True (the reference forwards
    both to fla's fused_recurrent_gla, ccq/ops/ccq_gla/fused_recurrent.py:41-49): inference on the
    decode kernels, and with reverse also the gradients (the cleaning, then the GLA backbone on the
    time-reversed sequences), against the oracle."""
    dev = _cuda()
    from ccq_amd import fused_recurrent_ccq_gla
    B, T, H, K, V, use_gv, rev, cu = case
    print(f"gla option case {case}", flush=True)
    gen = torch.Generator().manual_seed(17)
    # unit rows already (the op's own l2norm rounds its output to bf16; on unit rows that is a no-op
    # up to rounding, so the fp64 oracle and the kernels see the same query and key)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    v = bf(torch.randn(B, T, H, V, generator=gen))
    lam = bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen)))
    gk = (F.logsigmoid(torch.randn(B, T, H, K, generator=gen)) / 16).float()
    gv = (F.logsigmoid(torch.randn(B, T, H, V, generator=gen)) / 16).float() if use_gv else None
    N = B if cu is None else len(cu) - 1
    S0 = (torch.randn(N, H, K, V, generator=gen) * 0.1).float()
    cu_t = torch.tensor(cu, dtype=torch.int64) if cu is not None else None
    d = torch.float64
    o_r, S_r, C_r, m_r, _ = O.ccq_decode_gla(q.to(d), k.to(d), v.to(d), lam.to(d).squeeze(-1), gk.to(d), S0.to(d),
                                             None, None, 0, gv=None if gv is None else gv.to(d), reverse=rev,
                                             cu_seqlens=cu_t)
    dv_ = lambda x: None if x is None else x.to(dev)  # noqa: E731
    with torch.no_grad():
        o, S2, C2, m2 = fused_recurrent_ccq_gla(q.to(dev), k.to(dev), v.to(dev), lam.to(dev), gk=gk.to(dev),
                                                gv=dv_(gv), initial_state=S0.to(dev), output_final_state=True,
                                                reverse=rev, cu_seqlens=dv_(cu_t))
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "S": rel(S2, S_r), "C": rel(C2, C_r), "m": rel(m2, m_r)}
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    assert errs["o"] <= TOL_BF16
    for n in ("S", "C", "m"):
        assert errs[n] <= 1e-3, n
    if not rev or use_gv:
        return
    # gradients through the reversed backbone.  This path hands the cleaned query to the backbone
    # in q's dtype, as the reference's _CCQCleanQ does (ccq/ops/common/clean.py): the oracle rounds
    # it to bf16 at the same place
    do = bf(torch.randn(B, T, H, V, generator=gen))
    xs = [x.to(d).requires_grad_() for x in (q, k, v)]
    qn, kn = O.l2norm(xs[0]), O.l2norm(xs[1])
    qc, _, _ = O.clean_fwd_bruteforce(qn, kn, lam.to(d).squeeze(-1), cu_seqlens=cu_t)
    o_r, _ = O.gla_recurrent(O.round_through(qc, torch.bfloat16), kn, xs[2], gk.to(d), h0=S0.to(d), reverse=True,
                             cu_seqlens=cu_t)
    g_r = torch.autograd.grad(o_r, xs, do.to(d))
    xg = [x.to(dev).requires_grad_() for x in (q, k, v)]
    o, _, _, _ = fused_recurrent_ccq_gla(xg[0], xg[1], xg[2], lam.to(dev), gk=gk.to(dev), initial_state=S0.to(dev),
                                         reverse=True, cu_seqlens=dv_(cu_t))
    g = torch.autograd.grad(o, xg, do.to(dev).to(o.dtype))
    gerrs = {n: rel(a, b) for n, a, b in zip(("dq", "dk", "dv"), g, g_r)}
    print("grads", {n: f"{e:.2e}" for n, e in gerrs.items()}, flush=True)
    assert rel(o, o_r) <= TOL_BF16
    # the gradient of the cleaned query also crosses back from the backbone in bf16 (as fla returns
    # it in q's dtype to the reference's _CCQCleanQ): one more bf16 rounding (2^-9 relative) on dq
    # and dk than the fused path has, against an oracle whose gradients stay in fp64
    for n, e in gerrs.items():
        assert e <= 4e-3, n


def test_gdn_recurrent_key_value_decays():
    """fused_recurrent_ccq_gdn with the per-key / per-value decays gk, gv (forwarded by the
    reference to fla's fused_recurrent_gated_delta_rule, ccq/ops/ccq_gdn/fused_recurrent.py:66-74)
    on the decode kernels, against the oracle."""
    dev = _cuda()
    from ccq_amd import fused_recurrent_ccq_gdn
    B, T, H, K, V, pos = 2, 5, 2, 128, 128, 33
    gen = torch.Generator().manual_seed(23)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    v = bf(torch.randn(B, T, H, V, generator=gen))
    lam = bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen)))
    g = (-F.softplus(torch.randn(B, T, H, generator=gen)) * 0.3).float()
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float()
    gk = (F.logsigmoid(torch.randn(B, T, H, K, generator=gen)) / 8).float()
    gv = (F.logsigmoid(torch.randn(B, T, H, V, generator=gen)) / 8).float()
    S, C, m = _cache(B, H, K, V, gen, pos)
    d = torch.float64
    print("gdn gk/gv decode", flush=True)
    o_r, S_r, C_r, m_r, _ = O.ccq_decode_gdn(q.to(d), k.to(d), v.to(d), lam.to(d).squeeze(-1), g.to(d), beta.to(d),
                                             S.to(d), C.to(d), m.to(d), pos, use_qk_l2norm=False, gk=gk.to(d),
                                             gv=gv.to(d))
    with torch.no_grad():
        o, S2, C2, m2 = fused_recurrent_ccq_gdn(q.to(dev), k.to(dev), v.to(dev), lam.to(dev), g=g.to(dev),
                                                gk=gk.to(dev), gv=gv.to(dev), beta=beta.to(dev),
                                                initial_state=S.to(dev), initial_cov_state=C.to(dev),
                                                initial_mean_state=m.to(dev), output_final_state=True,
                                                position_offset=pos)
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "S": rel(S2, S_r), "C": rel(C2, C_r), "m": rel(m2, m_r)}
    print({n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    assert errs["o"] <= TOL_BF16
    for n in ("S", "C", "m"):
        assert errs[n] <= TOL_STATE, n
    with pytest.raises(NotImplementedError):
        fused_recurrent_ccq_gdn(q.to(dev).requires_grad_(), k.to(dev), v.to(dev), lam.to(dev), g=g.to(dev),
                                gk=gk.to(dev), beta=beta.to(dev))
