"""GPU checks of the public entry points that the layers do not reach directly, against the float64
CPU oracle on the same bf16-rounded inputs:

* ``fused_ccq_clean`` (reference ``ccq/ops/ccq_gdn/fused_clean.py:34-83``): l2norm, cleaning, final
  states, and the gradients of the reference's ``_CCQCleanQ`` pipeline -- q, k, lambda and the
  covariance states differentiated; the initial key sum not, and the final key sum's upstream gradient
  ignored (``ccq/ops/common/clean.py:691-748``);
* ``chunk_ccq_gdn`` called directly, with ``transpose_state_layout`` (backbone states ``[N, H, V, K]``,
  fla's option, ``ccq/ops/ccq_gdn/chunk.py:12-32``), and the same key-sum gradient rule, against
  ``fused_chunk_ccq_gdn``, whose gradients include the key sums (``fused_read.py:494-514``);
* ``chunk_ccq_gla`` called directly (``ccq/ops/ccq_gla/chunk.py:17-59``), with states;
* ``fused_recurrent_ccq_gdn`` in decode with ``transpose_state_layout``.

Tolerance (north star): relative L2 <= 2e-3 on bf16 outputs and gradients; fp32 states and
state gradients <= 1e-4.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import ccq_oracle as O
from tests._util import bf, gdn_inputs, l2n, rel, round_both

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-3
TOL_STATE = 1e-4
D = torch.float64


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401  (fails loudly if the library is missing)
    return torch.device("cuda")


def _spd(N, H, K, gen):
    a = torch.randn(N, H, K, 4, generator=gen)
    return (a @ a.transpose(-1, -2)).float()


def _check(case, errs, state_names=()):
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= (TOL_STATE if n in state_names else TOL_BF16), n


def test_fused_ccq_clean():
    dev = _cuda()
    from ccq_amd import fused_ccq_clean
    B, T, H, K, pos = 2, 150, 2, 64, 5
    print(f"test_fused_ccq_clean B={B} T={T} H={H} K={K}", flush=True)
    gen = torch.Generator().manual_seed(31)
    q = bf(torch.randn(B, T, H, K, generator=gen))   # un-normalised: use_qk_l2norm_in_kernel normalises
    k = bf(torch.randn(B, T, H, K, generator=gen))
    lam = bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen)))
    h0 = _spd(B, H, K, gen)
    m0 = torch.randn(B, H, K, generator=gen)
    dqc = bf(torch.randn(B, T, H, K, generator=gen))
    dhf = torch.randn(B, H, K, K, generator=gen) * 0.01
    dmf = torch.randn(B, H, K, generator=gen)

    r = {n: t.to(D).requires_grad_() for n, t in dict(q=q, k=k, lam=lam, h0=h0, m0=m0).items()}
    # the normalised q, k cross from the l2norm to the cleaning as bf16 tensors, value and gradient
    qn, kn = round_both(O.l2norm(r["q"])), round_both(O.l2norm(r["k"]))
    qc_r, hf_r, mf_r = O.clean_fwd_chunked(qn, kn, r["lam"], position_offset=pos, h0=r["h0"], m0=r["m0"].detach())
    # the final key sum's gradient is not taken (detached), the initial key sum is not differentiated
    ((qc_r * dqc.to(D)).sum() + (hf_r * dhf.to(D)).sum() + (mf_r.detach() * dmf.to(D)).sum()).backward()

    x = {n: t.to(dev).requires_grad_() for n, t in dict(q=q, k=k, lam=lam, h0=h0, m0=m0).items()}
    qc, k_out, hf, mf, flag = fused_ccq_clean(x["q"], x["k"], x["lam"], initial_cov_state=x["h0"],
                                              initial_mean_state=x["m0"], output_final_state=True,
                                              use_qk_l2norm_in_kernel=True, position_offset=pos)
    assert flag is False
    loss = (qc.float() * dqc.to(dev).float()).sum() + (hf * dhf.to(dev)).sum()
    if mf.requires_grad:
        loss = loss + (mf * dmf.to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    assert not mf.requires_grad, "the final key sum carries no gradient on this path"
    assert x["m0"].grad is None, "the initial key sum is not differentiated on this path"
    errs = {"q_clean": rel(qc, qc_r), "k": rel(k_out, kn), "C": rel(hf, hf_r), "m": rel(mf, mf_r),
            "dq": rel(x["q"].grad, r["q"].grad), "dk": rel(x["k"].grad, r["k"].grad),
            "dh0": rel(x["h0"].grad, r["h0"].grad)}
    # d(lambda) comes back in lambda's dtype (bf16), as the reference returns it
    errs["dlam"] = rel(x["lam"].grad, r["lam"].grad.to(torch.bfloat16))
    _check("fused_ccq_clean", errs, ("C", "m", "dh0"))


def test_chunk_ccq_gdn_transposed_states_and_key_sum_gradients():
    dev = _cuda()
    from ccq_amd import chunk_ccq_gdn, fused_chunk_ccq_gdn
    B, T, H, K, V = 2, 200, 2, 128, 128
    print(f"test_chunk_ccq_gdn B={B} T={T} H={H} K={K} V={V}", flush=True)
    x, gen = gdn_inputs(B, T, H, K, V, seed=32, with_state=True, device="cpu")
    lam = torch.sigmoid(torch.randn(B, T, H, 1, generator=gen))
    h0, m0 = _spd(B, H, K, gen), torch.randn(B, H, K, generator=gen)
    do = bf(torch.randn(B, T, H, V, generator=gen))
    dsf = torch.randn(B, H, K, V, generator=gen) * 0.1
    dmf = torch.randn(B, H, K, generator=gen)

    names = ("q", "k", "v", "g", "beta", "s0")
    r = {n: x[n].to(D).requires_grad_() for n in names}
    o_r, s_r, c_r, m_r = O.ccq_gdn_forward(r["q"], r["k"], r["v"], O.round_through(lam.to(D), torch.bfloat16),
                                           r["g"], r["beta"], h0=r["s0"], h0_cov=h0.to(D), m0=m0.to(D))
    ((o_r * do.to(D)).sum() + (s_r * dsf.to(D)).sum()).backward()

    def run(op, transpose):
        g = {n: x[n].to(dev).requires_grad_() for n in names}
        m0g = m0.to(dev).requires_grad_()
        s0 = g["s0"].transpose(-1, -2) if transpose else g["s0"]      # [N, H, V, K] when transposed
        kw = dict(transpose_state_layout=True) if transpose else {}
        o, s, c, m = op(g["q"], g["k"], g["v"], lam.to(dev), g["g"], g["beta"], initial_state=s0,
                        initial_cov_state=h0.to(dev), initial_mean_state=m0g, output_final_state=True, **kw)
        s_kv = s.transpose(-1, -2) if transpose else s
        loss = (o.float() * do.to(dev).float()).sum() + (s_kv * dsf.to(dev)).sum()
        if m.requires_grad:
            loss = loss + (m * dmf.to(dev)).sum()
        loss.backward()
        torch.cuda.synchronize()
        return o, s, s_kv, c, m, g, m0g

    o, s, s_kv, c, m, g, m0g = run(chunk_ccq_gdn, True)
    assert s.shape == (B, H, V, K), "transpose_state_layout returns [N, H, V, K] states"
    assert m0g.grad is None and not m.requires_grad, "stock chunk mode: no key-sum gradients"
    errs = {"o": rel(o, o_r), "S": rel(s_kv, s_r), "C": rel(c, c_r), "m": rel(m, m_r)}
    for n in names:
        errs["d" + n] = rel(g[n].grad, r[n].grad)
    _check("chunk_ccq_gdn transposed", errs, ("S", "C", "m"))

    # the fused path differentiates the key sums: the same outputs, a gradient for the initial key sum,
    # and with the final key sum's gradient in the loss only dk changes (m_final = m0 + sum of the keys)
    o2, s2, _, _, m2, g2, m0g2 = run(fused_chunk_ccq_gdn, False)
    assert m0g2.grad is not None and m2.requires_grad
    assert torch.equal(o2, o) and torch.equal(s2, s_kv)
    for n in ("q", "v", "g", "beta", "s0"):
        assert rel(g2[n].grad, g[n].grad) <= 1e-6, n
    assert rel(g2["k"].grad, g["k"].grad) > 1e-3


def test_chunk_ccq_gla_direct():
    dev = _cuda()
    from ccq_amd import chunk_ccq_gla
    B, T, H, K, V = 2, 170, 2, 64, 128
    print(f"test_chunk_ccq_gla B={B} T={T} H={H} K={K} V={V}", flush=True)
    gen = torch.Generator().manual_seed(33)
    x = {
        "q": bf(torch.randn(B, T, H, K, generator=gen)),
        "k": bf(torch.randn(B, T, H, K, generator=gen)),
        "v": bf(torch.randn(B, T, H, V, generator=gen)),
        "gk": (F.logsigmoid(torch.randn(B, T, H, K, generator=gen) * 2.0) / 16).float(),
        "s0": torch.randn(B, H, K, V, generator=gen) * 0.1,
    }
    lam = bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen)))
    h0 = _spd(B, H, K, gen)
    do = bf(torch.randn(B, T, H, V, generator=gen))
    dsf = torch.randn(B, H, K, V, generator=gen) * 0.1
    r = {n: t.to(D).requires_grad_() for n, t in x.items()}
    o_r, s_r, c_r, _ = O.ccq_gla_forward(r["q"], r["k"], r["v"], lam.to(D), r["gk"], h0=r["s0"], h0_cov=h0.to(D),
                                         position_offset=3, l2norm_dtype=torch.bfloat16)
    ((o_r * do.to(D)).sum() + (s_r * dsf.to(D)).sum()).backward()
    g = {n: t.to(dev).requires_grad_() for n, t in x.items()}
    o, s, c, m = chunk_ccq_gla(g["q"], g["k"], g["v"], lam.to(dev), g["gk"], initial_state=g["s0"],
                               initial_cov_state=h0.to(dev), output_final_state=True, position_offset=3)
    ((o.float() * do.to(dev).float()).sum() + (s * dsf.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "S": rel(s, s_r), "C": rel(c, c_r)}
    for n in x:
        errs["d" + n] = rel(g[n].grad, r[n].grad)
    _check("chunk_ccq_gla", errs, ("S", "C"))


def test_recurrent_gdn_transposed_state_layout():
    dev = _cuda()
    from ccq_amd import fused_recurrent_ccq_gdn
    B, T, H, K, V, pos = 2, 3, 2, 128, 256, 40
    print("test_recurrent_gdn_transposed_state_layout", flush=True)
    gen = torch.Generator().manual_seed(34)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen))).to(dev)
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen))).to(dev)
    v = bf(torch.randn(B, T, H, V, generator=gen)).to(dev)
    lam = torch.sigmoid(torch.randn(B, T, H, 1, generator=gen)).to(dev)
    g = (-F.softplus(torch.randn(B, T, H, generator=gen)) * 0.3).float().to(dev)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float().to(dev)
    S = (torch.randn(B, H, K, V, generator=gen) * 0.1).to(dev)
    C = _spd(B, H, K, gen).to(dev)
    m = torch.randn(B, H, K, generator=gen).to(dev)
    with torch.no_grad():
        common = dict(g=g, beta=beta, initial_cov_state=C, initial_mean_state=m, output_final_state=True,
                      position_offset=pos)
        o1, s1, c1, m1 = fused_recurrent_ccq_gdn(q, k, v, lam, initial_state=S, **common)
        o2, s2, c2, m2 = fused_recurrent_ccq_gdn(q, k, v, lam, initial_state=S.transpose(-1, -2).contiguous(),
                                                 transpose_state_layout=True, **common)
    torch.cuda.synchronize()
    assert s2.shape == (B, H, V, K)
    assert torch.equal(o1, o2) and torch.equal(s1, s2.transpose(-1, -2)) and torch.equal(c1, c2)
    assert torch.equal(m1, m2)
