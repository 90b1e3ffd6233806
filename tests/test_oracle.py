"""Pins the CPU oracle (oracle/ccq_oracle.py) without trusting its own formulas.

The reference ships no tests, golden vectors or fixtures (it has no tests/ at all), so each
oracle function is pinned by what the mathematics fixes: closed forms on special inputs,
invariants (chunk size, packing, state hand-off), agreement between independently written
forms (per-token loops vs chunked algebra), and finite differences for the gradients.  Each
check is chosen so that a plausible mistake (a dropped mean term, 1/pos instead of 1/pos^2,
a transposed state, a wrong decay exponent) fails it.
"""

import math

import pytest
import torch

from oracle import ccq_oracle as O

D = torch.float64


def _qk(B, T, H, K, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = O.l2norm(torch.randn(B, T, H, K, generator=g, dtype=D))
    k = O.l2norm(torch.randn(B, T, H, K, generator=g, dtype=D))
    lam = torch.rand(B, T, H, generator=g, dtype=D)
    return q, k, lam, g


# ----------------------------------------------------------------------------- cleaning


def test_lambda_zero_is_identity():
    q, k, _, _ = _qk(2, 50, 2, 8)
    for fn in (O.clean_fwd_bruteforce, O.clean_fwd_chunked):
        out, _, _ = fn(q, k, 0.0)
        assert torch.equal(out, q)


def test_first_token_has_zero_covariance():
    # t = 1 with the mean term: Sigma_1 = k k^T - k k^T = 0, so q_clean_1 = q_1 (a dropped or
    # mis-scaled mean term breaks this)
    q, k, lam, _ = _qk(1, 5, 3, 16)
    out, _, _ = O.clean_fwd_bruteforce(q, k, lam)
    assert torch.allclose(out[:, 0], q[:, 0], atol=1e-14)


def test_identical_keys_have_zero_covariance():
    q, k, lam, _ = _qk(1, 40, 2, 16)
    k = k[:, :1].expand_as(k).clone()
    for fn in (O.clean_fwd_bruteforce, O.clean_fwd_chunked):
        out, _, _ = fn(q, k, lam)
        assert torch.allclose(out, q, atol=1e-12)


def test_orthonormal_keys_closed_form():
    # keys e_1..e_T: Sigma_t = diag(1_{<=t})/t - 1_{<=t} 1_{<=t}^T / t^2
    T, K = 12, 16
    q, _, lam, _ = _qk(1, T, 1, K)
    k = torch.zeros(1, T, 1, K, dtype=D)
    for t in range(T):
        k[0, t, 0, t] = 1.0
    out, _, _ = O.clean_fwd_chunked(q, k, lam, BT=4)
    for t in range(T):
        n = t + 1
        ind = torch.zeros(K, dtype=D)
        ind[:n] = 1.0
        sigma = torch.diag(ind) / n - torch.outer(ind, ind) / n ** 2
        expect = q[0, t, 0] - lam[0, t, 0] * (sigma @ q[0, t, 0])
        assert torch.allclose(out[0, t, 0], expect, atol=1e-13)


def test_no_mean_term_closed_form():
    q, k, lam, _ = _qk(1, 30, 2, 8)
    out, _, _ = O.clean_fwd_chunked(q, k, lam, subtract_mean=False, BT=8)
    C = torch.zeros(2, 8, 8, dtype=D)
    for t in range(30):
        C = C + torch.einsum("ha,hb->hab", k[0, t], k[0, t])
        expect = q[0, t] - lam[0, t][:, None] * torch.einsum("hab,ha->hb", C, q[0, t]) / (t + 1)
        assert torch.allclose(out[0, t], expect, atol=1e-13)


@pytest.mark.parametrize("bt", [16, 32, 64])
def test_chunk_size_independence(bt):
    q, k, lam, _ = _qk(2, 130, 2, 16)
    ref = O.clean_fwd_bruteforce(q, k, lam, position_offset=3)
    got = O.clean_fwd_chunked(q, k, lam, position_offset=3, BT=bt)
    for a, b in zip(got, ref):
        assert torch.allclose(a, b, atol=1e-12)


def test_varlen_equals_separate_runs():
    q, k, lam, _ = _qk(1, 90, 2, 8)
    cu = torch.tensor([0, 17, 60, 90])
    out, hf, mf = O.clean_fwd_chunked(q, k, lam, cu_seqlens=cu, BT=16)
    for n in range(3):
        s, e = int(cu[n]), int(cu[n + 1])
        o1, h1, m1 = O.clean_fwd_chunked(q[:, s:e], k[:, s:e], lam[:, s:e], BT=16)
        assert torch.allclose(out[:, s:e], o1, atol=1e-12)
        assert torch.allclose(hf[n], h1[0], atol=1e-12)
        assert torch.allclose(mf[n], m1[0], atol=1e-12)


def test_state_handoff_equals_full_run():
    q, k, lam, _ = _qk(2, 100, 2, 8)
    full = O.clean_fwd_chunked(q, k, lam, BT=16)
    t1 = 37
    a = O.clean_fwd_chunked(q[:, :t1], k[:, :t1], lam[:, :t1], BT=16)
    b = O.clean_fwd_chunked(q[:, t1:], k[:, t1:], lam[:, t1:], h0=a[1], m0=a[2], position_offset=t1, BT=16)
    assert torch.allclose(torch.cat([a[0], b[0]], 1), full[0], atol=1e-12)
    assert torch.allclose(b[1], full[1], atol=1e-12)
    assert torch.allclose(b[2], full[2], atol=1e-12)


def test_positions_clamp_and_segments():
    cu = torch.tensor([0, 3, 7])
    p = O.positions(7, cu, position_offset=-2)
    assert p.tolist() == [1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 2.0]


@pytest.mark.parametrize("sub", [True, False])
def test_closed_form_backward_matches_autograd(sub):
    q, k, lam, g = _qk(2, 45, 2, 8, seed=4)
    h0 = torch.randn(2, 2, 8, 3, generator=g, dtype=D)
    h0 = h0 @ h0.transpose(-1, -2)
    m0 = torch.randn(2, 2, 8, generator=g, dtype=D)
    dqc = torch.randn(2, 45, 2, 8, generator=g, dtype=D)
    dhf = torch.randn(2, 2, 8, 8, generator=g, dtype=D)
    dmf = torch.randn(2, 2, 8, generator=g, dtype=D)
    leaves = [t.clone().requires_grad_() for t in (q, k, lam, h0, m0)]
    out, hf, mf = O.clean_fwd_bruteforce(*leaves[:3], position_offset=2, h0=leaves[3], m0=leaves[4],
                                         subtract_mean=sub)
    loss = (out * dqc).sum() + (hf * dhf).sum() + ((mf * dmf).sum() if sub else 0.0)
    loss.backward()
    got = O.clean_bwd_closed(q, k, lam, dqc, position_offset=2, h0=h0, m0=m0, subtract_mean=sub, dh_final=dhf,
                             dm_final=dmf if sub else None, BT=16)
    names = ["dq", "dk", "dlam", "dh0", "dm0"]
    for i, (name, a) in enumerate(zip(names, got)):
        if a is None:
            assert not sub and name == "dm0"
            continue
        assert torch.allclose(a, leaves[i].grad, atol=1e-11), name


def test_cleaning_gradcheck_finite_differences():
    q, k, lam, _ = _qk(1, 6, 1, 4, seed=5)
    leaves = [t.clone().requires_grad_() for t in (q, k, lam)]
    assert torch.autograd.gradcheck(lambda a, b, c: O.clean_fwd_chunked(a, b, c, BT=4)[0], leaves)


# ----------------------------------------------------------------------------- backbones


def _gdn_in(B, T, H, K, V, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = O.l2norm(torch.randn(B, T, H, K, generator=g, dtype=D))
    k = O.l2norm(torch.randn(B, T, H, K, generator=g, dtype=D))
    v = torch.randn(B, T, H, V, generator=g, dtype=D)
    gg = -torch.rand(B, T, H, generator=g, dtype=D)
    beta = torch.rand(B, T, H, generator=g, dtype=D)
    s0 = torch.randn(B, H, K, V, generator=g, dtype=D)
    return q, k, v, gg, beta, s0


def test_gdn_chunked_equals_recurrence_with_grads():
    q, k, v, g, beta, s0 = _gdn_in(2, 70, 2, 8, 6)
    leaves1 = [t.clone().requires_grad_() for t in (q, k, v, g, beta, s0)]
    leaves2 = [t.clone().requires_grad_() for t in (q, k, v, g, beta, s0)]
    o1, s1 = O.gdn_recurrent(*leaves1[:5], h0=leaves1[5])
    o2, s2 = O.gdn_chunked(*leaves2[:5], h0=leaves2[5], BT=16)
    assert torch.allclose(o1, o2, atol=1e-11) and torch.allclose(s1, s2, atol=1e-11)
    w = torch.randn_like(o1)
    ((o1 * w).sum() + s1.sum()).backward()
    ((o2 * w).sum() + s2.sum()).backward()
    for a, b in zip(leaves1, leaves2):
        assert torch.allclose(a.grad, b.grad, atol=1e-10)


def test_gdn_beta_zero_only_decays():
    q, k, v, g, beta, s0 = _gdn_in(1, 20, 2, 4, 3)
    o, s = O.gdn_chunked(q, k, v, g, torch.zeros_like(beta), h0=s0, BT=8)
    G = torch.cumsum(g, 1)
    assert torch.allclose(s, torch.exp(G[:, -1])[..., None, None] * s0, atol=1e-13)
    expect = 0.5 * torch.exp(G)[..., None] * torch.einsum("bhkv,bthk->bthv", s0, q)
    assert torch.allclose(o, expect, atol=1e-13)


def test_gdn_orthonormal_memory_readback():
    # g = 0, beta = 1, keys e_j: the delta rule stores v_j at e_j; a later query e_i reads scale * v_i
    K, V, T = 8, 3, 6
    k = torch.zeros(1, T, 1, K, dtype=D)
    for t in range(T):
        k[0, t, 0, t] = 1.0
    q = torch.zeros_like(k)
    q[0, :, 0, 0] = 1.0  # always read slot 0
    v = torch.randn(1, T, 1, V, dtype=D)
    o, _ = O.gdn_chunked(q, k, v, torch.zeros(1, T, 1, dtype=D), torch.ones(1, T, 1, dtype=D), scale=1.0, BT=4)
    assert torch.allclose(o[0, :, 0], v[0, 0, 0].expand(T, V), atol=1e-13)


def test_gdn_delta_rule_overwrites():
    # the same key written twice with beta = 1 keeps only the second value
    K, V = 4, 2
    k = torch.zeros(1, 2, 1, K, dtype=D)
    k[0, :, 0, 1] = 1.0
    v = torch.tensor([[[[1.0, 2.0]], [[-3.0, 5.0]]]], dtype=D)
    _, s = O.gdn_recurrent(k, k, v, torch.zeros(1, 2, 1, dtype=D), torch.ones(1, 2, 1, dtype=D))
    assert torch.allclose(s[0, 0, 1], v[0, 1, 0], atol=1e-14)


def test_gdn_decayed_prediction_closed_form():
    # q_t = k_t (unit keys), scale 1: o_t = S_t^T k_t.  With S_{-1} = s0 and any g, beta:
    #   o_0 = (1 - b0) a0 s0^T k0 + b0 v0
    #   o_1 = (1 - b1) a1 S_0^T k1 + b1 v1,  S_0^T k1 = a0 s0^T k1 + b0 (v0 - a0 s0^T k0) (k0 . k1)
    # The prediction inside the write must use the decayed state: an undecayed prediction, a
    # missing (1 - beta) or a transposed state each break it.
    q, k, v, g, beta, s0 = _gdn_in(1, 2, 3, 8, 5, seed=11)
    g = g * 3.0  # strong decay, well away from 1
    a = torch.exp(g)
    for fn in (O.gdn_recurrent, O.gdn_chunked):
        o, _ = fn(k, k, v, g, beta, scale=1.0, h0=s0)
        for h in range(3):
            k0, k1, v0, v1 = k[0, 0, h], k[0, 1, h], v[0, 0, h], v[0, 1, h]
            a0, a1, b0, b1 = a[0, 0, h], a[0, 1, h], beta[0, 0, h], beta[0, 1, h]
            S = s0[0, h]
            e0 = (1 - b0) * a0 * (S.T @ k0) + b0 * v0
            S0k1 = a0 * (S.T @ k1) + b0 * (v0 - a0 * (S.T @ k0)) * (k0 @ k1)
            e1 = (1 - b1) * a1 * S0k1 + b1 * v1
            assert torch.allclose(o[0, 0, h], e0, atol=1e-13), fn.__name__
            assert torch.allclose(o[0, 1, h], e1, atol=1e-13), fn.__name__


def test_gdn_overwrite_with_decay():
    # beta = 1 and a unit key: S_t^T k_t = v_t exactly, whatever the decay and the history
    q, k, v, g, beta, s0 = _gdn_in(1, 37, 2, 8, 4, seed=12)
    beta = torch.ones_like(beta)
    for fn in (O.gdn_recurrent, lambda *a, **kw: O.gdn_chunked(*a, BT=16, **kw)):
        o, _ = fn(k, k, v, g * 4.0, beta, scale=1.0, h0=s0)
        assert torch.allclose(o, v, atol=1e-12)


def test_gla_single_write_decayed_readback():
    # one write at t = 0 (k_t = 0 afterwards): S_t = diag(e^{G_t - G_0}) k_0 v_0^T, so
    # o_t = scale (q_t . (k_0 o e^{G_t - G_0})) v_0, with G the running sum of gk (decay applied
    # before the write of the same step)
    B, T, H, K, V = 1, 70, 2, 8, 3
    g = torch.Generator().manual_seed(13)
    q = torch.randn(B, T, H, K, generator=g, dtype=D)
    k = torch.zeros(B, T, H, K, dtype=D)
    k[:, 0] = torch.randn(B, H, K, generator=g, dtype=D)
    v = torch.randn(B, T, H, V, generator=g, dtype=D)
    gk = torch.nn.functional.logsigmoid(torch.randn(B, T, H, K, generator=g, dtype=D)) / 4
    G = torch.cumsum(gk, 1)
    decay = torch.exp(G - G[:, :1])                                  # [B,T,H,K]
    expect = (8 ** -0.5) * (q * decay * k[:, :1]).sum(-1, keepdim=True) * v[:, :1]
    for fn in (O.gla_recurrent, lambda *a, **kw: O.gla_chunked(*a, BT=16, **kw)):
        o, s = fn(q, k, v, gk)
        assert torch.allclose(o, expect, atol=1e-13)
        assert torch.allclose(s[0], (decay[0, -1][..., None] * k[0, 0][..., None]) * v[0, 0][:, None, :],
                              atol=1e-13)


def test_gla_no_decay_is_masked_linear_attention():
    q, k, v, _, _, _ = _gdn_in(1, 40, 2, 8, 5)
    o, _ = O.gla_chunked(q, k, v, None, BT=16)
    att = torch.einsum("bthk,bshk->bhts", q, k) * torch.tril(torch.ones(40, 40, dtype=D))
    expect = 8 ** -0.5 * torch.einsum("bhts,bshv->bthv", att, v)
    assert torch.allclose(o, expect, atol=1e-12)


def test_gla_chunked_equals_recurrence():
    q, k, v, _, _, s0 = _gdn_in(2, 70, 2, 8, 6)
    gk = torch.nn.functional.logsigmoid(torch.randn(2, 70, 2, 8, dtype=D)) / 16
    o1, s1 = O.gla_recurrent(q, k, v, gk, h0=s0)
    o2, s2 = O.gla_chunked(q, k, v, gk, h0=s0, BT=16)
    assert torch.allclose(o1, o2, atol=1e-11) and torch.allclose(s1, s2, atol=1e-11)


def test_decode_steps_equal_prefill():
    q, k, v, g, beta, _ = _gdn_in(1, 40, 2, 8, 8, seed=7)
    lam = torch.rand(1, 40, 2, dtype=D)
    o_full, s_full, c_full, m_full = O.ccq_gdn_forward(q, k, v, lam, g, beta, use_qk_l2norm=True)
    S = torch.zeros(1, 2, 8, 8, dtype=D)
    C = torch.zeros(1, 2, 8, 8, dtype=D)
    m = torch.zeros(1, 2, 8, dtype=D)
    pos = 0
    outs = []
    for t in range(40):
        sl = slice(t, t + 1)
        o, S, C, m, pos = O.ccq_decode_gdn(q[:, sl], k[:, sl], v[:, sl], lam[:, sl], g[:, sl], beta[:, sl], S, C, m,
                                           pos)
        outs.append(o)
    assert torch.allclose(torch.cat(outs, 1), o_full, atol=1e-11)
    assert torch.allclose(S, s_full, atol=1e-11) and torch.allclose(C, c_full, atol=1e-11)
    assert torch.allclose(m, m_full, atol=1e-11) and pos == 40


def test_l2norm_matches_normalize():
    x = torch.randn(5, 7, 32, dtype=D)
    assert torch.allclose(O.l2norm(x, eps=0.0), torch.nn.functional.normalize(x, dim=-1), atol=1e-14)


def test_gate_weight_zero_is_sigmoid_bias():
    q = torch.randn(2, 5, 3, 4, dtype=D)
    b = torch.tensor([0.1, -2.0, 3.0], dtype=D)
    lam = O.lambda_gate(q, torch.zeros(3, 4, dtype=D), b)
    assert torch.allclose(lam, torch.sigmoid(b).expand(2, 5, 3))


def test_gate_one_hot_row_reads_one_coordinate():
    # W[h] = c_h e_{j_h}: the contraction W[h]·q_t,h must pick coordinate j_h of head h's own query,
    # scaled by c_h, so lambda = sigmoid(c_h q[b, t, h, j_h] + b_h).  A dropped or transposed
    # contraction, or one that mixes heads, fails this.
    B, T, H, K = 2, 6, 3, 5
    q = torch.randn(B, T, H, K, dtype=D)
    js, cs = [4, 0, 2], [1.0, -3.0, 0.5]
    w = torch.zeros(H, K, dtype=D)
    for h in range(H):
        w[h, js[h]] = cs[h]
    b = torch.tensor([0.25, -1.0, 2.0], dtype=D)
    lam = O.lambda_gate(q, w, b)
    want = torch.empty(B, T, H, dtype=D)
    for bb in range(B):
        for t in range(T):
            for h in range(H):
                want[bb, t, h] = 1.0 / (1.0 + math.exp(-(cs[h] * float(q[bb, t, h, js[h]]) + float(b[h]))))
    assert torch.allclose(lam, want, atol=1e-15)


def test_reshape_lambda_every_form_written_out():
    B, T, H = 2, 3, 2
    # python scalar and 0-d tensor: one value everywhere
    assert torch.equal(O.reshape_lambda(0.75, B, T, H), torch.full((B, T, H), 0.75, dtype=D))
    assert torch.equal(O.reshape_lambda(torch.tensor(0.5), B, T, H), torch.full((B, T, H), 0.5, dtype=D))
    # (H,): head h's value at every token
    lam_h = torch.tensor([0.1, 0.9])
    want = torch.tensor([[[0.1, 0.9]] * T] * B, dtype=D)
    assert torch.equal(O.reshape_lambda(lam_h, B, T, H), lam_h.to(D).expand(B, T, H))
    assert torch.equal(O.reshape_lambda(lam_h, B, T, H), want.to(torch.float32).to(D))
    # [B, T, H, 1]: the trailing unit dimension dropped, values kept in place
    lam4 = torch.arange(B * T * H, dtype=D).view(B, T, H, 1) / 10
    out = O.reshape_lambda(lam4, B, T, H)
    assert out.shape == (B, T, H)
    for bb in range(B):
        for t in range(T):
            for h in range(H):
                assert out[bb, t, h] == (bb * T * H + t * H + h) / 10
    # [B, T, H]: unchanged
    lam3 = torch.rand(B, T, H, dtype=D)
    assert torch.equal(O.reshape_lambda(lam3, B, T, H), lam3)


def test_round_through_keeps_gradient():
    x = torch.randn(10, dtype=D, requires_grad=True)
    y = O.round_through(x, torch.bfloat16)
    assert torch.equal(y.detach(), x.detach().to(torch.bfloat16).to(D))
    y.sum().backward()
    assert torch.equal(x.grad, torch.ones(10, dtype=D))


# ----------------------------------------------------------------------------- stock `chunk` blocks


def test_covariance_read_closed_form_and_gla_identity():
    # z_t = (h0 + sum_{j<=t} k_j k_j^T)^T q_t: with orthonormal keys e_1..e_T and no h0, z_t is the
    # projection of q_t onto span(e_1..e_t); and the read is GLA with v = k, no decay, scale 1.
    T, K = 5, 8
    k = torch.eye(K, dtype=D)[:T].view(1, T, 1, K)
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, T, 1, K, generator=g, dtype=D)
    z, hf = O.covariance_read(q, k)
    for t in range(T):
        expect = torch.zeros(K, dtype=D)
        expect[: t + 1] = q[0, t, 0, : t + 1]
        assert torch.allclose(z[0, t, 0], expect)
    assert torch.allclose(hf[0, 0], torch.diag(torch.tensor([1.0] * T + [0.0] * (K - T), dtype=D)))
    q2, k2, _, g2 = _qk(2, 40, 2, 8, seed=4)
    a = torch.randn(2, 2, 8, 8, generator=g2, dtype=D)
    z2, h2 = O.covariance_read(q2, k2, h0=a)
    zg, hg = O.gla_recurrent(q2, k2, k2, None, scale=1.0, h0=a)
    assert torch.allclose(z2, zg) and torch.allclose(h2, hg)


@pytest.mark.parametrize("sub", [True, False])
def test_clean_given_z_composes_to_bruteforce(sub):
    # the stock path (read, then clean given z) is the fused closed form, including m0, h0,
    # position offsets and varlen segments
    q, k, lam, g = _qk(1, 60, 2, 8, seed=5)
    cu = torch.tensor([0, 17, 18, 60])
    h0 = torch.randn(3, 2, 8, 8, generator=g, dtype=D)
    m0 = torch.randn(3, 2, 8, generator=g, dtype=D)
    z, hf = O.covariance_read(q, k, h0=h0, cu_seqlens=cu)
    qc, mf = O.clean_given_z(q, k, z, lam, position_offset=3, m0=m0, subtract_mean=sub, cu_seqlens=cu)
    ref, hr, mr = O.clean_fwd_bruteforce(q, k, lam, position_offset=3, h0=h0, m0=m0, subtract_mean=sub,
                                         cu_seqlens=cu)
    assert torch.allclose(qc, ref) and torch.allclose(hf, hr)
    if sub:
        assert torch.allclose(mf, mr)
    else:
        assert mf is None and mr is None



# ----------------------------------------------------------------------------- BASELINE C0


def test_c0_fp32_chunked_vs_fp64_bruteforce():
    """C0: the cleaning op alone on the CPU in fp32 (chunked path, gate lambda = sigma(W q + b)),
    B=1, T=512, H=4, d_k=64, chunk 64, seed 0, q and k ~ N(0, 1) L2-normalised, W ~ N(0, 0.02^2),
    b = 0, ones upstream gradient; q_clean, dq, dk, dW and db against the per-token fp64 loop."""
    B, T, H, K = 1, 512, 4, 64
    g = torch.Generator().manual_seed(0)
    q = O.l2norm(torch.randn(B, T, H, K, generator=g))
    k = O.l2norm(torch.randn(B, T, H, K, generator=g))
    w = torch.randn(H, K, generator=g) * 0.02
    b = torch.zeros(H)
    res = {}
    for dt, fn in ((torch.float32, O.clean_fwd_chunked), (D, O.clean_fwd_bruteforce)):
        leaves = [t.detach().to(dt).clone().requires_grad_() for t in (q, k, w, b)]
        lam = O.lambda_gate(leaves[0], leaves[2], leaves[3])
        qc, _, _ = fn(leaves[0], leaves[1], lam)
        qc.sum().backward()
        res[dt] = [qc.detach()] + [t.grad for t in leaves]
    for name, a, r in zip(("q_clean", "dq", "dk", "dW", "db"), res[torch.float32], res[D]):
        err = ((a.double() - r).norm() / r.norm()).item()
        assert err <= 1e-5, (name, err)


def test_gla_value_decay_single_write_readback():
    # gv only, one write at t = 0: S_t = k_0 (v_0 o e^{Gv_t - Gv_0})^T, so
    # o_t = scale (q_t . k_0) (v_0 o e^{Gv_t - Gv_0}), with Gv the running sum of gv
    B, T, H, K, V = 1, 30, 2, 6, 5
    g = torch.Generator().manual_seed(21)
    q = torch.randn(B, T, H, K, generator=g, dtype=D)
    k = torch.zeros(B, T, H, K, dtype=D)
    k[:, 0] = torch.randn(B, H, K, generator=g, dtype=D)
    v = torch.randn(B, T, H, V, generator=g, dtype=D)
    gv = torch.nn.functional.logsigmoid(torch.randn(B, T, H, V, generator=g, dtype=D)) / 3
    Gv = torch.cumsum(gv, 1)
    expect = (6 ** -0.5) * (q * k[:, :1]).sum(-1, keepdim=True) * v[:, :1] * torch.exp(Gv - Gv[:, :1])
    o, s = O.gla_recurrent(q, k, v, None, gv=gv)
    assert torch.allclose(o, expect, atol=1e-13)
    # with both decays the state's rows and columns decay independently
    gk = torch.nn.functional.logsigmoid(torch.randn(B, T, H, K, generator=g, dtype=D)) / 3
    G = torch.cumsum(gk, 1)
    o, s = O.gla_recurrent(q, k, v, gk, gv=gv)
    rows = torch.exp(G - G[:, :1]) * k[:, :1]
    expect = (6 ** -0.5) * (q * rows).sum(-1, keepdim=True) * v[:, :1] * torch.exp(Gv - Gv[:, :1])
    assert torch.allclose(o, expect, atol=1e-13)


def test_gla_reverse_is_the_time_reversed_recurrence():
    # reverse=True on each sequence equals the forward recurrence on the sequence read backwards
    q, k, v, _, _, s0 = _gdn_in(1, 50, 2, 8, 6)
    gk = torch.nn.functional.logsigmoid(torch.randn(1, 50, 2, 8, dtype=D)) / 8
    gv = torch.nn.functional.logsigmoid(torch.randn(1, 50, 2, 6, dtype=D)) / 8
    cu = [0, 17, 17, 50]
    cu_t = torch.tensor(cu)
    o, s = O.gla_recurrent(q, k, v, gk, gv=gv, h0=s0[:1].expand(3, -1, -1, -1).contiguous(), cu_seqlens=cu_t,
                           reverse=True)
    for n, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        if a == b:
            assert torch.allclose(s[n], s0[0])
            continue
        f = lambda x: x[:, a:b].flip(1)  # noqa: E731
        o_f, s_f = O.gla_recurrent(f(q), f(k), f(v), f(gk), gv=f(gv), h0=s0[:1])
        assert torch.allclose(o[:, a:b], o_f.flip(1), atol=1e-12)
        assert torch.allclose(s[n], s_f[0], atol=1e-12)
    # and differs from the forward recurrence (the order matters)
    o_fwd, _ = O.gla_recurrent(q, k, v, gk, gv=gv, h0=s0[:1].expand(3, -1, -1, -1).contiguous(), cu_seqlens=cu_t)
    assert not torch.allclose(o, o_fwd, atol=1e-6)


def test_gdn_key_value_decays_closed_forms():
    # beta = 0 (no writes): S_T = S_0 o exp(sum g) exp(sum gk)[:, None] exp(sum gv)[None, :]
    q, k, v, g, beta, s0 = _gdn_in(1, 20, 2, 6, 5, seed=3)
    gk = torch.nn.functional.logsigmoid(torch.randn(1, 20, 2, 6, dtype=D)) / 4
    gv = torch.nn.functional.logsigmoid(torch.randn(1, 20, 2, 5, dtype=D)) / 4
    _, s = O.gdn_recurrent(q, k, v, g, torch.zeros_like(beta), h0=s0, gk=gk, gv=gv)
    expect = s0[0] * torch.exp(g[0].sum(0))[:, None, None] * torch.exp(gk[0].sum(0))[:, :, None] \
        * torch.exp(gv[0].sum(0))[:, None, :]
    assert torch.allclose(s[0], expect, atol=1e-12)
    # beta = 1 with a unit key overwrites the decayed state's read-back along k exactly:
    # S_1^T k_1 = v_1 whatever the decays did to S_0
    _, s1 = O.gdn_recurrent(q[:, :1], k[:, :1], v[:, :1], g[:, :1], torch.ones_like(beta[:, :1]), h0=s0,
                            gk=gk[:, :1], gv=gv[:, :1])
    assert torch.allclose(torch.einsum("hkv,hk->hv", s1[0], k[0, 0]), v[0, 0], atol=1e-12)
    # gk = gv = 0 is the plain gated delta rule
    o_a, _ = O.gdn_recurrent(q, k, v, g, beta, h0=s0, gk=torch.zeros_like(gk), gv=torch.zeros_like(gv))
    o_b, _ = O.gdn_recurrent(q, k, v, g, beta, h0=s0)
    assert torch.allclose(o_a, o_b, atol=1e-14)
