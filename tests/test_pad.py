"""Head sizes between the kernels' (ccq_amd/_pad.py), on the CPU.

The Python operators run such sizes zero-padded to the sizes the kernels take and slice the results
back.  That rests on the reference algorithm being unchanged by zero key and value channels: pinned
here on the float64 oracle (CCQ-GDN and CCQ-GLA, with initial states, the running key sum and the
l2norm), outputs, final states and every input gradient; plus the size rules of the helpers.
"""

import pytest
import torch

from ccq_amd._pad import CHUNK_K, STEP_K, cut_tail, key_size, pad_tail, value_size
from oracle import ccq_oracle as O

D = torch.float64


def test_sizes():
    assert [key_size(k, CHUNK_K) for k in (1, 64, 65, 96, 128, 129, 256)] == [64, 64, 128, 128, 128, 256, 256]
    assert [key_size(k, STEP_K) for k in (1, 32, 33, 40)] == [32, 32, 64, 64]
    assert [value_size(v) for v in (1, 64, 65, 300, 1024)] == [64, 64, 128, 320, 1024]
    with pytest.raises(ValueError):
        key_size(257, CHUNK_K)
    with pytest.raises(ValueError):
        value_size(1025)


def test_pad_and_cut():
    x = torch.randn(2, 3, 5, 7)
    y = pad_tail(x, 8, 9)
    assert y.shape == (2, 3, 8, 9) and torch.equal(y[..., :5, :7], x)
    assert y[..., 5:, :].abs().sum() == 0 and y[..., :, 7:].abs().sum() == 0
    assert torch.equal(cut_tail(y, 5, 7), x) and cut_tail(y, 5, 7).is_contiguous()
    assert pad_tail(None, 4) is None and cut_tail(None, 4) is None
    assert pad_tail(x, 7) is x


def _inputs(K, V, seed):
    gen = torch.Generator().manual_seed(seed)
    B, T, H = 1, 40, 2
    x = dict(q=torch.randn(B, T, H, K, generator=gen), k=torch.randn(B, T, H, K, generator=gen),
             v=torch.randn(B, T, H, V, generator=gen),
             lam=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
             g=-torch.rand(B, T, H, generator=gen) * 0.2,
             gk=-torch.rand(B, T, H, K, generator=gen) * 0.2,
             beta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
             s0=torch.randn(B, H, K, V, generator=gen) * 0.1,
             m0=torch.randn(B, H, K, generator=gen))
    a = torch.randn(B, H, K, 3, generator=gen)
    x["h0"] = a @ a.transpose(-1, -2)
    return {n: t.to(D) for n, t in x.items()}


def _padded(x, Kp, Vp):
    pads = dict(q=(Kp,), k=(Kp,), v=(Vp,), gk=(Kp,), s0=(Kp, Vp), m0=(Kp,), h0=(Kp, Kp))
    return {n: (pad_tail(t, *pads[n]) if n in pads else t) for n, t in x.items()}


@pytest.mark.parametrize("kind", ["gdn", "gla"])
def test_zero_channels_change_nothing(kind):
    K, V, Kp, Vp = 40, 24, 64, 64
    x = _inputs(K, V, seed=3)

    def run(inp, k_dim):
        leaves = {n: t.clone().requires_grad_() for n, t in inp.items()}
        common = dict(scale=K ** -0.5, h0=leaves["s0"], h0_cov=leaves["h0"], m0=leaves["m0"], position_offset=2)
        if kind == "gdn":
            out = O.ccq_gdn_forward(leaves["q"], leaves["k"], leaves["v"], leaves["lam"], leaves["g"], leaves["beta"],
                                    use_qk_l2norm=True, **common)
        else:
            out = O.ccq_gla_forward(leaves["q"], leaves["k"], leaves["v"], leaves["lam"], leaves["gk"], **common)
        o, S, C, m = out
        gen = torch.Generator().manual_seed(9)
        w_o = torch.randn(o.shape[:-1] + (V,), generator=gen).to(D)
        w_s = torch.randn(S.shape[:-2] + (K, V), generator=gen).to(D)
        # the loss reads the real channels only (as the sliced results of the padded run do)
        loss = (o[..., :V] * w_o).sum() + (S[..., :K, :V] * w_s).sum() + C[..., :K, :K].sum() + m[..., :K].sum()
        loss.backward()
        return o[..., :V], S[..., :K, :V], C[..., :K, :K], m[..., :K], leaves

    o1, S1, C1, m1, l1 = run(x, K)
    o2, S2, C2, m2, l2 = run(_padded(x, Kp, Vp), Kp)
    for a, b in ((o1, o2), (S1, S2), (C1, C2), (m1, m2)):
        assert torch.allclose(a, b, rtol=1e-12, atol=1e-12)
    shapes = dict(q=(K,), k=(K,), v=(V,), gk=(K,), s0=(K, V), m0=(K,), h0=(K, K))
    for n, t in l1.items():
        if t.grad is None:
            continue
        g2 = l2[n].grad
        g2 = cut_tail(g2, *shapes[n]) if n in shapes else g2
        assert torch.allclose(t.grad, g2, rtol=1e-10, atol=1e-12), n


def test_decode_step_refuses_sizes_it_cannot_hold():
    # the captured decode step's static buffers are the kernels' sizes (checked before any allocation)
    from ccq_amd.graph import DecodeStep
    for K, V in ((96, 128), (128, 100), (512, 128)):
        with pytest.raises(ValueError, match="DecodeStep takes K"):
            DecodeStep(1, 2, K, V, device="cpu")
