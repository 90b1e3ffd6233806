"""GPU parity over long sequences at the paper configurations' head shapes, against the float64 CPU
oracle on the same bf16-rounded inputs.

The K = 256 walks (cleaning column walks cut into time segments, the GDN state walks, the GLA state
walks) carry fp32 states through every 64-token chunk of a sequence; a drift that grows with the
number of chunks shows only over many chunks.  Cases:

* CCQ-GDN at K = 256, V = 512 (C2, C4 and ``configs/ccq_gdn_500M.json``: head_dim 256, expand_v 2)
  over 4096 tokens (64 chunks) under the benchmark's full decay (g = -softplus(N) exp(A_log), A_log ~
  U(0, log 16): down to about -55 per token) and the fused per-head gate (W ~ N(0, 0.02^2),
  b ~ U(-1, 1)), with the final states;
* CCQ-GLA at K = 256, V = 512 (``configs/ccq_gla_500M.json``: hidden 1024, expand_k 1.5 ->
  per-head 256 at 6 heads, expand_v 3 -> 512) and at K = 128, V = 256 (C3) with C3's log gate
  gk = logsigmoid(x W_g) / 16 through a rank-16 W_g ~ N(0, 0.02^2) on x ~ N(0, 1) of width 1024,
  over 2048 / 8192 tokens; and K = 256, V = 512 over 4096 tokens under a wider decay
  (logsigmoid(2 N) / 16, down to about -0.8 per token).

Tolerance (north star): relative L2 <= 2e-3 on outputs and gradients; the kernels' own error on bf16
outputs (against the oracle rounded to bf16) <= 5e-4.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import ccq_oracle as O
from tests._util import bf, kern, l2n, rel

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-3
TOL_KERNEL = 5e-4
D = torch.float64


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401  (fails loudly if the library is missing)
    return torch.device("cuda")


def _report(case, errs, kerrs):
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, "kernel", {n: f"{e:.2e}" for n, e in kerrs.items()},
          flush=True)
    for n, e in errs.items():
        assert e <= TOL_BF16, n
    for n, e in kerrs.items():
        assert e <= TOL_KERNEL, n


@pytest.mark.parametrize("T,H", [(4096, 2)])
def test_ccq_gdn_k256_v512_long(T, H):
    dev = _cuda()
    from ccq_amd import fused_chunk_ccq_gdn
    B, K, V = 1, 256, 512
    print(f"test_ccq_gdn_k256_v512_long B={B} T={T} H={H} K={K} V={V}", flush=True)
    gen = torch.Generator().manual_seed(11)
    x = {
        "q": bf(l2n(torch.randn(B, T, H, K, generator=gen))),
        "k": bf(l2n(torch.randn(B, T, H, K, generator=gen))),
        "w": torch.randn(H, K, generator=gen) * 0.02,
        "b": torch.empty(H).uniform_(-1.0, 1.0, generator=gen),
        "v": bf(torch.randn(B, T, H, V, generator=gen)),
    }
    a_log = torch.empty(H).uniform_(0.0, math.log(16.0), generator=gen)
    x["g"] = (-F.softplus(torch.randn(B, T, H, generator=gen)) * a_log.exp()).float()
    x["beta"] = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float()
    do = bf(torch.randn(B, T, H, V, generator=gen))
    dsf = torch.randn(B, H, K, V, generator=gen) * 0.1

    ref = {n: t.to(D).requires_grad_() for n, t in x.items()}
    lam = O.lambda_gate(ref["q"], ref["w"], ref["b"]).unsqueeze(-1)
    o_r, s_r, c_r, m_r = O.ccq_gdn_forward(ref["q"], ref["k"], ref["v"], lam, ref["g"], ref["beta"])
    ((o_r * do.to(D)).sum() + (s_r * dsf.to(D)).sum()).backward()

    g = {n: t.to(dev).requires_grad_() for n, t in x.items()}
    o, s, c, m = fused_chunk_ccq_gdn(g["q"], g["k"], g["v"], None, g["g"], g["beta"], gate_w=g["w"], gate_b=g["b"],
                                     output_final_state=True)
    ((o.float() * do.to(dev).float()).sum() + (s * dsf.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    errs = {"o": rel(o, o_r), "S": rel(s, s_r), "C": rel(c, c_r), "m": rel(m, m_r)}
    kerrs = {"o": kern(o, o_r)}
    for n in x:
        errs["d" + n] = rel(g[n].grad, ref[n].grad)
        if g[n].grad.dtype == torch.bfloat16:
            kerrs["d" + n] = kern(g[n].grad, ref[n].grad)
    _report(("gdn", T, H, K, V), errs, kerrs)


def _c3_log_gate(B, T, H, K, gen, width=1024, rank=16):
    """C3's per-channel log gate: logsigmoid(x W_1 W_2 + b) / 16, x ~ N(0, 1) [B, T, width],
    W_1 [width, rank], W_2 [rank, H K], both ~ N(0, 0.02^2), b = 0 (``ccq/gla/layer.py:162-163, 249``)."""
    xh = torch.randn(B, T, width, generator=gen)
    w1 = torch.randn(width, rank, generator=gen) * 0.02
    w2 = torch.randn(rank, H * K, generator=gen) * 0.02
    return (F.logsigmoid(xh @ w1 @ w2) / 16).view(B, T, H, K).float()


GLA_LONG = [
    # T, H, K, V, decay ("c3": C3's low-rank gate; "wide": logsigmoid(2 N) / 16)
    (2048, 1, 256, 512, "c3"),
    (8192, 1, 128, 256, "c3"),
    (4096, 1, 256, 512, "wide"),
]


@pytest.mark.parametrize("case", GLA_LONG, ids=[f"T{c[0]}_K{c[2]}_V{c[3]}_{c[4]}" for c in GLA_LONG])
def test_ccq_gla_long(case):
    dev = _cuda()
    from ccq_amd import fused_chunk_ccq_gla
    T, H, K, V, decay = case
    B = 1
    print(f"test_ccq_gla_long {case}", flush=True)
    gen = torch.Generator().manual_seed(12)
    x = {
        "q": bf(torch.randn(B, T, H, K, generator=gen)),     # the op L2-normalises q and k
        "k": bf(torch.randn(B, T, H, K, generator=gen)),
        "v": bf(torch.randn(B, T, H, V, generator=gen)),
        "lam": bf(torch.sigmoid(torch.randn(B, T, H, 1, generator=gen))),
    }
    if decay == "c3":
        x["gk"] = _c3_log_gate(B, T, H, K, gen)
    else:
        x["gk"] = (F.logsigmoid(torch.randn(B, T, H, K, generator=gen) * 2.0) / 16).float()
    do = bf(torch.randn(B, T, H, V, generator=gen))

    ref = {n: t.to(D).requires_grad_() for n, t in x.items()}
    o_r, s_r, c_r, m_r = O.ccq_gla_forward(ref["q"], ref["k"], ref["v"], ref["lam"], ref["gk"],
                                           l2norm_dtype=torch.bfloat16)
    (o_r * do.to(D)).sum().backward()

    g = {n: t.to(dev).requires_grad_() for n, t in x.items()}
    o, s, c, m = fused_chunk_ccq_gla(g["q"], g["k"], g["v"], g["lam"], g["gk"], output_final_state=True)
    (o.float() * do.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    errs = {"o": rel(o, o_r), "S": rel(s, s_r), "C": rel(c, c_r), "m": rel(m, m_r)}
    for n in ("q", "k", "v", "gk"):
        errs["d" + n] = rel(g[n].grad, ref[n].grad)
    # d(lambda) is returned in lambda's dtype (bf16), as the reference returns it
    errs["dlam"] = rel(g["lam"].grad, ref["lam"].grad.to(torch.bfloat16))
    kerrs = {"o": kern(o, o_r), "dq": kern(g["q"].grad, ref["q"].grad), "dk": kern(g["k"].grad, ref["k"].grad),
             "dv": kern(g["v"].grad, ref["v"].grad)}
    _report(("gla",) + tuple(case), errs, kerrs)
