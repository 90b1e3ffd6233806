"""GPU parity of the narrow linear map (the layers' gate projections, ``ccq_narrow_linear_fwd`` /
``_bwd`` through ``prologue.narrow_linear``) against a float64 torch restatement of nn.Linear on the
same bf16 inputs (the reference layers' erase_lambda_proj, a_proj, b_proj, gk_proj[0]:
``ccq/gdn/layer.py:174, 183-184, 292, 312, 316``; ``ccq/gla/layer.py:131, 162, 237-238``).

Tolerance: y, dx are bf16 (rounded once from an fp32 accumulation): relative L2 <= 2e-3 and, against the
float64 value rounded to bf16, <= 5e-4 (the accumulation order moves a few elements across a tie); dW
and db are fp32 sums over the rows: relative L2 <= 1e-5.
"""

import pytest
import torch

from tests._util import kern, rel

pytestmark = pytest.mark.gpu

D = torch.float64
BF = torch.bfloat16


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


CASES = [
    # rows, K, N, bias, strided x (a column slice of a wider tensor)
    (16384, 1024, 8, False, False),   # C2: b_proj + a_proj of d_model 1024, H 4
    (16384, 1024, 4, True, False),    # C2: erase_lambda_proj on q (key_dim 1024)
    (32768, 1024, 16, False, False),  # C3: gk_proj[0], rank 16
    (1000, 512, 4, True, True),       # ragged rows, strided x
    (7, 96, 3, True, False),          # tiny: fewer rows than a tile, odd N
    (130, 2016, 16, True, False),     # the widest K
]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_narrow_linear(case):
    dev = _cuda()
    from ccq_amd.prologue import narrow_linear
    M, K, N, with_bias, strided = case
    print("test_narrow_linear", case, flush=True)
    gen = torch.Generator().manual_seed(M + K + N)
    xw = torch.randn(M, K + (64 if strided else 0), generator=gen).to(BF)
    x_cpu = xw[:, 32:32 + K] if strided else xw
    w = (torch.randn(N, K, generator=gen) * 0.05).to(BF)
    b = (torch.randn(N, generator=gen) * 0.5).to(BF) if with_bias else None
    dy = torch.randn(M, N, generator=gen).to(BF)

    xr = x_cpu.to(D).requires_grad_()
    wr = w.to(D).requires_grad_()
    br = b.to(D).requires_grad_() if b is not None else None
    yr = xr @ wr.T + (br if br is not None else 0)
    (yr * dy.to(D)).sum().backward()

    xg = xw.to(dev)
    xg = (xg[:, 32:32 + K] if strided else xg).requires_grad_()
    wg = w.to(dev).requires_grad_()
    bg = b.to(dev).requires_grad_() if b is not None else None
    y = narrow_linear(xg, wg, bg)
    (y.float() * dy.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    errs = {"y": rel(y, yr), "dx": rel(xg.grad, xr.grad), "dW": rel(wg.grad.float(), wr.grad)}
    kerrs = {"y": kern(y, yr), "dx": kern(xg.grad, xr.grad)}
    if b is not None:
        errs["db"] = rel(bg.grad.float(), br.grad)
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, "kernel", {n: f"{e:.2e}" for n, e in kerrs.items()},
          flush=True)
    assert errs["y"] <= 2e-3 and errs["dx"] <= 2e-3
    assert kerrs["y"] <= 5e-4 and kerrs["dx"] <= 5e-4
    # dW / db come back in the parameter's dtype (bf16 here): one rounding of an fp32 sum
    assert kern(wg.grad, wr.grad) <= 5e-4
    if b is not None:
        assert kern(bg.grad, br.grad) <= 5e-4


def test_narrow_linear_rejects_wide_outputs():
    dev = _cuda()
    from ccq_amd.prologue import narrow_linear
    x = torch.zeros(4, 64, device=dev, dtype=BF)
    with pytest.raises(ValueError):
        narrow_linear(x, torch.zeros(17, 64, device=dev, dtype=BF))
