"""GPU parity of the reference's stock `chunk` building blocks: the covariance read
(_ccq_compute_z_and_sum_kk) and the cleaning given z (_CCQCleanQ), forward and backward, against
the CPU oracle (float64, same bf16-rounded inputs).  Tolerance: relative L2 <= 2e-3 (north star);
fp32 states and per-token fp32 gradients 1e-4."""

import pytest
import torch

from oracle import ccq_oracle as O
from tests._util import bf, l2n, rel

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-3


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


READ_CASES = [
    # B, T, H, K, with h0, varlen
    (2, 130, 2, 64, True, None),
    (1, 200, 2, 128, False, None),
    (1, 150, 2, 256, True, [0, 40, 41, 150]),
    (1, 120, 2, 96, True, None),   # K between the kernels' sizes: zero-padded to 128, results sliced back
]


@pytest.mark.parametrize("case", READ_CASES, ids=[str(i) for i in range(len(READ_CASES))])
def test_covariance_read(case):
    dev = _cuda()
    from ccq_amd import _ccq_compute_z_and_sum_kk
    B, T, H, K, wh0, cu = case
    N = B if cu is None else len(cu) - 1
    gen = torch.Generator().manual_seed(21)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    h0 = None
    if wh0:
        a = torch.randn(N, H, K, 4, generator=gen)
        h0 = (a @ a.transpose(-1, -2)).float()
    cu_t = torch.tensor(cu, dtype=torch.int64) if cu is not None else None
    dz = bf(torch.randn(B, T, H, K, generator=gen))
    dhf = torch.randn(N, H, K, K, generator=gen) * 0.01
    d = torch.float64
    qr, kr = q.to(d).requires_grad_(), k.to(d).requires_grad_()
    h0r = h0.to(d).requires_grad_() if wh0 else None
    z_r, h_r = O.covariance_read(qr, kr, h0=h0r, cu_seqlens=cu_t)
    ((z_r * dz.to(d)).sum() + (h_r * dhf.to(d)).sum()).backward()
    print(f"test_covariance_read {case}", flush=True)
    qg, kg = q.to(dev).requires_grad_(), k.to(dev).requires_grad_()
    h0g = h0.to(dev).requires_grad_() if wh0 else None
    z, hf = _ccq_compute_z_and_sum_kk(qg, kg, True, cu_t.to(dev) if cu_t is not None else None, initial_state=h0g)
    ((z.float() * dz.to(dev).float()).sum() + (hf * dhf.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    errs = {"z": rel(z, z_r), "h_final": rel(hf, h_r), "dq": rel(qg.grad, qr.grad), "dk": rel(kg.grad, kr.grad)}
    if wh0:
        errs["dh0"] = rel(h0g.grad, h0r.grad)
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n in ("z", "dq", "dk"):
        assert errs[n] <= TOL_BF16, n
    for n in ("h_final", "dh0"):
        if n in errs:
            assert errs[n] <= 1e-4, n


CLEANQ_CASES = [
    # B, T, H, K, m0, pos_off, subtract_mean, varlen
    (2, 130, 2, 64, True, 0, True, None),
    (1, 300, 2, 128, False, 5, True, None),
    (1, 90, 2, 32, True, 0, False, None),
    (1, 200, 2, 256, True, 2, True, [0, 64, 65, 200]),
    (1, 110, 2, 48, True, 3, True, None),   # K between the kernels' sizes: zero-padded to 64
]


@pytest.mark.parametrize("case", CLEANQ_CASES, ids=[str(i) for i in range(len(CLEANQ_CASES))])
def test_clean_given_z(case):
    dev = _cuda()
    from ccq_amd import _CCQCleanQ
    B, T, H, K, wm0, off, sub, cu = case
    N = B if cu is None else len(cu) - 1
    gen = torch.Generator().manual_seed(22)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    z = bf(torch.randn(B, T, H, K, generator=gen) * 3.0)
    lam = torch.sigmoid(torch.randn(B, T, H, 1, generator=gen))   # fp32: its gradient stays fp32
    m0 = torch.randn(N, H, K, generator=gen) if wm0 else None
    cu_t = torch.tensor(cu, dtype=torch.int64) if cu is not None else None
    dqc = bf(torch.randn(B, T, H, K, generator=gen))
    dmf = torch.randn(N, H, K, generator=gen) * 0.1
    d = torch.float64
    ref = {n: (t.to(d).requires_grad_() if t is not None else None) for n, t in
           dict(q=q, k=k, z=z, lam=lam.to(torch.bfloat16), m0=m0).items()}
    qc_r, mf_r = O.clean_given_z(ref["q"], ref["k"], ref["z"], ref["lam"], position_offset=off, m0=ref["m0"],
                                 subtract_mean=sub, cu_seqlens=cu_t)
    # the reference's _CCQCleanQ.backward (clean.py:720-748) ignores the gradient of final_state_K
    # and returns none for initial_state_K: its gradients are those of q_clean alone
    (qc_r * dqc.to(d)).sum().backward()
    print(f"test_clean_given_z {case}", flush=True)
    g = {n: (t.to(dev).requires_grad_() if t is not None else None) for n, t in
         dict(q=q, k=k, z=z, lam=lam, m0=m0).items()}
    qc, mf = _CCQCleanQ.apply(g["q"], g["k"], g["z"], g["lam"], off, g["m0"], True, sub,
                              cu_t.to(dev) if cu_t is not None else None)
    loss = (qc.float() * dqc.to(dev).float()).sum()
    if sub:
        loss = loss + (mf * dmf.to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    if not sub:  # k enters only through the mean term: the reference returns dk = 0 (clean.py:684-686)
        assert ref["k"].grad is None and torch.count_nonzero(g["k"].grad).item() == 0
        ref["k"].grad = torch.zeros_like(ref["k"])
    errs = {"q_clean": rel(qc, qc_r), "dq": rel(g["q"].grad, ref["q"].grad), "dk": rel(g["k"].grad, ref["k"].grad),
            "dz": rel(g["z"].grad, ref["z"].grad), "dlam": rel(g["lam"].grad, ref["lam"].grad)}
    if sub:
        errs["m_final"] = rel(mf, mf_r)
    if wm0:
        assert g["m0"].grad is None
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n in ("q_clean", "dq", "dk", "dz"):
        assert errs[n] <= TOL_BF16, n
    for n in ("m_final", "dm0", "dlam"):
        if n in errs:
            assert errs[n] <= 1e-4, n
