"""GPU checks of the decode step's projection kernels: ``decode_linear`` (``ccq_decode_linear``), its
split-contraction form (``ccq_decode_linear_split``) and its gated up-projection form
(``ccq_decode_linear_glu``) against a float64 restatement with the bf16
roundings of the torch ops they replace (``residual + linear(x)``; ``silu(gate) * up`` of
``linear(x).chunk(2, -1)``), and the
gated RMSNorm that reads its gate rows in place (``ccq_gated_rmsnorm_fwd_strided``) against the
contiguous kernel on a copy of those rows.

Tolerance: outputs are bf16 rounded once from an fp32 accumulation: against the float64 value
rounded at the same points, relative L2 <= 5e-4 (the accumulation order moves a few elements across
a tie); the strided and contiguous norms must agree bit for bit.
"""

import pytest
import torch
import torch.nn.functional as F

from tests._util import kern

pytestmark = pytest.mark.gpu

D = torch.float64
BF = torch.bfloat16


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


def _r(x):
    return x.to(BF).to(D)


CASES = [
    # M, K, N, residual
    (16, 1024, 6160, False),   # C4: a layer's concatenated input projections
    (16, 2048, 1024, True),    # C4: o_proj with the residual
    (3, 1024, 5632, False),    # three tokens
    (1, 4096, 100, True),      # one token, the widest K, N not a multiple of 16
    (16, 1024, 32000, False),  # C4's LM head: four column tiles per workgroup
    (5, 512, 17000, True),     # wide, the last workgroup's tiles partly past N
]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_decode_linear(case):
    dev = _cuda()
    from ccq_amd.graph import decode_linear
    M, K, N, with_res = case
    print("test_decode_linear", case, flush=True)
    gen = torch.Generator().manual_seed(M * 7 + K + N)
    x = torch.randn(M, K, generator=gen).to(BF)
    w = (torch.randn(N, K, generator=gen) * 0.03).to(BF)
    res = torch.randn(M, N, generator=gen).to(BF) if with_res else None
    ref = _r(x.to(D) @ w.to(D).T)
    if res is not None:
        ref = res.to(D) + ref
    y = decode_linear(x.to(dev), w.to(dev), res.to(dev) if res is not None else None)
    torch.cuda.synchronize()
    e = kern(y, ref)
    print(case, f"kernel {e:.2e}", flush=True)
    assert y.shape == (M, N) and e <= 5e-4


@pytest.mark.parametrize("M,K,N", [(16, 1024, 2816), (5, 512, 100)])
def test_decode_linear_glu(M, K, N):
    dev = _cuda()
    from ccq_amd.graph import decode_linear_glu
    print("test_decode_linear_glu", M, K, N, flush=True)
    gen = torch.Generator().manual_seed(K + N)
    x = torch.randn(M, K, generator=gen).to(BF).to(dev)
    w = (torch.randn(2 * N, K, generator=gen) * 0.03).to(BF).to(dev)
    gt, up = (x.double().cpu() @ w.double().cpu().T).chunk(2, -1)
    # torch's bf16 ops restated: each projection rounded, silu rounded, the product rounded
    ref = _r(_r(F.silu(_r(gt))) * _r(up))
    y = decode_linear_glu(x, w)
    torch.cuda.synchronize()
    e = kern(y, ref)
    print((M, K, N), f"kernel {e:.2e}", flush=True)
    assert y.shape == (M, N) and e <= 5e-4


@pytest.mark.parametrize("glu,N", [(False, 1024), (True, 1024), (False, 32000)])
def test_decode_linear_folded_rmsnorm(glu, N):
    """The RMSNorm folded into the projection equals torch's bf16 nn.RMSNorm followed by the same
    projection kernel (the norm's output is rounded once; the row's sum of squares runs in another
    order, which can move a rare element of the normalised row by one ulp); N = 32000 is the LM head
    with the final norm folded in (four column tiles per workgroup)."""
    dev = _cuda()
    import torch.nn as nn
    from ccq_amd.graph import decode_linear, decode_linear_glu
    M, K = 16, 1024
    gen = torch.Generator().manual_seed(5)
    norm = nn.RMSNorm(K, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(K, generator=gen) * 2)
    norm = norm.to(dev, BF)
    x = (torch.randn(M, K, generator=gen) * 3).to(BF).to(dev)
    w = (torch.randn((2 if glu else 1) * N, K, generator=gen) * 0.03).to(BF).to(dev)
    if glu:
        ref = decode_linear_glu(norm(x), w)
        y = decode_linear_glu(x, w, norm_weight=norm.weight, norm_eps=norm.eps)
    else:
        ref = decode_linear(norm(x), w)
        y = decode_linear(x, w, norm_weight=norm.weight, norm_eps=norm.eps)
    torch.cuda.synchronize()
    e = kern(y, ref.double().cpu())
    print("folded rmsnorm", glu, f"{e:.2e}", flush=True)
    assert e <= 5e-4


def test_gated_rmsnorm_strided_gate_rows():
    dev = _cuda()
    from ccq_amd import _lib
    from ccq_amd._lib import call, ptr
    T, H, V, width = 16, 4, 512, 6160
    gen = torch.Generator().manual_seed(3)
    proj = torch.randn(T, width, generator=gen).to(BF).to(dev)
    o = torch.randn(T * H, V, generator=gen).to(BF).to(dev)
    w = torch.rand(V, generator=gen).float().to(dev)
    og = 2 * 1024 + 2048
    g = proj[:, og:og + H * V].contiguous().view(T * H, V)
    y0, y1 = torch.empty_like(o), torch.empty_like(o)
    r0 = torch.empty(T * H, device=dev)
    r1 = torch.empty(T * H, device=dev)
    s = _lib.stream_of(o)
    call("ccq_gated_rmsnorm_fwd", ptr(o), ptr(g), ptr(w), ptr(y0), ptr(r0), T * H, V, 1e-5, s)
    call("ccq_gated_rmsnorm_fwd_strided", ptr(o), proj.data_ptr() + 2 * og, width, H, ptr(w), ptr(y1), ptr(r1),
         T * H, V, 1e-5, s)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1) and torch.equal(r0, r1)


@pytest.mark.parametrize("M,K,N,splits", [(16, 2816, 1024, 4), (16, 2048, 1024, 4), (3, 1024, 100, 3),
                                          (1, 96, 40, 3), (16, 4096, 520, 8)])
def test_decode_linear_split(M, K, N, splits):
    """The split contraction (partial tiles added by the last workgroup of each column block) against
    float64, over three calls in a row on one workspace (its counters must come back to zero; the
    second call with other inputs), and against the unsplit kernel."""
    dev = _cuda()
    from ccq_amd.graph import decode_linear, decode_linear_split, split_workspace
    print("test_decode_linear_split", M, K, N, splits, flush=True)
    ws = split_workspace(N, splits, dev)  # (the block counters lead it)
    gen = torch.Generator().manual_seed(K + N + splits)
    for call in range(3):
        x = torch.randn(M, K, generator=gen).to(BF)
        w = (torch.randn(N, K, generator=gen) * 0.03).to(BF)
        res = torch.randn(M, N, generator=gen).to(BF)
        ref = res.to(D) + _r(x.to(D) @ w.to(D).T)
        y = decode_linear_split(x.to(dev), w.to(dev), res.to(dev), splits, ws)
        y1 = decode_linear(x.to(dev), w.to(dev), res.to(dev))
        torch.cuda.synchronize()
        e, e1 = kern(y, ref), kern(y, y1.double().cpu())
        print((M, K, N, splits), call, f"kernel {e:.2e} vs unsplit {e1:.2e}", flush=True)
        assert y.shape == (M, N) and e <= 5e-4 and e1 <= 5e-4
        blocks = (N + 15) // 16
        assert int(ws[:4 * blocks].view(torch.int32).abs().sum()) == 0, "counters not back to zero"


@pytest.mark.parametrize("M,H,V,N,weighted", [(16, 4, 512, 1024, True), (1, 8, 128, 200, False), (5, 1, 256, 64, True)])
def test_decode_linear_folded_gated_norm(M, H, V, N, weighted):
    """The gated output norm folded into the output projection (``ccq_decode_linear_gnorm``: the
    contraction split per head, the gate rows read in place from a wider projection output) against
    the strided gated-norm kernel followed by ``decode_linear`` (the head's sum of squares runs in
    another order, which can move a rare normed element by one bf16 unit) and against float64, over
    two calls on one workspace."""
    dev = _cuda()
    from ccq_amd import _lib
    from ccq_amd._lib import call, ptr
    from ccq_amd.graph import decode_linear, decode_linear_gnorm, split_workspace
    print("test_decode_linear_folded_gated_norm", M, H, V, N, weighted, flush=True)
    K, og = H * V, 96
    width = og + K + 40
    ws = split_workspace(N, H, dev) if H > 1 else None
    gen = torch.Generator().manual_seed(M + H + V)
    for call_no in range(2):
        proj = (torch.randn(M, width, generator=gen) * 2).to(BF).to(dev)
        o = (torch.randn(M, K, generator=gen) * 3).to(BF).to(dev)
        nw = (torch.rand(V, generator=gen) * 2).float().to(dev) if weighted else None
        w = (torch.randn(N, K, generator=gen) * 0.03).to(BF).to(dev)
        res = torch.randn(M, N, generator=gen).to(BF).to(dev)
        gate = proj[:, og:og + K]
        y = decode_linear_gnorm(o, gate, nw, V, 1e-5, w, res, ws)
        normed = torch.empty_like(o)
        rstd = torch.empty(M * H, device=dev)
        call("ccq_gated_rmsnorm_fwd_strided", ptr(o), ptr(gate), width, H, ptr(nw), ptr(normed), ptr(rstd), M * H, V,
             1e-5, _lib.stream_of(o))
        ref = decode_linear(normed, w, res)
        torch.cuda.synchronize()
        e = kern(y, ref.double().cpu())
        od, gd = o.double().cpu().view(M, H, V), gate.double().cpu().view(M, H, V)
        r = 1.0 / torch.sqrt((od * od).mean(-1, keepdim=True) + 1e-5)
        wd = nw.double().cpu() if weighted else torch.ones(V, dtype=D)
        xn = _r((od * r * wd * F.silu(gd)).reshape(M, K))
        e64 = kern(y, res.double().cpu() + _r(xn @ w.double().cpu().T))
        print((M, H, V, N), call_no, f"vs unfolded {e:.2e} vs float64 {e64:.2e}", flush=True)
        assert y.shape == (M, N) and e <= 5e-4 and e64 <= 5e-4
        if ws is not None:
            assert int(ws[:4 * ((N + 15) // 16)].view(torch.int32).abs().sum()) == 0, "counters"


@pytest.mark.parametrize("M,N,rows,D", [(16, 32000, 32000, 1024), (3, 1003, 1003, 200), (2, 64, 40, 24)])
def test_greedy_embed(M, N, rows, D):
    """``greedy_embed`` against ``logits.argmax(-1)`` and the embedding lookup: planted ties (the first
    index wins), NaNs (the first NaN wins, as torch.argmax), a row of -inf (index 0), a width that is
    not a multiple of 8, and ids past the table's rows (zero rows)."""
    dev = _cuda()
    from ccq_amd.graph import greedy_embed
    print("test_greedy_embed", M, N, rows, D, flush=True)
    gen = torch.Generator().manual_seed(N + M)
    logits = torch.randn(M, N, generator=gen).to(BF)
    if M >= 3:
        top = logits[0].max()
        logits[0, N // 3] = top + 1
        logits[0, N - 1] = top + 1                     # tie: the first index wins
        logits[1, 7] = float("nan")
        logits[1, N // 2] = float("nan")               # NaNs: the first wins
        logits[2] = float("-inf")                      # all -inf: index 0
    else:
        logits[0, N - 1] = logits[0].max() + 1         # an id past the table (rows < N)
    table = torch.randn(rows, D, generator=gen).to(BF)
    ref_ids = logits.argmax(-1)
    ref_x = torch.zeros(M, D, dtype=BF)
    ok = ref_ids < rows
    ref_x[ok] = table[ref_ids[ok]]
    ids = torch.full((M, 1), -1, dtype=torch.int64, device=dev)
    x = torch.full((M, 1, D), 7.0, dtype=BF, device=dev)
    greedy_embed(logits.to(dev), table.to(dev), ids, x)
    torch.cuda.synchronize()
    assert torch.equal(ids[:, 0].cpu(), ref_ids), (ids[:, 0].cpu(), ref_ids)
    assert torch.equal(x[:, 0].cpu(), ref_x)
