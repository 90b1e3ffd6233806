"""GPU checks of the layer prologue / epilogue kernels (ccq_amd.prologue): the short causal
convolution (+ SiLU, + per-head L2 normalisation) and the gated RMSNorm, forward and backward,
against plain float32 PyTorch restatements of the same operations on the same bf16 inputs; and a
bf16 CCQ-GDN layer with the fused prologue against the same layer with the unfused one.

Tolerances: relative L2 <= 2e-3 on bf16 outputs and gradients (north star; the bf16 rounding of
the output alone is ~1.66e-3 of it), and the kernels' own error -- the bf16 output against the fp32
restatement rounded to bf16 -- <= 5e-4; fp32 weight gradients <= 1e-3; caches exact (they are
copies of inputs).  The fused-versus-unfused layer comparison at the end compares two bf16 layers
(both sides rounded), so it is a consistency check at 1e-2; the layer's bar is held against the
fp64 restatement in test_gpu_layers_bf16.py."""

import copy

import pytest
import torch
import torch.nn.functional as F

from tests._util import kern, rel

pytestmark = pytest.mark.gpu

TOL = 2e-3
TOL_KERNEL = 5e-4


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


def _bf16_through(x):
    """x rounded to bf16, gradient straight through (as the kernel normalises the rounded y)."""
    return x + (x.to(torch.bfloat16).float() - x).detach()


def _conv_ref(x, w, b, cache, cu, act, head_dim):
    """fp32 restatement: per sequence, window of the cached inputs then the sequence's inputs."""
    W = w.shape[-1]
    outs, normed, caches = [], [], []
    bounds = [0, x.shape[1]] if cu is None else cu
    rows = range(x.shape[0]) if cu is None else [0] * (len(bounds) - 1)
    for n, bi in enumerate(rows):
        s0, s1 = (0, x.shape[1]) if cu is None else (bounds[n], bounds[n + 1])
        xs = x[bi, s0:s1].t()                                        # [D, L]
        c = cache[n] if cache is not None else torch.zeros(x.shape[-1], W - 1, device=x.device)
        full = torch.cat([c, xs], -1)
        if s1 > s0:
            y = F.conv1d(full[None], w.view(-1, 1, W), b, groups=x.shape[-1])[0]
            if act:
                y = F.silu(y)
            y = y.t()
        else:
            y = x.new_zeros(0, x.shape[-1])
        outs.append(y)
        if head_dim:
            yb = _bf16_through(y).view(y.shape[0], y.shape[1] // head_dim, head_dim)
            normed.append((yb / torch.sqrt((yb * yb).sum(-1, keepdim=True) + 1e-6)).view(y.shape))
        caches.append(full[:, full.shape[-1] - (W - 1):] if W > 1 else full[:, :0])
    if cu is None:
        y = torch.stack(outs, 0)
        yn = torch.stack(normed, 0) if head_dim else None
    else:
        y = torch.cat(outs, 0)[None]
        yn = torch.cat(normed, 0)[None] if head_dim else None
    return y, yn, torch.stack(caches, 0)


CONV_CASES = [
    # B, T, D, W, act, head_dim, bias, cu, cache
    (2, 100, 256, 4, True, 64, False, None, False),
    (1, 120, 512, 4, True, 128, True, [0, 3, 3, 50, 120], True),
    (2, 70, 128, 3, False, None, True, None, True),
    (1, 300, 1024, 4, True, 256, False, [0, 1, 2, 300], False),
    # enough tokens for the forward's multi-token tiles (16 per tile from 16,384 tokens, 5 at 5,202),
    # with sequence starts inside tiles (window refills mid-tile)
    (1, 16500, 256, 4, True, 64, False, [0, 5, 4099, 9000, 16500], True),
    (2, 2601, 128, 4, True, 128, True, None, True),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[str(i) for i in range(len(CONV_CASES))])
def test_short_conv(case):
    dev = _cuda()
    from ccq_amd.prologue import short_conv
    B, T, D, W, act, hd, with_bias, cu, with_cache = case
    print(f"short conv case {case}", flush=True)
    gen = torch.Generator().manual_seed(3)
    N = B if cu is None else len(cu) - 1
    x = torch.randn(B, T, D, generator=gen).bfloat16().to(dev)
    w = (torch.randn(D, 1, W, generator=gen) * 0.5).to(dev)
    b = (torch.randn(D, generator=gen) * 0.1).to(dev) if with_bias else None
    cache = torch.randn(N, D, W - 1, generator=gen).bfloat16().float().to(dev) if with_cache else None
    cu_t = torch.tensor(cu, dtype=torch.int64, device=dev) if cu is not None else None
    dy = torch.randn(B, T, D, generator=gen).bfloat16().to(dev)
    dyn = torch.randn(B, T, D, generator=gen).bfloat16().to(dev) if hd else None

    xk = x.clone().requires_grad_()
    wk = w.clone().requires_grad_()
    bk = b.clone().requires_grad_() if b is not None else None
    y, yn, c_out = short_conv(xk, wk, bk, cache, cu_t, act, hd, True, True)
    loss = (y.float() * dy.float()).sum() + ((yn.float() * dyn.float()).sum() if hd else 0.0)
    grads = torch.autograd.grad(loss, [xk, wk] + ([bk] if bk is not None else []))

    xr = x.float().requires_grad_()
    wr = w.clone().requires_grad_()
    br = b.clone().requires_grad_() if b is not None else None
    y_r, yn_r, c_r = _conv_ref(xr, wr.view(D, W), br, cache, cu, act, hd)
    loss_r = (_bf16_through(y_r) * dy.float()).sum() + ((yn_r * dyn.float()).sum() if hd else 0.0)
    grads_r = torch.autograd.grad(loss_r, [xr, wr] + ([br] if br is not None else []))
    torch.cuda.synchronize()

    errs = {"y": rel(y, y_r), "dx": rel(grads[0], grads_r[0]), "dw": rel(grads[1], grads_r[1])}
    kerrs = {"y": kern(y, y_r), "dx": kern(grads[0], grads_r[0])}
    if hd:
        errs["yn"] = rel(yn, yn_r)
        kerrs["yn"] = kern(yn, yn_r)
    if b is not None:
        errs["db"] = rel(grads[2], grads_r[2])
    print(case, {n: f"{e:.2e}" for n, e in errs.items()}, "kernel", {n: f"{e:.2e}" for n, e in kerrs.items()},
          flush=True)
    for n in ("y", "yn", "dx"):
        if n in errs:
            assert errs[n] <= TOL, n
            assert kerrs[n] <= TOL_KERNEL, n
    for n in ("dw", "db"):
        if n in errs:
            assert errs[n] <= 1e-3, n
    if W > 1:
        assert torch.equal(c_out.float(), c_r), "final cache"


def test_short_conv_matches_the_layer_module_path():
    """The module's fused path and its plain PyTorch path give the same y (fp32 model runs the
    latter)."""
    dev = _cuda()
    from ccq_amd.layers import ShortConvolution
    torch.manual_seed(0)
    m = ShortConvolution(256, 4, bias=False, activation='silu').to(dev)
    x = torch.randn(2, 90, 256, device=dev).bfloat16()
    y_f, s_f = m(x, None, True)
    y_t, s_t = ShortConvolution.forward(m.float(), x.float(), None, True)  # fp32 inputs: the torch path
    torch.cuda.synchronize()
    assert rel(y_f, y_t) <= TOL and kern(y_f, y_t) <= TOL_KERNEL
    assert torch.equal(s_f.float(), s_t.float())


@pytest.mark.parametrize("rows,dv,with_w", [(300, 128, True), (1000, 512, True), (77, 64, False)])
def test_gated_rmsnorm(rows, dv, with_w):
    dev = _cuda()
    from ccq_amd.prologue import gated_rmsnorm
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(rows, dv, generator=gen).bfloat16().to(dev)
    g = torch.randn(rows, dv, generator=gen).bfloat16().to(dev)
    w = (1 + 0.1 * torch.randn(dv, generator=gen)).to(dev) if with_w else None
    dy = torch.randn(rows, dv, generator=gen).bfloat16().to(dev)
    print(f"gated rmsnorm {rows} {dv} {with_w}", flush=True)
    xk, gk = x.clone().requires_grad_(), g.clone().requires_grad_()
    wk = w.clone().requires_grad_() if w is not None else None
    y = gated_rmsnorm(xk, gk, wk, 1e-5)
    grads = torch.autograd.grad((y.float() * dy.float()).sum(), [xk, gk] + ([wk] if wk is not None else []))
    xr, gr = x.float().requires_grad_(), g.float().requires_grad_()
    wr = w.clone().requires_grad_() if w is not None else None
    yr = xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-5)
    if wr is not None:
        yr = yr * wr
    yr = yr * F.silu(gr)
    grads_r = torch.autograd.grad((yr * dy.float()).sum(), [xr, gr] + ([wr] if wr is not None else []))
    torch.cuda.synchronize()
    errs = {"y": rel(y, yr), "dx": rel(grads[0], grads_r[0]), "dg": rel(grads[1], grads_r[1])}
    kerrs = {"y": kern(y, yr), "dx": kern(grads[0], grads_r[0]), "dg": kern(grads[1], grads_r[1])}
    if w is not None:
        errs["dw"] = rel(grads[2], grads_r[2])
    print({n: f"{e:.2e}" for n, e in errs.items()}, "kernel", {n: f"{e:.2e}" for n, e in kerrs.items()},
          flush=True)
    for n, e in errs.items():
        assert e <= (1e-3 if n == "dw" else TOL), n
    for n, e in kerrs.items():
        assert e <= TOL_KERNEL, n


def test_gdn_layer_fused_prologue_matches_unfused():
    """A bf16 CCQ-GDN layer (C2 head shape, reduced T) with the fused prologue (conv + SiLU +
    per-head l2norm in one pass, the operator told not to normalise again) and the fused gated
    RMSNorm, against the same layer with the unfused PyTorch prologue / epilogue and the operator's
    own l2norm: outputs and every gradient."""
    dev = _cuda()
    from ccq_amd import CCQGDN
    import ccq_amd.layers as L
    torch.manual_seed(0)
    fused = CCQGDN(hidden_size=1024, head_dim=256, num_heads=4, expand_v=2, mode="fused_chunk",
                   layer_idx=0).to(dev, torch.bfloat16)
    plain = copy.deepcopy(fused)
    plain.fused_prologue = False
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(2, 300, 1024, generator=gen).bfloat16().to(dev)
    do = torch.randn(2, 300, 1024, generator=gen).bfloat16().to(dev)
    print("fused prologue layer", flush=True)

    def run(m, unfused_epilogue):
        xi = x.clone().requires_grad_()
        saved = L.FusedRMSNormGated.forward
        if unfused_epilogue:
            # the module's PyTorch path (fp32 arithmetic), as taken by non-bf16 inputs
            def torch_path(self, a, g):
                y = L._at_least_f32(L.RMSNorm.forward(self, a)) * F.silu(L._at_least_f32(g))
                return y.to(a.dtype)
            L.FusedRMSNormGated.forward = torch_path
        try:
            o = m(xi)[0]
            grads = torch.autograd.grad((o.float() * do.float()).sum(), [xi] + list(m.parameters()), allow_unused=True)
        finally:
            L.FusedRMSNormGated.forward = saved
        return o, grads

    o_f, g_f = run(fused, False)
    o_p, g_p = run(plain, True)
    torch.cuda.synchronize()
    errs = {"o": rel(o_f, o_p), "dx": rel(g_f[0], g_p[0])}
    for (n, _), a, b in zip(fused.named_parameters(), g_f[1:], g_p[1:]):
        assert (a is None) == (b is None), n
        if a is not None:
            errs["d" + n] = rel(a, b)
    print({n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= 1e-2, n


@pytest.mark.parametrize("rows,D,dy32", [(1000, 128, True), (333, 256, False), (77, 64, True), (50, 512, False),
                                         (41, 100, True), (9, 24, False)])
def test_l2norm(rows, D, dy32):
    """Row L2 normalisation (the op's l2norm, fla's at ccq/ops/ccq_gdn/fused_chunk.py:43-44) and its
    backward against fp32 PyTorch on the same bf16 inputs: the 16-byte kernels (D % 8 == 0, several
    rows per wavefront below D = 512) and the scalar ones (D = 100); fp32 and bf16 upstream
    gradients, row counts that leave a wavefront partly filled."""
    dev = _cuda()
    from ccq_amd.clean import l2norm_bwd, l2norm_fwd
    print(f"l2norm rows={rows} D={D} dy32={dy32}", flush=True)
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(rows, D, generator=gen).bfloat16().to(dev)
    dy = torch.randn(rows, D, generator=gen)
    dy = dy.to(dev) if dy32 else dy.bfloat16().to(dev)
    y, rstd = l2norm_fwd(x, 1e-6)
    dx = l2norm_bwd(x, rstd, dy)
    xr = x.float().requires_grad_()
    yr = xr / torch.sqrt((xr * xr).sum(-1, keepdim=True) + 1e-6)
    (dxr,) = torch.autograd.grad(yr, xr, dy.float())
    torch.cuda.synchronize()
    errs = {"y": rel(y, yr), "rstd": rel(rstd, 1.0 / torch.sqrt((xr * xr).sum(-1) + 1e-6)), "dx": rel(dx, dxr)}
    print(errs, flush=True)
    assert errs["y"] <= TOL and errs["dx"] <= TOL and errs["rstd"] <= 1e-6
