"""GPU parity of the CCQ layers (CCQGDN, CCQGLA): the same layer code runs on the GPU with the HIP
operators and on the CPU in float64 with the oracle in place of the operators, from identical
weights and inputs.  Covers the attn_mode dispatch (chunk / fused_chunk in training, the
recurrent mode for short inputs in eval), the recurrent cache (prefill, then single-token decode
carrying (S, C, m, position) and the short-convolution state) and attention-mask unpadding.

Tolerance: relative L2 <= 2e-3 on outputs and parameter gradients (north star).  Both sides run
the projections in fp32 and cross the operator boundary in the operators' dtypes (q, k, v and o in
bf16 -- so the upstream gradient of o arrives in bf16 on both sides), and the difference is the
kernels' own error."""

import copy

import pytest
import torch

from oracle import ccq_oracle as O
from tests._util import rel

pytestmark = pytest.mark.gpu

TOL = 2e-3
D = torch.float64


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


def _lam64(lambda_h, dtype):
    # the operators round lambda's value through their operand type (bf16) inside the autograd
    # function, so its gradient is not rounded (straight through)
    lam = lambda_h.squeeze(-1) if lambda_h.ndim == 4 else lambda_h
    return O.round_through(lam.to(D), dtype)


def q_dtype_of(x):
    """The dtype the operators see q in: bf16 for every accepted input dtype."""
    return torch.bfloat16


def _f64(x):
    return None if x is None else x.to(D)


def _operands(q, k, v):
    """q, k, v as the operators use them: values rounded to bf16 (their operand type, whatever the
    layer's dtype), gradients passed straight through the rounding as through the operators' cast."""
    return tuple(O.round_through(x.to(D), torch.bfloat16) for x in (q, k, v))


def _output(o, v):
    """o as the operators return it: computed into bf16 and handed back in v's dtype, so that its
    gradient also arrives through bf16."""
    return o.to(torch.bfloat16).to(v.dtype)


def oracle_gdn(q, k, v, lambda_h, g=None, beta=None, initial_state=None, initial_cov_state=None,
               initial_mean_state=None, output_final_state=False, cu_seqlens=None, use_qk_l2norm_in_kernel=False,
               position_offset=0, subtract_mean=True, enable_ccq=True, **_):
    v_in = v
    q, k, v = _operands(q, k, v)
    o, S, C, m = O.ccq_gdn_forward(q, k, v, _lam64(lambda_h, q_dtype_of(v_in)), g.to(D), beta.to(D),
                                   h0=_f64(initial_state), h0_cov=_f64(initial_cov_state),
                                   m0=_f64(initial_mean_state), position_offset=position_offset,
                                   subtract_mean=subtract_mean, cu_seqlens=cu_seqlens,
                                   use_qk_l2norm=use_qk_l2norm_in_kernel, enable_ccq=enable_ccq,
                                   l2norm_dtype=torch.bfloat16)
    o = _output(o, v_in)
    return (o, S, C, m) if output_final_state else (o, None, None, None)


def oracle_gla(q, k, v, lambda_h, g=None, gk=None, initial_state=None, initial_cov_state=None,
               initial_mean_state=None, output_final_state=False, cu_seqlens=None, position_offset=0,
               subtract_mean=True, **_):
    gate = g if g is not None else gk
    v_in = v
    q, k, v = _operands(q, k, v)
    o, S, C, m = O.ccq_gla_forward(q, k, v, _lam64(lambda_h, q_dtype_of(v_in)), gate.to(D),
                                   h0=_f64(initial_state), h0_cov=_f64(initial_cov_state),
                                   m0=_f64(initial_mean_state), position_offset=position_offset,
                                   subtract_mean=subtract_mean, cu_seqlens=cu_seqlens, l2norm_dtype=torch.bfloat16)
    o = _output(o, v_in)
    return (o, S, C, m) if output_final_state else (o, None, None, None)


@pytest.fixture(autouse=True)
def full_fp32_torch():
    """The layers' projections and short convolutions run in torch: keep them in full fp32 (no
    reduced-precision fp32 math) so that the comparison isolates the operators."""
    saved = (torch.backends.cudnn.allow_tf32, torch.backends.cuda.matmul.allow_tf32)
    torch.backends.cudnn.allow_tf32 = False
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cudnn.allow_tf32, torch.backends.cuda.matmul.allow_tf32 = saved


@pytest.fixture
def oracle_ops(monkeypatch):
    """Context in which ccq_amd.layers calls the oracle instead of the HIP operators."""
    import ccq_amd.layers as L

    class Ctx:
        def __enter__(self):
            for n in ("chunk_ccq_gdn", "fused_chunk_ccq_gdn", "fused_recurrent_ccq_gdn"):
                monkeypatch.setattr(L, n, oracle_gdn)
            for n in ("chunk_ccq_gla", "fused_chunk_ccq_gla", "fused_recurrent_ccq_gla"):
                monkeypatch.setattr(L, n, oracle_gla)
            return self

        def __exit__(self, *a):
            monkeypatch.undo()

    return Ctx()


def _make(kind, seed=0, **kw):
    from ccq_amd import CCQGDN, CCQGLA
    torch.manual_seed(seed)
    if kind == "gdn":
        m = CCQGDN(hidden_size=256, head_dim=64, num_heads=4, expand_v=2, layer_idx=0, **kw)
    else:
        m = CCQGLA(hidden_size=256, expand_k=0.5, expand_v=1.0, num_heads=2, use_short_conv=True, layer_idx=0, **kw)
    with torch.no_grad():   # lambda gate away from its 0.01 init so the cleaning matters
        m.erase_lambda_proj.bias.fill_(0.0)
    return m


def _x(B, T, seed=1):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, T, 256, generator=g).bfloat16().float()


@pytest.mark.parametrize("kind,mode", [("gdn", "chunk"), ("gdn", "fused_chunk"), ("gla", "chunk"),
                                       ("gla", "fused_chunk")])
def test_layer_train_step(kind, mode, oracle_ops):
    dev = _cuda()
    B, T = 2, 150
    ref = _make(kind, mode=mode).double()
    gpu = copy.deepcopy(ref).float().to(dev)
    ref.train()
    gpu.train()
    x = _x(B, T)
    gen = torch.Generator().manual_seed(2)
    do = torch.randn(B, T, 256, generator=gen)
    print(f"test_layer_train_step {kind} {mode}", flush=True)
    with oracle_ops:
        xr = x.to(D).requires_grad_()
        o_r, _, _ = ref(xr)
        (o_r * do.to(D)).sum().backward()
    xg = x.to(dev).requires_grad_()
    o, _, _ = gpu(xg)
    (o * do.to(dev)).sum().backward()
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "dx": rel(xg.grad, xr.grad)}
    for (n, p_r), (_, p) in zip(ref.named_parameters(), gpu.named_parameters()):
        if p_r.grad is not None:
            errs["d" + n] = rel(p.grad, p_r.grad)
    print(kind, mode, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= TOL, n


@pytest.mark.parametrize("kind", ["gdn", "gla"])
def test_layer_odd_head_sizes(kind, oracle_ops):
    """Layers whose head sizes the kernels do not take directly (the reference layers accept any
    head_dim): GDN head_dim 96 with expand_v 1.5 (V = 144), GLA K = V = 96; a training step against
    the layer running the oracle operators."""
    dev = _cuda()
    from ccq_amd import CCQGDN, CCQGLA
    torch.manual_seed(0)
    if kind == "gdn":
        ref = CCQGDN(hidden_size=256, head_dim=96, num_heads=2, expand_v=1.5, layer_idx=0, mode="chunk")
    else:
        ref = CCQGLA(hidden_size=256, expand_k=0.75, expand_v=0.75, num_heads=2, use_short_conv=True, layer_idx=0,
                     mode="chunk")
    with torch.no_grad():
        ref.erase_lambda_proj.bias.fill_(0.0)
    ref = ref.double().train()
    gpu = copy.deepcopy(ref).float().to(dev).train()
    B, T = 2, 100
    x = _x(B, T)
    gen = torch.Generator().manual_seed(2)
    do = torch.randn(B, T, 256, generator=gen)
    print(f"test_layer_odd_head_sizes {kind}", flush=True)
    with oracle_ops:
        xr = x.to(D).requires_grad_()
        o_r, _, _ = ref(xr)
        (o_r * do.to(D)).sum().backward()
    xg = x.to(dev).requires_grad_()
    o, _, _ = gpu(xg)
    (o * do.to(dev)).sum().backward()
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "dx": rel(xg.grad, xr.grad)}
    for (n, p_r), (_, p) in zip(ref.named_parameters(), gpu.named_parameters()):
        if p_r.grad is not None:
            errs["d" + n] = rel(p.grad, p_r.grad)
    print(kind, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= TOL, n


@pytest.mark.parametrize("kind", ["gdn", "gla"])
def test_layer_prefill_then_decode(kind, oracle_ops):
    """eval: chunked prefill of T0 tokens into a cache, then single-token calls (recurrent mode,
    decode kernels) carrying the recurrent and convolution states; checked against the oracle
    layer run through the same cache flow, and against one pass over all tokens."""
    dev = _cuda()
    from ccq_amd import LayerCache
    B, T0, T1 = 2, 100, 4
    ref = _make(kind).double().eval()
    gpu = copy.deepcopy(ref).float().to(dev).eval()
    x = _x(B, T0 + T1, seed=3)
    print(f"test_layer_prefill_then_decode {kind}", flush=True)

    def run(layer, xs, dtype, device):
        cache = LayerCache()
        outs = [layer(xs[:, :T0].to(device, dtype), past_key_values=cache, use_cache=True)[0]]
        for t in range(T0, T0 + T1):
            outs.append(layer(xs[:, t:t + 1].to(device, dtype), past_key_values=cache, use_cache=True)[0])
        return torch.cat(outs, 1), cache

    with torch.no_grad():
        with oracle_ops:
            o_r, cache_r = run(ref, x, D, "cpu")
        o, cache = run(gpu, x, torch.float32, dev)
        o_full = gpu(x.to(dev))[0]
    torch.cuda.synchronize()
    errs = {"prefill": rel(o[:, :T0], o_r[:, :T0]), "decode": rel(o[:, T0:], o_r[:, T0:]),
            "decode_vs_one_pass": rel(o[:, T0:], o_full[:, T0:])}
    S, C, m, pos = cache.get(0)["recurrent_state"]
    S_r, C_r, m_r, pos_r = cache_r.get(0)["recurrent_state"]
    errs.update(S=rel(S, S_r), C=rel(C, C_r), m=rel(m, m_r))
    print(kind, {n: f"{e:.2e}" for n, e in errs.items()}, "pos", pos, flush=True)
    assert pos == pos_r == T0 + T1
    for n, e in errs.items():
        assert e <= TOL, n


@pytest.mark.parametrize("kind", ["gdn", "gla"])
def test_layer_attention_mask(kind, oracle_ops):
    """Left-padded batch: the layer unpads to varlen sequences (cu_seqlens) and pads back."""
    dev = _cuda()
    B, T = 3, 130
    ref = _make(kind, mode="chunk").double().eval()
    gpu = copy.deepcopy(ref).float().to(dev).eval()
    x = _x(B, T, seed=4)
    mask = torch.ones(B, T, dtype=torch.long)
    mask[1, :40] = 0
    mask[2, :77] = 0
    print(f"test_layer_attention_mask {kind}", flush=True)
    with torch.no_grad():
        with oracle_ops:
            o_r = ref(x.to(D), attention_mask=mask)[0]
        o = gpu(x.to(dev), attention_mask=mask.to(dev))[0]
    torch.cuda.synchronize()
    keep = mask.bool()
    err = rel(o.cpu()[keep], o_r[keep])
    assert torch.count_nonzero(o.cpu()[~keep]).item() == 0
    print(kind, f"masked {err:.2e}", flush=True)
    assert err <= TOL


def test_layer_c2_shape(oracle_ops):
    """BASELINE C2's layer shape (d_model 1024, H 4, d_k 256, d_v 512: expand_v 2) at a reduced
    length: one training step, output and every parameter gradient."""
    dev = _cuda()
    from ccq_amd import CCQGDN
    B, T = 1, 140
    torch.manual_seed(5)
    ref = CCQGDN(hidden_size=1024, head_dim=256, num_heads=4, expand_v=2, mode="fused_chunk", layer_idx=0)
    with torch.no_grad():
        ref.erase_lambda_proj.bias.fill_(0.0)
    ref = ref.double().train()
    gpu = copy.deepcopy(ref).float().to(dev).train()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, T, 1024, generator=g).bfloat16().float()
    do = torch.randn(B, T, 1024, generator=g)
    print("test_layer_c2_shape", flush=True)
    with oracle_ops:
        xr = x.to(D).requires_grad_()
        o_r, _, _ = ref(xr)
        (o_r * do.to(D)).sum().backward()
    xg = x.to(dev).requires_grad_()
    o, _, _ = gpu(xg)
    (o * do.to(dev)).sum().backward()
    torch.cuda.synchronize()
    errs = {"o": rel(o, o_r), "dx": rel(xg.grad, xr.grad)}
    for (n, p_r), (_, p) in zip(ref.named_parameters(), gpu.named_parameters()):
        if p_r.grad is not None:
            errs["d" + n] = rel(p.grad, p_r.grad)
    print("C2 layer", {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
    for n, e in errs.items():
        assert e <= TOL, n
