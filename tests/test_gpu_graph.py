"""GPU checks of the captured decode loop (ccq_amd.graph): the in-place decode step with a
device-held position, recorded in one HIP graph over several layers, replayed token after token.

Each replay is compared with the eager, allocating decode op (``gdn_decode`` / ``gla_decode``,
itself held to the CPU oracle by test_gpu_decode.py) fed the same inputs and the previous step's
states: the same kernels see the same numbers, so outputs, states and positions must be
bit-identical.  Eager work and synchronisations run between the replays, and every replay is
checked, not only the last."""

import pytest
import torch

from tests._util import bf, l2n

pytestmark = pytest.mark.gpu


def _cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import ccq_amd  # noqa: F401
    return torch.device("cuda")


CASES = [
    # mode, layers, B, H, K, V, gate, subtract_mean, steps
    ("gdn", 2, 2, 2, 64, 128, True, True, 4),
    ("gdn", 3, 3, 4, 256, 512, False, True, 3),
    ("gdn", 1, 2, 2, 128, 64, True, False, 3),
    ("gla", 2, 2, 2, 128, 256, True, True, 3),
]


@pytest.mark.parametrize("case", CASES, ids=[str(i) for i in range(len(CASES))])
def test_captured_decode_matches_eager(case):
    dev = _cuda()
    from ccq_amd.decode import gdn_decode, gla_decode
    from ccq_amd.graph import CapturedDecode, DecodeStep

    mode, L, B, H, K, V, gate, sub, steps = case
    print(f"captured decode case {case}", flush=True)
    gen = torch.Generator().manual_seed(11)
    pos0 = 29
    layers = []
    for _ in range(L):
        st = DecodeStep(B, H, K, V, mode=mode, gate=gate, subtract_mean=sub, device=dev)
        kk = l2n(torch.randn(B, H, pos0, K, generator=gen))
        S0 = (torch.randn(B, H, K, V, generator=gen) * 0.1).float()
        st.load_state(S0.to(dev), (kk.transpose(-1, -2) @ kk).float().to(dev), kk.sum(-2).float().to(dev), pos0)
        if gate:
            st.gate_w.copy_(0.1 * torch.randn(H, K, generator=gen))
            st.gate_b.copy_(torch.rand(H, generator=gen) * 2 - 1)
        layers.append(st)
    # eager reference states (copies)
    ref = [[t.clone() if t is not None else None for t in (s.S, s.C, s.m)] for s in layers]
    graph = CapturedDecode(layers).capture()
    for step in range(steps):
        ins = []
        for st in layers:
            q = bf(torch.randn(B, 1, H, K, generator=gen) * 2)
            k = bf(torch.randn(B, 1, H, K, generator=gen) * 2)
            v = bf(torch.randn(B, 1, H, V, generator=gen))
            x = {"q": q, "k": k, "v": v}
            if not gate:
                # (the op rounds lambda to q's dtype, as the reference does; the step reads it as given)
                x["lam"] = torch.sigmoid(torch.randn(B, 1, H, generator=gen)).to(torch.bfloat16).float()
            if mode == "gdn":
                x["g"] = -torch.rand(B, 1, H, generator=gen) * 3
                x["beta"] = torch.rand(B, 1, H, generator=gen)
            else:
                x["gk"] = -torch.rand(B, 1, H, K, generator=gen) * 0.5
            for name, t in x.items():
                getattr(st, name).copy_(t)
            ins.append({n: t.to(dev) for n, t in x.items()})
        graph.replay()
        torch.cuda.synchronize()
        for li, (st, x) in enumerate(zip(layers, ins)):
            S, C, m = ref[li]
            gw, gb = (st.gate_w, st.gate_b) if gate else (None, None)
            if mode == "gdn":
                o, S2, C2, m2 = gdn_decode(x["q"], x["k"], x["v"], x.get("lam"), x["g"], x["beta"], st.scale,
                                           initial_state=S, initial_cov_state=C, initial_mean_state=m,
                                           position_offset=pos0 + step, subtract_mean=sub, gate_w=gw, gate_b=gb)
            else:
                o, S2, C2, m2 = gla_decode(x["q"], x["k"], x["v"], x.get("lam"), x["gk"], st.scale,
                                           initial_state=S, initial_cov_state=C, initial_mean_state=m,
                                           position_offset=pos0 + step, subtract_mean=sub, gate_w=gw, gate_b=gb)
            torch.cuda.synchronize()
            assert torch.equal(st.o, o), f"layer {li} step {step}: output"
            assert torch.equal(st.S, S2), f"layer {li} step {step}: S"
            assert torch.equal(st.C, C2), f"layer {li} step {step}: C"
            if sub:
                assert torch.equal(st.m, m2), f"layer {li} step {step}: m"
            assert int(st.position.item()) == pos0 + step + 1
            ref[li] = [S2, C2, m2 if sub else None]
        # eager work of the program between replays
        torch.cuda.synchronize()


def test_decode_step_rejects_missing_state():
    _cuda()
    from ccq_amd import _lib
    from ccq_amd.graph import DecodeStep
    st = DecodeStep(1, 1, 64, 64, device="cuda")
    lib = _lib.load()
    from ccq_amd._lib import ptr
    status = lib.ccq_gdn_decode_step(ptr(st.q), ptr(st.k), ptr(st.v), None, ptr(st.gate_w), ptr(st.gate_b),
                                     ptr(st.g), ptr(st.beta), ptr(st.S), ptr(st.C), ptr(st.m), None, ptr(st.o),
                                     ptr(st.workspace), 1, 1, 1, 64, 64, 1, 1, 1, 0.125, None)
    assert status == -2 and b"position" in lib.ccq_last_error()


def test_whole_model_decode_graph_matches_eager():
    """BASELINE C4's harness (``bench.run_c4``) at a reduced size: 2 CCQ-GDN layers (d_k 256, d_v
    512), 2 sequences of 256 tokens, 6 greedy decode steps.  The harness prefills, decodes eagerly
    through the layers' recurrent mode, then captures the whole model's token step (the layers'
    projections, prologue and output norm around the in-place decode kernels) in one graph and
    raises unless each of the first replays, fed the eager path's tokens, reproduces the eager
    logits."""
    dev = _cuda()
    import types

    import bench
    print("test_whole_model_decode_graph_matches_eager layers=2 b=2 t=256", flush=True)
    out = bench.run_c4(types.SimpleNamespace(steps=0, warmup=0), dev, layers=2, b=2, t=256, decode_steps=6,
                       check_steps=4)
    errs = out["config"]["graph_vs_eager_logits_rel_l2"]
    print("captured vs eager logits rel-L2", errs, flush=True)
    assert len(errs) == 4 and max(errs) <= 2e-2


@pytest.mark.parametrize("H,K,expand_v,T0", [(4, 256, 2, 70), (2, 128, 1, 33)])
def test_layer_decode_matches_recurrent_mode(H, K, expand_v, T0):
    """GDNLayerDecode (one GEMM for the input projections, the decode prologue kernel, the in-place
    decode step, the output norm and projection) against the bf16 layer's own recurrent mode
    (CCQGDN.forward with a LayerCache, one token per call) from the same chunked prefill: outputs,
    states, convolution caches and position after every token; then the same step captured in a
    graph and replayed token after token from the prefill state again."""
    dev = _cuda()
    import copy

    from ccq_amd import CCQGDN, LayerCache
    from ccq_amd.graph import GDNLayerDecode
    from tests._util import rel
    B, steps = 3, 4
    print(f"test_layer_decode_matches_recurrent_mode H={H} K={K} expand_v={expand_v}", flush=True)
    torch.manual_seed(0)
    layer = CCQGDN(hidden_size=512, head_dim=K, num_heads=H, expand_v=expand_v, mode="chunk", layer_idx=0)
    with torch.no_grad():
        layer.erase_lambda_proj.bias.fill_(0.0)
    layer = layer.to(dev, torch.bfloat16).eval()
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(B, T0 + steps, 512, generator=gen).to(dev, torch.bfloat16)
    with torch.no_grad():
        cache = LayerCache()
        layer(x[:, :T0], past_key_values=cache, use_cache=True)
        prefill = copy.deepcopy(cache)
        ld = GDNLayerDecode(layer, B)
        ld.load(prefill.get(0))
        for t in range(T0, T0 + steps):
            o_e = layer(x[:, t:t + 1], past_key_values=cache, use_cache=True)[0]
            o_f = ld(x[:, t:t + 1])
            torch.cuda.synchronize()
            S, C, m, pos = cache.get(0)["recurrent_state"]
            errs = {"o": rel(o_f, o_e), "S": rel(ld.step.S, S), "C": rel(ld.step.C, C), "m": rel(ld.step.m, m)}
            print(t, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
            assert errs["o"] <= 2e-3
            for n in ("S", "C", "m"):
                assert errs[n] <= 1e-5, n
            assert int(ld.step.position.item()) == pos == t + 1
            # the caches hold the projections' outputs, which here come from one GEMM over the
            # concatenated weights and there from one GEMM per projection: equal up to roundings
            # that the different summation orders move across a tie
            for a, b in zip(ld.conv, cache.get(0)["conv_state"]):
                assert rel(a, b) <= 1e-3, "convolution cache"
        # captured: the same steps replayed from the prefill state
        h = torch.zeros(B, 1, 512, device=dev, dtype=torch.bfloat16)
        ld.load(prefill.get(0))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            ld(h)                              # loads the kernels; its state change is undone below
        torch.cuda.current_stream().wait_stream(side)
        ld.load(prefill.get(0))
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = ld(h)
        ld.load(prefill.get(0))
        ref = GDNLayerDecode(layer, B)
        ref.load(prefill.get(0))
        # (the projection GEMM may take another algorithm under capture than eagerly, so the replays are
        # held to the same tolerances, not to bit equality)
        for t in range(T0, T0 + steps):
            h.copy_(x[:, t:t + 1])
            graph.replay()
            o_r = ref(x[:, t:t + 1])
            torch.cuda.synchronize()
            errs = {"o": rel(out, o_r), "S": rel(ld.step.S, ref.step.S), "C": rel(ld.step.C, ref.step.C),
                    "conv": rel(ld.conv[0], ref.conv[0])}
            print("replay", t, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
            assert errs["o"] <= 2e-3 and errs["conv"] <= 1e-3
            assert errs["S"] <= 1e-5 and errs["C"] <= 1e-5
            assert int(ld.step.position.item()) == t + 1


@pytest.mark.parametrize("H,K,expand_v,T,flags", [(4, 256, 2, 1, {}), (2, 128, 1, 2, {}), (2, 64, 2, 3, {}),
                                                   (2, 128, 1, 2, {"subtract_mean": False}),
                                                   (2, 128, 1, 1, {"enable_ccq": False})])
def test_layer_decode_in_proj_path_matches_prologue_path(H, K, expand_v, T, flags):
    """GDNLayerDecode's two paths on the same inputs: the short convolutions, g and beta in the input
    projections' epilogue with the decode step normalising q and k and forming lambda
    (``ccq_gdn_decode_in_proj`` + ``ccq_gdn_layer_decode_step``) and the gated output norm folded into
    the output projection (``ccq_decode_linear_gnorm``), against the input projections, the decode
    prologue kernel, the decode step, the gated norm kernel and the output projection.  Outputs within a bf16 unit on rare elements (the
    per-head sums of squares and the lambda logit run in another order), states to fp32 roundings,
    convolution caches and position equal; T tokens per call.  Also a layer without the running mean
    (``subtract_mean=False``) and one without cleaning (``enable_ccq=False``: no covariance, no lambda)."""
    dev = _cuda()
    import copy

    from ccq_amd import CCQGDN, LayerCache
    from ccq_amd.graph import GDNLayerDecode
    from tests._util import rel
    B, T0, steps = 3, 37, 3
    print(f"test_layer_decode_in_proj_path_matches_prologue_path H={H} K={K} expand_v={expand_v} T={T} {flags}",
          flush=True)
    torch.manual_seed(0)
    layer = CCQGDN(hidden_size=256, head_dim=K, num_heads=H, expand_v=expand_v, mode="chunk", layer_idx=0, **flags)
    layer = layer.to(dev, torch.bfloat16).eval()
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(B, T0 + steps * T, 256, generator=gen).to(dev, torch.bfloat16)
    with torch.no_grad():
        cache = LayerCache()
        layer(x[:, :T0], past_key_values=cache, use_cache=True)
        fused, plain = GDNLayerDecode(layer, B, T), GDNLayerDecode(layer, B, T)
        assert fused.conv_in_proj and fused.fast and fused.gnorm_in_proj
        plain.conv_in_proj = plain.gnorm_in_proj = False
        for ld in (fused, plain):
            ld.load(copy.deepcopy(cache).get(0))
        for s in range(steps):
            h = x[:, T0 + s * T:T0 + (s + 1) * T]
            o_f, o_p = fused(h), plain(h)
            torch.cuda.synchronize()
            errs = {"o": rel(o_f, o_p), "S": rel(fused.step.S, plain.step.S)}
            for n in ("C", "m"):
                a, b = getattr(fused.step, n), getattr(plain.step, n)
                assert (a is None) == (b is None), n
                if a is not None:
                    errs[n] = rel(a, b)
            print(s, {n: f"{e:.2e}" for n, e in errs.items()}, flush=True)
            assert errs["o"] <= 1e-3
            for n in errs.keys() - {"o"}:
                assert errs[n] <= 1e-5, n
            for a, b in zip(fused.conv, plain.conv):
                assert torch.equal(a, b), "convolution cache"
            assert torch.equal(fused.step.g, plain.step.g) and torch.equal(fused.step.beta, plain.step.beta)
            assert int(fused.step.position.item()) == int(plain.step.position.item()) == T0 + (s + 1) * T
