"""Benchmark of the north-star path on one MI355X: fused CCQ cleaning (per-head gate, fp32
statistics) + gated-delta-rule chunk forward and backward at B=8, T=4096, H=8, d_k=d_v=128, bf16.

Prints ONE JSON line (driver contract).  `value` is whole-job tokens/s of fwd+bwd with all
inputs resident in HBM; `roofline` is measured live for the dominant kernel with HIP events on
the stream the kernel runs on; `cpu_baseline` times the float32 PyTorch restatement of the
reference's non-fused algorithm (oracle/) on the host on a bounded sample.

The per-kernel breakdown comes from a pass with an event pair around every kernel; each pair puts a
marker between two kernels, so that pass is not the timed one.  The timed pass records events around
the dominant kernel only (one pair per step), for the roofline's live launch time.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import torch  # noqa: E402

B, T, H, K, V = 8, 4096, 8, 128, 128
PEAK_BF16 = 2.5e15   # MI355X dense bf16 MFMA, FLOP/s
PEAK_HBM = 8.0e12    # MI355X HBM3E, B/s

# Algorithmic work per token x head: BT = 64 dense tiles (no causal discount), each GEMM counted
# once at 2 M N K, fwd+bwd = 3 x fwd.
BT = 64
FLOP_CLEAN = 3 * (4 * K * K + 4 * BT * K)
FLOP_GDN = 3 * (6 * K * V + BT * (6 * K + 4 * V) + (2 * BT * BT) // 3)
FLOP_PER_TOKEN_HEAD = FLOP_CLEAN + FLOP_GDN


def make_inputs(device, seed=0, b=B, t=T):
    """Seeded synthetic inputs of BASELINE.json configs[1] (+ the GDN conventions of configs[2])."""
    gen = torch.Generator().manual_seed(seed)

    def l2n(x):
        return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)

    q = l2n(torch.randn(b, t, H, K, generator=gen)).to(torch.bfloat16)
    k = l2n(torch.randn(b, t, H, K, generator=gen)).to(torch.bfloat16)
    w = torch.randn(H, K, generator=gen) * 0.02
    bias = torch.empty(H).uniform_(-1.0, 1.0, generator=gen)
    v = torch.randn(b, t, H, V, generator=gen).to(torch.bfloat16)
    a_log = torch.empty(H).uniform_(0.0, math.log(16.0), generator=gen)
    g = -torch.nn.functional.softplus(torch.randn(b, t, H, generator=gen)) * a_log.exp()
    beta = torch.sigmoid(torch.randn(b, t, H, generator=gen))
    do = torch.randn(b, t, H, V, generator=gen).to(torch.bfloat16)
    xs = dict(q=q, k=k, v=v, g=g.float(), beta=beta.float(), w=w.float(), b=bias.float(), do=do)
    return {n: x.to(device) for n, x in xs.items()}


LEAVES = ("q", "k", "v", "g", "beta", "w", "b")


def gpu_step(x):
    """One training step of the path: forward, then the gradients of every input."""
    from ccq_amd import fused_chunk_ccq_gdn
    o, _, _, _ = fused_chunk_ccq_gdn(x["q"], x["k"], x["v"], None, x["g"], x["beta"], gate_w=x["w"],
                                     gate_b=x["b"], use_qk_l2norm_in_kernel=False)
    return torch.autograd.grad(o, [x[n] for n in LEAVES], x["do"])


MULTI_KERNEL_STAGES = ("clean_bwd_gate",)

# HBM bytes per launch at the metric shape, read from the committed rocprofv3 FETCH_SIZE /
# WRITE_SIZE summary (written by `bench.py --ingest-pmc`, which scales the counters by the
# reading for a known-size copy); a stage absent there reports traffic null.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_fused_ccq_gdn_B8_T4096_H8_K128.json")


def measured_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return {k: tuple(v) for k, v in json.load(f)["per_launch_bytes"].items()}
    except (OSError, ValueError, KeyError):
        return {}


# Compulsory work per token x head of each phase of the step: FLOP (dense BT x BT tiles, fwd+bwd = 3 x fwd, the backward = 2 x fwd) and bytes (each
# input read once, each output written once, bf16 activations, fp32 lambda / g / beta).
def phase_work(k=K, v=V, bt=BT):
    clean_fwd = 4 * k * k + 4 * bt * k
    gdn_fwd = 6 * k * v + bt * (6 * k + 4 * v) + (2 * bt * bt) // 3
    return {
        "cleaning fwd": (clean_fwd, 6 * k + 4),
        "cleaning bwd": (2 * clean_fwd, 10 * k + 8),
        "GDN fwd": (gdn_fwd, 4 * k + 4 * v + 8),
        "GDN bwd": (2 * gdn_fwd, 8 * k + 6 * v + 16),
    }


PHASE_OF = {
    "clean_fwd_sum": "cleaning fwd", "clean_fwd": "cleaning fwd",
    "clean_bwd_dq": "cleaning bwd", "clean_bwd_gsum": "cleaning bwd", "clean_bwd_dk": "cleaning bwd",
    "clean_bwd_gate": "cleaning bwd",
    "gdn_prep": "GDN fwd", "gdn_fwd_state": "GDN fwd",
    "gdn_bwd_state": "GDN bwd", "gdn_bwd_dqkw": "GDN bwd", "gdn_bwd_wy": "GDN bwd",
}


def kernel_work(k=K, v=V, bt=BT, cb=64):
    """The design's own FLOP and bytes per token x head of each timed stage (its inputs read once,
    its outputs written once, in the formats this implementation uses: fp32 q_clean into the
    delta rule, fp32 upstream gradients, per-chunk state snapshots), for comparison with the
    compulsory figures of phase_work()."""
    # fp32 K x K totals of 4 time segments per (sequence, head), each written once and read by
    # the later segments: about 4 K^2 bytes per segment of T / 4 tokens
    seg = 4 * k * k * 4 // T
    return {
        "clean_fwd_sum": (2 * k * k, 2 * k + seg),
        "clean_fwd": (4 * k * k + 4 * k * cb, 2 * k + 2 * k + 4 * k + 4 + seg),
        "clean_bwd_dq": (4 * k * k + 6 * k * cb, 2 * k + 2 * k + 4 * k + 4 + 2 * k + 16 + seg),
        "clean_bwd_gsum": (2 * k * k + 2 * k * cb, 2 * k + 4 * k + 16 + seg),
        "clean_bwd_dk": (6 * k * k + 8 * k * cb, 2 * k + 2 * k + 4 * k + 16 + 4 * k + 2 * k + seg),
        "gdn_prep": (2 * bt * (2 * k + v) + (2 * bt * bt) // 3, 2 * k + 2 * v + 8 + 2 * k + 4 * v + 4 + 4 * bt),
        # the forward walk with the chunk output fused in: state path (U = u - w S, S update) plus
        # Y = Qc S, P = Qc K^T and P U; reads k, w / wl, Qc (fp32), g, u; writes U, o, P^T and the
        # per-chunk state snapshots (int16 rows + one fp32 scale per row)
        "gdn_fwd_state": (4 * k * v + 2 * bt * k + 2 * k * v + 2 * bt * v,
                          2 * k + 4 * k + 4 * k + 4 + 4 * v + 4 * v + 2 * v + 4 * bt + (2 * k + 4) * v // bt),
        "gdn_bwd_state": (2 * bt * v + 6 * k * v,
                          4 * bt + 2 * v + 2 * k + 4 * k + 2 * k + 4 * v + (2 * k + 4) * v // bt),
        "gdn_bwd_dqkw": (6 * k * v + 2 * bt * v + 4 * bt * k,
                         2 * (2 * k + 4) * v // bt + 2 * v + 4 * v + 4 * v + 4 * k + 2 * k + 4 * bt + 12 * k + 4),
        "gdn_bwd_wy": (10 * bt * k + 4 * bt * v + 4 * bt * bt,
                       4 * bt + 4 * k + 4 * v + 2 * k + 2 * v + 4 * k + 4 * k + 2 * v + 8),
    }


def step_roofline(ms_per_step, units=B * T * H):
    """Whole step against min(MFMA peak, AI x HBM bandwidth) with the compulsory figures."""
    flop = sum(f for f, _ in phase_work().values()) * units
    byts = sum(b for _, b in phase_work().values()) * units
    ideal_s = max(flop / PEAK_BF16, byts / PEAK_HBM)
    return {"flop": flop, "bytes": byts, "ai": flop / byts, "bound": "hbm" if byts / PEAK_HBM >= flop / PEAK_BF16
            else "mfma", "ideal_us": ideal_s * 1e6, "frac": ideal_s / (ms_per_step * 1e-3)}


def dominant_kernel(step_kernel_ms):
    """The single-kernel stage with the largest share of the step."""
    single = [n for n in step_kernel_ms if n in PHASE_OF and n not in MULTI_KERNEL_STAGES]
    return max(single, key=lambda n: step_kernel_ms[n])


def roofline(name, avg_s, units=B * T * H):
    """Roofline object for kernel `name` (average launch time `avg_s` seconds).  Its algorithmic work is
    the compulsory work of the whole phase it belongs to (phase_work(): defined per phase, not per
    kernel), charged to this one kernel -- an upper bound of the kernel's share, so `frac` is an upper
    bound too.  The design's own per-kernel bytes are kept beside it."""
    phase = PHASE_OF[name]
    flop, byts = phase_work()[phase]
    if flop / byts >= PEAK_BF16 / PEAK_HBM:
        achieved, peak, unit, bound = flop * units / avg_s / 1e12, PEAK_BF16 / 1e12, "TFLOP/s", "mfma"
    else:
        achieved, peak, unit, bound = byts * units / avg_s / 1e9, PEAK_HBM / 1e9, "GB/s", "hbm"
    traffic = measured_traffic().get(name)
    dflop, dbytes = kernel_work()[name]
    return {"kernel": name, "phase": phase, "bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
            "frac": achieved / peak, "traffic": sum(traffic) if traffic else None,
            "avg_launch_us": avg_s * 1e6, "algorithmic_flop_per_launch": flop * units,
            "algorithmic_bytes_per_launch": byts * units,
            "attribution": f"compulsory work of the whole {phase} phase charged to this kernel (upper bound)",
            "design_bytes_per_launch": dbytes * units, "design_flop_per_launch": dflop * units,
            "mfma_frac_design_flop": dflop * units / avg_s / PEAK_BF16}


def cpu_model_name() -> str:
    """The host CPU's model name, as ``lscpu`` reports it (read from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds_budget=25.0):
    """fp32 PyTorch restatement of the reference's non-fused algorithm (oracle/) on the host:
    lambda gate, cleaning (chunked), gated delta rule (chunked WY form), autograd fwd+bwd,
    on a bounded sample (one sequence of T_s tokens, all H heads)."""
    from oracle import ccq_oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    t_s = 4096
    x = make_inputs("cpu", seed=0, b=1, t=t_s)
    for n in LEAVES:
        x[n] = x[n].float().requires_grad_()

    def step():
        lam = O.lambda_gate(x["q"], x["w"], x["b"])
        qc, _, _ = O.clean_fwd_chunked(x["q"], x["k"], lam)
        o, _ = O.gdn_chunked(qc, x["k"], x["v"], x["g"], x["beta"])
        o.backward(x["do"].float())

    step()  # warm-up
    times = []
    t_end = time.perf_counter() + seconds_budget
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 10):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": t_s / med, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": cpu_model_name(),
            "sample": f"1 sequence x {t_s} tokens x {H} heads (d_k=d_v={K}), fp32 autograd fwd+bwd, "
                      f"median of {len(times)} after 1 warm-up"}


def _timed_steps(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _line(metric, value, unit, args, ms, dtype, data, config, higher=True, **extra):
    out = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": higher, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
           "data": data, "config": config}
    out.update(extra)
    return out


def copy_calibration(dev):
    """One elementwise kernel of known traffic (512 MiB read, 512 MiB written): the reference that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE readings to bytes."""
    src = torch.ones(256 << 20, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def run_c1(args, dev):
    x = make_inputs(dev)
    for n in LEAVES:
        x[n].requires_grad_()
    from ccq_amd import _lib

    for _ in range(args.warmup):
        gpu_step(x)
    torch.cuda.synchronize()
    # breakdown pass: every kernel between its own event pair
    _lib.timing_reset()
    _lib.timing_select(None)
    _lib.timing_enable(True)
    for _ in range(args.steps):
        gpu_step(x)
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    kms, klaunch = {}, {}
    for name in _lib.KERNELS:
        ms_tot, n = _lib.timing_read(name)
        if n:
            kms[name], klaunch[name] = ms_tot / args.steps, n / args.steps
    dom = dominant_kernel(kms)
    # timed pass: events around the dominant kernel only
    _lib.timing_reset()
    _lib.timing_select(dom)
    _lib.timing_enable(True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        gpu_step(x)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.timing_enable(False)
    _lib.timing_select(None)
    dom_ms, dom_n = _lib.timing_read(dom)
    if args.copy_calibration:
        copy_calibration(dev)
    ms = elapsed / args.steps * 1e3
    flops = FLOP_PER_TOKEN_HEAD * B * T * H
    out = _line("cleaning+chunk fwd+bwd tokens/s at B8·T4096·H8·dk128 bf16; % MFMA peak", B * T * args.steps / elapsed,
                "tokens/s", args, ms, "bf16", "synthetic (seeded, BASELINE.json configs[1] + configs[2] GDN conventions)",
                {"workload": "fused CCQ cleaning (per-head gate) + GDN chunk fwd+bwd", "B": B, "T": T, "H": H,
                 "d_k": K, "d_v": V, "chunk": BT, "algorithmic_flop_per_step": flops,
                 "mfma_peak_fraction": flops / (ms * 1e-3) / PEAK_BF16,
                 "kernel_ms_per_step": {n: round(v, 4) for n, v in kms.items()},
                 "kernel_ms_note": "breakdown pass with an event pair around every kernel; the timed pass "
                                   "records events around the dominant kernel only"},
                roofline=roofline(dom, dom_ms / dom_n * 1e-3), step_roofline=step_roofline(ms))
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    return out


def run_decode(args, dev, layers=24, b=16, h=4, k=256, v=512):
    """C4's recurrent decode at its per-layer state shapes: `layers` CCQ-GDN decode steps (per-head
    gate, subtract_mean, l2norm) captured in one HIP graph, one token per sequence per replay.
    Inputs of the token are written into the steps' buffers once (their values do not change the
    work); the states carry over from replay to replay."""
    from ccq_amd.graph import CapturedDecode, DecodeStep
    gen = torch.Generator().manual_seed(0)
    steps = []
    for _ in range(layers):
        st = DecodeStep(b, h, k, v, mode="gdn", gate=True, device=dev)
        st.q.copy_(torch.randn(b, 1, h, k, generator=gen))
        st.k.copy_(torch.randn(b, 1, h, k, generator=gen))
        st.v.copy_(torch.randn(b, 1, h, v, generator=gen))
        st.g.copy_(-torch.rand(b, 1, h, generator=gen))
        st.beta.copy_(torch.rand(b, 1, h, generator=gen))
        st.gate_b.uniform_(-1.0, 1.0)
        kk = torch.nn.functional.normalize(torch.randn(b, h, 64, k, generator=gen), dim=-1)
        st.load_state((0.01 * torch.randn(b, h, k, v, generator=gen)).to(dev), (kk.transpose(-1, -2) @ kk).to(dev),
                      kk.sum(-2).to(dev), 16384)
        steps.append(st)
    cap = CapturedDecode(steps).capture()
    t_graph = _timed_steps(cap.replay, args.steps, args.warmup)
    t_eager = _timed_steps(cap.eager, args.steps, args.warmup)
    if args.copy_calibration:
        copy_calibration(dev)
    state_bytes = sum(s.state_bytes() for s in steps)
    io_bytes = layers * b * h * (2 * k + 2 * k + 2 * v + 2 * v + 4 + 4)
    byts = state_bytes + io_bytes
    achieved = byts / t_graph / 1e9
    return _line("CCQ-GDN decode step latency (24 layers, B16, H4, d_k256, d_v512; captured HIP graph)",
                 t_graph * 1e3, "ms/step", args, t_graph * 1e3, "f32 states, bf16 q/k/v/o",
                 "synthetic (seeded; states of a 16,384-token prefill shape, random values)",
                 {"workload": "C4 decode: recurrent CCQ-GDN step of every layer, one token per sequence",
                  "layers": layers, "B": b, "H": h, "d_k": k, "d_v": v, "tokens_per_s": b / t_graph,
                  "eager_ms_per_step": t_eager * 1e3, "state_bytes_per_step": state_bytes,
                  "bound_ms_with_weights_at_8tbs": 0.42},
                 higher=False,
                 roofline={"kernel": "decode step (clean + backbone kernels, all layers)", "bound": "hbm",
                           "achieved": achieved, "peak": PEAK_HBM / 1e9, "unit": "GB/s", "frac": achieved * 1e9 /
                           PEAK_HBM, "traffic": None, "algorithmic_bytes_per_step": byts,
                           "ideal_ms": byts / PEAK_HBM * 1e3})


def _gdn_inputs(dev, b, t, h, k, v, seed=0):
    gen = torch.Generator().manual_seed(seed)
    l2 = lambda x: torch.nn.functional.normalize(x, dim=-1)  # noqa: E731
    q = l2(torch.randn(b, t, h, k, generator=gen)).to(torch.bfloat16)
    kk = l2(torch.randn(b, t, h, k, generator=gen)).to(torch.bfloat16)
    vv = torch.randn(b, t, h, v, generator=gen).to(torch.bfloat16)
    a_log = torch.empty(h).uniform_(0.0, math.log(16.0), generator=gen)
    g = (-torch.nn.functional.softplus(torch.randn(b, t, h, generator=gen)) * a_log.exp()).float()
    beta = torch.sigmoid(torch.randn(b, t, h, generator=gen)).float()
    w = (torch.randn(h, k, generator=gen) * 0.02).float()
    bias = torch.empty(h).uniform_(-1.0, 1.0, generator=gen).float()
    do = torch.randn(b, t, h, v, generator=gen).to(torch.bfloat16)
    xs = dict(q=q, k=kk, v=vv, g=g, beta=beta, w=w, b=bias, do=do)
    return {n: x.to(dev) for n, x in xs.items()}


def run_readme(args, dev, b=1, t=32768, h=6, k=256, v=512):
    """The reference README's published shape (32K tokens, 6 heads, K=256, V=512, fwd+bwd): the
    cleaning overhead = fused CCQ-GDN fwd+bwd minus the plain GDN chunk fwd+bwd on the same inputs."""
    from ccq_amd import chunk_gated_delta_rule, fused_chunk_ccq_gdn
    x = _gdn_inputs(dev, b, t, h, k, v)
    for n in LEAVES:
        x[n].requires_grad_()

    def ccq():
        o, _, _, _ = fused_chunk_ccq_gdn(x["q"], x["k"], x["v"], None, x["g"], x["beta"], gate_w=x["w"],
                                         gate_b=x["b"])
        torch.autograd.grad(o, [x[n] for n in LEAVES], x["do"])

    plain_leaves = ("q", "k", "v", "g", "beta")

    def plain():
        o, _ = chunk_gated_delta_rule(x["q"], x["k"], x["v"], x["g"], x["beta"])
        torch.autograd.grad(o, [x[n] for n in plain_leaves], x["do"])

    t_ccq = _timed_steps(ccq, args.steps, args.warmup)
    t_plain = _timed_steps(plain, args.steps, args.warmup)
    return _line("CCQ cleaning overhead over plain GDN, fwd+bwd, 32K tokens, H6, d_k256, d_v512 (README shape)",
                 (t_ccq - t_plain) * 1e3, "ms", args, t_ccq * 1e3, "bf16",
                 "synthetic (seeded; q, k L2-normalised, C2 decay convention, per-head gate)",
                 {"workload": "fused_chunk_ccq_gdn vs chunk_gated_delta_rule fwd+bwd", "B": b, "T": t, "H": h,
                  "d_k": k, "d_v": v, "ccq_gdn_ms": t_ccq * 1e3, "plain_gdn_ms": t_plain * 1e3,
                  "tokens_per_s": b * t / t_ccq,
                  "reference_published_overhead_ms_h200": [4.2, 7.1]},
                 higher=False)


def run_layer(args, dev, which):
    """C2 (CCQ-GDN layer, d_model 1024, H4, K256, V512, B4 T4096) or C3 (CCQ-GLA layer, H4, K128,
    V256, B4 T8192, short conv on) forward + backward, random init, bf16."""
    from ccq_amd.layers import CCQGDN, CCQGLA
    torch.manual_seed(0)
    if which == "c2":
        b, t = 4, 4096
        layer = CCQGDN(hidden_size=1024, head_dim=256, num_heads=4, expand_v=2, mode="fused_chunk", layer_idx=0)
        desc = "CCQ-GDN layer fwd+bwd, d_model1024, H4, d_k256, d_v512, B4, T4096 (fused_chunk)"
    else:
        b, t = 4, 8192
        layer = CCQGLA(mode="fused_chunk", hidden_size=1024, expand_k=0.5, expand_v=1.0, num_heads=4,
                       use_short_conv=True, layer_idx=0)
        desc = "CCQ-GLA layer fwd+bwd, d_model1024, H4, d_k128, d_v256, B4, T8192 (fused_chunk, short conv)"
    layer = layer.to(dev, torch.bfloat16)
    gen = torch.Generator().manual_seed(0)
    xin = torch.randn(b, t, 1024, generator=gen).to(dev, torch.bfloat16).requires_grad_()
    dy = torch.randn(b, t, 1024, generator=gen).to(dev, torch.bfloat16)
    params = [p for p in layer.parameters() if p.requires_grad]

    def step():
        y = layer(xin)[0]
        torch.autograd.grad(y, [xin] + params, dy)

    dt = _timed_steps(step, args.steps, args.warmup)
    if args.copy_calibration:
        copy_calibration(dev)
    return _line(desc, b * t / dt, "tokens/s", args, dt * 1e3, "bf16",
                 "synthetic (seeded; x ~ N(0,1); the reference layer's own random init)",
                 {"workload": f"{which.upper()} single layer fwd+bwd", "B": b, "T": t})


def run_c4(args, dev, layers=24, b=16, t=16384, d=1024, vocab=32000, decode_steps=256, check_steps=4):
    """C4: a random-init 24-layer CCQ-GDN stack (RMSNorm -> CCQGDN -> residual, RMSNorm -> gated MLP
    -> residual; token embedding, final norm, LM head; bf16) over B x T uniform-random token ids:
    chunked prefill with the recurrent cache, then greedy decode steps carrying (S, C, m, position)
    and the short-convolution states.  The blocks around the layer are the measurement harness
    (the reference takes them from its HF model classes, which this library does not provide).

    Decode runs two ways from the same prefill state: eager (the layers' own recurrent mode, one
    launch per op from Python) and as one captured HIP graph of the whole model's step, in which
    each layer's token step is the library's ``GDNLayerDecode`` (one GEMM for the layer's input
    projections, the decode prologue kernel, the in-place decode step with the position held on the
    device, the output norm and projection) and the greedy token is written back into the graph's
    input.  The graph is replayed on the eager path's first tokens and each replay's logits are
    checked against the eager layers' before it is timed."""
    import torch.nn as nn
    import torch.nn.functional as F
    from ccq_amd.graph import (GDNLayerDecode, decode_linear, decode_linear_glu, decode_linear_split, greedy_embed,
                               split_plan, split_workspace)
    from ccq_amd.layers import CCQGDN, LayerCache

    inter = 256 * ((int(d * 4 * 2 / 3) + 255) // 256)  # fla GatedMLP's intermediate size (hidden_ratio 4)

    # block norms: torch's RMSNorm (x rsqrt(mean(x^2) + eps) w, as fla's), one fused op per call
    def RMSNorm(n):
        return nn.RMSNorm(n, eps=1e-5)

    class Block(nn.Module):
        def __init__(self, i):
            super().__init__()
            self.attn_norm = RMSNorm(d)
            self.attn = CCQGDN(hidden_size=d, head_dim=256, num_heads=4, expand_v=2, mode="chunk", layer_idx=i)
            self.mlp_norm = RMSNorm(d)
            self.gate_up = nn.Linear(d, 2 * inter, bias=False)
            self.down = nn.Linear(inter, d, bias=False)

        def mlp(self, x):
            gt, up = self.gate_up(self.mlp_norm(x)).chunk(2, -1)
            return x + self.down(F.silu(gt) * up)

        def mlp_step(self, x):
            # the captured decode step's MLP: the norm folded into the up projection's kernel, which
            # also forms silu(gate) * up; the down projection with the residual added in it, its
            # contraction split over several workgroups per column block (workspace: zeroed once)
            h = decode_linear_glu(x, self.gate_up.weight, norm_weight=self.mlp_norm.weight,
                                  norm_eps=self.mlp_norm.eps)
            if not hasattr(self, "down_ws"):
                self.down_splits = split_plan(inter, d)
                self.down_ws = split_workspace(d, self.down_splits, x.device)
            return decode_linear_split(h, self.down.weight, x, self.down_splits, self.down_ws)

        def forward(self, x, cache):
            return self.mlp(x + self.attn(self.attn_norm(x), past_key_values=cache, use_cache=True)[0])

    torch.manual_seed(0)
    embed = nn.Embedding(vocab, d).to(dev, torch.bfloat16)
    blocks = nn.ModuleList(Block(i) for i in range(layers)).to(dev, torch.bfloat16).eval()
    norm = RMSNorm(d).to(dev, torch.bfloat16)
    head = nn.Linear(d, vocab, bias=False).to(dev, torch.bfloat16)
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, vocab, (b, t), generator=gen).to(dev)

    def forward(ids, cache):
        x = embed(ids)
        for blk in blocks:
            x = blk(x, cache)
        return head(norm(x[:, -1]))  # logits of the last position only

    def snapshot(cache):
        out = []
        for st in cache.states:
            S, C, m, pos = st["recurrent_state"]
            out.append(((S.clone(), C.clone(), m.clone(), pos), tuple(c.clone() for c in st["conv_state"])))
        return out

    # the captured step: static token ids and input rows, one GDNLayerDecode (static buffers) per layer
    ids = torch.zeros(b, 1, dtype=torch.long, device=dev)
    xin = torch.zeros(b, 1, d, dtype=torch.bfloat16, device=dev)
    lds = [GDNLayerDecode(blk.attn, b) for blk in blocks]

    def feed(tok):
        """The step's input: token ids [b] and their embedding rows."""
        ids.copy_(tok[:, None])
        xin.copy_(embed(ids))

    def load(snap):
        for ld, (state, convs) in zip(lds, snap):
            ld.load({"recurrent_state": state, "conv_state": convs})

    def graph_step():
        x = xin
        for blk, ld in zip(blocks, lds):
            x = blk.mlp_step(ld(x, x, norm=blk.attn_norm))
        # the final RMSNorm folded into the LM head's projection (one launch, the same kernel)
        logits = decode_linear(x[:, -1], head.weight, norm_weight=norm.weight, norm_eps=norm.eps)
        # the greedy pick and its embedding row, the next step's input, in one launch
        greedy_embed(logits, embed.weight, ids, xin)
        return logits

    with torch.no_grad():
        forward(prompt, LayerCache())  # warm-up at full size (kernel loads, the allocator's pools)
        torch.cuda.synchronize()
        cache = LayerCache()
        t0 = time.perf_counter()
        logits = forward(prompt, cache)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        tok0 = logits.argmax(-1)
        snap = snapshot(cache)

        # eager decode (the first check_steps tokens and logits are the captured graph's reference)
        ref_in, ref_logits, nxt = [], [], tok0
        warm = min(3, decode_steps)
        for i in range(decode_steps):
            if i == warm:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
            ref_in.append(nxt)
            lg = forward(nxt[:, None], cache)
            if i < check_steps:
                ref_logits.append(lg.float())
            nxt = lg.argmax(-1)
        torch.cuda.synchronize()
        t_eager = (time.perf_counter() - t0) / max(decode_steps - warm, 1)
        assert cache.get_seq_length() == t + decode_steps

        # captured decode: warm up the step eagerly (libraries pick their kernels), restore the
        # prefill state, capture, then replay on the eager tokens and compare every replay
        load(snap)
        feed(tok0)
        graph_step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits_g = graph_step()
        load(snap)
        errs = []
        for i in range(check_steps):
            feed(ref_in[i])
            graph.replay()
            torch.cuda.synchronize()
            errs.append(((logits_g.float() - ref_logits[i]).norm() / ref_logits[i].norm()).item())
        if max(errs) > 2e-2:
            raise RuntimeError(f"captured decode step disagrees with the eager layers: rel-L2 {errs}")
        load(snap)
        feed(tok0)
        for _ in range(warm):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(decode_steps - warm):
            graph.replay()
        torch.cuda.synchronize()
        t_graph = (time.perf_counter() - t0) / max(decode_steps - warm, 1)
    return _line("C4 whole-model prefill tokens/s (24 CCQ-GDN layers, d_model1024, H4, d_k256, d_v512, B16, "
                 "T16384) + greedy decode", b * t / t_prefill, "tokens/s", args, t_prefill * 1e3, "bf16",
                 "synthetic (uniform-random token ids; random-init weights)",
                 {"workload": "C4: chunked prefill with the recurrent cache, then greedy recurrent decode",
                  "layers": layers, "B": b, "T": t, "d_model": d, "vocab": vocab, "mlp_intermediate": inter,
                  "prefill_s": t_prefill, "decode_steps": decode_steps,
                  "decode_ms_per_step_graph": t_graph * 1e3, "decode_ms_per_step_eager": t_eager * 1e3,
                  "graph_vs_eager_logits_rel_l2": errs})


def ingest_pmc(fetch_dir, write_dir, out_path):
    """Per-launch HBM bytes of each timed stage from two rocprofv3 --pmc runs of this script with
    --copy-calibration (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch), each scaled by the counter's
    reading for the calibration copy (torch neg over 512 MiB read + 512 MiB written)."""
    import csv
    import glob
    import re
    kernel_stage = {
        "cs_sum_kernel": "clean_fwd_sum", "cs_fwd_kernel": "clean_fwd", "cs_dq_kernel": "clean_bwd_dq",
        "cs_gsum_kernel": "clean_bwd_gsum", "cs_dk_kernel": "clean_bwd_dk", "gdn_prep": "gdn_prep",
        "gdn_fwd_state": "gdn_fwd_state", "gdn_bwd_state": "gdn_bwd_state", "gdn_bwd_dqkw": "gdn_bwd_dqkw",
        "gdn_bwd_wy": "gdn_bwd_wy",
    }

    def read(d, counter):
        per, calib = {}, []
        for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(fn)):
                if r["Counter_Name"] != counter:
                    continue
                name = r["Kernel_Name"]
                val = float(r["Counter_Value"]) * 1024.0
                if "neg" in name:
                    calib.append(val)
                    continue
                for key, stage in kernel_stage.items():
                    if re.search(r"\b" + key, name):
                        per.setdefault(stage, []).append(val)
        return {k: sum(v) / len(v) for k, v in per.items()}, (max(calib) if calib else None)

    fetch, fcal = read(fetch_dir, "FETCH_SIZE")
    write, wcal = read(write_dir, "WRITE_SIZE")
    ref = 512.0 * 2 ** 20
    fs, ws = ref / fcal, ref / wcal
    data = {"scale": {"fetch": fs, "write": ws},
            "per_launch_bytes": {k: [fetch[k] * fs, write.get(k, 0.0) * ws] for k in sorted(fetch)}}
    with open(out_path, "w") as f:
        json.dump(data, f, indent=1)
    print(json.dumps(data))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=("c1", "decode", "readme", "c2", "c3", "c4"), default="c1",
                    help="c1: the metric (default); decode: C4's captured decode step; readme: the reference "
                         "README's cleaning-overhead shape; c2 / c3: single-layer fwd+bwd; c4: the 24-layer "
                         "model's prefill and greedy decode")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--c4-prefill", type=int, default=16384,
                    help="c4: prompt tokens per sequence (BASELINE C4: 16384; a short prompt profiles the decode step)")
    ap.add_argument("--c4-decode-steps", type=int, default=256, help="c4: greedy decode steps")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed steps, run one elementwise copy of 512 MiB (read) + 512 MiB (write), "
                         "the known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counts")
    ap.add_argument("--ingest-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="write the per-launch traffic file from two rocprofv3 --pmc output folders and exit")
    args = ap.parse_args()
    if args.ingest_pmc:
        ingest_pmc(args.ingest_pmc[0], args.ingest_pmc[1], TRAFFIC_FILE)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    if args.workload == "c1":
        out = run_c1(args, dev)
    elif args.workload == "decode":
        out = run_decode(args, dev)
    elif args.workload == "readme":
        out = run_readme(args, dev)
    elif args.workload == "c4":
        out = run_c4(args, dev, t=args.c4_prefill, decode_steps=args.c4_decode_steps)
    else:
        out = run_layer(args, dev, args.workload)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
