"""Benchmark of the north-star path on one MI355X: fused CCQ cleaning (per-head gate, fp32
statistics) + gated-delta-rule chunk forward and backward at B=8, T=4096, H=8, d_k=d_v=128, bf16.

Prints ONE JSON line (driver contract).  `value` is whole-job tokens/s of fwd+bwd with all
inputs resident in HBM; `roofline` is measured live for the dominant kernel with HIP events on
the stream the kernel runs on; `cpu_baseline` times the float32 PyTorch restatement of the
reference's non-fused algorithm (oracle/) on the host on a bounded sample.
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

# Algorithmic work per token x head (BT = 64 dense tiles, fwd+bwd = 3 x fwd).
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

# HBM bytes per launch at the metric shape, measured with rocprofv3 --pmc FETCH_SIZE and
# --pmc WRITE_SIZE on this workload (bench.py --copy-calibration), each scaled by the counter's
# reading for a known-size elementwise copy (fetch x2.000, write x1.000).  Re-measured whenever a
# kernel changes; a stage absent here reports traffic null.
MEASURED_TRAFFIC_BYTES = {
    "gdn_bwd_dqkw": (1166.9e6, 419.4e6),
    "gdn_fwd_state": (478.5e6, 537.5e6),
    "gdn_bwd_state": (478.4e6, 402.7e6),
    "clean_bwd_dk": (438.6e6, 67.1e6),
    "clean_fwd": (148.9e6, 287.3e6),
    "clean_bwd_dq": (371.6e6, 67.1e6),
    "gdn_bwd_wy": (638.0e6, 218.1e6),
    "clean_bwd_rows": (428.8e6, 153.6e6),
    "gdn_prep": (151.3e6, 343.9e6),
}


def kernel_work(k=K, v=V, bt=BT, cb=64):
    """Algorithmic FLOP and bytes per token x head of each timed stage (its own inputs read once,
    its own outputs written once), for the metric's call (fp32 q_clean into the delta rule, fp32
    upstream gradients, bf16 dq / dk).  Cleaning walks over cb-token chunks: per token a K x K state
    read and update (2 K^2 each) plus causal scores over the chunk (K cb per product, two products
    forward / dq, four in the dk walk with a second K x K update)."""
    return {
        "clean_fwd": (4 * k * k + 2 * k * cb, 2 * k + 2 * k + 4 + 4 * k + 4 * k + 4 + 4 * k // cb),
        "clean_bwd_rows": (6 * k, 4 * k + 4 * k + 2 * k + 2 * k + 4 + 4 + 4 * k // cb + 16 + 4 * k // cb + 4 * k),
        "clean_bwd_dq": (4 * k * k + 2 * k * cb, 4 * k + 2 * k + 16 + 4 * k // cb + 2 * k),
        "clean_bwd_dk": (6 * k * k + 4 * k * cb, 2 * k + 2 * k + 4 * k + 16 + 4 * k + 2 * k),
        "gdn_prep": (2 * bt * (2 * k + v) + (2 * bt * bt) // 3, 2 * k + 2 * v + 8 + 2 * k + 4 * v + 4 + 4 * bt),
        # the forward walk with the chunk output fused in: state path (U = u - w S, S update) plus
        # Y = Qc S, P = Qc K^T and P U; reads k, w / wl, Qc (fp32), g, u; writes U, o, P^T and the
        # per-chunk state snapshots (hi/lo)
        "gdn_fwd_state": (4 * k * v + 2 * bt * k + 2 * k * v + 2 * bt * v,
                          2 * k + 4 * k + 4 * k + 4 + 4 * v + 4 * v + 2 * v + 4 * bt + 4 * k * v // bt),
        "gdn_bwd_state": (2 * bt * v + 6 * k * v, 4 * bt + 2 * v + 2 * k + 4 * k + 2 * k + 4 * v + 4 * k * v // bt),
        "gdn_bwd_dqkw": (6 * k * v + 2 * bt * v + 4 * bt * k,
                         8 * k * v // bt + 2 * v + 4 * v + 4 * v + 4 * k + 2 * k + 4 * bt + 12 * k + 4),
        "gdn_bwd_wy": (10 * bt * k + 4 * bt * v + 4 * bt * bt,
                       4 * bt + 4 * k + 4 * v + 2 * k + 2 * v + 4 * k + 4 * k + 2 * v + 8),
    }


def roofline(step_kernel_ms, launches_per_step):
    """Roofline object for the kernel with the largest share of the step."""
    work = kernel_work()
    # stages that launch several kernels (the gate's two row sums) are left out so that the average
    # launch time compares one-to-one with a kernel trace
    single = [n for n in step_kernel_ms if n in work and n not in MULTI_KERNEL_STAGES]
    name = max(single, key=lambda n: step_kernel_ms[n])
    flop, byts = work[name]
    units = B * T * H
    avg_s = step_kernel_ms[name] / launches_per_step[name] * 1e-3
    ai = flop / byts
    if ai >= PEAK_BF16 / PEAK_HBM:
        achieved, peak, unit, bound = flop * units / avg_s / 1e12, PEAK_BF16 / 1e12, "TFLOP/s", "mfma"
    else:
        achieved, peak, unit, bound = byts * units / avg_s / 1e9, PEAK_HBM / 1e9, "GB/s", "hbm"
    traffic = sum(MEASURED_TRAFFIC_BYTES[name]) if name in MEASURED_TRAFFIC_BYTES else None
    return {"kernel": name, "bound": bound, "achieved": achieved, "peak": peak, "unit": unit,
            "frac": achieved / peak, "traffic": traffic, "avg_launch_us": avg_s * 1e6,
            "algorithmic_flop_per_launch": flop * units, "algorithmic_bytes_per_launch": byts * units}


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
            "sample": f"1 sequence x {t_s} tokens x {H} heads (d_k=d_v={K}), fp32 autograd fwd+bwd, "
                      f"median of {len(times)} after 1 warm-up"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed steps, run one elementwise copy of 512 MiB (read) + 512 MiB (write), "
                         "the known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counts")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    x = make_inputs(dev)
    for n in LEAVES:
        x[n].requires_grad_()
    from ccq_amd import _lib

    for _ in range(args.warmup):
        gpu_step(x)
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        gpu_step(x)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.timing_enable(False)
    if args.copy_calibration:
        src = torch.ones(256 << 20, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    kms, klaunch = {}, {}
    for name in _lib.KERNELS:
        ms_tot, n = _lib.timing_read(name)
        if n:
            kms[name], klaunch[name] = ms_tot / args.steps, n / args.steps
    ms = elapsed / args.steps * 1e3
    tokens_per_s = B * T * args.steps / elapsed
    flops = FLOP_PER_TOKEN_HEAD * B * T * H
    out = {
        "metric": "cleaning+chunk fwd+bwd tokens/s at B8·T4096·H8·dk128 bf16; % MFMA peak",
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE.json configs[1] + configs[2] GDN conventions)",
        "config": {"workload": "fused CCQ cleaning (per-head gate) + GDN chunk fwd+bwd", "B": B, "T": T, "H": H,
                   "d_k": K, "d_v": V, "chunk": BT, "algorithmic_flop_per_step": flops,
                   "mfma_peak_fraction": flops / (ms * 1e-3) / PEAK_BF16,
                   "kernel_ms_per_step": {n: round(v, 4) for n, v in kms.items()}},
        "roofline": roofline(kms, klaunch),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
