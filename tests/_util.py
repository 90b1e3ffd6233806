"""Shared helpers of the test-suite: seeded inputs (generated on the CPU) and error measures."""

import math

import torch


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """Relative L2 error ||a - b|| / ||b||, computed in float64 on the CPU."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.norm().item()
    return (a - b).norm().item() / (den if den > 0 else 1.0)


def kern(a: torch.Tensor, b: torch.Tensor) -> float:
    """Error of a kernel output `a` against the oracle `b` rounded to `a`'s dtype: zero for an exact
    kernel, apart from the rare element where the two roundings fall on different sides."""
    return rel(a, b.detach().to(a.dtype))


def faithful_excess(a: torch.Tensor, b: torch.Tensor) -> float:
    """Largest amount by which an element of the kernel output `a` (bf16) lies further than one bf16
    ulp from the exact value `b`, relative to the rms of `b`.  Zero when every element is one of the
    two bf16 neighbours of the exact value (faithful rounding); unlike `kern`, a single near-tie on
    a large element does not move it."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    mag = b.abs().clamp_min(torch.finfo(torch.float32).tiny)
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)  # bf16 keeps 8 significant bits
    excess = ((a - b).abs() - ulp).clamp_min(0)
    return float(excess.max() / b.pow(2).mean().sqrt())


def bf(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16)


def l2n(x: torch.Tensor) -> torch.Tensor:
    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def gdn_inputs(B, T, H, K, V, seed=0, with_state=False, device="cuda"):
    """q, k (L2-normalised, bf16), v (bf16), g (fp32 log decay), beta (fp32) and optional s0."""
    gen = torch.Generator().manual_seed(seed)
    q = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    k = bf(l2n(torch.randn(B, T, H, K, generator=gen)))
    v = bf(torch.randn(B, T, H, V, generator=gen))
    a_log = torch.empty(H).uniform_(0.0, math.log(16.0), generator=gen)
    g = (-torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen)) * a_log.exp() * 0.1).float()
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen)).float()
    s0 = torch.randn(B, H, K, V, generator=gen) * 0.1 if with_state else None
    out = dict(q=q, k=k, v=v, g=g, beta=beta, s0=s0)
    return {n: (t.to(device) if t is not None else None) for n, t in out.items()}, gen


class _RoundBoth(torch.autograd.Function):
    """A tensor boundary in a narrower dtype between two operators: the value is rounded to that dtype
    and so is the gradient that crosses it (what autograd does to a bf16 tensor that one op returns and
    the next consumes)."""

    @staticmethod
    def forward(ctx, x, dtype):
        ctx.dtype = dtype
        return x.to(dtype).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dtype).to(g.dtype), None


def round_both(x: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    return _RoundBoth.apply(x, dtype)
