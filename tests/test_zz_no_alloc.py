"""The decode entry point that allocates nothing (ccq_gdn_decode_noalloc: fixed per-device scratch)
against the one that takes a workspace (ccq_gdn_decode), called through the C ABI: identical
outputs and updated states on two calls in a row, the second with a smaller input (the scratch
keeps the first call's contents, which the second must not read)."""

import pytest
import torch

from ccq_amd import _lib
from ccq_amd._lib import ptr, stream_of

pytestmark = pytest.mark.gpu


def _inputs(B, T, H, K, V, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    f = dict(q=torch.randn(B, T, H, K, generator=gen).bfloat16(), k=torch.randn(B, T, H, K, generator=gen).bfloat16(),
             v=torch.randn(B, T, H, V, generator=gen).bfloat16(),
             lam=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
             g=-torch.nn.functional.softplus(torch.randn(B, T, H, generator=gen)),
             beta=torch.sigmoid(torch.randn(B, T, H, generator=gen)),
             S=torch.randn(B, H, K, V, generator=gen) * 0.1, C=torch.randn(B, H, K, K, generator=gen) * 0.1,
             m=torch.randn(B, H, K, generator=gen))
    return {n: t.to(dev).contiguous() for n, t in f.items()}


def _run(x, B, T, H, K, V, pos, noalloc):
    lib = _lib.load()
    dev = x["q"].device
    o = torch.empty(B, T, H, V, device=dev, dtype=torch.bfloat16)
    S = torch.empty(B, H, K, V, device=dev)
    C = torch.empty(B, H, K, K, device=dev)
    m = torch.empty(B, H, K, device=dev)
    head = [ptr(x["q"]), ptr(x["k"]), ptr(x["v"]), ptr(x["lam"]), None, None, ptr(x["g"]), ptr(x["beta"]), None,
            None, ptr(x["S"]), ptr(x["C"]), ptr(x["m"]), None, ptr(o), ptr(S), ptr(C), ptr(m)]
    tail = [B, T, H, K, V, B, pos, 1, 1, 1, K ** -0.5, stream_of(x["q"])]
    if noalloc:
        st = lib.ccq_gdn_decode_noalloc(*head, *tail)
    else:
        ws = torch.empty(lib.ccq_decode_workspace_bytes(B * T, H, K), device=dev, dtype=torch.uint8)
        st = lib.ccq_gdn_decode(*head, ptr(ws), *tail)
    _lib.check(st, "decode")
    torch.cuda.synchronize()
    return o, S, C, m


def test_decode_noalloc_matches_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda")
    # the second call is smaller (fewer sequences, tokens, heads and channels)
    for case in ((4, 3, 4, 256, 512, 9, 1), (2, 1, 2, 128, 128, 40, 2)):
        B, T, H, K, V, pos, seed = case
        print("decode noalloc", case, flush=True)
        x = _inputs(B, T, H, K, V, seed, dev)
        want = _run(x, B, T, H, K, V, pos, noalloc=False)
        got = _run(x, B, T, H, K, V, pos, noalloc=True)
        for name, a, b in zip(("o", "S", "C", "m"), got, want):
            assert torch.equal(a, b), (case, name)
