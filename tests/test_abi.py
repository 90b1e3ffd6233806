"""C-ABI checks that need no GPU: the library loads, exports every entry point that
include/ccq_hip.h declares, and rejects invalid arguments with the documented status codes
before launching anything."""

import ctypes
import os
import re

import pytest

from ccq_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "ccq_hip.h")

CCQ_ERR_SHAPE, CCQ_ERR_NULL, CCQ_ERR_ALIGN = -1, -2, -3


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ccq_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared()
    assert len(names) >= 12
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"
    assert lib.ccq_abi_version() == 1


def _fake():
    return ctypes.c_void_p(0x1000)  # never dereferenced: argument checks fail first


def _clean_fwd(lib, *, lam=True, saved=True, out=True, cu=False, B=1, K=64, N=1):
    p = _fake()
    return lib.ccq_clean_fwd(p, p, p if lam else None, None, None, None, None, None, p if cu else None,
                             p if saved else None, p if out else None, None, None, None, B, 64, 2, K, N, 0, 1, None)


def test_clean_fwd_rejects_bad_k():
    lib = _lib.load()
    assert _clean_fwd(lib, K=48) == CCQ_ERR_SHAPE
    assert b"K=48" in lib.ccq_last_error()


def test_clean_fwd_rejects_missing_lambda_saved_and_output():
    lib = _lib.load()
    assert _clean_fwd(lib, lam=False) == CCQ_ERR_NULL
    assert _clean_fwd(lib, saved=False) == CCQ_ERR_NULL
    assert _clean_fwd(lib, out=False) == CCQ_ERR_NULL


def test_varlen_requires_batch_one():
    lib = _lib.load()
    assert _clean_fwd(lib, cu=True, B=2, N=3) == CCQ_ERR_SHAPE


def test_clean_bwd_requires_saved_gradient_and_outputs():
    lib = _lib.load()
    p = _fake()

    def call(saved=p, dqc=p, dq=p, dk=p, ws=p):
        return lib.ccq_clean_bwd(p, p, p, None, None, dqc, None, None, None, None, None, saved, None, None, dq, None,
                                 dk, None, None, None, None, None, None, ws, 1, 64, 2, 64, 1, 0, 1, None)

    assert call(saved=None) == CCQ_ERR_NULL
    assert call(ws=None) == CCQ_ERR_NULL
    assert call(dqc=None) == CCQ_ERR_NULL
    assert call(dq=None) == CCQ_ERR_NULL
    assert call(dk=None) == CCQ_ERR_NULL


def test_gdn_rejects_bad_shapes():
    lib = _lib.load()
    p = _fake()
    # V not a multiple of 64
    st = lib.ccq_gdn_fwd(p, None, p, p, p, p, None, None, None, None, 1, p, None, p, 1, 64, 2, 64, 100, 1, 0.1, None)
    assert st == CCQ_ERR_SHAPE
    # K unsupported
    st = lib.ccq_gdn_fwd(p, None, p, p, p, p, None, None, None, None, 1, p, None, p, 1, 64, 2, 96, 64, 1, 0.1, None)
    assert st == CCQ_ERR_SHAPE
    # wrong chunk count for dense inputs
    st = lib.ccq_gdn_fwd(p, None, p, p, p, p, None, None, None, None, 3, p, None, p, 1, 64, 2, 64, 64, 1, 0.1, None)
    assert st == CCQ_ERR_SHAPE
    # varlen without the chunk index
    st = lib.ccq_gdn_fwd(p, None, p, p, p, p, None, p, None, None, 3, p, None, p, 1, 64, 2, 64, 64, 2, 0.1, None)
    assert st == CCQ_ERR_NULL


def test_l2norm_rejects_wide_rows():
    lib = _lib.load()
    p = _fake()
    assert lib.ccq_l2norm_fwd(p, p, p, 10, 1024, 1e-6, None) == CCQ_ERR_SHAPE


@pytest.mark.parametrize("K,V", [(64, 64), (128, 128), (256, 512)])
def test_workspace_sizes_are_consistent(K, V):
    lib = _lib.load()
    tokens, H = 4096, 4
    nt = tokens // 64
    saved = lib.ccq_gdn_saved_bytes(tokens, nt, H, K, V)
    # gcum + T + w (hi, lo) + u + hT + U + P^T, each rounded up to 256 bytes; at these shapes the state
    # snapshots hT are int16 rows with one fp32 scale per row
    expect = tokens * H * 4 + nt * H * 4096 * 4 + 2 * tokens * H * K * 2 + tokens * H * V * 4 \
        + nt * H * V * (K * 2 + 4) + tokens * H * V * 4 + nt * H * 4096 * 4
    assert expect <= saved <= expect + 8 * 256
    # the backward's workspace: dU + dhT + dk (state part) + dw + per-block dg partials; the
    # state-gradient snapshots dhT are int16 rows with row scales at K = V = 128, hi/lo pairs elsewhere,
    # and there dk (state part) and dw are int16 with an fp32 scale per row and 32 columns
    gws = lib.ccq_gdn_bwd_workspace_bytes(tokens, nt, H, K, V)
    dh = nt * H * V * (K * 2 + 4) if (K, V) == (128, 128) else 2 * nt * H * V * K * 2
    dkw = 2 * tokens * H * (K * 2 + K // 32 * 4) if (K, V) == (128, 128) else 2 * tokens * H * K * 4
    gexpect = tokens * H * V * 4 + dh + dkw + (K // 64) * tokens * H * 4
    assert gexpect <= gws <= gexpect + 8 * 256
    csaved = lib.ccq_clean_saved_bytes(tokens, 1, tokens, 1, H, K, 0)
    ws = lib.ccq_clean_bwd_workspace_bytes(tokens, 1, tokens, 1, H, K, 0, 0)
    if K in (64, 128):
        # segment walks: saved = per-segment sums of k k^T and k; workspace = four fp32 row scalars
        # per token + per-segment sums of q dz^T and dm.  The segment count (1..16, at least two
        # chunks each) depends on the device's CU count; no per-token tensor is saved
        per_seg = H * (K * K + K) * 4
        nseg = [n for n in range(1, 17) if n * per_seg <= csaved <= n * per_seg + 2 * 256]
        assert len(nseg) == 1
        wexpect = tokens * H * 16 + nseg[0] * per_seg
        assert wexpect <= ws <= wexpect + 3 * 256
    else:
        # column walks: saved = z (fp32 per token) + s_t + key sum before each chunk; workspace = four
        # fp32 row scalars per token + per-chunk column sums of dm (+ gate partials).  K = 256 cuts
        # the walks into time segments and adds the segment totals to both
        cb = 32 if K > 128 else 64
        nc = tokens // cb
        per_seg = H * (K * K + K) * 4
        cexpect = tokens * H * K * 4 + tokens * H * 4 + nc * H * K * 4
        nseg = [n for n in range(2, 17) if cexpect + n * per_seg <= csaved <= cexpect + n * per_seg + 5 * 256]
        assert len(nseg) == 1
        wexpect = tokens * H * 16 + nc * H * K * 4 + nseg[0] * per_seg
        assert wexpect <= ws <= wexpect + 6 * 256
    assert lib.ccq_clean_bwd_workspace_bytes(tokens, 1, tokens, 1, H, K, 0, 1) > ws
    assert lib.ccq_clean_saved_bytes(tokens, 1, tokens, 1, H, K, 1) > csaved  # varlen adds the indexes


def test_gla_rejects_bad_shapes_and_missing_buffers():
    lib = _lib.load()
    p = _fake()

    def fwd(K=64, V=64, nc=1, cu=None, ci=None, out=p):
        return lib.ccq_gla_fwd(p, None, p, p, p, None, cu, ci, ci, nc, out, None, p, 1, 64, 2, K, V, 1 if cu is None
                               else 2, 0.1, None)

    assert fwd(V=96) == CCQ_ERR_SHAPE
    assert fwd(K=32) == CCQ_ERR_SHAPE
    assert fwd(nc=2) == CCQ_ERR_SHAPE
    assert fwd(cu=p, nc=3) == CCQ_ERR_NULL
    assert fwd(out=None) == CCQ_ERR_NULL

    def bwd(dgk=p, gk=p, dsf=None, sf=None):
        return lib.ccq_gla_bwd(p, None, p, p, gk, None, None, None, 1, p, p, dsf, sf, p, p, p, p, None, dgk, None, 1,
                               64, 2, 64, 64, 1, 0.1, None)

    assert bwd(gk=None) == CCQ_ERR_NULL          # dgk without gk
    assert bwd(dsf=p, sf=None) == CCQ_ERR_NULL   # final-state gradient without the final state


@pytest.mark.parametrize("K,V", [(64, 64), (128, 256), (256, 512)])
def test_gla_buffer_sizes(K, V):
    lib = _lib.load()
    tokens, H = 4096, 4
    nt = tokens // 64
    saved = lib.ccq_gla_saved_bytes(tokens, nt, H, K, V)
    # bcum + A + hT (hi, lo), each rounded up to 256 bytes
    expect = tokens * H * K * 4 + nt * H * 4096 * 4 + 2 * nt * H * V * K * 2
    assert expect <= saved <= expect + 4 * 256
    ws = lib.ccq_gla_bwd_workspace_bytes(tokens, nt, H, K, V)
    expect = 2 * nt * H * V * K * 2 + nt * H * K * 4
    assert expect <= ws <= expect + 3 * 256


def test_decode_noalloc_rejects_calls_beyond_its_scratch():
    # 2048 tokens x 4 heads x K=256 need 16 MiB of scratch, above the fixed 8 MiB: refused on the
    # host, before any device work
    lib = _lib.load()
    p = _fake()
    st = lib.ccq_gdn_decode_noalloc(p, p, p, p, None, None, None, p, None, None, None, None, None, None, p, None,
                                    None, None, 1, 2048, 4, 256, 512, 1, 0, 1, 1, 1, 0.0625, None)
    assert st == CCQ_ERR_SHAPE
    assert b"scratch" in lib.ccq_last_error()


def test_decode_step_checks_and_workspace():
    lib = _lib.load()
    p = _fake()
    # position (device int) and state are required; checked before any device work
    st = lib.ccq_gdn_decode_step(p, p, p, None, p, p, p, p, p, p, p, None, p, p, 2, 1, 4, 256, 512, 1, 1, 1, 0.0625,
                                 None)
    assert st == CCQ_ERR_NULL and b"position" in lib.ccq_last_error()
    st = lib.ccq_gla_decode_step(p, p, p, None, p, p, p, None, p, p, p, p, p, 2, 1, 4, 256, 512, 1, 1, 0.0625, None)
    assert st == CCQ_ERR_NULL
    # the decode workspace plus the new key sum [B, H, K] fp32
    B, T, H, K = 16, 1, 4, 256
    ws = lib.ccq_decode_step_workspace_bytes(B, T, H, K)
    base = lib.ccq_decode_workspace_bytes(B * T, H, K)
    assert base + B * H * K * 4 <= ws <= base + B * H * K * 4 + 256


def test_decode_rejects_unaligned_states_and_gv():
    # the decode kernels move state slices and gv as 16-byte pieces: an unaligned pointer is refused
    # on the host, before any device work
    lib = _lib.load()
    p, odd, m_out = _fake(), ctypes.c_void_p(0x1004), ctypes.c_void_p(0x2000)   # m_out may not alias m

    def call(state=p, cov=p, state_out=p, cov_out=p, gv=None):
        return lib.ccq_gdn_decode(p, p, p, p, None, None, None, p, None, gv, state, cov, p, None, p, state_out,
                                  cov_out, m_out, p, 2, 1, 4, 64, 64, 2, 0, 1, 1, 1, 0.125, None)

    for kw in ({"state": odd}, {"cov": odd}, {"state_out": odd}, {"cov_out": odd}, {"gv": odd}):
        assert call(**kw) == CCQ_ERR_ALIGN, kw
        assert b"aligned" in lib.ccq_last_error()
    st = lib.ccq_gla_decode(p, p, p, p, None, None, None, odd, p, p, p, None, p, p, p, m_out, p, 2, 1, 4, 64, 64, 2, 0, 1,
                            1, 0, 0.125, None)
    assert st == CCQ_ERR_ALIGN


def test_decode_linear_split_checks_and_workspace():
    # counters (one per 16 output columns, rounded up to 256 bytes) then splits x blocks partial tiles
    lib = _lib.load()
    p = _fake()
    assert lib.ccq_decode_linear_split_workspace_bytes(1024, 4) == 256 + 4 * 64 * 256 * 4
    assert lib.ccq_decode_linear_split_workspace_bytes(100, 3) == 256 + 3 * 7 * 256 * 4
    # splits outside [1, min(8, K/32)] and a split call without its workspace are refused on the host
    assert lib.ccq_decode_linear_split(p, 64, p, None, 0, p, 40, 1, 64, 40, 3, p, None) == CCQ_ERR_SHAPE
    assert lib.ccq_decode_linear_split(p, 2048, p, None, 0, p, 40, 1, 2048, 40, 9, p, None) == CCQ_ERR_SHAPE
    assert lib.ccq_decode_linear_split(p, 2048, p, None, 0, p, 40, 1, 2048, 40, 4, None, None) == CCQ_ERR_NULL


def test_greedy_embed_checks():
    # shapes, required pointers and the logits' alignment are refused on the host, before any launch
    lib = _lib.load()
    p = _fake()
    ids = _fake()
    assert lib.ccq_greedy_embed(p, 32, 2, 40, p, 40, 8, ids, 1, p, 8, None) == CCQ_ERR_SHAPE    # ldl < N
    assert lib.ccq_greedy_embed(p, 32, 2, 32, p, 0, 8, ids, 1, p, 8, None) == CCQ_ERR_SHAPE     # no table rows
    assert lib.ccq_greedy_embed(p, 32, 2, 32, p, 32, 8, ids, 1, p, 4, None) == CCQ_ERR_SHAPE    # ldx < D
    assert lib.ccq_greedy_embed(p, 32, 2, 32, None, 32, 8, ids, 1, p, 8, None) == CCQ_ERR_NULL
    assert lib.ccq_greedy_embed(ctypes.c_void_p(0x1001), 32, 2, 32, p, 32, 8, ids, 1, p, 8, None) == CCQ_ERR_ALIGN
