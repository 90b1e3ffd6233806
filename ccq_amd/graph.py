"""Captured decode loop: the per-token CCQ-GDN / CCQ-GLA recurrent step of one or more layers in a
single HIP graph.

The reference generates one token at a time by calling ``fused_recurrent_ccq_gdn`` (or ``_gla``)
once per layer with the cache tuple ``(S, C, m, position_offset)`` (``ccq/gdn/layer.py:318-336,
397``; ``ccq/ops/ccq_gdn/fused_recurrent.py:18-75``).  Per layer and token that is a handful of
launches plus host work, and the token's latency is launch-bound.  Here each layer's step is the
library's ``ccq_gdn_decode_step`` / ``ccq_gla_decode_step``: two kernels over static buffers,
with the states updated in place and the position offset held in device memory (advanced by the
step itself), so the same captured graph is replayed for every generated token.

``DecodeStep`` owns one layer's buffers: the token inputs (``q``, ``k``, ``v``, ``g``/``beta`` or
``gk``, ``lam``), the per-head gate (``gate_w``, ``gate_b``), the states ``S``, ``C``, ``m``, the
position and the output ``o``.  A caller writes the new token's inputs into the input buffers
(``copy_``), replays, and reads ``o``.  ``CapturedDecode`` captures the steps of several layers
in order (e.g. the 24 layers of a model) and replays them as one graph.

``GDNLayerDecode`` is a whole ``CCQGDN`` layer's token step around a ``DecodeStep``: one GEMM for the
layer's input projections, one kernel for everything between them and the recurrent op
(``ccq_gdn_decode_prologue``), the in-place decode step, and the layer's output norm and projection --
five launches per layer and token instead of the recurrent mode's few dozen small ones, on static
buffers, so that a model's whole token step can be captured.
"""

from __future__ import annotations

from typing import List, Optional, Sequence

import torch

import torch.nn.functional as F

from . import _lib
from ._lib import call, ptr

__all__ = ["DecodeStep", "CapturedDecode", "GDNLayerDecode", "decode_linear", "decode_linear_glu",
           "decode_linear_ok", "greedy_embed"]


def decode_linear_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``decode_linear`` takes this call: bf16 on the GPU, at most 16 rows, a contraction
    width that is a multiple of 32 in [32, 4096], 16-byte aligned operands."""
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    return (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and weight.dim() == 2
            and weight.shape[1] == K and 1 <= rows <= 16 and K % 32 == 0 and 32 <= K <= 4096
            and weight.is_contiguous() and weight.data_ptr() % 16 == 0)


def _rows(x: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2


def _norm_arg(x: torch.Tensor, norm_weight: Optional[torch.Tensor]):
    if norm_weight is None:
        return None
    if (norm_weight.shape != (x.shape[-1],) or norm_weight.dtype != torch.bfloat16 or not norm_weight.is_contiguous()
            or norm_weight.data_ptr() % 16):
        raise ValueError(f"norm_weight {tuple(norm_weight.shape)} {norm_weight.dtype}: expected a contiguous bf16 "
                         f"[{x.shape[-1]}]")
    return norm_weight


def decode_linear(x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor] = None,
                  norm_weight: Optional[torch.Tensor] = None, norm_eps: float = 1e-5) -> torch.Tensor:
    """``x @ weight.T (+ residual)`` for a decode step's few token rows (``ccq_decode_linear``: the
    weight streamed once by MFMA tiles; fp32 accumulation rounded to bf16, then the residual added
    and rounded again, as ``residual + linear(x)`` on bf16 tensors).  With ``norm_weight`` the rows
    of x first go through a bf16 RMSNorm (``x * norm_weight / sqrt(mean(x^2) + norm_eps)``, one
    rounding, as ``nn.RMSNorm`` does) inside the same kernel.  Inference only (no autograd).
    ``decode_linear_ok`` gives the shapes it takes."""
    if not decode_linear_ok(x, weight):
        raise ValueError(f"decode_linear: x {tuple(x.shape)} {x.dtype}, weight {tuple(weight.shape)} {weight.dtype}: "
                         f"needs bf16 on the GPU, <= 16 rows and a width that is a multiple of 32 in [32, 4096]")
    K, N = x.shape[-1], weight.shape[0]
    x2 = _rows(x)
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=torch.bfloat16)
    r2 = None
    if residual is not None:
        if residual.shape != y.shape or residual.dtype != torch.bfloat16:
            raise ValueError(f"decode_linear: residual {tuple(residual.shape)} {residual.dtype}, expected "
                             f"{tuple(y.shape)} bf16")
        r2 = residual.reshape(-1, N)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
    call("ccq_decode_linear", ptr(x2), x2.stride(0), ptr(weight), ptr(r2), r2.stride(0) if r2 is not None else 0,
         ptr(y), N, x2.shape[0], K, N, ptr(_norm_arg(x, norm_weight)), float(norm_eps), _lib.stream_of(x))
    return y


def split_plan(K: int, N: int) -> int:
    """Workgroups per 16 output columns for ``decode_linear_split``: enough for about 256 workgroups
    (one per CU), at most 8 and at least 4 contraction steps of 32 per workgroup."""
    blocks = (N + 15) // 16
    return max(1, min(8, (K // 32) // 4, -(-256 // blocks)))


def split_workspace(N: int, splits: int, device) -> torch.Tensor:
    """A zeroed workspace for ``decode_linear_split`` (its counters start at zero; every call leaves
    them so)."""
    n = _lib.load().ccq_decode_linear_split_workspace_bytes(N, splits)
    return torch.zeros(max(n, 16), device=device, dtype=torch.uint8)


def decode_linear_split(x: torch.Tensor, weight: torch.Tensor, residual: Optional[torch.Tensor], splits: int,
                        workspace: Optional[torch.Tensor]) -> torch.Tensor:
    """``decode_linear`` with the contraction split over ``splits`` workgroups per 16 output columns
    (``ccq_decode_linear_split``): the partial tiles are added by the last workgroup of each block to
    finish, in split order.  ``workspace`` from ``split_workspace(N, splits)``; calls sharing one
    workspace must not overlap (one stream)."""
    if not decode_linear_ok(x, weight):
        raise ValueError(f"decode_linear_split: x {tuple(x.shape)} {x.dtype}, weight {tuple(weight.shape)} "
                         f"{weight.dtype}: needs bf16 on the GPU, <= 16 rows, a width that is a multiple of 32 "
                         f"in [32, 4096]")
    K, N = x.shape[-1], weight.shape[0]
    x2 = _rows(x)
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=torch.bfloat16)
    r2 = None
    if residual is not None:
        if residual.shape != y.shape:
            raise ValueError(f"residual {tuple(residual.shape)}: expected {tuple(y.shape)}")
        r2 = _rows(residual)
    call("ccq_decode_linear_split", ptr(x2), x2.stride(0), ptr(weight), ptr(r2), 0 if r2 is None else r2.stride(0),
         ptr(y), N, x2.shape[0], K, N, int(splits), ptr(workspace), _lib.stream_of(x))
    return y


def decode_linear_gnorm(x: torch.Tensor, gate: torch.Tensor, norm_weight: Optional[torch.Tensor], dv: int,
                        norm_eps: float, weight: torch.Tensor, residual: Optional[torch.Tensor],
                        workspace: Optional[torch.Tensor]) -> torch.Tensor:
    """A gated-norm layer's output projection with the norm folded in (``ccq_decode_linear_gnorm``):
    ``linear(bf16(x r w silu(gate)), weight) (+ residual)``, ``r`` the reciprocal RMS of each
    ``dv``-wide head of ``x``, the contraction split per head.  ``gate`` a [rows, K] bf16 view (rows
    may be strided, e.g. columns of the input projections' output); ``norm_weight`` fp32 [dv] or
    None; ``workspace`` from ``split_workspace(N, K // dv)`` (None for one head)."""
    K = x.shape[-1]
    if not decode_linear_ok(x, weight) or dv % 32 or K % dv or K // dv > 8:
        raise ValueError(f"decode_linear_gnorm: x {tuple(x.shape)} {x.dtype}, weight {tuple(weight.shape)}, dv={dv}: "
                         f"needs bf16 on the GPU, <= 16 rows, K a multiple of 32 in [32, 4096] and dv a multiple "
                         f"of 32 dividing K into at most 8 heads")
    x2 = _rows(x)
    M, N = x2.shape[0], weight.shape[0]
    if gate.dtype != torch.bfloat16 or gate.shape != (M, K) or gate.stride(1) != 1:
        raise ValueError(f"gate {tuple(gate.shape)} {gate.dtype}: expected a bf16 [{M}, {K}] view, unit column stride")
    if norm_weight is not None and (norm_weight.shape != (dv,) or norm_weight.dtype != torch.float32):
        raise ValueError(f"norm_weight {tuple(norm_weight.shape)} {norm_weight.dtype}: expected fp32 [{dv}]")
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=torch.bfloat16)
    r2 = None
    if residual is not None:
        if residual.shape != y.shape:
            raise ValueError(f"residual {tuple(residual.shape)}: expected {tuple(y.shape)}")
        r2 = _rows(residual)
    call("ccq_decode_linear_gnorm", ptr(x2), x2.stride(0), ptr(gate), gate.stride(0), ptr(norm_weight), dv,
         float(norm_eps), ptr(weight), ptr(r2), 0 if r2 is None else r2.stride(0), ptr(y), N, M, K, N,
         ptr(workspace), _lib.stream_of(x))
    return y


def greedy_embed(logits: torch.Tensor, table: torch.Tensor, ids: torch.Tensor, x: torch.Tensor) -> None:
    """Greedy step of a generate loop (``ccq_greedy_embed``): ``ids[:, 0] = logits.argmax(-1)`` (int64,
    torch's tie and NaN rules) and ``x[:, 0] = table[ids[:, 0]]``, the next decode step's input rows,
    in one launch on logits' stream.  logits bf16 [M, N] (unit column stride); table bf16 [rows, D];
    ids int64 [M, 1]; x bf16 [M, 1, D]."""
    M, N = logits.shape
    D = table.shape[1]
    if (logits.dtype != torch.bfloat16 or logits.stride(1) != 1 or table.dtype != torch.bfloat16
            or not table.is_contiguous() or ids.dtype != torch.int64 or ids.shape != (M, 1)
            or x.dtype != torch.bfloat16 or x.shape != (M, 1, D) or x.stride(2) != 1):
        raise ValueError(f"greedy_embed: logits {tuple(logits.shape)} {logits.dtype}, table {tuple(table.shape)} "
                         f"{table.dtype}, ids {tuple(ids.shape)} {ids.dtype}, x {tuple(x.shape)} {x.dtype}")
    call("ccq_greedy_embed", ptr(logits), logits.stride(0), M, N, ptr(table), table.shape[0], D, ptr(ids),
         ids.stride(0), ptr(x), x.stride(0), _lib.stream_of(logits))


def decode_linear_glu(x: torch.Tensor, weight: torch.Tensor, norm_weight: Optional[torch.Tensor] = None,
                      norm_eps: float = 1e-5) -> torch.Tensor:
    """A gated MLP's up projection for a decode step: ``silu(gate) * up`` with
    ``gate, up = (x @ weight.T).chunk(2, -1)`` (``ccq_decode_linear_glu``; the bf16 roundings of those
    torch ops made in the kernel, the [rows, 2N] projection never written).  weight [2N, K];
    ``norm_weight`` / ``norm_eps`` as in ``decode_linear``."""
    if not decode_linear_ok(x, weight) or weight.shape[0] % 2:
        raise ValueError(f"decode_linear_glu: x {tuple(x.shape)} {x.dtype}, weight {tuple(weight.shape)} "
                         f"{weight.dtype}: needs bf16 on the GPU, <= 16 rows, an even number of weight rows and a "
                         f"width that is a multiple of 32 in [32, 4096]")
    K, N = x.shape[-1], weight.shape[0] // 2
    x2 = _rows(x)
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=torch.bfloat16)
    call("ccq_decode_linear_glu", ptr(x2), x2.stride(0), ptr(weight), ptr(y), N, x2.shape[0], K, N,
         ptr(_norm_arg(x, norm_weight)), float(norm_eps), _lib.stream_of(x))
    return y


class DecodeStep:
    """Static buffers and the in-place decode step of one CCQ-GDN (``mode="gdn"``) or CCQ-GLA
    (``mode="gla"``) layer: ``B`` sequences, ``T`` new tokens each (normally 1), ``H`` heads.

    ``gate=True`` computes lambda in the kernel from ``gate_w [H, K]`` / ``gate_b [H]`` (the
    per-head gate of the reference layer); otherwise ``lam [B, T, H]`` (fp32) is read as given
    (the reference ops round lambda to q's dtype first; a caller that mirrors them writes
    bf16-rounded values).  GLA takes the
    per-channel log decay ``gk [B, T, H, K]`` (``use_gk=False``: no decay) and always
    L2-normalises q and k, as the reference's recurrent GLA op does."""

    def __init__(self, B: int, H: int, K: int, V: int, *, T: int = 1, mode: str = "gdn", gate: bool = True,
                 use_gk: bool = True, subtract_mean: bool = True, use_l2norm: bool = True, enable_ccq: bool = True,
                 scale: Optional[float] = None, device=None):
        if mode not in ("gdn", "gla"):
            raise ValueError(f"mode must be 'gdn' or 'gla' (got {mode!r})")
        if mode == "gla" and not enable_ccq:
            raise ValueError("the GLA step always cleans the query (enable_ccq=True)")
        if K not in (32, 64, 128, 256) or V < 64 or V % 64 or V > 1024:
            # (its static buffers are the kernels' own; the operators pad other sizes, ccq_amd/_pad.py)
            raise ValueError(f"DecodeStep takes K in {{32, 64, 128, 256}} and V a multiple of 64 up to 1024 "
                             f"(got K={K}, V={V})")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        if dev.type != "cuda":
            raise ValueError(f"DecodeStep runs on a GPU (got device {dev})")
        self.B, self.T, self.H, self.K, self.V, self.mode = B, T, H, K, V, mode
        self.gate, self.subtract_mean, self.use_l2norm = gate, subtract_mean, use_l2norm
        self.enable_ccq = enable_ccq
        self.scale = float(K ** -0.5 if scale is None else scale)
        bf, f32 = torch.bfloat16, torch.float32
        z = lambda *shape, dtype=f32: torch.zeros(*shape, device=dev, dtype=dtype)  # noqa: E731
        self.q, self.k, self.v = z(B, T, H, K, dtype=bf), z(B, T, H, K, dtype=bf), z(B, T, H, V, dtype=bf)
        self.lam = None if gate or not enable_ccq else z(B, T, H)
        self.gate_w = z(H, K) if gate and enable_ccq else None
        self.gate_b = z(H) if gate and enable_ccq else None
        if mode == "gdn":
            self.g, self.beta, self.gk = z(B, T, H), torch.ones(B, T, H, device=dev, dtype=f32), None
        else:
            self.g, self.beta = None, None
            self.gk = z(B, T, H, K) if use_gk else None
        self.S = z(B, H, K, V)
        self.C = z(B, H, K, K) if enable_ccq else None
        self.m = z(B, H, K) if enable_ccq and subtract_mean else None
        self.position = torch.zeros(1, device=dev, dtype=torch.int32)
        self.o = z(B, T, H, V, dtype=bf)
        nbytes = _lib.load().ccq_decode_step_workspace_bytes(B, T, H, K)
        self.workspace = torch.empty(nbytes, device=dev, dtype=torch.uint8)

    # ---- state ----
    def load_state(self, S: torch.Tensor, C: Optional[torch.Tensor] = None, m: Optional[torch.Tensor] = None,
                   position: int = 0) -> None:
        """Copy a cached state (e.g. the prefill's final S, C, m and its token count) into the
        step's buffers (absent C / m: zero)."""
        self.S.copy_(S)
        for buf, src in ((self.C, C), (self.m, m)):
            if buf is None:
                continue
            if src is None:
                buf.zero_()
            else:
                buf.copy_(src)
        self.position.fill_(int(position))

    def state(self):
        """(S, C, m, position) -- the buffers themselves (position as a 1-element int32 tensor)."""
        return self.S, self.C, self.m, self.position

    # ---- one step ----
    def launch(self, stream=None) -> None:
        """Run the step on ``stream`` (default: the current stream; under capture, the capture
        stream)."""
        st = _lib.stream_of(self.q) if stream is None else stream
        if self.mode == "gdn":
            call("ccq_gdn_decode_step", ptr(self.q), ptr(self.k), ptr(self.v), ptr(self.lam), ptr(self.gate_w),
                 ptr(self.gate_b), ptr(self.g), ptr(self.beta), ptr(self.S), ptr(self.C), ptr(self.m),
                 ptr(self.position), ptr(self.o), ptr(self.workspace), self.B, self.T, self.H, self.K, self.V,
                 int(self.subtract_mean), int(self.use_l2norm), int(self.enable_ccq), self.scale, st)
        else:
            call("ccq_gla_decode_step", ptr(self.q), ptr(self.k), ptr(self.v), ptr(self.lam), ptr(self.gate_w),
                 ptr(self.gate_b), ptr(self.gk), ptr(self.S), ptr(self.C), ptr(self.m), ptr(self.position),
                 ptr(self.o), ptr(self.workspace), self.B, self.T, self.H, self.K, self.V, int(self.subtract_mean),
                 1, self.scale, st)

    def state_bytes(self) -> int:
        """HBM bytes of the states one step reads and writes (each element once each way)."""
        n = self.S.numel() + (self.C.numel() if self.C is not None else 0) + (self.m.numel() if self.m is not None
                                                                               else 0)
        return 2 * 4 * n


class CapturedDecode:
    """The steps of several layers captured in one graph.  ``capture()`` records them in order;
    ``replay()`` runs one token for all of them (inputs from the steps' input buffers, states and
    positions advanced in place).  The capture itself runs no step: the steps' kernels are loaded
    by one eager step whose state changes are undone before recording."""

    def __init__(self, steps: Sequence[DecodeStep]):
        if not steps:
            raise ValueError("no steps")
        self.steps: List[DecodeStep] = list(steps)
        self.graph: Optional[torch.cuda.CUDAGraph] = None

    def _snapshot(self):
        return [[t.clone() if t is not None else None for t in (s.S, s.C, s.m, s.position, s.o)] for s in self.steps]

    def _restore(self, snap) -> None:
        for s, saved in zip(self.steps, snap):
            for dst, src in zip((s.S, s.C, s.m, s.position, s.o), saved):
                if dst is not None:
                    dst.copy_(src)

    def capture(self) -> "CapturedDecode":
        snap = self._snapshot()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for s in self.steps:
                s.launch()
        torch.cuda.current_stream().wait_stream(side)
        self._restore(snap)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            for s in self.steps:
                s.launch()
        torch.cuda.synchronize()
        return self

    def replay(self) -> None:
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()

    def eager(self) -> None:
        """The same steps launched one by one (no graph)."""
        for s in self.steps:
            s.launch()


class GDNLayerDecode:
    """The token step of one ``CCQGDN`` layer (recurrent mode with a cache, ``ccq/gdn/layer.py:253-412``)
    on static buffers: ``__call__(h, residual=None, norm=None)`` maps the layer input ``h [B, T, hidden]``
    (bf16; normally T = 1; with ``norm``, an ``nn.RMSNorm`` with a bf16 weight and an explicit eps, the
    input before that norm, which the input projection then applies) to the layer output (plus
    ``residual``, with the roundings of ``residual + output``),
    advancing the layer's states, convolution caches and position in place.

    The step is the layer's input projections as one GEMM over their concatenated weights (taken at
    construction; ``refresh()`` after the weights change), ``ccq_gdn_decode_prologue`` (short
    convolutions + SiLU with in-place caches, lambda, beta, g, per-head l2norm of q and k, with the
    roundings of the layer's own bf16 operations), the in-place decode step (``DecodeStep``, lambda as
    given, no l2norm), the gated output norm and the output projection.  With at most 16 token rows
    per step the two projections are ``decode_linear`` launches (the weights streamed once).  For a
    bf16 layer on the GPU with short convolutions and one key / value head per query head (the
    reference configurations); other layers run their recurrent mode as usual."""

    def __init__(self, layer, B: int, T: int = 1):
        L = layer
        if not L.use_short_conv:
            raise ValueError("GDNLayerDecode needs a layer with short convolutions")
        if L.num_kv_heads != L.num_heads or L.num_v_heads != L.num_heads:
            raise ValueError("GDNLayerDecode needs one key / value head per query head")
        params = [L.q_proj.weight, L.k_proj.weight, L.v_proj.weight, L.a_proj.weight, L.b_proj.weight,
                  L.erase_lambda_proj.weight, L.A_log, L.dt_bias, L.q_conv1d.weight]
        if any(p.dtype != torch.bfloat16 or not p.is_cuda for p in params):
            raise ValueError("GDNLayerDecode runs a bf16 layer on the GPU")
        self.layer, self.B, self.T = L, B, T
        self.H, self.K, self.V, self.W = L.num_heads, L.head_k_dim, L.head_v_dim, L.conv_size
        dev = L.q_proj.weight.device
        self.step = DecodeStep(B, self.H, self.K, self.V, T=T, mode="gdn", gate=False,
                               subtract_mean=L.subtract_mean, use_l2norm=False, enable_ccq=L.enable_ccq,
                               device=dev)
        dq, dv = self.H * self.K, self.H * self.V
        self.conv = [torch.zeros(B, d, self.W - 1, device=dev, dtype=torch.bfloat16) for d in (dq, dq, dv)]
        # rows of the concatenated projection: q, k, v, g (output gate), a, b, zero padding to 8 elements
        widths = [dq, dq, dv, dv if L.use_gate else 0, self.H, self.H]
        self.offsets = [sum(widths[:i]) for i in range(len(widths))]
        self.pad = (-sum(widths)) % 8
        self.width = sum(widths) + self.pad
        self.refresh()
        # the projections as decode_linear launches when the step has at most 16 token rows
        self.fast = B * T <= 16 and decode_linear_ok(torch.empty(B * T, L.hidden_size, device=dev,
                                                                 dtype=torch.bfloat16), self.w_in)
        # the short convolutions in the input projections' epilogue (width 4) and the decode step over
        # their rows where its limits allow (H K <= 2048)
        self.conv_in_proj = self.W == 4 and self.H * self.K <= 2048
        # the output projection (N = hidden, about 1024: few column blocks) with its contraction split
        self.o_splits = split_plan(dv, L.o_proj.weight.shape[0])
        # the gated output norm folded into the output projection (split per head) where its limits allow
        self.gnorm_in_proj = L.use_gate and self.V % 32 == 0 and self.H <= 8 and self.conv_in_proj
        if self.gnorm_in_proj:
            self.o_splits = self.H
        self.o_ws = split_workspace(L.o_proj.weight.shape[0], self.o_splits, dev) if self.o_splits > 1 else None

    def refresh(self) -> None:
        """Concatenate the layer's current input-projection weights."""
        L = self.layer
        parts = [L.q_proj.weight, L.k_proj.weight, L.v_proj.weight]
        if L.use_gate:
            parts.append(L.g_proj.weight)
        parts += [L.a_proj.weight, L.b_proj.weight]
        if self.pad:
            parts.append(L.q_proj.weight.new_zeros(self.pad, L.hidden_size))
        with torch.no_grad():
            self.w_in = torch.cat([p.detach() for p in parts]).contiguous()
            w = getattr(L.o_norm, "weight", None)
            self.norm_w = w.detach().float().contiguous() if w is not None else None

    def load(self, entry) -> None:
        """Copy one layer's entry of a ``LayerCache`` (``{'recurrent_state': (S, C, m, pos),
        'conv_state': (q, k, v caches)}``, e.g. after a chunked prefill) into the step's buffers."""
        from .layers import unpack_recurrent_state
        from .prologue import last_inputs
        S, C, m, pos = unpack_recurrent_state(entry["recurrent_state"])
        self.step.load_state(S, C, m, pos)
        for dst, src in zip(self.conv, entry["conv_state"]):
            dst.copy_(last_inputs(src, self.W))

    def __call__(self, h: torch.Tensor, residual: Optional[torch.Tensor] = None,
                 norm: Optional[torch.nn.Module] = None) -> torch.Tensor:
        L, st = self.layer, self.step
        B, T, H, K, V = self.B, self.T, self.H, self.K, self.V
        if h.shape[:2] != (B, T) or h.dtype != torch.bfloat16:
            raise ValueError(f"expected bf16 input [{B}, {T}, hidden] (got {tuple(h.shape)} {h.dtype})")
        o_q, o_k, o_v, o_g, o_a, o_b = self.offsets
        cw = [c.weight for c in (L.q_conv1d, L.k_conv1d, L.v_conv1d)]
        cb = [c.bias for c in (L.q_conv1d, L.k_conv1d, L.v_conv1d)]
        nw, neps = (None, 1e-5) if norm is None else (norm.weight, norm.eps)
        if self.fast and self.conv_in_proj:
            # the input projections with the short convolutions, g and beta in their epilogue
            # (ccq_gdn_decode_in_proj), then the decode step over those rows, which normalises q and k
            # and forms lambda (ccq_gdn_layer_decode_step): three launches fewer than the prologue path
            x = torch.empty(B, T, self.width, device=h.device, dtype=torch.bfloat16)
            h2 = _rows(h)
            call("ccq_gdn_decode_in_proj", ptr(h2), h2.stride(0), ptr(self.w_in), ptr(x), self.width, B * T,
                 L.hidden_size, self.width, ptr(_norm_arg(h, nw)), float(neps), o_q, o_k, o_v, o_a, o_b, H, H * K,
                 H * V, T, ptr(cw[0]), ptr(cw[1]), ptr(cw[2]), ptr(cb[0]), ptr(cb[1]), ptr(cb[2]),
                 ptr(self.conv[0]), ptr(self.conv[1]), ptr(self.conv[2]), ptr(L.A_log), ptr(L.dt_bias), ptr(st.g),
                 ptr(st.beta), int(L.allow_neg_eigval), _lib.stream_of(h))
            call("ccq_gdn_layer_decode_step", ptr(x), self.width, o_q, o_k, o_v, ptr(L.erase_lambda_proj.weight),
                 ptr(L.erase_lambda_proj.bias), ptr(st.g), ptr(st.beta), ptr(st.S), ptr(st.C), ptr(st.m),
                 ptr(st.position), ptr(st.o), ptr(st.workspace), B, T, H, K, V, int(st.subtract_mean),
                 int(st.enable_ccq), st.scale, 1e-6, _lib.stream_of(x))
        else:
            if self.fast:
                # (with norm: the block's RMSNorm of h folded into the input projection)
                x = decode_linear(h, self.w_in, norm_weight=nw, norm_eps=neps)
            else:
                x = F.linear(h if norm is None else norm(h), self.w_in)
            call("ccq_gdn_decode_prologue", x.data_ptr() + 2 * o_q, x.data_ptr() + 2 * o_k, x.data_ptr() + 2 * o_v,
                 x.data_ptr() + 2 * o_a, x.data_ptr() + 2 * o_b, self.width,
                 ptr(cw[0]), ptr(cw[1]), ptr(cw[2]), ptr(cb[0]), ptr(cb[1]), ptr(cb[2]),
                 ptr(self.conv[0]), ptr(self.conv[1]), ptr(self.conv[2]),
                 ptr(L.erase_lambda_proj.weight), ptr(L.erase_lambda_proj.bias), ptr(L.A_log), ptr(L.dt_bias),
                 ptr(st.q), ptr(st.k), ptr(st.v), ptr(st.lam), ptr(st.g), ptr(st.beta),
                 B, T, H, K, V, self.W, int(L.allow_neg_eigval), 1e-6, _lib.stream_of(x))
            st.launch()
        base = x.data_ptr()
        at = lambda off: base + 2 * off  # noqa: E731  (bf16 elements)
        if self.fast and self.gnorm_in_proj and decode_linear_ok(st.o.view(B, T, H * V), L.o_proj.weight):
            # the gated output norm folded into the output projection, the gate rows read in place
            gate = x.view(B * T, self.width)[:, o_g:o_g + H * V]
            return decode_linear_gnorm(st.o.view(B, T, H * V), gate, self.norm_w, V, float(L.o_norm.eps),
                                       L.o_proj.weight, residual, self.o_ws)
        if L.use_gate:
            # the gated RMSNorm kernel reading the gate rows in place from the projection output (H rows
            # of V per token, the projection's row width apart), with the weight converted in refresh()
            o = torch.empty_like(st.o)
            rstd = torch.empty(B * T * H, device=x.device, dtype=torch.float32)
            call("ccq_gated_rmsnorm_fwd_strided", ptr(st.o), at(o_g), self.width, H, ptr(self.norm_w), ptr(o),
                 ptr(rstd), B * T * H, V, float(L.o_norm.eps), _lib.stream_of(x))
        else:
            o = L.o_norm(st.o)
        o = o.reshape(B, T, H * V)
        if self.fast and decode_linear_ok(o, L.o_proj.weight):
            if self.o_splits > 1:
                return decode_linear_split(o, L.o_proj.weight, residual, self.o_splits, self.o_ws)
            return decode_linear(o, L.o_proj.weight, residual)
        y = L.o_proj(o)
        return y if residual is None else residual + y
