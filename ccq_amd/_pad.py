"""Head sizes the kernels do not take directly.

The reference layers accept any ``head_dim`` (``ccq/gdn/layer.py:96``, ``ccq/gla/layer.py``; fla's
kernels take any size).  The kernels here take key sizes K in {64, 128, 256} (the chunk kernels) or
{32, 64, 128, 256} (the cleaning and the decode step) and value sizes V that are multiples of 64 up
to 1024.  Other sizes run zero-padded: q, k (and the per-key decays, the gate weights, the
covariance and key-sum states) along the key dimension to the next size the kernels take, v (and the
per-value decays, the backbone states) along the value dimension to the next multiple of 64; every
output and final state is sliced back.

Zero key channels add nothing to q . k, k k^T, the L2 norms or the running key sums, and a zero
value channel stays zero in the backbone state and the output (its state column starts at zero and
receives k times the channel's zero value (GLA) or beta (0 - S^T k) taken over that zero column
(GDN)), so the sliced results are those of the unpadded problem.  torch's ``pad`` and slicing carry
the gradients back to the unpadded inputs.  The padded channels cost their share of the work.
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

CHUNK_K = (64, 128, 256)
STEP_K = (32, 64, 128, 256)
V_STEP, V_MAX = 64, 1024


def key_size(K: int, sizes: Sequence[int]) -> int:
    for s in sizes:
        if K <= s:
            return s
    raise ValueError(f"head size K={K} is above the largest key size the kernels take ({sizes[-1]})")


def value_size(V: int) -> int:
    Vp = -(-V // V_STEP) * V_STEP
    if V < 1 or Vp > V_MAX:
        raise ValueError(f"value size V={V} must be in [1, {V_MAX}]")
    return Vp


def padded_sizes(K: int, V: Optional[int], sizes: Sequence[int]) -> Tuple[int, Optional[int]]:
    return key_size(K, sizes), (None if V is None else value_size(V))


def pad_tail(x: Optional[torch.Tensor], *sizes: int) -> Optional[torch.Tensor]:
    """x zero-padded so that its last len(sizes) dimensions have the given sizes (None stays None)."""
    if x is None:
        return None
    tail = x.shape[x.dim() - len(sizes):]
    if tuple(tail) == tuple(sizes):
        return x
    spec = []
    for have, want in zip(reversed(tail), reversed(sizes)):
        if want < have:
            raise ValueError(f"cannot pad a dimension of {have} down to {want}")
        spec += [0, want - have]
    return F.pad(x, spec)


def cut_tail(x: Optional[torch.Tensor], *sizes: int) -> Optional[torch.Tensor]:
    """The leading part of x's last len(sizes) dimensions (contiguous; None stays None)."""
    if x is None:
        return None
    tail = x.shape[x.dim() - len(sizes):]
    if tuple(tail) == tuple(sizes):
        return x
    idx = (Ellipsis,) + tuple(slice(0, s) for s in sizes)
    return x[idx].contiguous()
