"""Row L2 normalisation ``x / sqrt(sum x^2 + eps)`` with its backward, on the GPU
(stands in for fla's ``l2norm``, which the reference calls at
``ccq/ops/ccq_gdn/fused_chunk.py:43-44`` and in every orchestrator)."""

from __future__ import annotations

import torch

from .clean import as_kernel_dtype, in_dtype, l2norm_bwd, l2norm_fwd

__all__ = ["l2norm", "L2NormFunction"]


class L2NormFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, eps):
        if not x.is_cuda or x.dtype != torch.bfloat16:
            raise TypeError("ccq_amd l2norm runs on bf16 CUDA tensors (l2norm() converts other dtypes)")
        x = x.contiguous()
        y, rstd = l2norm_fwd(x, eps)
        ctx.save_for_backward(x, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, rstd = ctx.saved_tensors
        return l2norm_bwd(x, rstd, dy), None


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """fp16 / fp32 rows are normalised as bf16 and returned in their own dtype."""
    (xb,) = as_kernel_dtype(x)
    return in_dtype(L2NormFunction.apply(xb, float(eps)), x.dtype)
