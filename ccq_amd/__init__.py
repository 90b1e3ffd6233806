"""ccq_amd -- the CCQ read-side cleaning operator and the chunked linear-attention
path it feeds, written for AMD Instinct MI355X (gfx950).

Public surface mirrors the reference ``ccq.ops`` packages (``ccq/ops/ccq_gdn``, ``ccq/ops/ccq_gla``,
``ccq/ops/common/fused_read.py``).  All compute runs in hand-written HIP
kernels of ``libccq_hip.so`` (C ABI in ``include/ccq_hip.h``).
"""

from .ccq_gdn import (chunk_ccq_gdn, chunk_gated_delta_rule, fused_ccq_clean, fused_chunk_ccq_gdn,
                      fused_recurrent_ccq_gdn)
from .ccq_gla import chunk_ccq_gla, chunk_gla, fused_chunk_ccq_gla, fused_recurrent_ccq_gla
from .clean import FusedCCQCleanRead, _ccq_compute_z_and_sum_kk, _CCQCleanQ, fused_ccq_clean_read
from .l2norm import l2norm
from .layers import CCQGDN, CCQGLA, LayerCache

__all__ = [
    "chunk_ccq_gdn",
    "fused_chunk_ccq_gdn",
    "fused_recurrent_ccq_gdn",
    "fused_ccq_clean",
    "chunk_gated_delta_rule",
    "chunk_ccq_gla",
    "fused_chunk_ccq_gla",
    "fused_recurrent_ccq_gla",
    "chunk_gla",
    "fused_ccq_clean_read",
    "FusedCCQCleanRead",
    "_CCQCleanQ",
    "_ccq_compute_z_and_sum_kk",
    "l2norm",
    "CCQGDN",
    "CCQGLA",
    "LayerCache",
]
