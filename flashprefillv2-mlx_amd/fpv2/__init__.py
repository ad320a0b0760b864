"""FlashPrefill V2 block-sparse prefill attention for MI355X (gfx950).

Public surface of the reference package (``fpv2/__init__.py``): the SDPA hook
(``enable``/``disable``/``is_enabled``/``fpv2_sdpa``/``block_sparsity``) and the
selection front end (``FPV2Config``/``pool_blocks``/``block_scores_and_select``/
``density``).  ``fpv2.kernel`` holds ``compact_block_indices`` and
``sparse_attention``.  ``ChunkedPrefill`` (``fpv2.chunked``) drives one
layer's chunked prefill over a growing KV cache with incremental pooling.
"""

from fpv2.chunked import ChunkedPrefill
from fpv2.patch import block_sparsity, disable, enable, fpv2_sdpa, is_enabled
from fpv2.selection import FPV2Config, block_scores_and_select, density, pool_blocks

__all__ = [
    "ChunkedPrefill",
    "FPV2Config",
    "block_scores_and_select",
    "block_sparsity",
    "density",
    "disable",
    "enable",
    "fpv2_sdpa",
    "is_enabled",
    "pool_blocks",
]
