"""Import name of the reference's kernel module (``src/triton_block_attn.py``).

Harness code imports ``block_sparse_attn``, ``block_sparse_attn_v2``,
``_compute_kv_idx`` and ``reference_attn`` from ``triton_block_attn``; on
MI355X they are the HIP launchers and helpers of ``block_attn``.  Nothing
here uses Triton.
"""

from block_attn import (  # noqa: F401
    _compute_kv_idx,
    attn_workspace,
    block_sparse_attn,
    block_sparse_attn_v2,
    reference_attn,
)
