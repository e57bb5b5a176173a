"""usagi_amd — MI355X (gfx950) block-sparse causal attention forward.

The reference's submission-module names are re-exported here:
VARIANT_MANIFEST, setup, block_sparse_attn_fwd (kernels/v7_blockptr_warpspec.py:24, 201, 251),
plus block_sparse_attn_fwd_generic, the order-free CSR walk (kernels/v1_baseline.py:331-406),
and block_sparse_attn_fwd_window, the analytic window / window + global-prefix path
(kernels/v1_baseline.py:141-322).
"""

from .submission import (  # noqa: F401
    BLOCK_SIZE,
    HEAD_DIM,
    VARIANT_MANIFEST,
    block_sparse_attn_fwd,
    block_sparse_attn_fwd_generic,
    block_sparse_attn_fwd_window,
    clear_csr_cache,
    setup,
)

__version__ = "0.2.0"
