"""Block-sparse flash attention, Matrix-Game-3.0 entry point.

Same signature as ``longcat_flash_attn``
(matrix-game-3.0/files/wan/modules/longcat_kernel.py:137-190): non-half inputs
are cast to bf16 and a K length that is not a multiple of the block size fails
an ``assert`` (longcat_kernel.py:161); indices are not range-checked on the
host, as in the reference (the HIP kernel skips out-of-range ids instead of
reading out of bounds).
"""
from .. import _core
from ..hy.longcat_kernel import _prepare


def longcat_flash_attn(q, k, v, block_indices, block_counts, sm_scale=None, logical_block_size=128):
    q, k, v = _prepare(q, k, v)
    block_indices = block_indices.contiguous().int()
    block_counts = block_counts.contiguous().int()
    B, H, Q_len, HEAD_DIM = q.shape
    K_len = k.shape[2]
    if sm_scale is None:
        sm_scale = 1.0 / (HEAD_DIM ** 0.5)
    BLOCK_N = logical_block_size
    assert K_len % BLOCK_N == 0, f"K Length ({K_len}) must be divisible by logical_block_size ({BLOCK_N})"
    return _core.bsa_forward(q, k, v, block_indices, block_counts, sm_scale, BLOCK_N)
