"""Block-sparse flash attention, HY-WorldPlay entry point.

Same signature and error behaviour as ``longcat_flash_attn``
(hy-worldplay/files/hyvideo/models/transformers/modules/longcat_kernel.py:158-233);
the Triton kernel ``_attn_fwd_bsa_align`` (longcat_kernel.py:27-155) is replaced
by the gfx950 HIP kernel behind ``li_bsa_fwd``.
"""
from .. import _core
import torch

_HALF = (torch.float16, torch.bfloat16)


def _prepare(q, k, v):
    # Non-half inputs are computed in bf16 (matrix-game-3.0 longcat_kernel.py:139-147);
    # K and V follow Q's (possibly cast) dtype, since the kernels take one element type.
    q = q if q.dtype in _HALF else q.to(torch.bfloat16)
    k = k.to(q.dtype) if k.dtype != q.dtype else k
    v = v.to(q.dtype) if v.dtype != q.dtype else v
    return q.contiguous(), k.contiguous(), v.contiguous()


def longcat_flash_attn(q, k, v, block_indices, block_counts, sm_scale=None, logical_block_size=128):
    """Block-sparse flash attention.

    Args:
        q: Query ``(B, H, Q_len, D)``.
        k: Key ``(B, H, K_len, D)``.
        v: Value ``(B, H, K_len, D)``.
        block_indices: ``(B, H, ceil(Q_len / logical_block_size), K_blk)`` int32 key-block ids.
        block_counts: ``(B, H, ceil(Q_len / logical_block_size))`` int32 valid ids per query tile.
        sm_scale: softmax scale (default ``1/sqrt(D)``).
        logical_block_size: key block size, also the query tile size (64 or 128).

    Returns:
        Attention output ``(B, H, Q_len, D)`` in q's dtype, as ``torch.empty_like(q)``
        gives it in the reference (longcat_kernel.py:198); a float32 (or other
        non-half) q is computed in bf16 and the output cast back.

    Raises:
        ValueError: if K_len is not divisible by logical_block_size or a block
        index is out of bounds (checked on the host, as the reference does).
    """
    out_dtype = q.dtype
    q, k, v = _prepare(q, k, v)
    block_indices = block_indices.contiguous()
    block_counts = block_counts.contiguous()
    if block_indices.dtype != torch.int32:
        block_indices = block_indices.int()
    if block_counts.dtype != torch.int32:
        block_counts = block_counts.int()
    B, H, Q_len, HEAD_DIM = q.shape
    K_len = k.shape[2]
    if sm_scale is None:
        sm_scale = 1.0 / (HEAD_DIM ** 0.5)
    BLOCK_N = logical_block_size
    if K_len % BLOCK_N != 0:
        raise ValueError(f"K Length ({K_len}) must be divisible by logical_block_size ({BLOCK_N})")
    if block_indices.numel() and (int(block_indices.max()) >= K_len // BLOCK_N or int(block_indices.min()) < 0):
        raise ValueError("Sparse indices out of bounds.")
    o = _core.bsa_forward(q, k, v, block_indices, block_counts, sm_scale, BLOCK_N)
    return o if o.dtype == out_dtype else o.to(out_dtype)
