"""Tile gather, mean pool and untile (oracle, test infrastructure only).

Restates the Triton kernels ``_fused_q_prep_kernel`` / ``_fused_kv_prep_kernel``
/ ``_fused_untile_kernel`` (ar_sparse_operation.py:26-161, identical copies in
bi_sparse_operation_for_KV_cache.py:27-163 and bi_sparse_operation.py:25-140):

* gather: tiled[b,h,blk,f,:] = x[b,h,l(blk,f),:] or 0 outside the grid
  (ar_sparse_operation.py:58-66);
* pool:   bf16( fp32-sum over the BS rows of the tile / float(BS) ) with the
  padding rows included (ar_sparse_operation.py:69-70);
* untile: x[b,h,l(blk,f),:] = tiled[b,h,blk,f,:] for valid slots only
  (ar_sparse_operation.py:158-161).

The reference's fp32 sum order (Triton ``tl.sum``) is not observable, so the
oracle fixes one: ``NG = 256 // (D // 8)`` row groups; group ``g`` sums rows
``g, g+NG, g+2NG, ...`` sequentially starting from +0.0; the NG partials are
then combined by the pairwise tree ``s[g] += s[g+stride]`` for
``stride = NG/2, NG/4, ..., 1``.  This is the order the HIP gather kernel uses,
so pooled values are compared bit-exactly.

Pinned by tests/test_oracle_tile.py: gather/untile round trip is the identity
on valid tokens and padding rows are zero (brute force over small grids);
the pool agrees with an exact (float64) mean rounded to bf16 to within one
bf16 ulp and exactly on power-of-two-friendly inputs.
"""
import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16
from .geometry import tile_permutation


def tile_gather(x_bits, T, H, W, tile):
    """x_bits: uint16 (B, NH, L, D) with L >= T*H*W -> tiles uint16 (B, NH, nblk, BS, D)."""
    tt, th, tw = tile
    bs = tt * th * tw
    perm = tile_permutation(T, H, W, tile)
    B, NH, _, D = x_bits.shape
    out = np.zeros((B, NH, perm.size, D), dtype=np.uint16)
    valid = perm >= 0
    out[:, :, valid, :] = x_bits[:, :, perm[valid], :]
    return out.reshape(B, NH, perm.size // bs, bs, D)


def pool_mean(tiles_bits):
    """Fixed-order fp32 mean over the BS rows of each tile -> uint16 bf16 (B, NH, nblk, D)."""
    B, NH, nblk, bs, D = tiles_bits.shape
    ng = 256 // (D // 8)
    x = bf16_to_f32(tiles_bits)
    part = np.zeros((B, NH, nblk, ng, D), dtype=np.float32)
    for f in range(bs):
        g = f % ng
        part[:, :, :, g, :] = part[:, :, :, g, :] + x[:, :, :, f, :]
    stride = ng // 2
    while stride >= 1:
        part[:, :, :, :stride, :] = part[:, :, :, :stride, :] + part[:, :, :, stride:2 * stride, :]
        stride //= 2
    s = part[:, :, :, 0, :]
    return f32_to_bf16(s / np.float32(bs))


def untile(tiles_bits, L, T, H, W, tile):
    """Inverse scatter: uint16 (B, NH, nblk, BS, D) -> uint16 (B, NH, L, D); untouched rows are zero."""
    B, NH, nblk, bs, D = tiles_bits.shape
    perm = tile_permutation(T, H, W, tile)
    flat = tiles_bits.reshape(B, NH, nblk * bs, D)
    out = np.zeros((B, NH, L, D), dtype=np.uint16)
    valid = perm >= 0
    out[:, :, perm[valid], :] = flat[:, :, valid, :]
    return out
