"""Block geometry and the 3D tile permutation (oracle, test infrastructure only).

Restates ar_sparse_operation.py:319-327 (block counts, also
bi_sparse_operation_for_KV_cache.py:347-361 and bi_sparse_operation.py:253-265)
and the index maps of the Triton gather kernels, ar_sparse_operation.py:42-59:

* block ``blk`` -> ``(ct, ch, cw) = (blk // (nh*nw), (blk // nw) % nh, blk % nw)``
* in-tile row ``f`` -> ``(ft, fh, fw) = (f // (tw*th), (f // tw) % th, f % tw)``
* linear token ``l = (ct*tt+ft)*H*W + (ch*th+fh)*W + (cw*tw+fw)``, valid iff
  ``t < T and h < H and w < W`` (otherwise the tile row is zero fill).

Pinned by tests/test_oracle_geometry.py: brute-force bijection between valid
tile slots and linear tokens on small grids, hand-computed block counts for
the HY (30x52, 2x8x8), MG (22x40) and toy (32x32, 4x4x4) shapes, and the
reference's own ``(x + (t - x % t) % t) // t`` padding formula.
"""
import numpy as np


def ceil_div(a, b):
    return (a + b - 1) // b


def pad_blocks(x, t):
    """The reference's block-count formula ``(x + (t - x % t) % t) // t`` (ar_sparse_operation.py:322-324)."""
    return (x + (t - x % t) % t) // t


def block_geometry(lq, lk_vis, latent_hw, tile, text_len=0):
    """Block geometry of one sparse call (ar_sparse_operation.py:319-327).

    Returns a dict with BS, nh, nw, T_q, T_k, nt_q, nt_k, num_txt_blk,
    nq_blk, nk_blk (visual), lq_pad, lk_pad (text + visual padded key length).
    """
    H, W = latent_hw
    tt, th, tw = tile
    bs = tt * th * tw
    nh, nw = pad_blocks(H, th), pad_blocks(W, tw)
    T_q, T_k = lq // (H * W), lk_vis // (H * W)
    nt_q, nt_k = pad_blocks(T_q, tt), pad_blocks(T_k, tt)
    num_txt_blk = pad_blocks(text_len, bs) if text_len > 0 else 0
    nq_blk, nk_blk = nt_q * nh * nw, nt_k * nh * nw
    return dict(BS=bs, nh=nh, nw=nw, T_q=T_q, T_k=T_k, nt_q=nt_q, nt_k=nt_k,
                num_txt_blk=num_txt_blk, nq_blk=nq_blk, nk_blk=nk_blk,
                lq_pad=nq_blk * bs, lk_pad=(num_txt_blk + nk_blk) * bs)


def tile_permutation(T, H, W, tile):
    """Linear token index for every (block, row) slot of the tiled layout, -1 for padding.

    Shape ``(nblk * BS,)`` with ``nblk = ceil(T/tt) * ceil(H/th) * ceil(W/tw)``.
    """
    tt, th, tw = tile
    nh, nw, nt = ceil_div(H, th), ceil_div(W, tw), ceil_div(T, tt)
    bs = tt * th * tw
    blk = np.arange(nt * nh * nw)[:, None]
    f = np.arange(bs)[None, :]
    ct, ch, cw = blk // (nh * nw), (blk // nw) % nh, blk % nw
    ft, fh, fw = f // (tw * th), (f // tw) % th, f % tw
    t, h, w = ct * tt + ft, ch * th + fh, cw * tw + fw
    valid = (t < T) & (h < H) & (w < W)
    lin = t * (H * W) + h * W + w
    return np.where(valid, lin, -1).reshape(-1).astype(np.int64)


def key_block_coords(nk, nh, nw):
    """(t, h, w) block-grid coordinates of key blocks 0..nk-1 (bi_sparse_operation_for_KV_cache.py:268-272)."""
    idx = np.arange(nk)
    return idx // (nh * nw), (idx % (nh * nw)) // nw, idx % nw
