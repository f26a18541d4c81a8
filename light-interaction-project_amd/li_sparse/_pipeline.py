"""The sparse-attention call shared by the HY and MG entry points.

Steps (ar_sparse_operation.py:316-362, bi_sparse_operation_for_KV_cache.py:347-395,
bi_sparse_operation.py:246-348): block geometry; tile buffers; text K/V
zero-padded into the leading blocks; Q tile gather + pool; K/V tile gather +
K pool; block selection; block-sparse attention; untile into ``empty_like(q)``.
Every stage except the text copy is one HIP kernel of this package; the
index lists come from the mask kernel, so the attention launch needs no
host-side range check (the reference's ``block_indices.max()`` sync is gone).
"""
import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _core


@dataclass(frozen=True)
class Geometry:
    """Block geometry of one call (ar_sparse_operation.py:319-327)."""
    H: int
    W: int
    tt: int
    th: int
    tw: int
    bs: int
    nh: int
    nw: int
    T_q: int
    T_k: int
    nt_q: int
    nt_k: int
    num_txt_blk: int
    nq_blk: int
    nk_blk: int


def pad_blocks(x, t):
    return (x + (t - x % t) % t) // t


def geometry(latent_hw, tile, vis_len_q, vis_len_k, text_len):
    H, W = latent_hw
    tt, th, tw = tile
    bs = tt * th * tw
    nh, nw = pad_blocks(H, th), pad_blocks(W, tw)
    T_q, T_k = vis_len_q // (H * W), vis_len_k // (H * W)
    nt_q, nt_k = pad_blocks(T_q, tt), pad_blocks(T_k, tt)
    num_txt_blk = pad_blocks(text_len, bs)
    return Geometry(H, W, tt, th, tw, bs, nh, nw, T_q, T_k, nt_q, nt_k, num_txt_blk, nt_q * nh * nw, nt_k * nh * nw)


def _stage(events, name):
    if events is not None:
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        events[name] = e


def _fusable(*ts):
    """Token views the fused kernel reads directly: unit d stride, 16-byte aligned, non-overlapping rows."""
    for t in ts:
        st = t.stride()
        if st[3] != 1 or any(x % 8 for x in st[:3]) or st[2] < t.shape[3] or t.data_ptr() % 16:
            return False
    return True


def uses_fused(q, k_vis, v_vis, tile, latent_hw):
    """True when ``sparse_attention(..., fused=True)`` takes the fused kernel for these inputs."""
    return _core.fused_supported(q.shape[3], tile, latent_hw) and _fusable(q, k_vis, v_vis)


def ragged(sparse_params):
    """Whether the rows have their own budgets (then the attention starts its longest tiles first)."""
    return sparse_params.get("row_budget") is not None


def qk_fp8(sparse_params):
    """The ``qk_fp8`` extension key: Q K^T on e4m3 codes with per-tile-block scales."""
    return bool(sparse_params.get("qk_fp8", False))


def _fused(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance):
    """Pools, block selection, then one kernel that gathers, attends and untiles."""
    B, NH, _, D = q.shape
    dev, dt = q.device, q.dtype
    _stage(events, "alloc_start")
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=dt)
    k_pool = torch.empty((B, NH, g.nk_blk, D), device=dev, dtype=dt)
    kt = vt = None
    if text_len > 0:
        pad = g.num_txt_blk * g.bs - text_len
        kt = (F.pad(k_txt, (0, 0, 0, pad)) if pad > 0 else k_txt).contiguous()
        vt = (F.pad(v_txt, (0, 0, 0, pad)) if pad > 0 else v_txt).contiguous()
    o_out = torch.empty_like(q)
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    _core.pool(q, q_pool, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.pool(k_vis, k_pool, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = select(q_pool, k_pool, text_len, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw))
    _stage(events, "index_end")
    _stage(events, "attn_start")
    _core.bsa_forward_gather(q, k_vis, v_vis, kt, vt, g.num_txt_blk, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw,
                             g.nh, g.nw, indices, counts, 1.0 / math.sqrt(D), o_out, balance=balance)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def fp8_supported(D, tile):
    """Shapes the e4m3 (qk_fp8) path is built for: D = 128 and 128-token tiles."""
    return D == 128 and tile[0] * tile[1] * tile[2] == 128


def _tiled_fp8(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance):
    """Tiled sequence with Q and K quantized to e4m3 per tile block (scale amax / 448) in their gathers.

    The pools (and so the block selection) are those of the bf16 path; V, P V and the output stay bf16.
    """
    B, NH, _, D = q.shape
    dev = q.device
    f8 = _core.FP8
    _stage(events, "alloc_start")
    q8 = torch.empty((B, NH, g.nq_blk, g.bs, D), device=dev, dtype=f8)
    q_scale = torch.empty((B, NH, g.nq_blk), device=dev, dtype=torch.float32)
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=q.dtype)
    nkb = g.num_txt_blk + g.nk_blk
    k8 = torch.empty((B, NH, nkb, g.bs, D), device=dev, dtype=f8)
    k_scale = torch.empty((B, NH, nkb), device=dev, dtype=torch.float32)
    v_all = torch.empty((B, NH, nkb, g.bs, D), device=dev, dtype=q.dtype)
    k_pool = torch.empty((B, NH, g.nk_blk, D), device=dev, dtype=q.dtype)
    if text_len > 0:
        pad = g.num_txt_blk * g.bs - text_len
        kt = F.pad(k_txt, (0, 0, 0, pad)) if pad > 0 else k_txt
        vt = F.pad(v_txt, (0, 0, 0, pad)) if pad > 0 else v_txt
        v_all[:, :, :g.num_txt_blk].copy_(vt.reshape(B, NH, g.num_txt_blk, g.bs, D))
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    if text_len > 0:
        # Contiguous text blocks: the trivial grid T = blocks, H = 1, W = BS, tile (1, 1, BS).
        _core.tile_prep_fp8(kt, k8, k_scale, None, 0, 0, g.num_txt_blk, 1, g.bs, 1, 1, g.bs, 1, 1)
    _core.tile_prep_fp8(q, q8, q_scale, q_pool, 0, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.kv_prep_fp8(k_vis, v_vis, k8, k_scale, v_all, k_pool, g.num_txt_blk, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw,
                      g.nh, g.nw)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = select(q_pool, k_pool, text_len, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw))
    _stage(events, "index_end")
    _stage(events, "attn_start")
    o_flat = _core.bsa_forward_fp8(q8.flatten(2, 3), q_scale, k8.flatten(2, 3), k_scale, v_all.flatten(2, 3),
                                   indices, counts, 1.0 / math.sqrt(D), g.bs, balance=balance)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    o_out = torch.empty_like(q)
    _core.untile(o_flat.view(B, NH, g.nq_blk, g.bs, D), o_out, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def _fused_fp8(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance):
    """e4m3 Q/K tiles from the quantizing gathers, then one kernel that reads V and writes O in token order."""
    B, NH, _, D = q.shape
    dev = q.device
    f8 = _core.FP8
    _stage(events, "alloc_start")
    q8 = torch.empty((B, NH, g.nq_blk, g.bs, D), device=dev, dtype=f8)
    q_scale = torch.empty((B, NH, g.nq_blk), device=dev, dtype=torch.float32)
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=q.dtype)
    nkb = g.num_txt_blk + g.nk_blk
    k8 = torch.empty((B, NH, nkb, g.bs, D), device=dev, dtype=f8)
    k_scale = torch.empty((B, NH, nkb), device=dev, dtype=torch.float32)
    k_pool = torch.empty((B, NH, g.nk_blk, D), device=dev, dtype=q.dtype)
    vt = None
    if text_len > 0:
        pad = g.num_txt_blk * g.bs - text_len
        kt = F.pad(k_txt, (0, 0, 0, pad)) if pad > 0 else k_txt
        vt = (F.pad(v_txt, (0, 0, 0, pad)) if pad > 0 else v_txt).contiguous()
    o_out = torch.empty_like(q)
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    if text_len > 0:
        _core.tile_prep_fp8(kt, k8, k_scale, None, 0, 0, g.num_txt_blk, 1, g.bs, 1, 1, g.bs, 1, 1)
    _core.tile_prep_fp8(q, q8, q_scale, q_pool, 0, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.tile_prep_fp8(k_vis, k8, k_scale, k_pool, g.num_txt_blk, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = select(q_pool, k_pool, text_len, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw))
    _stage(events, "index_end")
    _stage(events, "attn_start")
    _core.bsa_forward_fp8_gather(q8.flatten(2, 3), q_scale, k8.flatten(2, 3), k_scale, v_vis, vt, g.num_txt_blk,
                                 g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, indices, counts,
                                 1.0 / math.sqrt(D), o_out, balance=balance)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def sparse_attention(q, k_txt, v_txt, k_vis, v_vis, latent_hw, tile, select, events=None, fused=True,
                     balance=False, qk_fp8=False):
    """One sparse-attention forward.

    q (B,H,Lq,D); k_txt/v_txt (B,H,N_txt,D) or None; k_vis/v_vis (B,H,Lk,D), any strides.
    ``select(q_pool, k_pool, text_len, grid_q, grid_k) -> (indices, counts)``.
    ``events`` (dict or None) collects CUDA events per stage for profiling.
    ``fused`` (default) runs pools + one gather/attend/untile kernel where the
    shape allows it (D = 128, 128-token tiles, tw and W multiples of 4, a grid
    at least one tile high and wide, token views with unit d stride);
    otherwise, or with ``fused=False``, the tiled sequence q_prep / kv_prep /
    attention / untile.  Both give the same bits.  ``balance`` (rows with their own budgets) starts
    the longest query tiles first.  ``qk_fp8`` takes Q K^T on e4m3 codes with one scale per tile
    block (bf16 only; D = 128 and 128-token tiles, ValueError otherwise); the selection is unchanged.
    """
    out_dtype = q.dtype
    if q.dtype not in (torch.bfloat16, torch.float16):
        q, k_vis, v_vis = q.to(torch.bfloat16), k_vis.to(torch.bfloat16), v_vis.to(torch.bfloat16)
        if k_txt is not None:
            k_txt, v_txt = k_txt.to(torch.bfloat16), v_txt.to(torch.bfloat16)
    text_len = 0 if k_txt is None else k_txt.shape[2]
    g = geometry(latent_hw, tile, q.shape[2], k_vis.shape[2], text_len)
    B, NH, _, D = q.shape
    dev, dt = q.device, q.dtype
    if qk_fp8:
        if dt != torch.bfloat16 or not fp8_supported(D, tile):
            raise ValueError(f"qk_fp8 is built for bfloat16, D = 128 and 128-token tiles (got {dt}, D = {D}, "
                             f"tile {tuple(tile)})")
        if fused and uses_fused(q, k_vis, v_vis, tile, (g.H, g.W)):
            return _fused_fp8(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance)
        return _tiled_fp8(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance)
    if fused and uses_fused(q, k_vis, v_vis, tile, (g.H, g.W)):
        return _fused(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance)
    _stage(events, "alloc_start")
    q_tiled = torch.empty((B, NH, g.nq_blk, g.bs, D), device=dev, dtype=dt)
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=dt)
    k_all = torch.empty((B, NH, g.num_txt_blk + g.nk_blk, g.bs, D), device=dev, dtype=dt)
    v_all = torch.empty((B, NH, g.num_txt_blk + g.nk_blk, g.bs, D), device=dev, dtype=dt)
    k_pool = torch.empty((B, NH, g.nk_blk, D), device=dev, dtype=dt)
    if text_len > 0:
        pad = g.num_txt_blk * g.bs - text_len
        kt = F.pad(k_txt, (0, 0, 0, pad)) if pad > 0 else k_txt
        vt = F.pad(v_txt, (0, 0, 0, pad)) if pad > 0 else v_txt
        k_all[:, :, :g.num_txt_blk].copy_(kt.reshape(B, NH, g.num_txt_blk, g.bs, D))
        v_all[:, :, :g.num_txt_blk].copy_(vt.reshape(B, NH, g.num_txt_blk, g.bs, D))
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    _core.q_prep(q, q_tiled, q_pool, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.kv_prep(k_vis, v_vis, k_all, v_all, k_pool, g.num_txt_blk, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw,
                  g.nh, g.nw)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = select(q_pool, k_pool, text_len, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw))
    _stage(events, "index_end")
    _stage(events, "attn_start")
    o_flat = _core.bsa_forward(q_tiled.flatten(2, 3), k_all.flatten(2, 3), v_all.flatten(2, 3), indices, counts,
                               1.0 / math.sqrt(D), g.bs, balance=balance)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    o_out = torch.empty_like(q)
    _core.untile(o_flat.view(B, NH, g.nq_blk, g.bs, D), o_out, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def dense_attention(q, k_txt, v_txt, k_vis, v_vis):
    """The reference's dense fallback ``F.scaled_dot_product_attention(q, cat(k_txt, k_vis), cat(v_txt, v_vis))``
    (ar_sparse_operation.py:316-317, bi_sparse_operation_for_KV_cache.py:331-343, bi_sparse_operation.py:246-248).

    Runs the dense HIP kernel (li_attn_fwd_dense: every key, no concatenation formed) for fp16/bf16, D = 128 and
    visual lengths that are multiples of 4; other inputs take the reference's own torch call.
    """
    if k_txt is not None and k_txt.shape[2] == 0:
        k_txt = v_txt = None
    if _core.dense_supported(q, k_vis, v_vis, k_txt):
        return _core.attn_dense(q, k_vis, v_vis, k_txt, v_txt)
    if k_txt is not None:
        k_vis, v_vis = torch.cat([k_txt, k_vis], dim=2), torch.cat([v_txt, v_vis], dim=2)
    return F.scaled_dot_product_attention(q, k_vis, v_vis, dropout_p=0.0, is_causal=False)


def recent_blocks(params, tt, nh, nw, nk):
    """Trailing key blocks protected by ``recent_protect`` frames (ar_sparse_operation.py:263-266)."""
    rp = params.get("recent_protect", 0)
    if rp > 0:
        return min(((rp + tt - 1) // tt) * nh * nw, nk)
    return 0


def extras(params):
    """Forced-block and ragged-budget extensions (unset = the reference's rules)."""
    return dict(force_diag=bool(params.get("force_diag", False)), force_sink=bool(params.get("force_sink", False)),
                row_budget=params.get("row_budget"))
