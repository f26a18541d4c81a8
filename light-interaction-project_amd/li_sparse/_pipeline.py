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


def cosine(sparse_params):
    """Whether the selection scores blocks by cosine similarity (the reference's default ``sim_metric``)."""
    return sparse_params.get("sim_metric", "cosine") == "cosine"


class ContextCache:
    """Prepared key-side blocks of the fixed context of K/V, kept across calls.

    HY-WorldPlay recomputes the current chunk's K/V at every denoise step while
    the memory frames' K/V and the text stay fixed for the chunk; the reference
    re-tiles all of it on every call (ar_sparse_operation.py:337-348).  Pass a
    cache as ``sparse_params["context_cache"]`` with
    ``sparse_params["context_frames"]``, the number of leading K frames that do
    not change until the next ``reset()``.  The first call per layer
    (``block_idx``) and shape prepares every key block (pools; e4m3 codes and
    scales; tiles on the tiled paths) and keeps the buffers; later calls
    prepare only the blocks from the first t-slab that is not entirely
    context (the context is rounded down to whole ``tt``-frame slabs) and the
    text blocks not at all.  Results are bit-identical to uncached calls.  Call
    ``reset()`` whenever the context or the text changes (a new chunk);
    calls that share a cache must run on one stream.
    """

    def __init__(self):
        self._entries = {}

    def reset(self):
        self._entries.clear()

    def __len__(self):
        return len(self._entries)


def context_of(sparse_params, block_idx):
    """(cache, layer, frames) from ``sparse_params`` for ``sparse_attention``, or None without a cache."""
    cache = sparse_params.get("context_cache")
    if cache is None:
        return None
    if not isinstance(cache, ContextCache):
        raise TypeError("sparse_params['context_cache'] must be a li_sparse.ContextCache")
    return cache, block_idx, int(sparse_params.get("context_frames", 0))


def _pad_text(x, g, text_len):
    pad = g.num_txt_blk * g.bs - text_len
    return (F.pad(x, (0, 0, 0, pad)) if pad > 0 else x).contiguous()


def _k_side(path, k_txt, v_txt, k_vis, v_vis, g, text_len, ctx, B, NH, D, dev, dt, q_pool_job=None, k_norm=False):
    """Key-side buffers of one call: text blocks, then the visual blocks from the first uncached frame.

    path: "fused" (K pool; padded text K/V), "fused_fp8" (e4m3 K tiles + scales, K pool; padded text V),
    "tiled" (K/V tiles, K pool), "tiled_fp8" (e4m3 K tiles + scales, V tiles, K pool).
    q_pool_job: (q, q_pool, pool_off, geometry) of the query pool, taken in the same launch as the K pool on
    the fused path (li_pool_pair), or on its own when there is no K pool to take (every frame cached).
    k_norm: on the fused path, also keep the K pool's rows normalised for the cosine selection (written by
    the same launch, ``k_pool_n``; the selection takes it as ``k_pool_normalized``).
    """
    cache, layer, cframes = ctx if ctx is not None else (None, None, 0)
    cf = min((max(cframes, 0) // g.tt) * g.tt, g.T_k) if cache is not None else 0
    k_norm = bool(k_norm) and path == "fused"
    key = (path, layer, B, NH, D, dt, str(dev), g, text_len, cf, k_norm)
    bufs = cache._entries.get(key) if cache is not None else None
    first = cf if bufs is not None else 0
    nkb = g.num_txt_blk + g.nk_blk
    if bufs is None:
        bufs = {"k_pool": torch.empty((B, NH, g.nk_blk, D), device=dev, dtype=dt), "k_pool_n": None}
        if k_norm:
            bufs["k_pool_n"] = torch.empty_like(bufs["k_pool"])
        if path in ("fused_fp8", "tiled_fp8"):
            bufs["k8"] = torch.empty((B, NH, nkb, g.bs, D), device=dev, dtype=_core.FP8)
            bufs["k_scale"] = torch.empty((B, NH, nkb), device=dev, dtype=torch.float32)
        if path == "tiled":
            bufs["k_all"] = torch.empty((B, NH, nkb, g.bs, D), device=dev, dtype=dt)
        if path in ("tiled", "tiled_fp8"):
            bufs["v_all"] = torch.empty((B, NH, nkb, g.bs, D), device=dev, dtype=dt)
        bufs["kt"] = bufs["vt"] = None
        if text_len > 0:
            kt, vt = _pad_text(k_txt, g, text_len), _pad_text(v_txt, g, text_len)
            if path == "fused":
                bufs["kt"], bufs["vt"] = kt, vt
            elif path == "fused_fp8":
                bufs["vt"] = vt
            if path in ("fused_fp8", "tiled_fp8"):
                # Contiguous text blocks: the trivial grid T = blocks, H = 1, W = BS, tile (1, 1, BS).
                _core.tile_prep_fp8(kt, bufs["k8"], bufs["k_scale"], None, 0, 0, g.num_txt_blk, 1, g.bs, 1, 1, g.bs,
                                    1, 1)
            if path == "tiled":
                bufs["k_all"][:, :, :g.num_txt_blk].copy_(kt.view(B, NH, g.num_txt_blk, g.bs, D))
            if path in ("tiled", "tiled_fp8"):
                bufs["v_all"][:, :, :g.num_txt_blk].copy_(vt.view(B, NH, g.num_txt_blk, g.bs, D))
        if cache is not None:
            cache._entries[key] = bufs
    T = g.T_k - first
    if T > 0:
        fb = (first // g.tt) * g.nh * g.nw
        tok = first * g.H * g.W
        kv, vv = k_vis[:, :, tok:], v_vis[:, :, tok:]
        geo = (T, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
        if path == "fused" and q_pool_job is not None:
            _core.pool_pair(*q_pool_job, kv, bufs["k_pool"], fb, geo, mean1_normalized=bufs["k_pool_n"])
            q_pool_job = None
        elif path == "fused":
            if k_norm:
                raise ValueError("the normalised key pool is written with the query pool (li_pool_pair)")
            _core.pool(kv, bufs["k_pool"], fb, *geo)
        elif path == "fused_fp8":
            _core.tile_prep_fp8(kv, bufs["k8"], bufs["k_scale"], bufs["k_pool"], g.num_txt_blk + fb, fb, *geo)
        elif path == "tiled":
            _core.kv_prep(kv, vv, bufs["k_all"], bufs["v_all"], bufs["k_pool"], g.num_txt_blk + fb, fb, *geo)
        else:
            _core.kv_prep_fp8(kv, vv, bufs["k8"], bufs["k_scale"], bufs["v_all"], bufs["k_pool"], g.num_txt_blk + fb,
                              fb, *geo)
    if q_pool_job is not None:
        src, mean, off, qgeo = q_pool_job
        _core.pool(src, mean, off, *qgeo)
    return bufs


def _select(select, q_pool, kb, text_len, g):
    """``select`` on the call's pools; the normalised key pool goes along only when the call wrote one."""
    kw = {} if kb.get("k_pool_n") is None else {"k_pool_normalized": kb["k_pool_n"]}
    return select(q_pool, kb["k_pool"], text_len, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), **kw)


def _fused(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance, ctx, sorted_lists,
           k_norm=False):
    """Pools, block selection, then one kernel that gathers, attends and untiles."""
    B, NH, _, D = q.shape
    dev, dt = q.device, q.dtype
    _stage(events, "alloc_start")
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=dt)
    o_out = torch.empty_like(q)
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    q_job = (q, q_pool, 0, (g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw))
    kb = _k_side("fused", k_txt, v_txt, k_vis, v_vis, g, text_len, ctx, B, NH, D, dev, dt, q_pool_job=q_job,
                 k_norm=k_norm)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = _select(select, q_pool, kb, text_len, g)
    _stage(events, "index_end")
    _stage(events, "attn_start")
    _core.bsa_forward_gather(q, k_vis, v_vis, kb["kt"], kb["vt"], g.num_txt_blk, g.T_q, g.T_k, g.H, g.W, g.tt, g.th,
                             g.tw, g.nh, g.nw, indices, counts, 1.0 / math.sqrt(D), o_out, balance=balance,
                             sorted_lists=sorted_lists)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def fp8_supported(D, tile):
    """Shapes the e4m3 (qk_fp8) path is built for: D = 128 and 128-token tiles."""
    return D == 128 and tile[0] * tile[1] * tile[2] == 128


def _q_fp8(q, g, B, NH, D, dev):
    q8 = torch.empty((B, NH, g.nq_blk, g.bs, D), device=dev, dtype=_core.FP8)
    q_scale = torch.empty((B, NH, g.nq_blk), device=dev, dtype=torch.float32)
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=q.dtype)
    _core.tile_prep_fp8(q, q8, q_scale, q_pool, 0, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    return q8, q_scale, q_pool


def _tiled_fp8(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance, ctx, sorted_lists):
    """Tiled sequence with Q and K quantized to e4m3 per tile block (scale amax / 448) in their gathers.

    The pools (and so the block selection) are those of the bf16 path; V, P V and the output stay bf16.
    """
    B, NH, _, D = q.shape
    dev = q.device
    _stage(events, "alloc_start")
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    q8, q_scale, q_pool = _q_fp8(q, g, B, NH, D, dev)
    kb = _k_side("tiled_fp8", k_txt, v_txt, k_vis, v_vis, g, text_len, ctx, B, NH, D, dev, q.dtype)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = _select(select, q_pool, kb, text_len, g)
    _stage(events, "index_end")
    _stage(events, "attn_start")
    o_flat = _core.bsa_forward_fp8(q8.flatten(2, 3), q_scale, kb["k8"].flatten(2, 3), kb["k_scale"],
                                   kb["v_all"].flatten(2, 3), indices, counts, 1.0 / math.sqrt(D), g.bs,
                                   balance=balance)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    o_out = torch.empty_like(q)
    _core.untile(o_flat.view(B, NH, g.nq_blk, g.bs, D), o_out, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def _fused_fp8(q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance, ctx, sorted_lists):
    """e4m3 Q/K tiles from the quantizing gathers, then one kernel that reads V and writes O in token order."""
    B, NH, _, D = q.shape
    dev = q.device
    _stage(events, "alloc_start")
    o_out = torch.empty_like(q)
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    q8, q_scale, q_pool = _q_fp8(q, g, B, NH, D, dev)
    kb = _k_side("fused_fp8", k_txt, v_txt, k_vis, v_vis, g, text_len, ctx, B, NH, D, dev, q.dtype)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = _select(select, q_pool, kb, text_len, g)
    _stage(events, "index_end")
    _stage(events, "attn_start")
    _core.bsa_forward_fp8_gather(q8.flatten(2, 3), q_scale, kb["k8"].flatten(2, 3), kb["k_scale"], v_vis, kb["vt"],
                                 g.num_txt_blk, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, indices, counts,
                                 1.0 / math.sqrt(D), o_out, balance=balance, sorted_lists=sorted_lists)
    _stage(events, "attn_end")
    _stage(events, "untile_start")
    _stage(events, "untile_end")
    return o_out if o_out.dtype == out_dtype else o_out.to(out_dtype)


def sparse_attention(q, k_txt, v_txt, k_vis, v_vis, latent_hw, tile, select, events=None, fused=True,
                     balance=False, qk_fp8=False, context=None, normalize_k_pool=False, sorted_lists=False):
    """One sparse-attention forward.

    q (B,H,Lq,D); k_txt/v_txt (B,H,N_txt,D) or None; k_vis/v_vis (B,H,Lk,D), any strides.
    ``select(q_pool, k_pool, text_len, grid_q, grid_k) -> (indices, counts)``.  ``sorted_lists``: every
    row ``select`` returns lists its text blocks before its visual blocks, as the block mask's ascending
    lists do; the token-order kernels then take their faster load path (a text block listed after a
    visual block would read as zeros, so leave it off for other selectors).
    ``events`` (dict or None) collects CUDA events per stage for profiling.
    ``fused`` (default) runs pools + one gather/attend/untile kernel where the
    shape allows it (D = 128, 128-token tiles, tw and W multiples of 4, a grid
    at least one tile high and wide, token views with unit d stride);
    otherwise, or with ``fused=False``, the tiled sequence q_prep / kv_prep /
    attention / untile.  Both give the same bits.  ``balance`` (rows with their own budgets) starts
    the longest query tiles first.  ``qk_fp8`` takes Q K^T on e4m3 codes with one scale per tile
    block (bf16 only; D = 128 and 128-token tiles, ValueError otherwise); the selection is unchanged.
    ``context`` = (ContextCache, layer key, context frames) keeps the key-side preparation of the
    fixed leading frames and the text across calls (see ContextCache).  ``normalize_k_pool`` (``select``
    scores by cosine similarity): the fused bf16/f16 path's pool launch also writes the key pool's rows
    normalised, once per key block, and the block mask takes them instead of normalising every key row in
    every workgroup of query rows (same selection, bit for bit); ``select`` then receives it as the
    keyword argument ``k_pool_normalized``.
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
    args = (q, k_txt, v_txt, k_vis, v_vis, g, select, text_len, out_dtype, events, balance, context, sorted_lists)
    if qk_fp8:
        if dt != torch.bfloat16 or not fp8_supported(D, tile):
            raise ValueError(f"qk_fp8 is built for bfloat16, D = 128 and 128-token tiles (got {dt}, D = {D}, "
                             f"tile {tuple(tile)})")
        if fused and uses_fused(q, k_vis, v_vis, tile, (g.H, g.W)):
            return _fused_fp8(*args)
        return _tiled_fp8(*args)
    if fused and uses_fused(q, k_vis, v_vis, tile, (g.H, g.W)):
        return _fused(*args, k_norm=normalize_k_pool)
    _stage(events, "alloc_start")
    q_tiled = torch.empty((B, NH, g.nq_blk, g.bs, D), device=dev, dtype=dt)
    q_pool = torch.empty((B, NH, g.nq_blk, D), device=dev, dtype=dt)
    _stage(events, "alloc_end")
    _stage(events, "prep_start")
    _core.q_prep(q, q_tiled, q_pool, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    kb = _k_side("tiled", k_txt, v_txt, k_vis, v_vis, g, text_len, context, B, NH, D, dev, dt)
    _stage(events, "prep_end")
    _stage(events, "index_start")
    indices, counts = _select(select, q_pool, kb, text_len, g)
    _stage(events, "index_end")
    _stage(events, "attn_start")
    o_flat = _core.bsa_forward(q_tiled.flatten(2, 3), kb["k_all"].flatten(2, 3), kb["v_all"].flatten(2, 3), indices,
                               counts, 1.0 / math.sqrt(D), g.bs, balance=balance)
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
