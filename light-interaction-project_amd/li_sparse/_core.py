"""Torch-facing launchers: host-side validation, then one ``torch.ops.li`` operator each.

Every function validates shapes on the host with the reference's error
types and messages, then calls its custom operator (li_sparse/_ops.py, a C++
layer over the C ABI) which enqueues the HIP kernel on torch's current stream
of the tensors' device.  Nothing here synchronises the stream or computes on
the CPU.
"""
import math
import re

import numpy as np
import torch

from . import _lib
from ._ops import ops

_DTYPES = {torch.bfloat16: _lib.LI_DTYPE_BF16, torch.float16: _lib.LI_DTYPE_F16}
_STATUS = re.compile(r"(li_\w+) failed: .*\(status (-?\d+)\)")


def _run(op, *args):
    """Calls a torch.ops.li operator; a failed C-ABI status becomes LiError (with its status code)."""
    try:
        return op(*args)
    except RuntimeError as e:
        m = _STATUS.search(str(e))
        if m is None:
            raise
        raise _lib.LiError(m.group(1), int(m.group(2))) from None
METRICS = {"cosine": _lib.LI_METRIC_COSINE, "scaled_dot_product": _lib.LI_METRIC_SCALED_DOT}


def dtype_code(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected bfloat16 or float16") from None


def _device_check(*ts):
    dev = ts[0].device
    if dev.type != "cuda":
        raise ValueError("sparse attention tensors must be on a ROCm (cuda) device")
    for t in ts[1:]:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _same_dtype(*ts):
    for t in ts[1:]:
        if t.dtype != ts[0].dtype:
            raise TypeError(f"dtype mismatch: {ts[0].dtype} vs {t.dtype}")


def ceil_div(a, b):
    return (a + b - 1) // b


def num_blocks(T, tt, nh, nw):
    return ceil_div(T, tt) * nh * nw


def q_prep(src, dst, mean, T, H, W, tt, th, tw, nh, nw):
    """Tile gather + mean pool of one tensor (see li_q_prep)."""
    _device_check(src, dst, mean)
    _same_dtype(src, dst, mean)
    B, NH, L, D = src.shape
    nblk, bs = num_blocks(T, tt, nh, nw), tt * th * tw
    if L < T * H * W:
        raise ValueError(f"source length {L} < T*H*W = {T * H * W}")
    if dst.shape[:2] != (B, NH) or dst.shape[2] < nblk or dst.shape[3:] != (bs, D):
        raise ValueError(f"tile buffer shape {tuple(dst.shape)} does not hold {nblk} tiles of ({bs}, {D})")
    if tuple(mean.shape[:2]) != (B, NH) or mean.shape[2] < nblk or mean.shape[3] != D:
        raise ValueError(f"pool buffer shape {tuple(mean.shape)} does not hold {nblk} rows of {D}")
    dtype_code(src)
    _run(ops.q_prep, src, dst, mean, [T, H, W, tt, th, tw, nh, nw])


def kv_prep(k_src, v_src, k_dst, v_dst, k_mean, dst_off, pool_off, T, H, W, tt, th, tw, nh, nw):
    """Tile gather of K and V (at block offset dst_off) + K mean pool (at pool_off) (see li_kv_prep)."""
    _device_check(k_src, v_src, k_dst, v_dst, k_mean)
    _same_dtype(k_src, v_src, k_dst, v_dst, k_mean)
    B, NH, L, D = k_src.shape
    if tuple(v_src.shape) != tuple(k_src.shape):
        raise ValueError(f"K/V source shapes differ: {tuple(k_src.shape)} vs {tuple(v_src.shape)}")
    nblk, bs = num_blocks(T, tt, nh, nw), tt * th * tw
    if L < T * H * W:
        raise ValueError(f"source length {L} < T*H*W = {T * H * W}")
    for name, t in (("k_dst", k_dst), ("v_dst", v_dst)):
        if t.shape[:2] != (B, NH) or t.shape[2] < nblk + dst_off or t.shape[3:] != (bs, D):
            raise ValueError(f"{name} shape {tuple(t.shape)} does not hold {nblk}+{dst_off} tiles of ({bs}, {D})")
    if tuple(k_mean.shape[:2]) != (B, NH) or k_mean.shape[2] < nblk + pool_off or k_mean.shape[3] != D:
        raise ValueError(f"pool buffer shape {tuple(k_mean.shape)} does not hold {nblk}+{pool_off} rows")
    dtype_code(k_src)
    _run(ops.kv_prep, k_src, v_src, k_dst, v_dst, k_mean, int(dst_off), int(pool_off),
         [T, H, W, tt, th, tw, nh, nw])


FP8 = torch.float8_e4m3fn


def _fp8_tiles_check(name, t, B, NH, nblk, bs, D):
    if t.dtype != FP8:
        raise TypeError(f"{name} must be float8_e4m3fn, got {t.dtype}")
    if t.dim() != 5 or tuple(t.shape[:2]) != (B, NH) or t.shape[2] < nblk or tuple(t.shape[3:]) != (bs, D):
        raise ValueError(f"{name} shape {tuple(t.shape)} does not hold {nblk} tiles of ({bs}, {D})")


def _scale_check(name, t, B, NH, nblk):
    if t.dtype != torch.float32 or t.dim() != 3 or tuple(t.shape[:2]) != (B, NH) or t.shape[2] < nblk:
        raise ValueError(f"{name} must be float32 (B, NH, >= {nblk}), got {t.dtype} {tuple(t.shape)}")


def tile_prep_fp8(src, dst, scales, mean, dst_off, pool_off, T, H, W, tt, th, tw, nh, nw):
    """Tile gather into e4m3 codes with one fp32 scale per block (+ optional mean pool) (see li_tile_prep_fp8).

    dst (B, NH, nblk, BS, D) float8_e4m3fn and scales (B, NH, nblk) float32, written at block blk + dst_off;
    mean (or None) as q_prep's pool, at block blk + pool_off.
    """
    _device_check(src, dst, scales, *([mean] if mean is not None else []))
    B, NH, L, D = src.shape
    dtype_code(src)
    nblk, bs = num_blocks(T, tt, nh, nw), tt * th * tw
    if L < T * H * W:
        raise ValueError(f"source length {L} < T*H*W = {T * H * W}")
    _fp8_tiles_check("dst", dst, B, NH, nblk + dst_off, bs, D)
    _scale_check("scales", scales, B, NH, nblk + dst_off)
    if mean is not None:
        _same_dtype(src, mean)
        if tuple(mean.shape[:2]) != (B, NH) or mean.shape[2] < nblk + pool_off or mean.shape[3] != D:
            raise ValueError(f"pool buffer shape {tuple(mean.shape)} does not hold {nblk}+{pool_off} rows of {D}")
    _run(ops.tile_prep_fp8, src, dst, scales, mean, int(dst_off), int(pool_off), [T, H, W, tt, th, tw, nh, nw])


def kv_prep_fp8(k_src, v_src, k_dst, k_scales, v_dst, k_mean, dst_off, pool_off, T, H, W, tt, th, tw, nh, nw):
    """kv_prep with K written as e4m3 codes + per-block scales and V copied unchanged (see li_kv_prep_fp8)."""
    _device_check(k_src, v_src, k_dst, k_scales, v_dst, k_mean)
    _same_dtype(k_src, v_src, v_dst, k_mean)
    B, NH, L, D = k_src.shape
    if tuple(v_src.shape) != tuple(k_src.shape):
        raise ValueError(f"K/V source shapes differ: {tuple(k_src.shape)} vs {tuple(v_src.shape)}")
    nblk, bs = num_blocks(T, tt, nh, nw), tt * th * tw
    if L < T * H * W:
        raise ValueError(f"source length {L} < T*H*W = {T * H * W}")
    _fp8_tiles_check("k_dst", k_dst, B, NH, nblk + dst_off, bs, D)
    _scale_check("k_scales", k_scales, B, NH, nblk + dst_off)
    if v_dst.shape[:2] != (B, NH) or v_dst.shape[2] < nblk + dst_off or v_dst.shape[3:] != (bs, D):
        raise ValueError(f"v_dst shape {tuple(v_dst.shape)} does not hold {nblk}+{dst_off} tiles of ({bs}, {D})")
    if tuple(k_mean.shape[:2]) != (B, NH) or k_mean.shape[2] < nblk + pool_off or k_mean.shape[3] != D:
        raise ValueError(f"pool buffer shape {tuple(k_mean.shape)} does not hold {nblk}+{pool_off} rows")
    dtype_code(k_src)
    _run(ops.kv_prep_fp8, k_src, v_src, k_dst, k_scales, v_dst, k_mean, int(dst_off), int(pool_off),
                    [T, H, W, tt, th, tw, nh, nw])


def pool(src, mean, pool_off, T, H, W, tt, th, tw, nh, nw):
    """Tile mean pool without writing tiles (see li_pool); same values as q_prep / kv_prep."""
    _device_check(src, mean)
    _same_dtype(src, mean)
    B, NH, L, D = src.shape
    nblk = num_blocks(T, tt, nh, nw)
    if L < T * H * W:
        raise ValueError(f"source length {L} < T*H*W = {T * H * W}")
    if tuple(mean.shape[:2]) != (B, NH) or mean.shape[2] < nblk + pool_off or mean.shape[3] != D:
        raise ValueError(f"pool buffer shape {tuple(mean.shape)} does not hold {nblk}+{pool_off} rows of {D}")
    dtype_code(src)
    _run(ops.pool, src, mean, int(pool_off), [T, H, W, tt, th, tw, nh, nw])


def pool_pair(src0, mean0, pool_off0, geom0, src1, mean1, pool_off1, geom1, mean1_normalized=None):
    """Two pools (see li_pool_pair) in one launch; geom = (T, H, W, tt, th, tw, nh, nw) of each job.

    Same values, bit for bit, as ``pool`` on each job.  ``mean1_normalized`` (optional, the shape and
    strides of ``mean1``) also receives job 1's rows normalised as the cosine block mask normalises a
    key pool row.
    """
    _device_check(src0, mean0, src1, mean1)
    _same_dtype(src0, mean0, src1, mean1)
    if mean1_normalized is not None:
        _device_check(mean1, mean1_normalized)
        _same_dtype(mean1, mean1_normalized)
        if mean1_normalized.shape != mean1.shape or mean1_normalized.stride() != mean1.stride():
            raise ValueError("mean1_normalized must have the shape and strides of mean1")
    B, NH, _, D = src0.shape
    if tuple(src1.shape[:2]) != (B, NH) or src1.shape[3] != D:
        raise ValueError(f"pool pair sources {tuple(src0.shape)} and {tuple(src1.shape)} differ in B, NH or D")
    gs = []
    for src, mean, off, geo in ((src0, mean0, pool_off0, geom0), (src1, mean1, pool_off1, geom1)):
        T, H, W, tt, th, tw, nh, nw = geo
        nblk = num_blocks(T, tt, nh, nw)
        if src.shape[2] < T * H * W:
            raise ValueError(f"source length {src.shape[2]} < T*H*W = {T * H * W}")
        if tuple(mean.shape[:2]) != (B, NH) or mean.shape[2] < nblk + off or mean.shape[3] != D:
            raise ValueError(f"pool buffer shape {tuple(mean.shape)} does not hold {nblk}+{off} rows of {D}")
        gs.append([int(x) for x in geo])
    dtype_code(src0)
    _run(ops.pool_pair, src0, mean0, int(pool_off0), gs[0], src1, mean1, int(pool_off1), gs[1], mean1_normalized)


def fused_supported(D, tile, latent_hw):
    """Whether li_bsa_fwd_gather covers this shape.

    D = 128, 128-token tiles, tw and W multiples of 4, and a latent grid at
    least one tile high and wide (H >= th, W >= tw).
    """
    tt, th, tw = tile
    H, W = latent_hw
    return D == 128 and tt * th * tw == 128 and tw % 4 == 0 and W % 4 == 0 and H >= th and W >= tw


def bsa_forward_gather(q, k, v, k_txt, v_txt, num_txt_blk, T_q, T_k, H, W, tt, th, tw, nh, nw, indices, counts,
                       sm_scale, out, return_lse=False, split=True, balance=False, sorted_lists=False):
    """Block-sparse attention reading Q/K/V in token order and writing ``out`` in token order (li_bsa_fwd_gather).

    q/out (B,NH,Lq,D) and k/v (B,NH,Lk,D) views with any strides the kernel accepts; k_txt/v_txt the
    zero-padded (B,NH,num_txt_blk*BS,D) contiguous text keys/values or None.  ``split`` and ``balance``
    as for ``bsa_forward``.  ``sorted_lists`` (LI_BSA_SORTED): every row lists its text blocks before its
    visual blocks, as the block mask's ascending lists do, which lets the kernel take its faster load path
    (same results; a text block listed after a visual block would read as zeros).  No host sync.
    """
    _device_check(q, k, v, out, indices, counts)
    _same_dtype(q, k, v, out)
    B, NH, Lq, D = q.shape
    if indices.dtype != torch.int32 or counts.dtype != torch.int32:
        raise TypeError("block indices and counts must be int32")
    nq = num_blocks(T_q, tt, nh, nw)
    if indices.dim() != 4 or tuple(indices.shape[:2]) != (B, NH) or indices.shape[2] < nq:
        raise ValueError(f"block_indices shape {tuple(indices.shape)} does not cover {nq} query tiles")
    if counts.dim() != 3 or tuple(counts.shape[:2]) != (B, NH) or counts.shape[2] < nq:
        raise ValueError(f"block_counts shape {tuple(counts.shape)} does not cover {nq} query tiles")
    if Lq < T_q * H * W or k.shape[2] < T_k * H * W or tuple(out.shape) != tuple(q.shape):
        raise ValueError("token tensors do not hold the grids")
    if num_txt_blk > 0:
        _same_dtype(q, k_txt, v_txt)
        if not (k_txt.is_contiguous() and v_txt.is_contiguous()):
            raise ValueError("padded text K/V must be contiguous")
        want = (B, NH, num_txt_blk * tt * th * tw, D)
        if tuple(k_txt.shape) != want or tuple(v_txt.shape) != want:
            raise ValueError(f"padded text K/V must be {want}, got {tuple(k_txt.shape)} / {tuple(v_txt.shape)}")
    dtype_code(q)
    lse = _run(ops.bsa_fwd_gather, q, k, v, k_txt if num_txt_blk > 0 else None,
               v_txt if num_txt_blk > 0 else None, int(num_txt_blk), [T_q, H, W, tt, th, tw, nh, nw],
               [T_k, H, W, tt, th, tw, nh, nw], indices, counts, float(sm_scale), out, bool(return_lse), bool(split),
               bool(balance), bool(sorted_lists))
    return (out, lse) if return_lse else out


def untile(src, dst, T, H, W, tt, th, tw, nh, nw):
    """Inverse scatter of tiles into the linear token layout (see li_untile)."""
    _device_check(src, dst)
    _same_dtype(src, dst)
    B, NH, L, D = dst.shape
    nblk, bs = num_blocks(T, tt, nh, nw), tt * th * tw
    if L < T * H * W:
        raise ValueError(f"destination length {L} < T*H*W = {T * H * W}")
    if src.shape[:2] != (B, NH) or src.shape[2] < nblk or src.shape[3:] != (bs, D):
        raise ValueError(f"tile buffer shape {tuple(src.shape)} does not hold {nblk} tiles of ({bs}, {D})")
    dtype_code(src)
    _run(ops.untile, src, dst, [T, H, W, tt, th, tw, nh, nw])


# ----------------------------------------------------------------------------
# Block-mask budgets (host side: the forced set and the budget depend only on
# the block geometry and the parameters, so the row length is known without
# reading any device data).
# ----------------------------------------------------------------------------
def forced_counts(nq, nk, nh, nw, n_recent=0, diag=False, sink=False, neighbors=False):
    """Number of forced key blocks for every query row (same rules as the mask kernel)."""
    return forced_blocks(nq, nk, nh, nw, n_recent, diag, sink, neighbors).sum(axis=1)


def forced_blocks(nq, nk, nh, nw, n_recent=0, diag=False, sink=False, neighbors=False):
    """Boolean (nq, nk) forced-block mask (same rules as the mask kernel)."""
    qb = np.arange(nq)
    pos = nk - nq + qb
    j = np.arange(nk)
    f = np.zeros((nq, nk), dtype=bool)
    if n_recent > 0:
        f[:, j >= nk - n_recent] = True
    if diag:
        f |= j[None, :] == pos[:, None]
    if sink:
        f |= j[None, :] == (qb % (nh * nw))[:, None]
    if neighbors:
        hw = nh * nw
        ok = (pos >= 0) & (pos < nk)
        p = np.where(ok, pos, 0)
        dist = (np.abs(p[:, None] // hw - j[None, :] // hw) + np.abs((p[:, None] % hw) // nw - (j[None, :] % hw) // nw)
                + np.abs(p[:, None] % nw - j[None, :] % nw))
        f |= (dist <= 1) & ok[:, None]
    return f


def row_budgets(nf, nk, mode, ratio, min_budget=7, row_budget=None):
    """Visual blocks kept per row (forced included), the same arithmetic as the mask kernel."""
    nf = np.asarray(nf, dtype=np.int64)
    if row_budget is not None:
        k = np.asarray(row_budget, dtype=np.int64)
        return np.minimum(np.maximum(k, nf), nk)
    out = np.empty_like(nf)
    for i, f in enumerate(nf.tolist()):
        if mode == _lib.LI_BUDGET_HISTORY:
            k = f + int((nk - f) * ratio)
            k = min(max(k, 1 if nk > 0 else 0), nk)
        else:
            k = min(max(int(nk * ratio), min_budget), nk)
        out[i] = max(k, f)
    return out


def tie_free_fraction(scores, counts, forced, num_txt_blk=0, margin=2):
    """Fraction of rows whose selection does not depend on score ties.

    ``scores`` (..., nq, nk) bf16/f16 block scores as ``block_mask`` returns them, ``counts`` (..., nq) the row
    lengths, ``forced`` the (nq, nk) forced-block mask.  A row is tie-free when its k-th and (k+1)-th largest
    non-forced scores are at least ``margin`` ulps apart (or it keeps all or none of them): then any summation order
    within an ulp selects the same blocks.
    """
    b = scores.detach().cpu().contiguous().view(torch.int16).numpy().astype(np.int32) & 0xFFFF
    key = np.where(b & 0x8000, -(b & 0x7FFF) - 1, b)  # monotone in the value
    nq, nk = key.shape[-2:]
    key = key.reshape(-1, nq, nk)
    cnt = counts.detach().cpu().numpy().reshape(-1, nq) - num_txt_blk
    nf = forced.sum(axis=1)
    free = ~forced
    ok = total = 0
    for r in range(key.shape[0]):
        for q in range(nq):
            kk = int(cnt[r, q]) - int(nf[q])
            vals = np.sort(key[r, q][free[q]])[::-1]
            total += 1
            ok += not (0 < kk < vals.size) or int(vals[kk - 1]) - int(vals[kk]) >= margin
    return ok / max(total, 1)


_MASK_PLANS = {}


def _mask_plan(dev, nq, nk, nh, nw, num_txt_blk, n_recent, force_diag, force_sink, force_neighbors, budget_mode,
               ratio, min_budget, row_budget):
    """Row length and device copy of explicit row budgets for one mask configuration.

    Both depend only on the configuration, so they are worked out once per configuration and device (the
    decode and prefill calls repeat the same one every layer and step), which also keeps the host-to-device
    copy of the budgets out of the steady state.
    """
    rb = None if row_budget is None else tuple(int(x) for x in np.asarray(row_budget).reshape(-1))
    key = (str(dev), nq, nk, nh, nw, num_txt_blk, n_recent, force_diag, force_sink, force_neighbors, budget_mode,
           ratio, min_budget, rb)
    plan = _MASK_PLANS.get(key)
    if plan is not None:
        return plan
    nf = forced_counts(nq, nk, nh, nw, n_recent, force_diag, force_sink, force_neighbors)
    rb_dev = None
    if rb is not None:
        if len(rb) != nq:
            raise ValueError(f"row_budget has {len(rb)} entries for {nq} query blocks")
        rb_dev = torch.tensor(rb, dtype=torch.int32, device=dev)
        k = row_budgets(nf, nk, budget_mode, ratio, min_budget, np.asarray(rb, dtype=np.int64))
    else:
        k = row_budgets(nf, nk, budget_mode, ratio, min_budget)
    plan = (int(num_txt_blk + (k.max() if nq > 0 else 0)), rb_dev)
    if len(_MASK_PLANS) >= 64:
        _MASK_PLANS.clear()
    _MASK_PLANS[key] = plan
    return plan


def block_mask(q_pool, k_pool, *, metric, budget_mode, ratio, nh, nw, num_txt_blk=0, n_recent=0,
               force_diag=False, force_sink=False, force_neighbors=False, min_budget=7, row_budget=None,
               return_scores=False, k_pool_normalized=None):
    """Block selection on the device (see li_block_mask).

    Returns ``(indices (B,H,nq,kmax) int32, counts (B,H,nq) int32)`` (+ scores if asked), where
    ``kmax = num_txt_blk + max row budget``.  ``k_pool_normalized``: ``k_pool`` with every row normalised
    for the cosine metric, as ``pool_pair``'s ``mean1_normalized`` writes it in the same launch as the
    pool; with ``metric="cosine"`` the mask scores against it instead of normalising every key row once
    per workgroup of query rows (same bits).  Other metrics ignore it.  The caller keeps the two in step.
    """
    dev = _device_check(q_pool, k_pool)
    _same_dtype(q_pool, k_pool)
    B, NH, nq, D = q_pool.shape
    nk = k_pool.shape[2]
    if tuple(k_pool.shape[:2]) != (B, NH) or k_pool.shape[3] != D:
        raise ValueError(f"pool shapes differ: {tuple(q_pool.shape)} vs {tuple(k_pool.shape)}")
    metric_code = METRICS.get(metric, _lib.LI_METRIC_DOT)
    kmax, rb_dev = _mask_plan(dev, nq, nk, nh, nw, num_txt_blk, n_recent, bool(force_diag), bool(force_sink),
                              bool(force_neighbors), budget_mode, float(ratio), int(min_budget), row_budget)
    dtype_code(q_pool)
    k_norm = k_pool_normalized if metric_code == _lib.LI_METRIC_COSINE else None
    if k_norm is not None:
        if k_norm.shape != k_pool.shape or k_norm.dtype != k_pool.dtype or k_norm.device != k_pool.device:
            raise ValueError("the normalised key pool does not match the key pool")
        k_pool = k_norm
    indices, counts, scores = _run(ops.block_mask, q_pool, k_pool, metric_code, int(budget_mode), float(ratio),
                                             int(min_budget), int(n_recent), bool(force_diag), bool(force_sink),
                                             bool(force_neighbors), int(nh), int(nw), int(num_txt_blk), int(kmax),
                                             rb_dev, bool(return_scores), k_norm is not None)
    if return_scores:
        return indices, counts, scores
    return indices, counts


def bsa_forward(q, k, v, indices, counts, sm_scale, block_size, return_lse=False, out=None, split=True,
                balance=False):
    """Block-sparse attention over contiguous (B,H,L,D) tensors (see li_bsa_fwd); no host sync.

    ``split=False`` runs every query tile whole (no tail split workspace).  ``balance=True`` (rows of
    unequal length) starts the query tiles longest first instead (LI_BSA_BALANCE; no tail split).
    """
    _device_check(q, k, v, indices, counts)
    _same_dtype(q, k, v)
    if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
        raise ValueError("q, k, v must be contiguous")
    B, NH, Lq, D = q.shape
    Lk = k.shape[2]
    if tuple(k.shape) != (B, NH, Lk, D) or tuple(v.shape) != (B, NH, Lk, D):
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    if indices.dtype != torch.int32 or counts.dtype != torch.int32:
        raise TypeError("block indices and counts must be int32")
    nqt = ceil_div(Lq, block_size)
    if indices.dim() != 4 or tuple(indices.shape[:2]) != (B, NH) or indices.shape[2] < nqt:
        raise ValueError(f"block_indices shape {tuple(indices.shape)} does not cover {nqt} query tiles")
    if counts.dim() != 3 or tuple(counts.shape[:2]) != (B, NH) or counts.shape[2] < nqt:
        raise ValueError(f"block_counts shape {tuple(counts.shape)} does not cover {nqt} query tiles")
    if Lk % block_size != 0:
        raise ValueError(f"K Length ({Lk}) must be divisible by logical_block_size ({block_size})")
    dtype_code(q)
    if out is None:
        out = torch.empty_like(q)
    # The operator allocates the workspace for splitting the query tiles of a
    # partial last round (or for the balanced tile order) through torch's
    # caching allocator; stream-ordered, so it is freed on return.
    lse = _run(ops.bsa_fwd, q, k, v, indices, counts, float(sm_scale), int(block_size), out, bool(return_lse),
               bool(split), bool(balance))
    return (out, lse) if return_lse else out


def bsa_forward_fp8(q8, q_scale, k8, k_scale, v, indices, counts, sm_scale, block_size=128, return_lse=False,
                    out=None, split=True, balance=False):
    """Block-sparse attention with e4m3 Q/K and per-block scales, bf16 V and output (see li_bsa_fwd_fp8).

    q8 (B,H,Lq,D) / k8 (B,H,Lk,D) float8_e4m3fn, contiguous; q_scale (B,H,ceil(Lq/128)) and
    k_scale (B,H,Lk/128) float32; v (B,H,Lk,D) bfloat16.  ``split`` / ``balance`` as for bsa_forward.
    """
    dev = _device_check(q8, q_scale, k8, k_scale, v, indices, counts)
    if q8.dtype != FP8 or k8.dtype != FP8:
        raise TypeError("q8 and k8 must be float8_e4m3fn")
    if v.dtype != torch.bfloat16:
        raise TypeError(f"v must be bfloat16, got {v.dtype}")
    if not (q8.is_contiguous() and k8.is_contiguous() and v.is_contiguous() and q_scale.is_contiguous()
            and k_scale.is_contiguous()):
        raise ValueError("q8, k8, v and the scales must be contiguous")
    B, NH, Lq, D = q8.shape
    Lk = k8.shape[2]
    if tuple(k8.shape) != (B, NH, Lk, D) or tuple(v.shape) != (B, NH, Lk, D):
        raise ValueError(f"shape mismatch q {tuple(q8.shape)} k {tuple(k8.shape)} v {tuple(v.shape)}")
    nqt = ceil_div(Lq, block_size)
    if tuple(q_scale.shape) != (B, NH, nqt) or q_scale.dtype != torch.float32:
        raise ValueError(f"q_scale must be float32 {(B, NH, nqt)}, got {q_scale.dtype} {tuple(q_scale.shape)}")
    if Lk % block_size == 0 and (tuple(k_scale.shape) != (B, NH, Lk // block_size) or k_scale.dtype != torch.float32):
        raise ValueError(f"k_scale must be float32 {(B, NH, Lk // block_size)}, got {tuple(k_scale.shape)}")
    if indices.dtype != torch.int32 or counts.dtype != torch.int32:
        raise TypeError("block indices and counts must be int32")
    if indices.dim() != 4 or tuple(indices.shape[:2]) != (B, NH) or indices.shape[2] < nqt:
        raise ValueError(f"block_indices shape {tuple(indices.shape)} does not cover {nqt} query tiles")
    if counts.dim() != 3 or tuple(counts.shape[:2]) != (B, NH) or counts.shape[2] < nqt:
        raise ValueError(f"block_counts shape {tuple(counts.shape)} does not cover {nqt} query tiles")
    if Lk % block_size != 0:
        raise ValueError(f"K Length ({Lk}) must be divisible by logical_block_size ({block_size})")
    if out is None:
        out = torch.empty((B, NH, Lq, D), dtype=torch.bfloat16, device=dev)
    lse = _run(ops.bsa_fwd_fp8, q8, q_scale, k8, k_scale, v, indices, counts, float(sm_scale), int(block_size),
               out, bool(return_lse), bool(split), bool(balance))
    return (out, lse) if return_lse else out


def bsa_forward_fp8_gather(q8, q_scale, k8, k_scale, v, v_txt, num_txt_blk, T_q, T_k, H, W, tt, th, tw, nh, nw,
                           indices, counts, sm_scale, out, return_lse=False, balance=False, sorted_lists=False):
    """e4m3 attention with V read and O written in token order (see li_bsa_fwd_fp8_gather).

    q8 (B,NH,nq_blk*128,D) / k8 (B,NH,(num_txt_blk+nk_blk)*128,D) e4m3 tiles with their (B,NH,nblk) scales;
    v (B,NH,Lk,D) bf16 token view; v_txt (B,NH,num_txt_blk*128,D) contiguous zero-padded or None;
    out (B,NH,Lq,D) bf16 token view, written at valid tokens.  ``sorted_lists`` as for bsa_forward_gather.
    """
    _device_check(q8, q_scale, k8, k_scale, v, indices, counts, out)
    if q8.dtype != FP8 or k8.dtype != FP8 or v.dtype != torch.bfloat16 or out.dtype != torch.bfloat16:
        raise TypeError("q8/k8 must be float8_e4m3fn, v and out bfloat16")
    if not (q8.is_contiguous() and k8.is_contiguous() and q_scale.is_contiguous() and k_scale.is_contiguous()):
        raise ValueError("the e4m3 tiles and scales must be contiguous")
    B, NH, _, D = v.shape
    nq, nk = num_blocks(T_q, tt, nh, nw), num_blocks(T_k, tt, nh, nw)
    if tuple(q8.shape) != (B, NH, nq * 128, D) or tuple(q_scale.shape) != (B, NH, nq):
        raise ValueError(f"q8 {tuple(q8.shape)} / q_scale {tuple(q_scale.shape)} do not hold {nq} tiles")
    nkb = num_txt_blk + nk
    if tuple(k8.shape) != (B, NH, nkb * 128, D) or tuple(k_scale.shape) != (B, NH, nkb):
        raise ValueError(f"k8 {tuple(k8.shape)} / k_scale {tuple(k_scale.shape)} do not hold {nkb} blocks")
    if indices.dtype != torch.int32 or counts.dtype != torch.int32:
        raise TypeError("block indices and counts must be int32")
    if num_txt_blk > 0 and (v_txt is None or not v_txt.is_contiguous()
                            or tuple(v_txt.shape) != (B, NH, num_txt_blk * 128, D)):
        raise ValueError("v_txt must be a contiguous (B, NH, num_txt_blk*128, D) buffer")
    lse = _run(ops.bsa_fwd_fp8_gather, q8, q_scale, k8, k_scale, v, v_txt if num_txt_blk > 0 else None,
               int(num_txt_blk), [T_q, H, W, tt, th, tw, nh, nw], [T_k, H, W, tt, th, tw, nh, nw], indices, counts,
               float(sm_scale), out, bool(return_lse), bool(balance), bool(sorted_lists))
    return (out, lse) if return_lse else out


def dense_supported(q, k, v, k_txt=None):
    """Inputs li_attn_fwd_dense takes: fp16/bf16, D = 128, Lk a multiple of 4, token views with unit d stride,
    8-element-multiple strides, 16-byte aligned, K/V token strides >= D."""
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype or q.shape[3] != 128:
        return False
    if k_txt is not None and k_txt.dtype != q.dtype:
        return False
    if k.shape[2] % 4 != 0:
        return False
    for t in ((q, k, v) if k.shape[2] > 0 else (q,)):
        st = t.stride()
        if st[3] != 1 or any(x % 8 for x in st[:3]) or st[2] < t.shape[3] or t.data_ptr() % 16:
            return False
    return True


def attn_dense(q, k, v, k_txt=None, v_txt=None, sm_scale=None, return_lse=False, out=None, split=True):
    """Dense attention over [text keys, visual keys] without forming the concatenation (see li_attn_fwd_dense).

    q (B,H,Lq,128), k/v (B,H,Lk,128) token views; k_txt/v_txt (B,H,N_txt,128) or None.  Output has q's strides
    (``empty_like(q)``).  Raises LiError(LI_ERR_UNSUPPORTED) for shapes it is not built for.
    """
    _device_check(q, k, v)
    _same_dtype(q, k, v)
    B, NH, Lq, D = q.shape
    Lk = k.shape[2]
    if tuple(k.shape) != (B, NH, Lk, D) or tuple(v.shape) != (B, NH, Lk, D):
        raise ValueError(f"shape mismatch q {tuple(q.shape)} k {tuple(k.shape)} v {tuple(v.shape)}")
    txt_len = 0 if k_txt is None else k_txt.shape[2]
    kt = vt = None
    if txt_len > 0:
        _device_check(q, k_txt, v_txt)
        _same_dtype(q, k_txt, v_txt)
        if tuple(k_txt.shape) != (B, NH, txt_len, D) or tuple(v_txt.shape) != (B, NH, txt_len, D):
            raise ValueError(f"text K/V shapes {tuple(k_txt.shape)} / {tuple(v_txt.shape)} do not match q")
        pad = (-txt_len) % 128
        kt = (torch.nn.functional.pad(k_txt, (0, 0, 0, pad)) if pad else k_txt).contiguous()
        vt = (torch.nn.functional.pad(v_txt, (0, 0, 0, pad)) if pad else v_txt).contiguous()
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty_like(q)
    dtype_code(q)
    lse = _run(ops.attn_dense, q, k, v, kt, vt, int(txt_len), float(sm_scale), out, bool(return_lse), bool(split))
    return (out, lse) if return_lse else out
