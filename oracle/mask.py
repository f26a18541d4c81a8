"""Block-mask selection (oracle, test infrastructure only).

Restates the reference index builders:

* ``fast_generate_indices`` (AR decode), ar_sparse_operation.py:223-284;
* ``generate_prefill_indices`` (prefill / bidirectional),
  bi_sparse_operation_for_KV_cache.py:220-296 and bi_sparse_operation.py:179-234;

plus the build-defined forced-block extension (``force_diag``/``force_sink``)
and the explicit per-row budget used for ragged rows; both reduce exactly to
the reference rules when unset.

Rounding model (the reference computes these with bf16 torch ops):

* cosine: ``xn = bf16(x / max(bf16(sqrt(sum x^2)), bf16(1e-12)))`` per pooled
  row (``F.normalize``, ar_sparse_operation.py:252), then
  ``sim = bf16(sum_d qn*kn)``;
* scaled_dot_product: ``sim = bf16(f32(bf16(sum_d q*k)) * f32(1/sqrt(d)))``
  (ar_sparse_operation.py:254, bi_sparse_operation_for_KV_cache.py:258-260);
* dot: ``sim = bf16(sum_d q*k)`` (ar_sparse_operation.py:256).

Sums over d are in fp32 with bf16*bf16 products exact in fp32 (so fused and
unfused multiply-add agree).  A dot product takes eight partial sums, partial
i over d = i, i+8, i+16, ... sequentially from +0.0, combined as
((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)); a sum of squares (the normaliser) is
sequential from +0.0 in increasing d.

float16 pools (``fmt="f16"``) follow the same model with every bf16 rounding
replaced by an IEEE half rounding (the reference's ops then run in float16);
the normaliser's floor becomes f16(1e-12) = 0.  f16*f16 products are exact in
fp32 as well.  The
reference's own sum order (cuBLAS) is not observable; rows whose k-th and
(k+1)-th non-forced scores are at least two bf16 ulps apart ("tie-free") are
insensitive to it.

Forced blocks: the reference adds +1e6 to their scores
(ar_sparse_operation.py:266, bi_sparse_operation_for_KV_cache.py:280) so they
always win the top-k; here they are selected unconditionally and the
remaining ``k - n_forced`` slots go to the highest non-forced scores, ties to
the lower block index.  Output rows are ascending (``torch.sort`` of the top-k
indices, ar_sparse_operation.py:276), offset by ``num_txt_blk`` and prefixed
with the text blocks ``0..num_txt_blk-1`` (ar_sparse_operation.py:277-282).

Pinned by tests/test_oracle_mask.py: one-hot pooled similarities with a known
answer, ratio 1 -> every block and ratio 0 -> forced blocks only, brute-force
top-k on tiny rows, the reference's budget arithmetic (``int(n * ratio)``
truncation) on hand-computed cases, and an independent torch-CPU formulation
with the reference's own library calls (``F.normalize``, ``matmul``, ``topk``,
``sort``) that must select the same blocks on tie-free rows.
"""
import math

import numpy as np

from .bf16 import bf16_order_key, bf16_to_f32, f32_to_bf16

METRICS = ("cosine", "scaled_dot_product", "dot")


def f16_to_f32(bits):
    """uint16 IEEE half bit patterns -> float32 values (exact)."""
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16(x):
    """float32 -> uint16 IEEE half bit patterns, round to nearest even (numpy's cast)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


# element format -> (bits to float32, float32 to bits)
FORMATS = {"bf16": (bf16_to_f32, f32_to_bf16), "f16": (f16_to_f32, f32_to_f16)}


def _dot8(a, b):
    """fp32 dot over the last axis: a (..., M, D), b (..., N, D) -> (..., M, N), D a multiple of 8.

    Eight partial sums, partial i over d = i, i+8, ... sequentially from +0.0, then
    ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)): the order both mask kernels use.
    """
    D = a.shape[-1]
    assert D % 8 == 0, "the dot order is defined for D a multiple of 8"
    s = [np.zeros(a.shape[:-1] + (b.shape[-2],), dtype=np.float32) for _ in range(8)]
    for d in range(D):
        s[d % 8] = s[d % 8] + a[..., :, None, d] * b[..., None, :, d]
    return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]))


def _normalize_bits(x_bits, fmt="bf16"):
    """F.normalize(x, dim=-1) in the element format with fp32 internals (sequential sum of squares)."""
    to32, from32 = FORMATS[fmt]
    x = to32(x_bits)
    D = x.shape[-1]
    ss = np.zeros(x.shape[:-1], dtype=np.float32)
    for d in range(D):
        ss = ss + x[..., d] * x[..., d]
    nrm = to32(from32(np.sqrt(ss)))
    eps = to32(from32(np.float32(1e-12)))
    den = np.maximum(nrm, eps)
    with np.errstate(divide="ignore", invalid="ignore"):
        return from32(x / den[..., None])


def similarity(q_pool_bits, k_pool_bits, metric, fmt="bf16"):
    """Pooled block similarity (B,H,Nq,D) x (B,H,Nk,D) -> uint16 scores (B,H,Nq,Nk) in the element format."""
    to32, from32 = FORMATS[fmt]
    if metric == "cosine":
        qn, kn = _normalize_bits(q_pool_bits, fmt), _normalize_bits(k_pool_bits, fmt)
        return from32(_dot8(to32(qn), to32(kn)))
    dot = from32(_dot8(to32(q_pool_bits), to32(k_pool_bits)))
    if metric == "scaled_dot_product":
        d = q_pool_bits.shape[-1]
        scale = np.float32(1.0 / math.sqrt(d))
        return from32(to32(dot) * scale)
    return dot


def forced_mask(nq, nk, nh, nw, *, n_recent=0, diag=False, sink=False, neighbors=False):
    """Boolean (nq, nk) forced-block mask.

    * ``n_recent``: the last ``n_recent`` key blocks (ar_sparse_operation.py:263-266).
    * ``neighbors``: key blocks at 3D Manhattan distance <= 1 from the query's
      position in the key grid (bi_sparse_operation_for_KV_cache.py:268-280,
      where Nq == Nk and the query's position is its own index).
    * ``diag``: the key block at the query's position in the key grid.
    * ``sink``: the key block of t-slab 0 at the query block's (h, w).

    The query block ``qb`` sits at key-grid position ``nk - nq + qb`` (the query
    chunk is the trailing ``nq`` key blocks; equal to ``qb`` when nq == nk).
    """
    m = np.zeros((nq, nk), dtype=bool)
    qb = np.arange(nq)
    pos = nk - nq + qb
    if n_recent > 0:
        m[:, max(0, nk - n_recent):] = True
    if diag:
        ok = (pos >= 0) & (pos < nk)
        m[qb[ok], pos[ok]] = True
    if sink:
        s = qb % (nh * nw)
        ok = s < nk
        m[qb[ok], s[ok]] = True
    if neighbors:
        kidx = np.arange(nk)
        kt, kh, kw = kidx // (nh * nw), (kidx % (nh * nw)) // nw, kidx % nw
        ok = (pos >= 0) & (pos < nk)
        p = np.where(ok, pos, 0)
        pt, ph, pw = p // (nh * nw), (p % (nh * nw)) // nw, p % nw
        dist = (np.abs(pt[:, None] - kt[None, :]) + np.abs(ph[:, None] - kh[None, :])
                + np.abs(pw[:, None] - kw[None, :]))
        m |= (dist <= 1) & ok[:, None]
    return m


def budgets(forced, ratio, *, mode, min_budget=None, row_budget=None):
    """Visual blocks kept per query row (forced included), shape (nq,).

    * ``mode='history'`` (decode): ``nf + int((nk - nf) * ratio)`` clamped to
      ``[1 if nk > 0 else 0, nk]`` (ar_sparse_operation.py:268-272).
    * ``mode='total'`` (prefill): ``min(max(int(nk * ratio), min_budget), nk)``
      with ``min_budget = 7`` (bi_sparse_operation_for_KV_cache.py:282-285).
    * ``row_budget`` (ragged rows): explicit per-row totals clamped to ``[nf, nk]``.

    Every budget is raised to at least the row's forced count.
    """
    nq, nk = forced.shape
    nf = forced.sum(axis=1)
    if row_budget is not None:
        k = np.asarray(row_budget, dtype=np.int64).copy()
        k = np.minimum(np.maximum(k, nf), nk)
        return k
    if mode == "history":
        k = np.array([int(f) + int((nk - int(f)) * ratio) for f in nf], dtype=np.int64)
        k = np.minimum(np.maximum(k, 1 if nk > 0 else 0), nk)
    elif mode == "total":
        mb = 7 if min_budget is None else min_budget
        k = np.full(nq, min(max(int(nk * ratio), mb), nk), dtype=np.int64)
    else:
        raise ValueError(mode)
    return np.maximum(k, nf)


def select_rows(score_bits, forced, k):
    """Per-row selection -> list of ascending int arrays.

    score_bits (nq, nk) uint16 (bf16 or f16 patterns: both order as sign and
    magnitude); forced (nq, nk) bool; k (nq,) totals.
    Forced blocks always; then the top ``k - nf`` non-forced by score, ties to the lower index.
    """
    key = bf16_order_key(score_bits)
    nq, nk = score_bits.shape
    out = []
    idx = np.arange(nk)
    for r in range(nq):
        f = forced[r]
        free = idx[~f]
        order = np.lexsort((free, -key[r, free]))
        take = int(k[r]) - int(f.sum())
        sel = np.concatenate([idx[f], free[order[:max(take, 0)]]])
        out.append(np.sort(sel))
    return out


def tie_free(score_bits, forced, k, margin=2):
    """True for rows whose k-th and (k+1)-th largest non-forced scores are >= margin ulps apart (bf16 or f16)."""
    key = bf16_order_key(score_bits)
    nq = score_bits.shape[0]
    res = np.ones(nq, dtype=bool)
    for r in range(nq):
        free = np.sort(key[r, ~forced[r]])[::-1]
        take = int(k[r]) - int(forced[r].sum())
        if 0 < take < free.size:
            res[r] = (free[take - 1] - free[take]) >= margin
    return res


def assemble(rows_per_bh, num_txt_blk, kmax=None):
    """Lists of per-row selections, shape [B][H][nq] -> (indices int32 (B,H,nq,kmax), counts int32 (B,H,nq))."""
    B, H, nq = len(rows_per_bh), len(rows_per_bh[0]), len(rows_per_bh[0][0])
    width = max(len(r) for bh in rows_per_bh for hh in bh for r in hh) + num_txt_blk
    kmax = width if kmax is None else kmax
    ind = np.zeros((B, H, nq, kmax), dtype=np.int32)
    cnt = np.zeros((B, H, nq), dtype=np.int32)
    txt = np.arange(num_txt_blk, dtype=np.int32)
    for b in range(B):
        for h in range(H):
            for q in range(nq):
                row = np.concatenate([txt, rows_per_bh[b][h][q].astype(np.int32) + num_txt_blk])
                ind[b, h, q, :row.size] = row
                cnt[b, h, q] = row.size
    return ind, cnt


def build_indices(q_pool_bits, k_pool_bits, *, metric, forced, k, num_txt_blk, kmax=None, fmt="bf16"):
    """Full selection for all (b, h): returns (indices, counts, scores, tie_free_mask)."""
    score = similarity(q_pool_bits, k_pool_bits, metric, fmt)
    B, H = score.shape[:2]
    rows = [[select_rows(score[b, h], forced, k) for h in range(H)] for b in range(B)]
    ind, cnt = assemble(rows, num_txt_blk, kmax)
    tf = np.stack([np.stack([tie_free(score[b, h], forced, k) for h in range(H)]) for b in range(B)])
    return ind, cnt, score, tf


def fast_generate_indices(q_pool_bits, k_pool_bits, text_len, grid_thw_q, grid_thw_k, params):
    """AR-decode selection, ar_sparse_operation.py:223-284 (+ force_diag / force_sink / row_budget)."""
    tt, th, tw = params["tile_size"]
    bs = tt * th * tw
    nq, nk = q_pool_bits.shape[2], k_pool_bits.shape[2]
    nh, nw = grid_thw_q[1], grid_thw_q[2]
    rp = params.get("recent_protect", 0)
    n_prot = min(((rp + tt - 1) // tt) * nh * nw, nk) if rp > 0 else 0
    forced = forced_mask(nq, nk, nh, nw, n_recent=n_prot, diag=params.get("force_diag", False),
                         sink=params.get("force_sink", False))
    k = budgets(forced, params.get("topk_ratio", 1.0), mode="history", row_budget=params.get("row_budget"))
    num_txt_blk = (text_len + bs - 1) // bs
    ind, cnt, _, _ = build_indices(q_pool_bits, k_pool_bits, metric=params.get("sim_metric", "cosine"),
                                   forced=forced, k=k, num_txt_blk=num_txt_blk)
    return ind, cnt


def generate_prefill_indices(q_pool_bits, k_pool_bits, text_len, grid_thw, params, default_ratio=None):
    """Prefill selection, bi_sparse_operation_for_KV_cache.py:220-296 (HY: ratio required;
    MG default 0.25, bi_sparse_operation.py:221)."""
    tt, th, tw = params["tile_size"]
    bs = tt * th * tw
    nq, nk = q_pool_bits.shape[2], k_pool_bits.shape[2]
    _, nh, nw = grid_thw
    ratio = params["topk_ratio"] if default_ratio is None else params.get("topk_ratio", default_ratio)
    forced = forced_mask(nq, nk, nh, nw, neighbors=True, diag=params.get("force_diag", False),
                         sink=params.get("force_sink", False))
    k = budgets(forced, ratio, mode="total", row_budget=params.get("row_budget"))
    num_txt_blk = (text_len + bs - 1) // bs
    ind, cnt, _, _ = build_indices(q_pool_bits, k_pool_bits, metric=params.get("sim_metric", "cosine"),
                                   forced=forced, k=k, num_txt_blk=num_txt_blk)
    return ind, cnt
