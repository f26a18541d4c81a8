"""The reference's index builders written with the reference's own torch calls, on the CPU.

Follows ar_sparse_operation.py:245-284 (decode) and
bi_sparse_operation_for_KV_cache.py:252-296 (prefill) step by step:
``F.normalize`` / ``torch.matmul`` / scalar scale in bf16, ``+1e6`` bias,
``torch.topk``, ``torch.sort``, text prefix.  The forced-diag/sink extension
adds the same +1e6 bias.  This is an independent formulation used to pin the
oracle's rounding model (it shares no code with ``oracle/``); ``torch.topk``'s
tie order is unspecified, so results are compared on tie-free rows only.
"""
import math

import torch
import torch.nn.functional as F


def sim(q_pool, k_pool, metric):
    d = q_pool.shape[-1]
    if metric == "cosine":
        return torch.matmul(F.normalize(q_pool, dim=-1), F.normalize(k_pool, dim=-1).transpose(-2, -1))
    s = torch.matmul(q_pool, k_pool.transpose(-2, -1))
    if metric == "scaled_dot_product":
        s = s * (1.0 / math.sqrt(d))
    return s


def _extra_bias(score, nq, nk, nh, nw, params):
    qb = torch.arange(nq)
    if params.get("force_diag", False):
        pos = nk - nq + qb
        ok = (pos >= 0) & (pos < nk)
        score[..., qb[ok], pos[ok]] += 1e6
    if params.get("force_sink", False):
        s = qb % (nh * nw)
        ok = s < nk
        score[..., qb[ok], s[ok]] += 1e6
    return score


def decode_select(q_pool, k_pool, text_len, grid_thw_q, grid_thw_k, params):
    tt, th, tw = params["tile_size"]
    bs = tt * th * tw
    b, h, nq, d = q_pool.shape
    nk = k_pool.shape[2]
    s = sim(q_pool, k_pool, params.get("sim_metric", "cosine"))
    score = s.clone()
    n_prot = 0
    Nh, Nw = grid_thw_q[1], grid_thw_q[2]
    if params.get("recent_protect", 0) > 0:
        n_prot = min(((params["recent_protect"] + tt - 1) // tt) * Nh * Nw, nk)
        if n_prot > 0:
            score[..., -n_prot:] += 1e6
    score = _extra_bias(score, nq, nk, Nh, Nw, params)
    # forced blocks (recent slabs, and the diag/sink extension) count towards the budget like n_prot
    nf = ((score.float() - s.float()) > 1e5).sum(dim=-1)
    if nf.numel() and not bool((nf == nf.flatten()[0]).all()):
        raise NotImplementedError("rows with different forced counts need per-row budgets")
    n_forced = int(nf.flatten()[0]) if nf.numel() else n_prot
    n_hist = max(0, nk - n_forced)
    k = n_forced + int(n_hist * params.get("topk_ratio", 1.0))
    k = min(max(k, 1 if nk > 0 else 0), nk)
    _, idx = torch.topk(score, k=k, dim=-1)
    idx, _ = torch.sort(idx, dim=-1)
    ntxt = (text_len + bs - 1) // bs
    idx = idx + ntxt
    txt = torch.arange(ntxt, dtype=torch.int32).view(1, 1, 1, -1).expand(b, h, nq, -1)
    final = torch.cat([txt, idx.int()], dim=-1).contiguous()
    return final, s, score


def prefill_select(q_pool, k_pool, text_len, grid_thw, params):
    tt, th, tw = params["tile_size"]
    bs = tt * th * tw
    s = sim(q_pool, k_pool, params.get("sim_metric", "cosine"))
    B, H, N_q, N_k = s.shape
    Nt, Nh, Nw = grid_thw
    score = s.clone()
    idx_arr = torch.arange(N_k)
    t_idx, rem = idx_arr // (Nh * Nw), idx_arr % (Nh * Nw)
    h_idx, w_idx = rem // Nw, rem % Nw
    dist = ((t_idx[:, None] - t_idx[None, :]).abs() + (h_idx[:, None] - h_idx[None, :]).abs()
            + (w_idx[:, None] - w_idx[None, :]).abs())
    score = score + (dist <= 1).to(score.dtype) * 1e6
    score = _extra_bias(score, N_q, N_k, Nh, Nw, params)
    k = min(max(int(N_k * params["topk_ratio"]), 7), N_k)
    _, idx = torch.topk(score, k=k, dim=-1)
    idx, _ = torch.sort(idx, dim=-1)
    ntxt = (text_len + bs - 1) // bs
    txt = torch.arange(ntxt).view(1, 1, 1, -1).expand(B, H, N_q, -1)
    final = torch.cat([txt, idx + ntxt], dim=-1).int().contiguous()
    return final, s, score
