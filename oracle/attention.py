"""Block-sparse attention forward (oracle, test infrastructure only).

Restates ``_attn_fwd_bsa_align`` (longcat_kernel.py:27-155, same math in
matrix-game-3.0/files/wan/modules/longcat_kernel.py:28-134) in float64:

for each (b, h) and query tile m (``block_m`` rows of the tiled Q), over the
kept key blocks ``indices[b,h,m,:counts[b,h,m]]`` (each ``block_n`` rows of the
tiled K/V), ``O = softmax(sm_scale * Q K^T) V``.  Zero-padded key rows inside
kept blocks take part in the softmax (the kernel has no key mask,
longcat_kernel.py:125-141).  ``lse`` is in log2 units like the kernel's ``M``
buffer: ``m + log2(l)`` with ``m`` the running max of ``sm_scale*log2(e)*S``
(longcat_kernel.py:146).  A row with ``counts == 0`` gives output 0 and
``lse = -inf`` (``l_i`` starts at 1 and ``acc`` at 0, longcat_kernel.py:102-104).

The reference kernel always tiles queries by 128 rows (longcat_kernel.py:202);
``block_m`` defaults to ``block_n`` here, which is the same thing for the
128-token blocks every reference call site uses.

Pinned by tests/test_oracle_attention.py: a single kept block equals
``torch.nn.functional.scaled_dot_product_attention`` (float64, CPU) over that
block, all blocks kept equals dense SDPA over the padded K/V, identical keys
reduce to the closed form ``sum_valid v / (n_valid + n_pad * exp(-s))``,
``lse`` matches ``torch.logsumexp / ln 2``, and the output is invariant under
reversing the kept-block order.
"""
import math

import numpy as np


def bsa_forward(q, k, v, indices, counts, sm_scale=None, block_n=128, block_m=None, heads=None):
    """Block-sparse attention in float64.

    q (B,H,Lq,D), k/v (B,H,Lk,D) float arrays; indices (B,H,Nq,K) int; counts (B,H,Nq) int.
    ``heads`` optionally restricts the work to a list of (b, h, m) query tiles; other rows stay 0.
    Returns (out float64 (B,H,Lq,D), lse float64 (B,H,Lq)).
    """
    B, H, Lq, D = q.shape
    bm = block_n if block_m is None else block_m
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, H, Lq, D), dtype=np.float64)
    lse = np.full((B, H, Lq), -np.inf, dtype=np.float64)
    nq = (Lq + bm - 1) // bm
    tiles = heads if heads is not None else [(b, h, m) for b in range(B) for h in range(H) for m in range(nq)]
    for (b, h, m) in tiles:
        n = int(counts[b, h, m])
        if n == 0:
            continue
        ids = np.asarray(indices[b, h, m, :n], dtype=np.int64)
        rows = (ids[:, None] * block_n + np.arange(block_n)[None, :]).reshape(-1)
        qt = np.asarray(q[b, h, m * bm:(m + 1) * bm], dtype=np.float64)
        kt = np.asarray(k[b, h][rows], dtype=np.float64)
        vt = np.asarray(v[b, h][rows], dtype=np.float64)
        s = (qt @ kt.T) * sm_scale
        mx = s.max(axis=1, keepdims=True)
        p = np.exp(s - mx)
        l = p.sum(axis=1, keepdims=True)
        out[b, h, m * bm:(m + 1) * bm] = (p @ vt) / l
        lse[b, h, m * bm:(m + 1) * bm] = (mx[:, 0] + np.log(l[:, 0])) / math.log(2.0)
    return out, lse


def expand_block_mask(indices, counts, nq_rows, nk_rows, block_n, block_m=None):
    """Boolean token mask (B,H,Lq,Lk) expanded from block lists (for small shapes)."""
    B, H, Nq, _ = indices.shape
    bm = block_n if block_m is None else block_m
    m = np.zeros((B, H, nq_rows, nk_rows), dtype=bool)
    for b in range(B):
        for h in range(H):
            for r in range(Nq):
                for j in indices[b, h, r, :counts[b, h, r]]:
                    m[b, h, r * bm:(r + 1) * bm, j * block_n:(j + 1) * block_n] = True
    return m


def dense_masked_cpu(q_bf16, k_bf16, v_bf16, indices, counts, sm_scale, block_n, head_list=None):
    """The reference's "PyTorch dense-masked" semantics on the CPU (torch, float32 from bf16).

    ``F.scaled_dot_product_attention`` with a boolean mask expanded from the kept
    blocks over the tiled/padded layout, one head at a time (a full
    (H, Lq_pad, Lk_pad) mask does not fit at the HY shape).  Used as the CPU
    baseline that the GPU op is timed against; ``head_list`` bounds the sample.
    Returns float32 (len(head_list), Lq, D).
    """
    import torch
    import torch.nn.functional as F

    B, H, Lq, D = q_bf16.shape
    Lk = k_bf16.shape[2]
    if head_list is None:
        head_list = [(b, h) for b in range(B) for h in range(H)]
    idx = torch.as_tensor(np.asarray(indices), dtype=torch.long)
    cnt = torch.as_tensor(np.asarray(counts), dtype=torch.long)
    nq = idx.shape[2]
    outs = []
    for (b, h) in head_list:
        blk_mask = torch.zeros(nq, Lk // block_n, dtype=torch.bool)
        for r in range(nq):
            blk_mask[r, idx[b, h, r, :cnt[b, h, r]]] = True
        mask = blk_mask.repeat_interleave(block_n, 0).repeat_interleave(block_n, 1)[:Lq]
        qf = q_bf16[b, h].float()
        kf = k_bf16[b, h].float()
        vf = v_bf16[b, h].float()
        o = F.scaled_dot_product_attention(qf[None], kf[None], vf[None], attn_mask=mask[None], scale=sm_scale)
        empty = ~blk_mask.any(dim=1).repeat_interleave(block_n)[:Lq]
        o = o[0]
        o[empty] = 0.0
        outs.append(o)
    return torch.stack(outs)
