"""Shared test helpers: bf16 bit views and the oracle version of the whole pipeline."""
import math

import numpy as np
import torch

from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import mask as omask
from oracle import tile as otile
from oracle.bf16 import bf16_to_f32
from oracle.geometry import block_geometry, tile_permutation


def bits(t):
    """bf16/f16 torch tensor (any device) -> uint16 numpy bit patterns (contiguous)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(dtype)


def oracle_forced(geo, params, mode):
    nq, nk, nh, nw = geo["nq_blk"], geo["nk_blk"], geo["nh"], geo["nw"]
    tt = params["tile_size"][0]
    rp = params.get("recent_protect", 0)
    n_recent = min(((rp + tt - 1) // tt) * nh * nw, nk) if rp > 0 else 0
    forced = omask.forced_mask(nq, nk, nh, nw, n_recent=n_recent, diag=params.get("force_diag", False),
                               sink=params.get("force_sink", False), neighbors=(mode == "prefill"))
    if mode == "prefill":
        k = omask.budgets(forced, params["topk_ratio"], mode="total", row_budget=params.get("row_budget"))
    else:
        k = omask.budgets(forced, params.get("topk_ratio", 1.0), mode="history", row_budget=params.get("row_budget"))
    return forced, k


def oracle_pipeline(q, k, v, latent_hw, params, mode="decode", text=None, heads=None):
    """Oracle of run_sparse_attention on CPU tensors.

    Returns dict with tiles/pools (bits), indices/counts, scores, tie_free, out (float64, linear layout).
    ``heads`` restricts the attention to a list of (b, h, m) tiles.  With ``params["qk_fp8"]`` the
    attention takes Q and K (text blocks included) as their per-block e4m3 quantizations, dequantized.
    """
    H, W = latent_hw
    tile = tuple(params["tile_size"])
    lq, lk = q.shape[2], k.shape[2]
    text_len = 0 if text is None else text[0].shape[2]
    geo = block_geometry(lq, lk, latent_hw, tile, text_len)
    qt = otile.tile_gather(bits(q), geo["T_q"], H, W, tile)
    kt = otile.tile_gather(bits(k), geo["T_k"], H, W, tile)
    vt = otile.tile_gather(bits(v), geo["T_k"], H, W, tile)
    qp, kp = otile.pool_mean(qt), otile.pool_mean(kt)
    forced, kk = oracle_forced(geo, params, mode)
    ind, cnt, score, tf = omask.build_indices(qp, kp, metric=params.get("sim_metric", "cosine"), forced=forced,
                                              k=kk, num_txt_blk=geo["num_txt_blk"])
    B, NH, _, D = q.shape
    bs = geo["BS"]
    kf = bf16_to_f32(kt.reshape(B, NH, -1, D))
    vf = bf16_to_f32(vt.reshape(B, NH, -1, D))
    if text_len:
        pad = geo["num_txt_blk"] * bs - text_len
        ktx = np.concatenate([bf16_to_f32(bits(text[0])), np.zeros((B, NH, pad, D), np.float32)], axis=2)
        vtx = np.concatenate([bf16_to_f32(bits(text[1])), np.zeros((B, NH, pad, D), np.float32)], axis=2)
        kf, vf = np.concatenate([ktx, kf], axis=2), np.concatenate([vtx, vf], axis=2)
    qf = bf16_to_f32(qt.reshape(B, NH, -1, D))
    if params.get("qk_fp8", False):
        qf = ofp8.dequantize_blocks(*ofp8.quantize_blocks(qf.reshape(B, NH, -1, bs, D))).reshape(B, NH, -1, D)
        kf = ofp8.dequantize_blocks(*ofp8.quantize_blocks(kf.reshape(B, NH, -1, bs, D))).reshape(B, NH, -1, D)
    o, lse = oatt.bsa_forward(qf, kf, vf, ind, cnt, 1.0 / math.sqrt(D), bs, heads=heads)
    perm = tile_permutation(geo["T_q"], H, W, tile)
    valid = perm >= 0
    out = np.zeros((B, NH, lq, D), dtype=np.float64)
    out[:, :, perm[valid], :] = o[:, :, valid, :]
    return dict(geo=geo, q_tiles=qt, k_tiles=kt, v_tiles=vt, q_pool=qp, k_pool=kp, indices=ind, counts=cnt,
                scores=score, tie_free=tf, forced=forced, budgets=kk, out=out, out_tiled=o, lse=lse, perm=perm)
