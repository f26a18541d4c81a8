"""GPU: the fused gather/attend/untile path gives the same bits as the tiled sequence.

The fused kernel (li_bsa_fwd_gather) reads Q/K/V in token order and writes
the output in token order; the tiled sequence (li_q_prep, li_kv_prep,
li_bsa_fwd, li_untile) materialises the tiles.  Both run the same arithmetic
in the same order, so their outputs must be equal bit for bit.  The tiled
sequence is itself checked against the oracle by test_gpu_attention /
test_gpu_pipeline.
"""
import math

import numpy as np
import pytest
import torch

from li_sparse import _core, _pipeline
from li_sparse.hy.ar_sparse_operation import fast_generate_indices

pytestmark = pytest.mark.gpu


def _qkv(seed, B, H, Lq, Lk, D, layout, text=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)

    def mk(L, scale=1.0):
        x = (torch.randn(B, L, H, D, generator=g) * scale).to(dtype)
        return x.permute(0, 2, 1, 3) if layout == "blhd" else x.permute(0, 2, 1, 3).contiguous()

    q, k, v = mk(Lq, 0.3), mk(Lk), mk(Lk)
    kt = vt = None
    if text:
        kt, vt = mk(text), mk(text)
    return q, k, v, kt, vt


def _select(params, dev, text_len_unused=None):
    def select(q_pool, k_pool, text_len, grid_q, grid_k):
        return fast_generate_indices(q_pool, k_pool, text_len, grid_q, grid_k, params, dev)
    return select


CASES = [
    # name, B, H, latent (H, W), tile, frames q, frames k, text tokens, layout, dtype
    ("hy_small_blhd", 1, 3, (30, 52), (2, 8, 8), 2, 6, 0, "blhd", torch.bfloat16),
    ("hy_small_bhld_text", 2, 2, (30, 52), (2, 8, 8), 3, 5, 300, "bhld", torch.bfloat16),
    ("mg_tile_4x4x8", 1, 2, (22, 40), (4, 4, 8), 4, 8, 0, "blhd", torch.bfloat16),
    ("odd_frames_edge", 1, 2, (12, 20), (2, 8, 8), 3, 7, 130, "blhd", torch.bfloat16),
    ("hy_small_f16_text", 1, 2, (30, 52), (2, 8, 8), 2, 6, 200, "blhd", torch.float16),
    # full HY shape with 200 text tokens: 896 tiles, so 16 of each XCD's 112 run as split halves, the first half
    # holding the text blocks
    ("hy_full_text_split", 1, 16, (30, 52), (2, 8, 8), 4, 12, 200, "blhd", torch.bfloat16),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_equals_tiled(dev, case):
    name, B, H, hw, tile, fq, fk, text, layout, dtype = case
    Hh, W = hw
    D = 128
    print(f"[gpu] fused vs tiled {name}", flush=True)
    q, k, v, kt, vt = _qkv(sum(map(ord, name)), B, H, fq * Hh * W, fk * Hh * W, D, layout, text, dtype)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    kt = kt.to(dev) if kt is not None else None
    vt = vt.to(dev) if vt is not None else None
    params = {"tile_size": tile, "topk_ratio": 0.3, "recent_protect": tile[0], "sim_metric": "scaled_dot_product",
              "force_diag": True, "force_sink": True}
    sel = _select(params, dev)
    assert _core.fused_supported(D, tile, hw)
    out_f = _pipeline.sparse_attention(q, kt, vt, k, v, hw, tile, sel, fused=True)
    out_t = _pipeline.sparse_attention(q, kt, vt, k, v, hw, tile, sel, fused=False)
    torch.cuda.synchronize()
    assert out_f.shape == out_t.shape and out_f.stride() == out_t.stride()
    same = torch.equal(out_f.view(torch.int16), out_t.view(torch.int16))
    diff = (out_f.float() - out_t.float()).abs().max().item()
    print(f"[gpu]   bitwise equal: {same} (max abs diff {diff:.3e})", flush=True)
    assert same


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_sorted_lists_path_gives_the_same_bits(dev, case):
    """LI_BSA_SORTED (the zero-region load path: text blocks first, out-of-grid chunks read from a zero region at
    the visual offsets) against the per-chunk source selection on the mask's own ascending lists: same bits,
    with text blocks, grids with partial tiles, the (4,4,8) tile, f16 and the tail split."""
    name, B, H, hw, tile, fq, fk, text, layout, dtype = case
    Hh, W = hw
    D = 128
    print(f"[gpu] sorted-lists path vs per-chunk selection {name}", flush=True)
    q, k, v, kt, vt = _qkv(sum(map(ord, name)) + 1, B, H, fq * Hh * W, fk * Hh * W, D, layout, text, dtype)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    g = _pipeline.geometry(hw, tile, q.shape[2], k.shape[2], text)
    k_txt = v_txt = None
    if text:
        k_txt = torch.zeros((B, H, g.num_txt_blk * g.bs, D), dtype=dtype, device=dev)
        v_txt = torch.zeros_like(k_txt)
        k_txt[:, :, :text] = kt.to(dev)
        v_txt[:, :, :text] = vt.to(dev)
    q_pool = torch.empty((B, H, g.nq_blk, D), device=dev, dtype=dtype)
    k_pool = torch.empty((B, H, g.nk_blk, D), device=dev, dtype=dtype)
    _core.pool(q, q_pool, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.pool(k, k_pool, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    params = {"tile_size": tile, "topk_ratio": 0.3, "recent_protect": tile[0], "sim_metric": "scaled_dot_product",
              "force_diag": True, "force_sink": True}
    ind, cnt = fast_generate_indices(q_pool, k_pool, text, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
    args = (q, k, v, k_txt, v_txt, g.num_txt_blk, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt,
            1.0 / math.sqrt(D))
    out_s, lse_s = _core.bsa_forward_gather(*args, torch.empty_like(q), return_lse=True, sorted_lists=True)
    out_u, lse_u = _core.bsa_forward_gather(*args, torch.empty_like(q), return_lse=True, sorted_lists=False)
    torch.cuda.synchronize()
    assert torch.equal(out_s.view(torch.int16), out_u.view(torch.int16))
    assert torch.equal(lse_s.view(torch.int32), lse_u.view(torch.int32))


def test_fused_hy_shape_with_split_and_lse(dev):
    """Full HY decode shape (896 query tiles: the tail split runs) and the LSE of both paths."""
    B, H, D, hw, tile = 1, 16, 128, (30, 52), (2, 8, 8)
    print("[gpu] fused vs tiled, HY shape, lse", flush=True)
    q, k, v, _, _ = _qkv(7, B, H, 4 * 1560, 12 * 1560, D, "blhd")
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    g = _pipeline.geometry(hw, tile, q.shape[2], k.shape[2], 0)
    q_pool = torch.empty((B, H, g.nq_blk, D), device=dev, dtype=q.dtype)
    k_pool = torch.empty((B, H, g.nk_blk, D), device=dev, dtype=q.dtype)
    _core.pool(q, q_pool, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.pool(k, k_pool, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    params = {"tile_size": tile, "topk_ratio": 0.3, "sim_metric": "scaled_dot_product",
              "force_diag": True, "force_sink": True}
    ind, cnt = fast_generate_indices(q_pool, k_pool, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
    scale = 1.0 / math.sqrt(D)
    out_f = torch.empty_like(q)
    _, lse_f = _core.bsa_forward_gather(q, k, v, None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh,
                                        g.nw, ind, cnt, scale, out_f, return_lse=True)
    # tiled sequence
    q_t = torch.empty((B, H, g.nq_blk, g.bs, D), device=dev, dtype=q.dtype)
    q_p2 = torch.empty_like(q_pool)
    k_all = torch.empty((B, H, g.nk_blk, g.bs, D), device=dev, dtype=q.dtype)
    v_all = torch.empty_like(k_all)
    k_p2 = torch.empty_like(k_pool)
    _core.q_prep(q, q_t, q_p2, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.kv_prep(k, v, k_all, v_all, k_p2, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    o_t, lse_t = _core.bsa_forward(q_t.flatten(2, 3), k_all.flatten(2, 3), v_all.flatten(2, 3), ind, cnt, scale,
                                   g.bs, return_lse=True)
    out_t = torch.empty_like(q)
    _core.untile(o_t.view(B, H, g.nq_blk, g.bs, D), out_t, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    torch.cuda.synchronize()
    assert torch.equal(q_pool.view(torch.int16), q_p2.view(torch.int16))
    assert torch.equal(k_pool.view(torch.int16), k_p2.view(torch.int16))
    same = torch.equal(out_f.view(torch.int16), out_t.view(torch.int16))
    print(f"[gpu]   out bitwise equal: {same}", flush=True)
    assert same
    assert torch.equal(lse_f, lse_t)


def test_fused_rejects_unsupported_shapes(dev):
    """Shapes the fused kernel does not take (W not a multiple of 4 here) run the tiled sequence."""
    assert not _core.fused_supported(128, (2, 8, 8), (30, 50))
    assert not _core.fused_supported(128, (4, 16, 2), (30, 48))
    assert not _core.fused_supported(64, (2, 8, 8), (30, 52))
    assert not _core.fused_supported(128, (2, 8, 8), (6, 52))     # grid lower than a tile
    assert not _core.fused_supported(128, (2, 8, 8), (30, 4))     # grid narrower than a tile
    assert _core.fused_supported(128, (2, 8, 8), (8, 8))
    B, H, D, hw, tile = 1, 2, 128, (16, 50), (2, 8, 8)
    q, k, v, _, _ = _qkv(3, B, H, 2 * 800, 4 * 800, D, "blhd")
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    params = {"tile_size": tile, "topk_ratio": 0.5, "sim_metric": "scaled_dot_product"}
    out = _pipeline.sparse_attention(q, None, None, k, v, hw, tile, _select(params, dev))
    torch.cuda.synchronize()
    assert out.shape == q.shape and torch.isfinite(out.float()).all()


def test_fused_balanced_order_gives_the_same_bits(dev):
    """The ragged-row order on the fused kernel: the same bits as whole tiles in natural order."""
    B, H, D, hw, tile = 1, 4, 128, (30, 52), (2, 8, 8)
    print("[gpu] fused balanced order, ragged budgets", flush=True)
    q, k, v, _, _ = _qkv(9, B, H, 4 * 1560, 16 * 1560, D, "blhd")
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    g = _pipeline.geometry(hw, tile, q.shape[2], k.shape[2], 0)
    q_pool = torch.empty((B, H, g.nq_blk, D), device=dev, dtype=q.dtype)
    k_pool = torch.empty((B, H, g.nk_blk, D), device=dev, dtype=q.dtype)
    _core.pool(q, q_pool, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.pool(k, k_pool, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    budgets = (np.random.default_rng(3).permutation(np.linspace(4, g.nk_blk, g.nq_blk)).astype(np.int64)).tolist()
    params = {"tile_size": tile, "topk_ratio": 0.1, "sim_metric": "scaled_dot_product", "force_diag": True,
              "force_sink": True, "row_budget": budgets}
    ind, cnt = fast_generate_indices(q_pool, k_pool, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
    scale = 1.0 / math.sqrt(D)
    args = (q, k, v, None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt, scale)
    out_b, lse_b = _core.bsa_forward_gather(*args, torch.empty_like(q), return_lse=True, balance=True)
    out_w, lse_w = _core.bsa_forward_gather(*args, torch.empty_like(q), return_lse=True, split=False)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), out_w.view(torch.int16))
    assert torch.equal(lse_b, lse_w)
    # the pipeline takes the balanced order for ragged budgets and still matches the tiled sequence
    sel = lambda qp, kp, tl, gq, gk: fast_generate_indices(qp, kp, tl, gq, gk, params, dev)  # noqa: E731
    o_f = _pipeline.sparse_attention(q, None, None, k, v, hw, tile, sel, balance=True)
    o_t = _pipeline.sparse_attention(q, None, None, k, v, hw, tile, sel, fused=False, balance=True)
    torch.cuda.synchronize()
    assert torch.equal(o_f.view(torch.int16), o_t.view(torch.int16))
