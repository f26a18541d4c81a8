"""GPU parity at the HY long-rollout shape: Lq = 6240, Lk = 99840 (64 frames), 896 key blocks, ragged rows.

The whole ``run_sparse_attention`` call (pools, block mask, fused attention
with the longest-first tile order and per-head XCD chunks) is compared with
the oracle pipeline on sampled query tiles, including the longest and the
shortest rows; the fused call, the tiled sequence and whole tiles in natural
order give the same bits.  Reference path: ar_sparse_operation.py:289-362.
"""
import math

import numpy as np
import pytest
import torch

from helpers import oracle_pipeline
from li_sparse import _core, _pipeline
from li_sparse.hy.ar_sparse_operation import fast_generate_indices, run_sparse_attention
from li_sparse.workloads import WORKLOADS, make_qkv

pytestmark = pytest.mark.gpu
TOL = 2e-2


@pytest.fixture(scope="module")
def long_case(dev):
    wl = WORKLOADS["hy_long"]
    print("[gpu] hy_long inputs (Lq=6240, Lk=99840, BLHD views)", flush=True)
    q, k, v = make_qkv(wl, seed=0, layout="blhd")
    g = _pipeline.geometry(wl.latent_hw, wl.tile, wl.lq, wl.lk, 0)
    return wl, q, k, v, g


def test_long_rollout_call_vs_oracle(dev, long_case):
    wl, q, k, v, g = long_case
    params = wl.sparse_params(g.nq_blk)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    e = torch.empty((1, wl.heads, 0, wl.head_dim), dtype=torch.bfloat16, device=dev)
    assert _pipeline.uses_fused(qd, kd, vd, wl.tile, wl.latent_hw) and _pipeline.ragged(params)
    print("[gpu] run_sparse_attention hy_long (fused, longest tiles first)", flush=True)
    out = run_sparse_attention(qd, e, e, kd, vd, 1, wl.latent_hw, params)
    torch.cuda.synchronize()
    # Sampled tiles: the longest and the shortest rows of two heads, plus random ones.
    budgets = np.asarray(params["row_budget"])
    longest, shortest = int(np.argmax(budgets)), int(np.argmin(budgets))
    rng = np.random.default_rng(3)
    tiles = [(0, 0, longest), (0, wl.heads - 1, longest), (0, 5, shortest), (0, wl.heads - 1, shortest)]
    tiles += [(0, int(h), int(m)) for h, m in zip(rng.integers(0, wl.heads, 14), rng.integers(0, g.nq_blk, 14))]
    print(f"[gpu]   oracle on {len(tiles)} tiles (row budgets {budgets.min()}..{budgets.max()})", flush=True)
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, heads=tiles)
    cnt = ref["counts"]
    assert cnt[0, 0, longest] == budgets.max() and cnt[0, 5, shortest] == budgets.min()
    got = out.float().cpu().numpy()
    bs, perm = ref["geo"]["BS"], ref["perm"]
    err = 0.0
    for b, h, m in tiles:
        rows = perm[m * bs:(m + 1) * bs]
        rows = rows[rows >= 0]
        err = max(err, np.abs(got[b, h, rows] - ref["out"][b, h, rows]).max())
    print(f"[gpu]   max abs err over {len(tiles)} sampled tiles {err:.3e}", flush=True)
    assert err <= TOL


def test_long_rollout_orders_and_paths_same_bits(dev, long_case):
    wl, q, k, v, g = long_case
    params = wl.sparse_params(g.nq_blk)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    print("[gpu] hy_long: fused balanced vs fused natural order vs tiled sequence", flush=True)

    def select(q_pool, k_pool, text_len, grid_q, grid_k):
        return fast_generate_indices(q_pool, k_pool, text_len, grid_q, grid_k, params, dev)

    out_bal = _pipeline.sparse_attention(qd, None, None, kd, vd, wl.latent_hw, wl.tile, select, balance=True)
    out_nat = _pipeline.sparse_attention(qd, None, None, kd, vd, wl.latent_hw, wl.tile, select, balance=False)
    out_til = _pipeline.sparse_attention(qd, None, None, kd, vd, wl.latent_hw, wl.tile, select, balance=True,
                                         fused=False)
    # Whole tiles in natural order, without the tail split, from the same lists.
    q_pool = torch.empty((1, wl.heads, g.nq_blk, wl.head_dim), dtype=torch.bfloat16, device=dev)
    k_pool = torch.empty((1, wl.heads, g.nk_blk, wl.head_dim), dtype=torch.bfloat16, device=dev)
    _core.pool(qd, q_pool, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.pool(kd, k_pool, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    ind, cnt = select(q_pool, k_pool, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw))
    out_whole = torch.empty_like(qd)
    _core.bsa_forward_gather(qd, kd, vd, None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt,
                             1.0 / math.sqrt(wl.head_dim), out_whole, split=False, balance=False)
    torch.cuda.synchronize()
    assert torch.equal(out_bal.view(torch.int16), out_whole.view(torch.int16))
    assert torch.equal(out_til.view(torch.int16), out_whole.view(torch.int16))
    # The natural order may split its last round's tiles (merged in fp32): within rounding of whole tiles.
    d = (out_nat.float() - out_whole.float()).abs().max().item()
    print(f"[gpu]   natural order (tail split) vs whole tiles: {d:.3e}", flush=True)
    assert d <= 1e-2


def test_long_rollout_e4m3_call_vs_oracle(dev, long_case):
    """The e4m3 call (qk_fp8) at the long-rollout shape: sampled tiles (longest and shortest rows included) against
    the oracle pipeline on the quantized Q and K, and the fused longest-first kernel bit-equal to the tiled e4m3
    sequence on the same lists."""
    wl, q, k, v, g = long_case
    params = WORKLOADS["hy_long_fp8"].sparse_params(g.nq_blk)
    assert params["qk_fp8"] and params["row_budget"] == wl.sparse_params(g.nq_blk)["row_budget"]
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    e = torch.empty((1, wl.heads, 0, wl.head_dim), dtype=torch.bfloat16, device=dev)
    print("[gpu] run_sparse_attention hy_long_fp8 (fused e4m3, longest tiles first)", flush=True)
    out = run_sparse_attention(qd, e, e, kd, vd, 1, wl.latent_hw, params)

    def select(q_pool, k_pool, text_len, grid_q, grid_k):
        return fast_generate_indices(q_pool, k_pool, text_len, grid_q, grid_k, params, dev)

    out_til = _pipeline.sparse_attention(qd, None, None, kd, vd, wl.latent_hw, wl.tile, select, balance=True,
                                         qk_fp8=True, fused=False)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), out_til.view(torch.int16))
    budgets = np.asarray(params["row_budget"])
    longest, shortest = int(np.argmax(budgets)), int(np.argmin(budgets))
    rng = np.random.default_rng(5)
    tiles = [(0, 1, longest), (0, wl.heads - 2, shortest)]
    tiles += [(0, int(h), int(m)) for h, m in zip(rng.integers(0, wl.heads, 8), rng.integers(0, g.nq_blk, 8))]
    print(f"[gpu]   oracle (quantized Q, K) on {len(tiles)} tiles", flush=True)
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, heads=tiles)
    got = out.float().cpu().numpy()
    bs, perm = ref["geo"]["BS"], ref["perm"]
    err = 0.0
    for b, h, m in tiles:
        rows = perm[m * bs:(m + 1) * bs]
        rows = rows[rows >= 0]
        err = max(err, np.abs(got[b, h, rows] - ref["out"][b, h, rows]).max())
    print(f"[gpu]   max abs err over {len(tiles)} sampled tiles {err:.3e}", flush=True)
    assert err <= TOL
