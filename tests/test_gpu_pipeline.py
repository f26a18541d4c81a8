"""GPU parity of the drop-in entry points (HY decode, HY prefill, MG) against the oracle pipeline."""
import math

import numpy as np
import pytest
import torch

from helpers import bits, oracle_pipeline
from li_sparse.hy import bi_sparse_operation_for_KV_cache as hykv
from li_sparse.hy.ar_sparse_operation import run_sparse_attention
from li_sparse.hy.infer_state import get_infer_state
from li_sparse.mg import bi_sparse_operation as mgs
from li_sparse.workloads import WORKLOADS, Workload, make_qkv

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _empty(wl, dev):
    return torch.empty((wl.batch, wl.heads, 0, wl.head_dim), dtype=torch.bfloat16, device=dev)


@pytest.mark.parametrize("layout", ["bhld", "blhd"])
def test_hy_decode_toy_full(dev, layout):
    wl = WORKLOADS["toy"]
    print(f"[gpu] run_sparse_attention toy layout={layout}", flush=True)
    q, k, v = make_qkv(wl, seed=0, layout=layout)
    params = wl.sparse_params()
    out = run_sparse_attention(q.to(dev), _empty(wl, dev), _empty(wl, dev), k.to(dev), v.to(dev), 1, wl.latent_hw,
                               params)
    torch.cuda.synchronize()
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params)
    assert out.shape == q.shape and out.stride() == q.to(dev).stride()
    err = np.abs(out.float().cpu().numpy() - ref["out"]).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("name", ["hy", "mg"])
def test_decode_full_shape_sampled(dev, name):
    wl = WORKLOADS[name]
    print(f"[gpu] run_sparse_attention {name} full shape", flush=True)
    q, k, v = make_qkv(wl, seed=0, layout="blhd")
    params = wl.sparse_params()
    out = run_sparse_attention(q.to(dev), _empty(wl, dev), _empty(wl, dev), k.to(dev), v.to(dev), 1, wl.latent_hw,
                               params)
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    nq = math.ceil(wl.frames_q / wl.tile[0]) * math.ceil(wl.latent_hw[0] / wl.tile[1]) * \
        math.ceil(wl.latent_hw[1] / wl.tile[2])
    tiles = [(0, int(h), int(m)) for h, m in zip(rng.integers(0, wl.heads, 16), rng.integers(0, nq, 16))]
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, heads=tiles)
    got = out.float().cpu().numpy()
    bs = ref["geo"]["BS"]
    perm = ref["perm"]
    err = 0.0
    for b, h, m in tiles:
        rows = perm[m * bs:(m + 1) * bs]
        rows = rows[rows >= 0]
        err = max(err, np.abs(got[b, h, rows] - ref["out"][b, h, rows]).max())
    print(f"[gpu]   max abs err over {len(tiles)} sampled tiles {err:.3e}", flush=True)
    assert err <= TOL


def test_hy_decode_reference_rule_with_text(dev):
    # the reference's own decode configuration: tile (4, 8, 4), recent_protect 4, ratio 0.175, text tokens
    wl = Workload("hy_ref", 2, 128, (30, 52), 4, 8, (4, 8, 4), 0.175, "scaled_dot_product", force_diag=False,
                  force_sink=False)
    print("[gpu] run_sparse_attention reference decode rule + 200 text tokens", flush=True)
    q, k, v = make_qkv(wl, seed=4, layout="blhd")
    g = torch.Generator().manual_seed(9)
    kt = torch.randn(1, 2, 200, 128, generator=g).to(torch.bfloat16)
    vt = torch.randn(1, 2, 200, 128, generator=g).to(torch.bfloat16)
    params = {"tile_size": (4, 8, 4), "topk_ratio": 0.175, "recent_protect": 4, "sim_metric": "scaled_dot_product"}
    out = run_sparse_attention(q.to(dev), kt.to(dev), vt.to(dev), k.to(dev), v.to(dev), 3, wl.latent_hw, params)
    torch.cuda.synchronize()
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, text=(kt, vt))
    err = np.abs(out.float().cpu().numpy() - ref["out"]).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_hy_prefill_gating_and_sparse(dev):
    wl = Workload("hy_prefill", 2, 128, (30, 52), 4, 4, (4, 8, 4), 0.3, "scaled_dot_product", force_diag=False,
                  force_sink=False)
    print("[gpu] run_sparse_prefill_attention (dense for chunk < 3, sparse after)", flush=True)
    q, k, v = make_qkv(wl, seed=5)
    params = {"tile_size": (4, 8, 4), "topk_ratio": 0.3, "sim_metric": "scaled_dot_product"}
    state = get_infer_state()
    e = _empty(wl, dev)
    state.current_chunk_index = 1
    dense = hykv.run_sparse_prefill_attention(q.to(dev), e, e, k.to(dev), v.to(dev), 2, wl.latent_hw, params)
    ref_dense = torch.nn.functional.scaled_dot_product_attention(q.to(dev).float(), k.to(dev).float(),
                                                                 v.to(dev).float())
    state.current_chunk_index = 5
    try:
        out = hykv.run_sparse_prefill_attention(q.to(dev), e, e, k.to(dev), v.to(dev), 2, wl.latent_hw, params)
    finally:
        state.current_chunk_index = 0
    torch.cuda.synchronize()
    assert (dense.float() - ref_dense).abs().max().item() <= TOL
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, mode="prefill")
    err = np.abs(out.float().cpu().numpy() - ref["out"]).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_mg_self_attention_entry(dev):
    # MG calls with Lq = Lk over memory + current clip, tile (4, 4, 8), cosine, text_len = 0
    wl = Workload("mg_self", 2, 128, (22, 40), 8, 8, (4, 4, 8), 0.2, "cosine", force_diag=False, force_sink=False)
    print("[gpu] MG run_sparse_attention (Lq = Lk)", flush=True)
    q, k, v = make_qkv(wl, seed=6)
    params = {"tile_size": (4, 4, 8), "topk_ratio": 0.2, "sim_metric": "cosine", "profile_layers": []}
    out = mgs.run_sparse_attention(q.to(dev), k.to(dev), v.to(dev), 0, 1, wl.latent_hw, params)
    torch.cuda.synchronize()
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, mode="prefill")
    err = np.abs(out.float().cpu().numpy() - ref["out"]).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL
