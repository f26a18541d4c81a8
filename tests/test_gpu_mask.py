"""GPU parity: block-mask builder vs the oracle (bit-exact scores, indices, counts) and the golden fixtures."""
import ctypes
import math
import os

import numpy as np
import pytest
import torch

from helpers import bits, from_bits, oracle_forced
from li_sparse import _core, _lib
from li_sparse.hy.ar_sparse_operation import fast_generate_indices
from li_sparse.hy.bi_sparse_operation_for_KV_cache import generate_prefill_indices
from li_sparse.workloads import WORKLOADS, make_qkv
from oracle import mask as omask
from oracle import tile as otile
from oracle.geometry import block_geometry
from test_oracle_mask import CASES

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mask_golden.npz")


@pytest.mark.parametrize("name", list(CASES))
def test_golden_cases_bit_exact(dev, name):
    print(f"[gpu] mask golden {name}", flush=True)
    g = np.load(GOLDEN)
    mode, (nt_q, nt_k, nh, nw), text_len, params = CASES[name]
    qp, kp = g[f"{name}/q_pool"], g[f"{name}/k_pool"]
    qd, kd = from_bits(qp).to(dev), from_bits(kp).to(dev)
    if mode == "decode":
        ind, cnt = fast_generate_indices(qd, kd, text_len, (nt_q, nh, nw), (nt_k, nh, nw), params, dev)
        oind, ocnt = omask.fast_generate_indices(qp, kp, text_len, (nt_q, nh, nw), (nt_k, nh, nw), params)
    else:
        ind, cnt = generate_prefill_indices(qd, kd, text_len, (nt_k, nh, nw), params, dev)
        oind, ocnt = omask.generate_prefill_indices(qp, kp, text_len, (nt_k, nh, nw), params)
    torch.cuda.synchronize()
    assert np.array_equal(ind.cpu().numpy(), oind)
    assert np.array_equal(cnt.cpu().numpy(), ocnt)
    tf = g[f"{name}/tie_free"]
    assert np.array_equal(ind.cpu().numpy()[tf], g[f"{name}/indices"][tf])


@pytest.mark.parametrize("name", ["toy", "hy", "mg", "hy_long"])
def test_workload_selection_bit_exact(dev, name):
    wl = WORKLOADS[name]
    print(f"[gpu] mask workload {name}", flush=True)
    q, k, _ = make_qkv(wl, seed=3)
    geo = block_geometry(wl.lq, wl.lk, wl.latent_hw, wl.tile)
    H, W = wl.latent_hw
    qp = otile.pool_mean(otile.tile_gather(bits(q), geo["T_q"], H, W, wl.tile))
    kp = otile.pool_mean(otile.tile_gather(bits(k), geo["T_k"], H, W, wl.tile))
    params = wl.sparse_params(geo["nq_blk"])
    forced, kk = oracle_forced(geo, params, "decode")
    oind, ocnt, oscore, tf = omask.build_indices(qp, kp, metric=wl.metric, forced=forced, k=kk, num_txt_blk=0)
    ind, cnt, sc = _core.block_mask(from_bits(qp).to(dev), from_bits(kp).to(dev), metric=wl.metric,
                                    budget_mode=_lib.LI_BUDGET_HISTORY, ratio=wl.ratio, nh=geo["nh"], nw=geo["nw"],
                                    force_diag=True, force_sink=True, row_budget=params.get("row_budget"),
                                    return_scores=True)
    torch.cuda.synchronize()
    assert np.array_equal(bits(sc), oscore)
    assert np.array_equal(cnt.cpu().numpy(), ocnt)
    assert np.array_equal(ind.cpu().numpy(), oind)
    print(f"[gpu]   rows tie-free (>= 2 bf16 ulps at the cut): {tf.mean():.3f}", flush=True)


@pytest.mark.parametrize("metric", ["cosine", "scaled_dot_product", "dot"])
@pytest.mark.parametrize("rule", ["recent", "prefill", "ragged"])
def test_rules_and_metrics(dev, metric, rule):
    print(f"[gpu] mask rule={rule} metric={metric}", flush=True)
    rng = np.random.default_rng(sum(map(ord, metric + rule)))
    nh, nw, nt_q, nt_k, D = 3, 5, 2, 6, 128
    if rule == "prefill":
        nt_q = nt_k
    nq, nk = nt_q * nh * nw, nt_k * nh * nw
    qp = torch.randn(2, 3, nq, D, generator=torch.Generator().manual_seed(int(rng.integers(1 << 30)))).to(torch.bfloat16)
    kp = torch.randn(2, 3, nk, D, generator=torch.Generator().manual_seed(int(rng.integers(1 << 30)))).to(torch.bfloat16)
    if rule == "recent":
        params = {"tile_size": (2, 8, 8), "topk_ratio": 0.2, "recent_protect": 4, "sim_metric": metric}
        ind, cnt = fast_generate_indices(qp.to(dev), kp.to(dev), 130, (nt_q, nh, nw), (nt_k, nh, nw), params, dev)
        oind, ocnt = omask.fast_generate_indices(bits(qp), bits(kp), 130, (nt_q, nh, nw), (nt_k, nh, nw), params)
    elif rule == "prefill":
        params = {"tile_size": (4, 4, 8), "topk_ratio": 0.25, "sim_metric": metric}
        ind, cnt = generate_prefill_indices(qp.to(dev), kp.to(dev), 0, (nt_k, nh, nw), params, dev)
        oind, ocnt = omask.generate_prefill_indices(bits(qp), bits(kp), 0, (nt_k, nh, nw), params)
    else:
        rb = rng.integers(0, nk + 5, size=nq).tolist()
        params = {"tile_size": (2, 8, 8), "topk_ratio": 0.1, "sim_metric": metric, "force_diag": True,
                  "force_sink": True, "row_budget": rb}
        ind, cnt = fast_generate_indices(qp.to(dev), kp.to(dev), 0, (nt_q, nh, nw), (nt_k, nh, nw), params, dev)
        oind, ocnt = omask.fast_generate_indices(bits(qp), bits(kp), 0, (nt_q, nh, nw), (nt_k, nh, nw), params)
    torch.cuda.synchronize()
    assert np.array_equal(cnt.cpu().numpy(), ocnt)
    assert np.array_equal(ind.cpu().numpy(), oind)


def test_five_d_input_and_ties(dev):
    # tiled (5-D) input is mean-pooled first; all-equal pools -> every score ties -> lower indices win
    print("[gpu] mask 5-D input + all ties", flush=True)
    nh, nw = 2, 2
    x = torch.ones(1, 1, 8, 16, 64, dtype=torch.bfloat16, device=dev)
    params = {"tile_size": (1, 4, 4), "topk_ratio": 0.3, "sim_metric": "dot"}
    ind, cnt = generate_prefill_indices(x, x, 0, (2, nh, nw), params, dev)
    torch.cuda.synchronize()
    forced = omask.forced_mask(8, 8, nh, nw, neighbors=True)
    for r in range(8):
        free = [j for j in range(8) if not forced[r, j]]
        want = sorted(list(np.nonzero(forced[r])[0]) + free[:max(0, 7 - int(forced[r].sum()))])
        assert ind[0, 0, r].tolist() == want


@pytest.mark.parametrize("metric", ["cosine", "dot"])
def test_no_key_blocks(dev, metric):
    """A key grid with no blocks (nk = 0), through the C ABI with a valid key-pool pointer (torch gives a
    zero-row tensor a null pointer, which the entry point rejects): the shared-pool kernel reads no pool row and
    every query row keeps only its text blocks, as the oracle's selection does; the rest of the row is zero."""
    print(f"[gpu] mask nk=0 metric={metric}", flush=True)
    D, nq, nh, nw, ntxt, kmax = 128, 6, 2, 3, 2, 3
    gen = torch.Generator().manual_seed(7)
    qp = torch.randn(1, 2, nq, D, generator=gen).to(torch.bfloat16)
    qd = qp.to(dev)
    kbuf = torch.randn(1, 2, 4, D, generator=gen).to(torch.bfloat16).to(dev)
    geo = {"nq_blk": nq, "nk_blk": 0, "nh": nh, "nw": nw}
    params = {"tile_size": (2, 8, 8), "topk_ratio": 0.3, "force_diag": True, "force_sink": True}
    forced, kk = oracle_forced(geo, params, "decode")
    oind, ocnt, _, _ = omask.build_indices(bits(qp), np.zeros((1, 2, 0, D), np.uint16), metric=metric,
                                           forced=forced, k=kk, num_txt_blk=ntxt)
    ind = torch.full((1, 2, nq, kmax), -7, dtype=torch.int32, device=dev)
    cnt = torch.full((1, 2, nq), -7, dtype=torch.int32, device=dev)
    code = _core.METRICS.get(metric, _lib.LI_METRIC_DOT)
    p = _lib.MaskParams(metric=code, budget_mode=_lib.LI_BUDGET_HISTORY, topk_ratio=0.3, min_budget=7,
                        force_diag=1, force_sink=1, nq=nq, nk=0, nh=nh, nw=nw, num_txt_blk=ntxt, kmax=kmax)
    stream = torch.cuda.current_stream(dev).cuda_stream
    st = _lib.lib.li_block_mask(_lib.LI_DTYPE_BF16, 1, 2, D, qd.data_ptr(), _lib.i64_array(qd.stride()),
                                kbuf.data_ptr(), _lib.i64_array(kbuf.stride()), ctypes.byref(p), ind.data_ptr(),
                                cnt.data_ptr(), None, ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    assert st == _lib.LI_OK
    assert np.array_equal(cnt.cpu().numpy(), ocnt)
    assert np.array_equal(ind[..., :ntxt].cpu().numpy(), oind)
    assert (ind[..., ntxt:] == 0).all()


@pytest.mark.parametrize("metric", ["cosine", "scaled_dot_product", "dot"])
@pytest.mark.parametrize("case", ["nk_above_shared_path", "strided_pools", "shared_path_partial_tiles",
                                  "shared_path_long_rows"])
def test_lds_key_path(dev, metric, case):
    """Both mask kernels: the generic one for more key blocks than the shared-pool kernel's LDS holds (nk = 1960 at
    D = 128) and for pool views without a unit d stride; the shared-pool one with a partial last tile and a last
    workgroup with fewer query rows than waves (D = 64), and with nk = 1120 (nine tiles, the widest key registers)."""
    print(f"[gpu] mask LDS path {case} metric={metric}", flush=True)
    rng = np.random.default_rng(sum(map(ord, metric + case)))
    D = 128
    if case == "nk_above_shared_path":
        nh, nw, nt_q, nt_k = 4, 7, 1, 70           # nk = 1960
    elif case == "strided_pools":
        nh, nw, nt_q, nt_k = 3, 5, 2, 6            # nk = 90
    elif case == "shared_path_partial_tiles":
        nh, nw, nt_q, nt_k, D = 3, 5, 2, 13, 64    # nq = 30, nk = 195
    else:
        nh, nw, nt_q, nt_k = 4, 7, 1, 40           # nq = 28, nk = 1120
    nq, nk = nt_q * nh * nw, nt_k * nh * nw
    gen = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    qp = torch.randn(1, 2, nq, D, generator=gen).to(torch.bfloat16)
    kp = torch.randn(1, 2, nk, D, generator=gen).to(torch.bfloat16)
    qd, kd = qp.to(dev), kp.to(dev)
    if case == "strided_pools":
        kd = kd.transpose(2, 3).contiguous().transpose(2, 3)   # d stride nk: element-wise loads
    geo = {"nq_blk": nq, "nk_blk": nk, "nh": nh, "nw": nw}
    params = {"tile_size": (2, 8, 8), "topk_ratio": 0.2, "force_diag": True, "force_sink": True}
    forced, kk = oracle_forced(geo, params, "decode")
    oind, ocnt, oscore, _ = omask.build_indices(bits(qp), bits(kp), metric=metric, forced=forced, k=kk,
                                                num_txt_blk=0)
    ind, cnt, sc = _core.block_mask(qd, kd, metric=metric, budget_mode=_lib.LI_BUDGET_HISTORY, ratio=0.2, nh=nh,
                                    nw=nw, force_diag=True, force_sink=True, return_scores=True)
    torch.cuda.synchronize()
    assert np.array_equal(bits(sc), oscore)
    assert np.array_equal(cnt.cpu().numpy(), ocnt)
    assert np.array_equal(ind.cpu().numpy(), oind)


@pytest.mark.parametrize("metric", ["cosine", "scaled_dot_product", "dot"])
@pytest.mark.parametrize("case", ["shared_pool", "generic_strided"])
def test_float16_pools(dev, metric, case):
    """float16 pools: scores, lists and counts bit-exact against the oracle's float16 model, on both kernels."""
    print(f"[gpu] mask float16 {case} metric={metric}", flush=True)
    rng = np.random.default_rng(sum(map(ord, metric + case)) + 16)
    D, nh, nw, nt_q, nt_k = 128, 4, 7, 2, 6                 # nq = 56, nk = 168
    nq, nk = nt_q * nh * nw, nt_k * nh * nw
    gen = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    qp = (torch.randn(1, 3, nq, D, generator=gen) * 0.5).to(torch.float16)
    kp = (torch.randn(1, 3, nk, D, generator=gen) * 0.5).to(torch.float16)
    qd, kd = qp.to(dev), kp.to(dev)
    if case == "generic_strided":
        kd = kd.transpose(2, 3).contiguous().transpose(2, 3)
    geo = {"nq_blk": nq, "nk_blk": nk, "nh": nh, "nw": nw}
    params = {"tile_size": (2, 8, 8), "topk_ratio": 0.3, "force_diag": True, "force_sink": True}
    forced, kk = oracle_forced(geo, params, "decode")
    oind, ocnt, oscore, _ = omask.build_indices(bits(qp), bits(kp), metric=metric, forced=forced, k=kk,
                                                num_txt_blk=0, fmt="f16")
    ind, cnt, sc = _core.block_mask(qd, kd, metric=metric, budget_mode=_lib.LI_BUDGET_HISTORY, ratio=0.3, nh=nh,
                                    nw=nw, force_diag=True, force_sink=True, return_scores=True)
    torch.cuda.synchronize()
    assert sc.dtype == torch.float16
    assert np.array_equal(bits(sc), oscore)
    assert np.array_equal(cnt.cpu().numpy(), ocnt)
    assert np.array_equal(ind.cpu().numpy(), oind)
