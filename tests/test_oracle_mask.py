"""Pins oracle.mask: golden fixtures from the reference's torch calls, known answers, budgets, brute force."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import mask as omask
from oracle.bf16 import bf16_order_key, bf16_to_f32, f32_to_bf16

import torch_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mask_golden.npz")

CASES = {  # name -> (mode, grid (nt_q, nt_k, nh, nw), text_len, params); must match tests/golden/make_golden.py
    "decode_recent_sdp": ("decode", (2, 6, 4, 7), 0,
                          {"tile_size": (2, 8, 8), "topk_ratio": 0.175, "recent_protect": 4,
                           "sim_metric": "scaled_dot_product"}),
    "decode_cosine_text": ("decode", (1, 5, 3, 5), 300,
                           {"tile_size": (4, 4, 8), "topk_ratio": 0.3, "recent_protect": 4, "sim_metric": "cosine"}),
    "decode_diag_sink": ("decode", (2, 6, 4, 7), 0,
                         {"tile_size": (2, 8, 8), "topk_ratio": 0.3, "sim_metric": "scaled_dot_product",
                          "force_diag": True, "force_sink": True}),
    "decode_dot": ("decode", (1, 4, 8, 8), 0,
                   {"tile_size": (4, 4, 4), "topk_ratio": 0.25, "recent_protect": 2, "sim_metric": "dot"}),
    "prefill_sdp": ("prefill", (3, 3, 4, 7), 0,
                    {"tile_size": (4, 8, 4), "topk_ratio": 0.3, "sim_metric": "scaled_dot_product"}),
    "prefill_cosine_mg": ("prefill", (5, 5, 3, 5), 0,
                          {"tile_size": (4, 4, 8), "topk_ratio": 0.2, "sim_metric": "cosine"}),
}


def oracle_case(mode, grid, text_len, params, qp, kp):
    nt_q, nt_k, nh, nw = grid
    q = np.asarray(qp)
    k = np.asarray(kp)
    if mode == "decode":
        return omask.fast_generate_indices(q, k, text_len, (nt_q, nh, nw), (nt_k, nh, nw), params)
    return omask.generate_prefill_indices(q, k, text_len, (nt_k, nh, nw), params)


def is_valid_topk(key_row, forced_row, sel):
    """sel (ascending visual ids) keeps every forced block and a top-k set of the rest."""
    s = np.zeros(key_row.size, dtype=bool)
    s[sel] = True
    if not np.all(s[forced_row]):
        return False
    free_in, free_out = key_row[s & ~forced_row], key_row[~s & ~forced_row]
    return free_in.size == 0 or free_out.size == 0 or free_in.min() >= free_out.max()


@pytest.mark.parametrize("name", list(CASES))
def test_golden_reference_calls(name):
    g = np.load(GOLDEN)
    mode, grid, text_len, params = CASES[name]
    qp, kp = g[f"{name}/q_pool"], g[f"{name}/k_pool"]
    gold_idx, gold_scores, tf = g[f"{name}/indices"], g[f"{name}/scores"], g[f"{name}/tie_free"]
    ind, cnt = oracle_case(mode, grid, text_len, params, qp, kp)
    assert ind.shape == gold_idx.shape and np.all(cnt == gold_idx.shape[-1])
    # 1. the oracle's rounding model reproduces the torch bf16 scores; the fp32 sum order may move
    # the bf16 dot by one ulp, which the x(1/sqrt(d)) rescale can widen to two
    score = omask.similarity(qp, kp, params["sim_metric"])
    ulp = np.abs(score.astype(np.int32) - gold_scores.astype(np.int32))
    assert ulp.max() <= (2 if params["sim_metric"] == "scaled_dot_product" else 1)
    same_rows = (ulp == 0).all(axis=-1)
    assert same_rows.mean() >= 0.75, f"only {same_rows.mean():.2f} of rows have bit-identical scores"
    # 2. identical selections on tie-free rows
    assert np.array_equal(ind[tf], gold_idx[tf])
    # 3. on rows with identical scores both are valid top-k sets of the same size
    nt_q, nt_k, nh, nw = grid
    bs = params["tile_size"][0] * params["tile_size"][1] * params["tile_size"][2]
    ntxt = (text_len + bs - 1) // bs
    nq, nk = nt_q * nh * nw, nt_k * nh * nw
    tt = params["tile_size"][0]
    rp = params.get("recent_protect", 0)
    forced = omask.forced_mask(nq, nk, nh, nw, n_recent=min(((rp + tt - 1) // tt) * nh * nw, nk) if rp else 0,
                               diag=params.get("force_diag", False), sink=params.get("force_sink", False),
                               neighbors=(mode == "prefill"))
    key = bf16_order_key(score)
    B, H = score.shape[:2]
    for b in range(B):
        for h in range(H):
            for r in range(nq):
                assert np.array_equal(ind[b, h, r, :ntxt], np.arange(ntxt))
                if not same_rows[b, h, r]:
                    continue
                mine, theirs = ind[b, h, r, ntxt:] - ntxt, gold_idx[b, h, r, ntxt:] - ntxt
                assert is_valid_topk(key[b, h, r], forced[r], mine)
                assert is_valid_topk(key[b, h, r], forced[r], theirs)


def test_one_hot_known_answer():
    # query pool e_0 (scaled), key pools c_j * e_0 with distinct c_j: dot ranking is the ranking of c_j
    D, nq, nk = 64, 3, 12
    c = np.array([0.5, 3.0, -1.0, 2.0, 0.25, 7.0, 1.5, -4.0, 6.0, 0.75, 5.0, 1.0], dtype=np.float32)
    q = np.zeros((1, 1, nq, D), np.float32)
    q[..., 0] = 1.0
    k = np.zeros((1, 1, nk, D), np.float32)
    k[0, 0, :, 0] = c
    qb, kb = f32_to_bf16(q), f32_to_bf16(k)
    params = {"tile_size": (1, 1, 1), "topk_ratio": 0.25, "sim_metric": "dot"}
    ind, cnt = omask.fast_generate_indices(qb, kb, 0, (3, 1, 1), (12, 1, 1), params)
    # k = int(12 * 0.25) = 3 largest: c = 7 (j=5), 6 (j=8), 5 (j=10)
    assert np.all(cnt == 3)
    assert np.array_equal(ind[0, 0, 0], [5, 8, 10])
    # cosine of one-hot vectors: +1 for c > 0, -1 for c < 0 -> ties broken towards the lower index
    params["sim_metric"] = "cosine"
    ind, _ = omask.fast_generate_indices(qb, kb, 0, (3, 1, 1), (12, 1, 1), params)
    assert np.array_equal(ind[0, 0, 0], [0, 1, 3])
    sc = omask.similarity(qb, kb, "cosine")
    assert np.array_equal(bf16_to_f32(sc[0, 0, 0]), np.sign(c))


def test_scaled_metric_rounding_points():
    # dot of exact small integers, then bf16(dot) * f32(1/sqrt(d)) rounded to bf16
    D = 128
    q = np.zeros((1, 1, 1, D), np.float32)
    k = np.zeros((1, 1, 2, D), np.float32)
    q[..., :3] = [1.0, 2.0, 3.0]
    k[0, 0, 0, :3] = [4.0, 5.0, 6.0]      # dot 32
    k[0, 0, 1, :3] = [100.0, 1.0, 0.0]    # dot 102
    s = bf16_to_f32(omask.similarity(f32_to_bf16(q), f32_to_bf16(k), "scaled_dot_product"))[0, 0, 0]
    scale = np.float32(1.0 / math.sqrt(D))
    expect = bf16_to_f32(f32_to_bf16(np.array([32.0, 102.0], np.float32) * scale))
    assert np.array_equal(s, expect)
    # and agrees with torch's bf16 arithmetic for the same expression
    t = (torch.tensor([[32.0, 102.0]]).to(torch.bfloat16) * (1.0 / math.sqrt(D))).float().numpy()[0]
    assert np.array_equal(s, t)


def test_budget_arithmetic():
    nq, nk = 4, 168
    f = np.zeros((nq, nk), bool)
    f[:, 0] = True
    f[:, 100] = True
    k = omask.budgets(f, 0.3, mode="history")
    assert np.all(k == 2 + int(166 * 0.3)) and k[0] == 51
    f2 = np.zeros((1, 100), bool)
    assert omask.budgets(f2, 0.29, mode="history")[0] == 28  # int(100*0.29) = int(28.999...) = 28
    assert omask.budgets(f2, 0.0, mode="history")[0] == 1    # clamp to >= 1
    assert omask.budgets(np.zeros((1, 0), bool), 0.5, mode="history")[0] == 0
    assert omask.budgets(np.zeros((1, 20), bool), 0.25, mode="total")[0] == 7   # max(int(5), 7)
    assert omask.budgets(np.zeros((1, 5), bool), 0.25, mode="total")[0] == 5    # min(., Nk)
    assert omask.budgets(np.zeros((1, 150), bool), 0.2, mode="total")[0] == 30
    fr = np.zeros((3, 50), bool)
    fr[:, :4] = True
    assert np.array_equal(omask.budgets(fr, 0.1, mode="history", row_budget=[2, 30, 99]), [4, 30, 50])


def test_forced_sets():
    nh, nw = 3, 3
    nk = 27
    m = omask.forced_mask(nk, nk, nh, nw, neighbors=True)
    assert m[13].sum() == 7 and m[0].sum() == 4        # centre of a 3x3x3 grid, corner
    assert np.array_equal(m, m.T)
    r = omask.forced_mask(4, 20, 2, 2, n_recent=8)
    assert np.all(r[:, 12:]) and not r[:, :12].any()
    d = omask.forced_mask(4, 12, 2, 2, diag=True, sink=True)
    for q in range(4):
        assert set(np.nonzero(d[q])[0]) == {12 - 4 + q, q % 4}


def test_ratio_extremes_and_bruteforce_ties():
    rng = np.random.default_rng(5)
    qp = f32_to_bf16(rng.standard_normal((1, 2, 6, 64)).astype(np.float32))
    kp = f32_to_bf16(rng.standard_normal((1, 2, 24, 64)).astype(np.float32))
    params = {"tile_size": (1, 2, 2), "topk_ratio": 1.0, "sim_metric": "dot"}
    ind, cnt = omask.fast_generate_indices(qp, kp, 0, (6, 2, 2), (24, 2, 2), params)
    assert np.all(cnt == 24) and np.all(ind == np.arange(24))
    params.update(topk_ratio=0.0, recent_protect=2)  # forced only: last ceil(2/1)*4 = 8 blocks
    ind, cnt = omask.fast_generate_indices(qp, kp, 0, (6, 2, 2), (24, 2, 2), params)
    assert np.all(cnt == 8) and np.all(ind == np.arange(16, 24))
    # brute force with heavy ties: integer-valued scores
    score = f32_to_bf16(rng.integers(-3, 4, size=(40, 30)).astype(np.float32))
    forced = np.zeros((40, 30), bool)
    forced[:, 7] = True
    k = np.full(40, 9)
    rows = omask.select_rows(score, forced, k)
    v = bf16_to_f32(score)
    for r in range(40):
        cand = [j for j in range(30) if not forced[r, j]]
        cand.sort(key=lambda j: (-v[r, j], j))
        assert np.array_equal(rows[r], np.sort([7] + cand[:8]))


def _f16_torch_bits(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def test_f16_conversions_match_torch():
    """The float16 element format: float32 -> half is torch's cast (ties, overflow, subnormals); half -> float32 exact."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-20, 14, 200000))).astype(np.float32)
    u = np.array([0x3F801000, 0x3F803000, 0x477FE000, 0x477FF000, 0x477FEFFF, 0x33800000, 0x33000000, 0x33000001,
                  0x387FC000, 0x80000000, 0x7F800000, 0xFF800000], dtype=np.uint32)
    x = np.concatenate([x, u.view(np.float32)])
    assert np.array_equal(omask.f32_to_f16(x), _f16_torch_bits(x))
    b = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    f = omask.f16_to_f32(b)
    fin = np.isfinite(f)
    assert np.array_equal(omask.f32_to_f16(f[fin]), b[fin])
    # half patterns order like bf16 ones (sign and magnitude): the same key function applies
    ks = bf16_order_key(b[fin])
    i, j = np.random.default_rng(6).integers(0, int(fin.sum()), (2, 100000))
    lt = f[fin][i] < f[fin][j]
    assert np.all(ks[i][lt] < ks[j][lt])


def test_f16_known_answers():
    """One-hot pools and a 3-4-5 vector in float16: dot ranking, cosine signs, the normaliser and the scale."""
    D, nq, nk = 64, 2, 12
    c = np.array([0.5, 3.0, -1.0, 2.0, 0.25, 7.0, 1.5, -4.0, 6.0, 0.75, 5.0, 1.0], dtype=np.float32)
    q = np.zeros((1, 1, nq, D), np.float32)
    q[..., 0] = 1.0
    k = np.zeros((1, 1, nk, D), np.float32)
    k[0, 0, :, 0] = c
    qb, kb = omask.f32_to_f16(q), omask.f32_to_f16(k)
    assert np.array_equal(omask.f16_to_f32(omask.similarity(qb, kb, "dot", "f16"))[0, 0, 0], c)
    assert np.array_equal(omask.f16_to_f32(omask.similarity(qb, kb, "cosine", "f16"))[0, 0, 0], np.sign(c))
    s = omask.f16_to_f32(omask.similarity(qb, kb, "scaled_dot_product", "f16"))[0, 0, 0]
    scale = np.float32(1.0 / math.sqrt(D))
    assert np.array_equal(s, (c * scale).astype(np.float16).astype(np.float32))
    ind, cnt, _, _ = omask.build_indices(qb, kb, metric="dot", forced=np.zeros((nq, nk), bool),
                                         k=np.full(nq, 3), num_txt_blk=0, fmt="f16")
    assert np.array_equal(ind[0, 0, 0], [5, 8, 10]) and np.all(cnt == 3)
    v = np.zeros((1, 1, 1, D), np.float32)
    v[..., :2] = [3.0, 4.0]
    n = omask.f16_to_f32(omask._normalize_bits(omask.f32_to_f16(v), "f16"))[0, 0, 0, :2]
    assert np.array_equal(n, np.array([0.6, 0.8], np.float16).astype(np.float32))
    # f16(1e-12) = 0: a zero vector divides by zero (NaN), as the float16 reference would
    z = omask._normalize_bits(np.zeros((1, 1, 1, D), np.uint16), "f16")
    assert np.all(np.isnan(omask.f16_to_f32(z)))


@pytest.mark.parametrize("metric", ["cosine", "scaled_dot_product", "dot"])
def test_f16_similarity_vs_torch_half(metric):
    """Scores of the float16 model against the reference's own torch calls run in float16 on the CPU: within one
    half ulp everywhere (the matmul sum order is the only freedom), equal selections on tie-free rows."""
    rng = np.random.default_rng(len(metric))
    B, H, nq, nk, D = 1, 2, 6, 40, 128
    q = (rng.standard_normal((B, H, nq, D)) * 0.5).astype(np.float32)
    k = (rng.standard_normal((B, H, nk, D)) * 0.5).astype(np.float32)
    qb, kb = omask.f32_to_f16(q), omask.f32_to_f16(k)
    ours = omask.similarity(qb, kb, metric, "f16")
    qt = torch.from_numpy(omask.f16_to_f32(qb)).to(torch.float16)
    kt = torch.from_numpy(omask.f16_to_f32(kb)).to(torch.float16)
    theirs = torch_ref.sim(qt, kt, metric).contiguous().view(torch.int16).numpy().view(np.uint16)
    d = np.abs(bf16_order_key(ours).astype(np.int64) - bf16_order_key(theirs).astype(np.int64))
    assert d.max() <= 1
    forced = np.zeros((nq, nk), bool)
    kk = np.full(nq, 9)
    for h in range(H):
        mine = omask.select_rows(ours[0, h], forced, kk)
        ref = omask.select_rows(theirs[0, h], forced, kk)
        tf = omask.tie_free(ours[0, h], forced, kk) & omask.tie_free(theirs[0, h], forced, kk)
        for r in np.nonzero(tf)[0]:
            assert np.array_equal(mine[r], ref[r])
