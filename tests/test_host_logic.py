"""Host-side logic of the product (geometry, forced counts, budgets) against the oracle; CPU only."""
import numpy as np
import pytest

from li_sparse import _core, _lib, _pipeline
from li_sparse.workloads import WORKLOADS, ragged_budgets
from oracle import mask as omask
from oracle.geometry import block_geometry


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_geometry_matches_oracle(name):
    wl = WORKLOADS[name]
    g = _pipeline.geometry(wl.latent_hw, wl.tile, wl.lq, wl.lk, 0)
    o = block_geometry(wl.lq, wl.lk, wl.latent_hw, wl.tile)
    assert (g.bs, g.nh, g.nw, g.nq_blk, g.nk_blk, g.num_txt_blk) == (o["BS"], o["nh"], o["nw"], o["nq_blk"],
                                                                   o["nk_blk"], o["num_txt_blk"])
    g2 = _pipeline.geometry(wl.latent_hw, wl.tile, wl.lq, wl.lk, 77)
    assert g2.num_txt_blk == block_geometry(wl.lq, wl.lk, wl.latent_hw, wl.tile, 77)["num_txt_blk"]


def test_forced_counts_and_budgets_match_oracle():
    rng = np.random.default_rng(0)
    for _ in range(300):
        nh, nw = int(rng.integers(1, 6)), int(rng.integers(1, 8))
        nq = int(rng.integers(1, 4)) * nh * nw
        nk = nq + int(rng.integers(0, 5)) * nh * nw
        kw = dict(n_recent=int(rng.integers(0, nk + 1)) if rng.random() < 0.3 else 0, diag=bool(rng.random() < .5),
                  sink=bool(rng.random() < .5), neighbors=bool(rng.random() < .3))
        if rng.random() < 0.2:
            nq, nk = nk, nq  # more query than key blocks
        f = omask.forced_mask(nq, nk, nh, nw, **kw)
        nf = _core.forced_counts(nq, nk, nh, nw, kw["n_recent"], kw["diag"], kw["sink"], kw["neighbors"])
        assert np.array_equal(nf, f.sum(axis=1))
        ratio = float(rng.choice([0.0, 0.1, 0.175, 0.25, 0.29, 0.3, 1.0]))
        for mode, code in (("history", _lib.LI_BUDGET_HISTORY), ("total", _lib.LI_BUDGET_TOTAL)):
            assert np.array_equal(_core.row_budgets(nf, nk, code, ratio), omask.budgets(f, ratio, mode=mode))
        rb = rng.integers(0, nk + 3, size=nq)
        assert np.array_equal(_core.row_budgets(nf, nk, 0, ratio, row_budget=rb),
                              omask.budgets(f, ratio, mode="history", row_budget=rb))


def test_workload_budgets():
    hy = WORKLOADS["hy"]
    g = _pipeline.geometry(hy.latent_hw, hy.tile, hy.lq, hy.lk, 0)
    nf = _core.forced_counts(g.nq_blk, g.nk_blk, g.nh, g.nw, 0, True, True)
    k = _core.row_budgets(nf, g.nk_blk, _lib.LI_BUDGET_HISTORY, hy.ratio)
    assert np.all(nf == 2) and np.all(k == 51)  # 2 forced + int(166 * 0.3)
    rb = ragged_budgets(56, 8, 200)
    assert min(rb) == 8 and max(rb) == 200 and 0.09 < np.mean(rb) / 896 < 0.115


def test_forced_blocks_and_tie_free_fraction_match_oracle():
    """The bench's tie-free row count (product code) against the oracle's per-row test on random bf16 scores."""
    import torch

    rng = np.random.default_rng(11)
    nq, nk, nh, nw = 28, 140, 4, 7
    for diag, sink, n_recent in [(True, True, 0), (False, False, 28), (True, False, 28)]:
        forced = _core.forced_blocks(nq, nk, nh, nw, n_recent, diag, sink)
        assert np.array_equal(forced, omask.forced_mask(nq, nk, nh, nw, n_recent=n_recent, diag=diag, sink=sink))
        # few distinct values so that ties are common
        vals = rng.integers(-40, 40, size=(2, nq, nk)).astype(np.float32) / 16.0
        bits = torch.from_numpy(vals).to(torch.bfloat16)
        k = omask.budgets(forced, 0.3, mode="history")
        counts = torch.from_numpy(np.broadcast_to(k, (2, nq)).astype(np.int32).copy())
        b = bits.view(torch.int16).numpy().view(np.uint16)
        want = np.mean([omask.tie_free(b[i], forced, k) for i in range(2)])
        got = _core.tie_free_fraction(bits, counts, forced)
        assert abs(got - want) < 1e-12 and 0.0 < got < 1.0


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and says so, before touching any device."""
    import os
    import subprocess
    import sys

    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(repo, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
