"""GPU: size-independent properties of the attention path at the full HY-WorldPlay shape.

The float64 oracle is too slow to compare every tile at this size (16 heads,
6240 queries, 18720 keys); the sampled-tile tests cover it tile by tile.
These tests check every tile through identities attention must satisfy,
with the block lists of the real mask:

* LSE combination: attention over a kept list equals the combination of
  attention over the list's first and second halves, weighted by their
  log-sum-exps, and the LSEs combine the same way (the identity the tail split
  and the reference's online softmax rest on, HYK:102-155);
* order invariance: each row's list in reverse order gives the same output
  (only the accumulation order changes);
* all blocks kept: on a grid without padding, the sparse kernel keeping
  every key block equals this library's dense kernel over the same keys.
"""
import math

import numpy as np
import pytest
import torch

from li_sparse import _core, _pipeline
from li_sparse.hy.ar_sparse_operation import fast_generate_indices
from li_sparse.workloads import WORKLOADS, Workload, make_qkv

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _setup(dev, wl):
    q, k, v = make_qkv(wl, seed=3, layout="blhd")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    g = _pipeline.geometry(wl.latent_hw, wl.tile, wl.lq, wl.lk, 0)
    B, H, D, bs = wl.batch, wl.heads, wl.head_dim, g.bs
    q_t = torch.empty((B, H, g.nq_blk, bs, D), dtype=torch.bfloat16, device=dev)
    q_p = torch.empty((B, H, g.nq_blk, D), dtype=torch.bfloat16, device=dev)
    k_all = torch.empty((B, H, g.nk_blk, bs, D), dtype=torch.bfloat16, device=dev)
    v_all = torch.empty_like(k_all)
    k_p = torch.empty((B, H, g.nk_blk, D), dtype=torch.bfloat16, device=dev)
    _core.q_prep(qd, q_t, q_p, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.kv_prep(kd, vd, k_all, v_all, k_p, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    ind, cnt = fast_generate_indices(q_p, k_p, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw),
                                     wl.sparse_params(g.nq_blk), dev)
    return dict(qd=qd, kd=kd, vd=vd, g=g, qf=q_t.flatten(2, 3), kf=k_all.flatten(2, 3), vf=v_all.flatten(2, 3),
                ind=ind, cnt=cnt, scale=1.0 / math.sqrt(D))


def test_lse_combination_of_list_halves_full_hy(dev):
    print("[gpu] LSE combination of list halves, full HY shape (896 tiles, real mask)", flush=True)
    s = _setup(dev, WORKLOADS["hy"])
    ind, cnt = s["ind"].cpu().numpy(), s["cnt"].cpu().numpy()
    ca = (cnt + 1) // 2
    cb = cnt - ca
    ind_b = np.zeros_like(ind)
    for b, h, m in zip(*np.nonzero(cb > 0)):
        ind_b[b, h, m, :cb[b, h, m]] = ind[b, h, m, ca[b, h, m]:cnt[b, h, m]]
    run = lambda ii, cc: _core.bsa_forward(s["qf"], s["kf"], s["vf"], torch.from_numpy(ii).to(dev),  # noqa: E731
                                           torch.from_numpy(cc).to(dev), s["scale"], 128, return_lse=True)
    o_all, l_all = run(ind, cnt)
    o_a, l_a = run(ind, ca)
    o_b, l_b = run(ind_b, cb)
    torch.cuda.synchronize()
    la, lb = l_a.double(), l_b.double()
    mx = torch.maximum(la, lb)
    wa, wb = torch.exp2(la - mx), torch.exp2(lb - mx)   # an empty half has LSE -inf: weight 0
    comb = (o_a.double() * wa[..., None] + o_b.double() * wb[..., None]) / (wa + wb)[..., None]
    l_comb = mx + torch.log2(wa + wb)
    err = (comb - o_all.double()).abs().max().item()
    lerr = (l_comb - l_all.double()).abs().max().item()
    print(f"[gpu]   rows with two halves {int((cb > 0).sum())} of {cb.size}; max |combined - whole| {err:.3e}, "
          f"LSE {lerr:.3e}", flush=True)
    assert (cb > 0).all() and torch.isfinite(l_all).all()
    assert err <= TOL and lerr <= 1e-3


def test_reversed_lists_full_hy(dev):
    print("[gpu] reversed block lists, full HY shape, fused kernel", flush=True)
    s = _setup(dev, WORKLOADS["hy"])
    g = s["g"]
    ind, cnt = s["ind"].cpu().numpy(), s["cnt"].cpu().numpy()
    ind_r = ind.copy()
    for b, h, m in np.ndindex(*cnt.shape):
        ind_r[b, h, m, :cnt[b, h, m]] = ind[b, h, m, :cnt[b, h, m]][::-1]
    outs = []
    for ii, sorted_lists in ((ind, True), (ind_r, False), (ind_r, True)):
        o = torch.empty_like(s["qd"])
        _, l = _core.bsa_forward_gather(s["qd"], s["kd"], s["vd"], None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th,
                                        g.tw, g.nh, g.nw, torch.from_numpy(ii).to(dev), s["cnt"], s["scale"], o,
                                        return_lse=True, sorted_lists=sorted_lists)
        outs.append((o, l))
    torch.cuda.synchronize()
    (o0, l0), (o1, l1), (o2, l2) = outs
    err = (o1.float() - o0.float()).abs().max().item()
    lerr = (l1 - l0).abs().max().item()
    print(f"[gpu]   max |reversed - ascending| {err:.3e}, LSE {lerr:.3e}", flush=True)
    assert err <= 1e-2 and lerr <= 1e-4
    # with no text blocks the zero-region loads take any order: the same bits as the general loads
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_all_blocks_kept_equals_dense_kernel(dev):
    """A 32 x 56 latent with 2x8x8 tiles has no padding rows, so keeping every key block is dense attention."""
    wl = Workload("dense_check", 8, 128, (32, 56), 4, 12, (2, 8, 8), 1.0, "scaled_dot_product")
    print("[gpu] all blocks kept vs the dense kernel (8 heads, 32x56 latent, Lq=7168, Lk=21504)", flush=True)
    q, k, v = make_qkv(wl, seed=5, layout="blhd")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    g = _pipeline.geometry(wl.latent_hw, wl.tile, wl.lq, wl.lk, 0)
    assert g.nq_blk * 128 == wl.lq and g.nk_blk * 128 == wl.lk
    B, H = wl.batch, wl.heads
    ind = torch.arange(g.nk_blk, dtype=torch.int32, device=dev).expand(B, H, g.nq_blk, g.nk_blk).contiguous()
    cnt = torch.full((B, H, g.nq_blk), g.nk_blk, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(wl.head_dim)
    o_s = torch.empty_like(qd)
    _core.bsa_forward_gather(qd, kd, vd, None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt,
                             scale, o_s, sorted_lists=True)
    o_d = _core.attn_dense(qd, kd, vd, sm_scale=scale)
    torch.cuda.synchronize()
    err = (o_s.float() - o_d.float()).abs().max().item()
    print(f"[gpu]   max |sparse, all blocks - dense| {err:.3e}", flush=True)
    assert err <= 1e-2
