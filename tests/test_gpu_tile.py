"""GPU parity: tile gather / pool / untile vs the oracle, bit-exact."""
import numpy as np
import pytest
import torch

from helpers import bits
from li_sparse import _core
from li_sparse.workloads import WORKLOADS, make_qkv
from oracle import tile as otile
from oracle.geometry import block_geometry

pytestmark = pytest.mark.gpu


def _geo(wl):
    g = block_geometry(wl.lq, wl.lk, wl.latent_hw, wl.tile)
    return g


@pytest.mark.parametrize("name,layout", [("toy", "bhld"), ("toy", "blhd"), ("hy", "blhd"), ("mg", "bhld")])
def test_q_and_kv_prep_bit_exact(dev, name, layout):
    wl = WORKLOADS[name]
    print(f"[gpu] tile gather {name} layout={layout}", flush=True)
    q, k, v = make_qkv(wl, seed=1, layout=layout)
    g = _geo(wl)
    H, W = wl.latent_hw
    tt, th, tw = wl.tile
    B, NH, D, bs = wl.batch, wl.heads, wl.head_dim, g["BS"]
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    q_t = torch.empty((B, NH, g["nq_blk"], bs, D), dtype=torch.bfloat16, device=dev)
    q_p = torch.empty((B, NH, g["nq_blk"], D), dtype=torch.bfloat16, device=dev)
    _core.q_prep(qd, q_t, q_p, g["T_q"], H, W, tt, th, tw, g["nh"], g["nw"])
    ntxt = 2
    k_all = torch.full((B, NH, ntxt + g["nk_blk"], bs, D), 7.0, dtype=torch.bfloat16, device=dev)
    v_all = torch.full_like(k_all, 7.0)
    k_p = torch.empty((B, NH, g["nk_blk"], D), dtype=torch.bfloat16, device=dev)
    _core.kv_prep(kd, vd, k_all, v_all, k_p, ntxt, 0, g["T_k"], H, W, tt, th, tw, g["nh"], g["nw"])
    torch.cuda.synchronize()
    oq = otile.tile_gather(bits(q), g["T_q"], H, W, wl.tile)
    ok_ = otile.tile_gather(bits(k), g["T_k"], H, W, wl.tile)
    ov = otile.tile_gather(bits(v), g["T_k"], H, W, wl.tile)
    assert np.array_equal(bits(q_t), oq)
    assert np.array_equal(bits(q_p), otile.pool_mean(oq))
    assert np.array_equal(bits(k_all[:, :, ntxt:]), ok_)
    assert np.array_equal(bits(v_all[:, :, ntxt:]), ov)
    assert torch.all(k_all[:, :, :ntxt] == 7.0) and torch.all(v_all[:, :, :ntxt] == 7.0)  # text blocks untouched
    assert np.array_equal(bits(k_p), otile.pool_mean(ok_))


@pytest.mark.parametrize("name,layout", [("toy", "blhd"), ("hy", "bhld"), ("hy", "blhd")])
def test_untile_roundtrip(dev, name, layout):
    wl = WORKLOADS[name]
    print(f"[gpu] untile {name} layout={layout}", flush=True)
    q, _, _ = make_qkv(wl, seed=2, layout=layout)
    g = _geo(wl)
    H, W = wl.latent_hw
    tt, th, tw = wl.tile
    qd = q.to(dev)
    q_t = torch.empty((wl.batch, wl.heads, g["nq_blk"], g["BS"], wl.head_dim), dtype=torch.bfloat16, device=dev)
    q_p = torch.empty((wl.batch, wl.heads, g["nq_blk"], wl.head_dim), dtype=torch.bfloat16, device=dev)
    _core.q_prep(qd, q_t, q_p, g["T_q"], H, W, tt, th, tw, g["nh"], g["nw"])
    out = torch.zeros_like(qd)                    # keeps q's strides, as empty_like(q) does
    assert out.stride() == qd.stride()
    _core.untile(q_t, out, g["T_q"], H, W, tt, th, tw, g["nh"], g["nw"])
    torch.cuda.synchronize()
    assert torch.equal(out, qd)


def test_f16_and_odd_strides(dev):
    # fp16 pooling and a non-unit innermost stride (scalar path)
    print("[gpu] tile gather f16 + strided d", flush=True)
    T, H, W, tile, D = 3, 10, 13, (2, 4, 8), 64
    g = block_geometry(T * H * W, T * H * W, (H, W), tile)
    rng = np.random.default_rng(3)
    base = torch.from_numpy(rng.standard_normal((1, 2, T * H * W, 2 * D)).astype(np.float32)).to(torch.float16)
    x = base.to(dev)[..., ::2]                    # d stride 2
    tt, th, tw = tile
    q_t = torch.empty((1, 2, g["nq_blk"], g["BS"], D), dtype=torch.float16, device=dev)
    q_p = torch.empty((1, 2, g["nq_blk"], D), dtype=torch.float16, device=dev)
    _core.q_prep(x, q_t, q_p, T, H, W, tt, th, tw, g["nh"], g["nw"])
    torch.cuda.synchronize()
    xt = base[..., ::2].contiguous()
    ot = otile.tile_gather(bits(xt), T, H, W, tile)
    assert np.array_equal(bits(q_t), ot)
    # f16 pool: fixed-order fp32 sum / BS rounded to f16
    ref = torch.from_numpy(ot.view(np.float16).astype(np.float32))
    ng = 256 // (D // 8)
    part = torch.zeros(1, 2, g["nq_blk"], ng, D)
    for f in range(g["BS"]):
        part[:, :, :, f % ng] += ref[:, :, :, f]
    s = ng // 2
    while s >= 1:
        part[:, :, :, :s] = part[:, :, :, :s] + part[:, :, :, s:2 * s]
        s //= 2
    expect = (part[:, :, :, 0] / g["BS"]).to(torch.float16)
    assert torch.equal(q_p.cpu(), expect)
