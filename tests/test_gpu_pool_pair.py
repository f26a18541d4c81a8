"""li_pool_pair: the query and key pools of one call in a single launch.

Checked bit for bit against two li_pool launches (whose means are pinned
against the oracle's tile pool in the tile tests), on the HY decode geometry
(different frame counts, a pool offset into a larger buffer) and on the
fallback cases: sources that differ in vector access, and a key job with no
blocks.  Rows of the pool buffers outside each job are checked untouched.
"""
import ctypes

import pytest
import torch

import li_sparse._lib as L
from li_sparse import _core


def _sentinel(shape, dev, dtype):
    return torch.full(shape, 3.0, device=dev, dtype=dtype)


def _case(q, k, hw, tile, Tq, Tk, k_off, dtype):
    H, W = hw
    tt, th, tw = tile
    nh, nw = -(-H // th), -(-W // tw)
    B, NH, _, D = q.shape
    nq = _core.num_blocks(Tq, tt, nh, nw)
    nk = _core.num_blocks(Tk, tt, nh, nw)
    gq = (Tq, H, W, tt, th, tw, nh, nw)
    gk = (Tk, H, W, tt, th, tw, nh, nw)
    dev = q.device
    qp1, qp2 = _sentinel((B, NH, nq + 2, D), dev, dtype), _sentinel((B, NH, nq + 2, D), dev, dtype)
    kp1, kp2 = _sentinel((B, NH, nk + k_off + 1, D), dev, dtype), _sentinel((B, NH, nk + k_off + 1, D), dev, dtype)
    _core.pool(q, qp1, 0, *gq)
    if nk:
        _core.pool(k, kp1, k_off, *gk)
    _core.pool_pair(q, qp2, 0, gq, k, kp2, k_off, gk)
    torch.cuda.synchronize()
    assert torch.equal(qp1.view(torch.int16), qp2.view(torch.int16))
    assert torch.equal(kp1.view(torch.int16), kp2.view(torch.int16))
    assert (qp2[:, :, nq:] == 3.0).all().item()
    assert (kp2[:, :, :k_off] == 3.0).all().item() and (kp2[:, :, nk + k_off:] == 3.0).all().item()


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["bhld", "blhd"])
def test_pair_matches_two_pools_hy_geometry(layout):
    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(11)
    B, NH, D, hw, tile = 1, 3, 128, (30, 52), (2, 8, 8)
    Lq, Lk = 4 * 30 * 52, 12 * 30 * 52
    if layout == "bhld":
        q = torch.randn((B, NH, Lq, D), generator=g).to(dev, torch.bfloat16)
        k = torch.randn((B, NH, Lk, D), generator=g).to(dev, torch.bfloat16)
    else:
        q = torch.randn((B, Lq, NH, D), generator=g).to(dev, torch.bfloat16).transpose(1, 2)
        k = torch.randn((B, Lk, NH, D), generator=g).to(dev, torch.bfloat16).transpose(1, 2)
    _case(q, k, hw, tile, 4, 12, 0, torch.bfloat16)
    # key frames from 4 on (a cached context prefix), written after the first 2 * 4 * 7 pool rows
    _case(q, k[:, :, 4 * 30 * 52:], hw, tile, 4, 8, 2 * 4 * 7, torch.bfloat16)


@pytest.mark.gpu
def test_pair_fallbacks():
    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(12)
    B, NH, D, hw, tile = 2, 2, 64, (9, 20), (1, 4, 4)
    q = torch.randn((B, NH, 3 * 180, D), generator=g).to(dev, torch.float16)
    kbig = torch.randn((B, NH, 5 * 180, 2 * D), generator=g).to(dev, torch.float16)
    k = kbig[..., ::2]  # innermost stride 2: element-wise loads, so the jobs launch one after the other
    _case(q, k, hw, tile, 3, 5, 1, torch.float16)
    _case(q, kbig[..., :D], hw, tile, 3, 5, 1, torch.float16)  # row stride 2D, still vector access
    _case(q, kbig[..., :D], hw, tile, 3, 0, 0, torch.float16)  # no key blocks: the query pool alone


def test_pair_host_validation_needs_no_gpu():
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    s4 = L.i64_array([1, 1, 1, 1])
    geo = L.TileGeom(2, 30, 52, 2, 8, 8, 4, 7)
    f = L.lib.li_pool_pair
    assert f(0, 1, 1, 128, None, s4, fake, s4, 0, ctypes.byref(geo), fake, s4, fake, s4, 0, ctypes.byref(geo), None) == L.LI_ERR_INVALID_ARG
    assert f(0, 1, 1, 128, fake, s4, fake, s4, 0, ctypes.byref(geo), fake, s4, fake, s4, -1, ctypes.byref(geo), None) == L.LI_ERR_INVALID_ARG
    bad = L.TileGeom(2, 30, 52, 2, 8, 8, 3, 7)  # nh does not cover H
    assert f(0, 1, 1, 128, fake, s4, fake, s4, 0, ctypes.byref(geo), fake, s4, fake, s4, 0, ctypes.byref(bad), None) == L.LI_ERR_SHAPE
