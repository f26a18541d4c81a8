"""li_pool_pair: the query and key pools of one call in a single launch.

Checked bit for bit against two li_pool launches (whose means are pinned
against the oracle's tile pool in the tile tests), on the HY decode geometry
(different frame counts, a pool offset into a larger buffer) and on the
fallback cases: sources that differ in vector access, and a key job with no
blocks.  Rows of the pool buffers outside each job are checked untouched.
The optional normalised key pool is checked bit for bit against the oracle's
cosine normalisation of the key pool, and the block mask scored through it
against the block mask normalising the raw pool itself.
"""
import ctypes

import pytest
import torch

import li_sparse._lib as L
from li_sparse import _core
from oracle import mask as omask


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


def _bits(x):
    return x.view(torch.int16).cpu().numpy().view("uint16")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,D,vec", [(torch.bfloat16, 128, True), (torch.float16, 64, True),
                                         (torch.bfloat16, 128, False)])
def test_pair_normalized_key_pool(dtype, D, vec):
    """mean1_normalized: the oracle's cosine normalisation of mean1, bit for bit; mean1 itself unchanged."""
    print(f"[gpu] pool_pair normalised key pool {dtype} D={D} vec={vec}", flush=True)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(13)
    B, NH, hw, tile = 1, 3, (30, 52), (2, 8, 8)
    H, W = hw
    nh, nw = -(-H // 8), -(-W // 8)
    q = torch.randn((B, NH, 2 * H * W, D), generator=g).to(dev, dtype)
    kbig = torch.randn((B, NH, 6 * H * W, 2 * D), generator=g).to(dev, dtype)
    kbig[:, :, 2 * H * W:4 * H * W] = 0  # the blocks of t-slab 1 pool to zero rows (normaliser = eps)
    kbig[:, 1, :H * W] *= 1e-3  # small rows
    k = kbig[..., :D] if vec else kbig[..., ::2]
    gq, gk = (2, H, W, 2, 8, 8, nh, nw), (6, H, W, 2, 8, 8, nh, nw)
    nq, nk, k_off = 1 * nh * nw, 3 * nh * nw, 5
    qp = _sentinel((B, NH, nq, D), dev, dtype)
    kp1, kp2, kn = (_sentinel((B, NH, nk + k_off + 1, D), dev, dtype) for _ in range(3))
    _core.pool_pair(q, qp, 0, gq, k, kp1, k_off, gk)
    _core.pool_pair(q, qp, 0, gq, k, kp2, k_off, gk, mean1_normalized=kn)
    torch.cuda.synchronize()
    assert torch.equal(kp1.view(torch.int16), kp2.view(torch.int16))
    rows = slice(k_off, k_off + nk)
    fmt = "bf16" if dtype == torch.bfloat16 else "f16"
    want = omask._normalize_bits(_bits(kp2[:, :, rows]), fmt)
    assert (_bits(kn[:, :, rows]) == want).all()
    assert (kn[:, :, :k_off] == 3.0).all().item() and (kn[:, :, nk + k_off:] == 3.0).all().item()
    zero_rows = kn[:, :, k_off + nh * nw:k_off + 2 * nh * nw]
    if dtype == torch.bfloat16:
        assert (zero_rows == 0).all().item()
    else:  # fp16 rounds the 1e-12 floor to 0, so 0 / 0, as F.normalize in half precision
        assert zero_rows.isnan().all().item()


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["tiled", "generic"])
def test_mask_through_normalized_pool(kernel):
    """The cosine block mask scored through the normalised pool equals the mask on the raw pool: indices,
    counts and scores, bit for bit (shared-pool kernel for aligned pools, per-row kernel for strided ones)."""
    print(f"[gpu] block mask through the normalised key pool ({kernel})", flush=True)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device="cpu").manual_seed(14)
    B, NH, D, H, W = 1, 4, 128, 22, 40
    nh, nw = -(-H // 8), -(-W // 8)
    q = torch.randn((B, NH, 4 * H * W, D), generator=g).to(dev, torch.bfloat16)
    k = torch.randn((B, NH, 20 * H * W, D), generator=g).to(dev, torch.bfloat16)
    gq, gk = (4, H, W, 2, 8, 8, nh, nw), (20, H, W, 2, 8, 8, nh, nw)
    nq, nk = 2 * nh * nw, 10 * nh * nw
    qp = torch.empty((B, NH, nq, D), dtype=torch.bfloat16, device=dev)
    def pool_buf():
        if kernel == "tiled":
            return torch.empty((B, NH, nk, D), dtype=torch.bfloat16, device=dev)
        return torch.empty((B, NH, nk, 2 * D), dtype=torch.bfloat16, device=dev)[..., ::2]

    kp, kn = pool_buf(), pool_buf()
    _core.pool_pair(q, qp, 0, gq, k, kp, 0, gk, mean1_normalized=kn)
    kw = dict(metric="cosine", budget_mode=L.LI_BUDGET_TOTAL, ratio=0.25, nh=nh, nw=nw, num_txt_blk=1,
              force_neighbors=True, return_scores=True)
    raw = _core.block_mask(qp, kp, **kw)
    kp2 = pool_buf().copy_(kp)
    via = _core.block_mask(qp, kp2, k_pool_normalized=kn, **kw)
    dot = _core.block_mask(qp, kp2, k_pool_normalized=kn, **dict(kw, metric="dot"))  # other metrics ignore it
    dot_raw = _core.block_mask(qp, kp, **dict(kw, metric="dot"))
    torch.cuda.synchronize()
    for a, b in zip(raw, via):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)
    for a, b in zip(dot, dot_raw):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)


def test_pair_host_validation_needs_no_gpu():
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    s4 = L.i64_array([1, 1, 1, 1])
    geo = L.TileGeom(2, 30, 52, 2, 8, 8, 4, 7)
    f = L.lib.li_pool_pair
    assert f(0, 1, 1, 128, None, s4, fake, s4, 0, ctypes.byref(geo), fake, s4, fake, s4, 0, ctypes.byref(geo), None, None) == L.LI_ERR_INVALID_ARG
    assert f(0, 1, 1, 128, fake, s4, fake, s4, 0, ctypes.byref(geo), fake, s4, fake, s4, -1, ctypes.byref(geo), None, None) == L.LI_ERR_INVALID_ARG
    bad = L.TileGeom(2, 30, 52, 2, 8, 8, 3, 7)  # nh does not cover H
    assert f(0, 1, 1, 128, fake, s4, fake, s4, 0, ctypes.byref(geo), fake, s4, fake, s4, 0, ctypes.byref(bad), None, None) == L.LI_ERR_SHAPE
