"""GPU: the allocation-free entry point li_bsa_fwd_gather_noalloc against li_bsa_fwd_gather.

Both run the same kernels with the same tail-split / tile-order decisions;
the allocation-free one keeps the split partials and the tile order in the
library's per-device scratch instead of a caller workspace, so the outputs
and LSE must be equal bit for bit.  Two calls in a row (the second with a
smaller input, reusing the scratch the first one wrote), with and without the
longest-first order.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from li_sparse import _core, _lib
from li_sparse._lib import TileGeom, i64_array, lib

pytestmark = pytest.mark.gpu


def _case(seed, heads, frames_q, frames_k, ragged, dev):
    H, W, tile = 30, 52, (2, 8, 8)
    nh, nw = 4, 7
    g = torch.Generator().manual_seed(seed)

    def tok(frames, scale=1.0):
        return (torch.randn(1, frames * H * W, heads, 128, generator=g) * scale).to(torch.bfloat16).to(dev) \
            .permute(0, 2, 1, 3)

    q, k, v = tok(frames_q, 0.3), tok(frames_k), tok(frames_k)
    nq, nk = (frames_q // 2) * nh * nw, (frames_k // 2) * nh * nw
    rng = np.random.default_rng(seed)
    kmax = min(nk, 60)
    ind = np.zeros((1, heads, nq, kmax), np.int32)
    cnt = np.zeros((1, heads, nq), np.int32)
    for h in range(heads):
        for r in range(nq):
            n = int(rng.integers(1, kmax + 1)) if ragged else kmax - 9
            ind[0, h, r, :n] = np.sort(rng.choice(nk, size=n, replace=False))
            cnt[0, h, r] = n
    geo = (frames_q, frames_k, H, W, tile, nh, nw)
    return q, k, v, torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev), geo


def _noalloc(q, k, v, ind, cnt, geo, out, lse, balance):
    fq, fk, H, W, (tt, th, tw), nh, nw = geo
    gq, gk = TileGeom(fq, H, W, tt, th, tw, nh, nw), TileGeom(fk, H, W, tt, th, tw, nh, nw)
    B, NH, _, D = q.shape
    st = lib.li_bsa_fwd_gather_noalloc(_lib.LI_DTYPE_BF16, B, NH, D, q.data_ptr(), i64_array(q.stride()),
                                       k.data_ptr(), i64_array(k.stride()), v.data_ptr(), i64_array(v.stride()),
                                       None, None, 0, ctypes.byref(gq), ctypes.byref(gk), ind.data_ptr(),
                                       i64_array(ind.stride()), ind.shape[3], cnt.data_ptr(),
                                       i64_array(cnt.stride()), ctypes.c_float(1.0 / math.sqrt(D)), out.data_ptr(),
                                       i64_array(out.stride()), lse.data_ptr(),
                                       _lib.LI_BSA_BALANCE if balance else 0,
                                       ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream))
    _lib.check("li_bsa_fwd_gather_noalloc", st)


@pytest.mark.parametrize("balance", [False, True])
def test_noalloc_equals_workspace_entry_point(dev, balance):
    assert lib.li_bsa_fwd_noalloc_scratch_bytes() == 32 << 20
    # HY shape (896 query tiles: 128 of them split on 256 CUs), then a smaller call (6 heads, 2 slabs).
    for seed, heads, fq, fk in ((1, 16, 4, 12), (2, 6, 4, 8)):
        print(f"[gpu] noalloc vs workspace entry point: heads={heads} frames q/k={fq}/{fk} balance={balance}",
              flush=True)
        q, k, v, ind, cnt, geo = _case(seed, heads, fq, fk, balance, dev)
        fq_, fk_, H, W, (tt, th, tw), nh, nw = geo
        scale = 1.0 / math.sqrt(128)
        ref = torch.empty_like(q)
        _, lse_ref = _core.bsa_forward_gather(q, k, v, None, None, 0, fq_, fk_, H, W, tt, th, tw, nh, nw, ind, cnt,
                                              scale, ref, return_lse=True, split=True, balance=balance)
        out = torch.full_like(q, float("nan"))
        lse = torch.full_like(lse_ref, float("nan"))
        _noalloc(q, k, v, ind, cnt, geo, out, lse, balance)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(lse.view(torch.int32), lse_ref.view(torch.int32))


def test_noalloc_rejects_invalid_arguments(dev):
    q, k, v, ind, cnt, geo = _case(3, 2, 2, 4, False, dev)
    fq, fk, H, W, (tt, th, tw), nh, nw = geo
    gq = TileGeom(fq, H, W, tt, th, tw, nh, nw)
    gk = TileGeom(fk, H, W, tt, th, tw, nh, nw + 1)   # inconsistent key grid
    out = torch.empty_like(q)
    st = lib.li_bsa_fwd_gather_noalloc(_lib.LI_DTYPE_BF16, 1, 2, 128, q.data_ptr(), i64_array(q.stride()),
                                       k.data_ptr(), i64_array(k.stride()), v.data_ptr(), i64_array(v.stride()),
                                       None, None, 0, ctypes.byref(gq), ctypes.byref(gk), ind.data_ptr(),
                                       i64_array(ind.stride()), ind.shape[3], cnt.data_ptr(),
                                       i64_array(cnt.stride()), ctypes.c_float(0.1), out.data_ptr(),
                                       i64_array(out.stride()), None, 0, None)
    assert st == _lib.LI_ERR_SHAPE
