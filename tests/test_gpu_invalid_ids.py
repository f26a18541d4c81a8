"""GPU: block ids outside [0, nkb) in the lists of the D = 128 attention kernels.

``longcat_flash_attn`` raises on such ids (longcat_kernel.py:192-195) before
any launch, but the C ABI and the MG entry point (which checks nothing,
matrix-game-3.0 longcat_kernel.py:137-190) hand them to the kernel.  The
D = 128 kernels fetch block 0 in their place and give it zero probability,
so an invalid id adds nothing: each launch below is compared with the float64
oracle run on the same lists with the invalid ids dropped.  Covered: the tiled
bf16 kernel (whole tiles and the balanced order), the fused kernel (token
order, with a text block), the tiled e4m3 kernel and the fused e4m3 kernel;
invalid ids first, last, in the middle and filling a whole row (zeros, LSE
-inf).  Also the lists with nothing to read: index tensors with no columns,
and split tiles whose second half is empty in a one-column index tensor.
"""
import math

import numpy as np
import pytest
import torch

from helpers import bits
from li_sparse import _core
from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import tile as otile
from oracle.bf16 import bf16_to_f32
from oracle.geometry import tile_permutation

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _lists(nq, nkb, H=2):
    """Rows with ids below 0 and at or above nkb; returns (indices, counts, cleaned indices, cleaned counts)."""
    bad = [-3, -1, nkb, nkb + 5, 1 << 20, -(1 << 30)]
    rng = np.random.default_rng(nkb * 31 + nq)
    kmax = 6
    ind = np.zeros((1, H, nq, kmax), np.int32)
    cnt = np.zeros((1, H, nq), np.int32)
    for h in range(H):
        for r in range(nq):
            kind = (h * nq + r) % 5
            n = int(rng.integers(2, kmax + 1))
            good = list(rng.choice(nkb, size=n, replace=False))
            if kind == 0:                      # invalid first
                row = [bad[r % len(bad)]] + good[:n - 1]
            elif kind == 1:                    # invalid last
                row = good[:n - 1] + [bad[(r + 1) % len(bad)]]
            elif kind == 2:                    # invalid in the middle, twice
                row = good[:1] + [bad[(r + 2) % len(bad)], bad[(r + 3) % len(bad)]] + good[1:n - 2]
            elif kind == 3:                    # only invalid ids: zeros and LSE -inf
                row = [bad[(r + j) % len(bad)] for j in range(n)]
            else:                              # all valid
                row = good
            ind[0, h, r, :len(row)] = row
            cnt[0, h, r] = len(row)
    ok_ind = np.zeros_like(ind)
    ok_cnt = np.zeros_like(cnt)
    for h in range(H):
        for r in range(nq):
            row = [int(x) for x in ind[0, h, r, :cnt[0, h, r]] if 0 <= x < nkb]
            ok_ind[0, h, r, :len(row)] = row
            ok_cnt[0, h, r] = len(row)
    assert (ok_cnt < cnt).any() and (ok_cnt == 0).any()
    return ind, cnt, ok_ind, ok_cnt


def _check(out, lse, o_ref, lse_ref, name):
    err = np.abs(out.float().cpu().numpy() - o_ref).max()
    print(f"[gpu]   {name}: max abs err {err:.3e}", flush=True)
    assert err <= TOL
    if lse is not None:
        lse_g = lse.cpu().numpy()
        fin = np.isfinite(lse_ref)
        assert np.array_equal(np.isneginf(lse_g), ~fin)
        assert np.abs(lse_g[fin] - lse_ref[fin]).max() < 1e-3


def _bf16(seed, shape, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("balance", [False, True])
def test_tiled_d128_kernel_skips_invalid_ids(dev, balance):
    B, H, nq, nkb, bs, D = 1, 2, 7, 9, 128, 128
    Lq, Lk = nq * bs - 30, nkb * bs
    print(f"[gpu] invalid ids, tiled D=128 kernel, balance={balance}", flush=True)
    q, k, v = _bf16(1, (B, H, Lq, D), 0.2), _bf16(2, (B, H, Lk, D)), _bf16(3, (B, H, Lk, D))
    ind, cnt, ok_ind, ok_cnt = _lists(nq, nkb, H)
    out, lse = _core.bsa_forward(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(ind).to(dev),
                                 torch.from_numpy(cnt).to(dev), 1.0 / math.sqrt(D), bs, return_lse=True,
                                 balance=balance)
    torch.cuda.synchronize()
    f64 = lambda t: bf16_to_f32(bits(t)).astype(np.float64)  # noqa: E731
    o_ref, lse_ref = oatt.bsa_forward(f64(q), f64(k), f64(v), ok_ind, ok_cnt, 1.0 / math.sqrt(D), bs)
    _check(out, lse, o_ref, lse_ref, "tiled")


def _grid_case(seed, text):
    """Token-order inputs on a 16 x 16 latent with 2x8x8 tiles (BLHD views) and their oracle tiles."""
    Hh, W, tile, fq, fk, H, D = 16, 16, (2, 8, 8), 6, 4, 2, 128
    q = _bf16(seed, (1, fq * Hh * W, H, D), 0.2).permute(0, 2, 1, 3)
    k = _bf16(seed + 1, (1, fk * Hh * W, H, D)).permute(0, 2, 1, 3)
    v = _bf16(seed + 2, (1, fk * Hh * W, H, D)).permute(0, 2, 1, 3)
    nh, nw = 2, 2
    nq, nk = (fq // 2) * nh * nw, (fk // 2) * nh * nw
    ntxt = 1 if text else 0
    kt = vt = None
    if text:
        kt = torch.zeros((1, H, 128, D), dtype=torch.bfloat16)
        vt = torch.zeros((1, H, 128, D), dtype=torch.bfloat16)
        kt[:, :, :text] = _bf16(seed + 3, (1, H, text, D))
        vt[:, :, :text] = _bf16(seed + 4, (1, H, text, D))
    qt = otile.tile_gather(bits(q), fq, Hh, W, tile)
    ktl = otile.tile_gather(bits(k), fk, Hh, W, tile)
    vtl = otile.tile_gather(bits(v), fk, Hh, W, tile)
    flat = lambda t: bf16_to_f32(t.reshape(1, H, -1, D))  # noqa: E731
    kf, vf = flat(ktl), flat(vtl)
    if text:
        kf = np.concatenate([bf16_to_f32(bits(kt)), kf], axis=2)
        vf = np.concatenate([bf16_to_f32(bits(vt)), vf], axis=2)
    return dict(q=q, k=k, v=v, kt=kt, vt=vt, qf=flat(qt), kf=kf, vf=vf, geo=(fq, fk, Hh, W, tile, nh, nw),
                nq=nq, nkb=ntxt + nk, ntxt=ntxt, H=H, D=D)


def _to_tokens(o_tiled, c):
    fq, _, Hh, W, tile, _, _ = c["geo"]
    perm = tile_permutation(fq, Hh, W, tile)
    out = np.zeros((1, c["H"], fq * Hh * W, c["D"]))
    valid = perm >= 0
    out[:, :, perm[valid]] = o_tiled[:, :, valid]
    return out


def test_fused_kernel_skips_invalid_ids(dev):
    c = _grid_case(11, text=77)
    print(f"[gpu] invalid ids, fused D=128 kernel (nq={c['nq']}, nkb={c['nkb']}, one text block)", flush=True)
    ind, cnt, ok_ind, ok_cnt = _lists(c["nq"], c["nkb"], c["H"])
    fq, fk, Hh, W, (tt, th, tw), nh, nw = c["geo"]
    qd, kd, vd = c["q"].to(dev), c["k"].to(dev), c["v"].to(dev)
    out = torch.empty_like(qd)
    _, lse = _core.bsa_forward_gather(qd, kd, vd, c["kt"].to(dev), c["vt"].to(dev), c["ntxt"], fq, fk, Hh, W, tt, th,
                                      tw, nh, nw, torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev),
                                      1.0 / math.sqrt(c["D"]), out, return_lse=True)
    torch.cuda.synchronize()
    o_ref, lse_ref = oatt.bsa_forward(c["qf"], c["kf"], c["vf"], ok_ind, ok_cnt, 1.0 / math.sqrt(c["D"]), 128)
    _check(out, lse, _to_tokens(o_ref, c), lse_ref, "fused")


def _e4m3(x):
    """float32 (1, H, nblk*128, D) -> (codes uint8, scales (1, H, nblk), dequantized float64)."""
    B, H, L, D = x.shape
    codes, sc = ofp8.quantize_blocks(x.reshape(B, H, L // 128, 128, D))
    deq = ofp8.dequantize_blocks(codes, sc).reshape(B, H, L, D).astype(np.float64)
    return torch.from_numpy(np.ascontiguousarray(codes.reshape(B, H, L, D))).view(_core.FP8), torch.from_numpy(sc), deq


def test_e4m3_kernels_skip_invalid_ids(dev):
    c = _grid_case(21, text=130 - 128)
    print(f"[gpu] invalid ids, tiled and fused e4m3 kernels (nq={c['nq']}, nkb={c['nkb']})", flush=True)
    ind, cnt, ok_ind, ok_cnt = _lists(c["nq"], c["nkb"], c["H"])
    fq, fk, Hh, W, (tt, th, tw), nh, nw = c["geo"]
    q8, qs, q_deq = _e4m3(c["qf"])
    k8, ks, k_deq = _e4m3(c["kf"])
    scale = 1.0 / math.sqrt(c["D"])
    o_ref, lse_ref = oatt.bsa_forward(q_deq, k_deq, c["vf"].astype(np.float64), ok_ind, ok_cnt, scale, 128)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    vf = torch.from_numpy(np.ascontiguousarray(c["vf"])).to(torch.bfloat16).to(dev)
    out_t, lse_t = _core.bsa_forward_fp8(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev), vf, ii, cc, scale, 128,
                                         return_lse=True)
    vd = c["v"].to(dev)
    out_f = torch.empty(c["q"].shape, dtype=torch.bfloat16, device=dev)
    _, lse_f = _core.bsa_forward_fp8_gather(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev), vd, c["vt"].to(dev),
                                            c["ntxt"], fq, fk, Hh, W, tt, th, tw, nh, nw, ii, cc, scale, out_f,
                                            return_lse=True)
    torch.cuda.synchronize()
    _check(out_t, lse_t, o_ref, lse_ref, "tiled e4m3")
    _check(out_f, lse_f, _to_tokens(o_ref, c), lse_ref, "fused e4m3")


def test_lists_without_columns_give_zeros(dev):
    """Index tensors with no columns (every count clamps to 0): zeros and LSE -inf from the tiled kernel (with
    and without the balanced order), the fused kernel and both e4m3 kernels.  An empty list runs as one block
    with an out-of-range id, and its row has no entry to read."""
    c = _grid_case(31, text=0)
    H, D, nq = c["H"], c["D"], c["nq"]
    print(f"[gpu] lists with no columns (nq={nq}, nkb={c['nkb']})", flush=True)
    fq, fk, Hh, W, (tt, th, tw), nh, nw = c["geo"]
    # zero-column view of a real allocation (a non-null pointer, n_cols = 0); counts above 0 clamp to 0
    ii = torch.full((1, H, nq, 1), 3, dtype=torch.int32, device=dev)[..., :0]
    cc = torch.full((1, H, nq), 2, dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)
    qf = torch.from_numpy(np.ascontiguousarray(c["qf"])).to(torch.bfloat16).to(dev)
    kf = torch.from_numpy(np.ascontiguousarray(c["kf"])).to(torch.bfloat16).to(dev)
    vf = torch.from_numpy(np.ascontiguousarray(c["vf"])).to(torch.bfloat16).to(dev)
    outs = []
    for balance in (False, True):
        o, l = _core.bsa_forward(qf, kf, vf, ii, cc, scale, 128, return_lse=True, balance=balance)
        outs.append((f"tiled balance={balance}", o, l))
    qd, kd, vd = c["q"].to(dev), c["k"].to(dev), c["v"].to(dev)
    o = torch.empty_like(qd)
    _, l = _core.bsa_forward_gather(qd, kd, vd, None, None, 0, fq, fk, Hh, W, tt, th, tw, nh, nw, ii, cc, scale, o,
                                    return_lse=True)
    outs.append(("fused", o, l))
    q8, qs, _ = _e4m3(c["qf"])
    k8, ks, _ = _e4m3(c["kf"])
    o, l = _core.bsa_forward_fp8(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev), vf, ii, cc, scale, 128,
                                 return_lse=True)
    outs.append(("tiled e4m3", o, l))
    o = torch.empty_like(qd)
    _, l = _core.bsa_forward_fp8_gather(q8.to(dev), qs.to(dev), k8.to(dev), ks.to(dev), vd, None, 0, fq, fk, Hh, W,
                                        tt, th, tw, nh, nw, ii, cc, scale, o, return_lse=True)
    outs.append(("fused e4m3", o, l))
    torch.cuda.synchronize()
    for name, o, l in outs:
        print(f"[gpu]   {name}: max |out| {o.float().abs().max().item():.3e}", flush=True)
        assert o.float().abs().max().item() == 0.0
        assert torch.isneginf(l).all()


def test_split_tiles_with_an_empty_second_half(dev):
    """Tail-split tiles whose lists hold 0 or 1 block in an index tensor of one column: the second half of a
    one-block list is empty and its row has no entry left.  Split against whole tiles and the oracle."""
    from li_sparse import _lib

    bs, D, B, H, nq, nkb = 128, 128, 1, 8, 44, 6
    Lq, Lk = nq * bs - 40, nkb * bs
    with torch.cuda.device(dev):
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        ws = _lib.lib.li_bsa_fwd_workspace_size(B, H, Lq, D, bs)
    print(f"[gpu] split tiles with one-column lists (B={B} H={H} Lq={Lq} Lk={Lk}, {cus} CUs)", flush=True)
    rng = np.random.default_rng(17)
    q, k, v = _bf16(41, (B, H, Lq, D), 0.2), _bf16(42, (B, H, Lk, D)), _bf16(43, (B, H, Lk, D))
    ind = rng.integers(0, nkb, size=(B, H, nq, 1)).astype(np.int32)
    cnt = rng.integers(0, 2, size=(B, H, nq)).astype(np.int32)
    cnt[0, H - 1, nq - 1] = 1          # the tensor's last row: its second half would start past the end
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    scale = 1.0 / math.sqrt(D)
    out_s, lse_s = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, return_lse=True, split=True)
    out_w, lse_w = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, return_lse=True, split=False)
    torch.cuda.synchronize()
    assert ws > 0
    f64 = lambda t: bf16_to_f32(bits(t)).astype(np.float64)  # noqa: E731
    o_ref, lse_ref = oatt.bsa_forward(f64(q), f64(k), f64(v), ind, cnt, scale, bs)
    d_out = (out_s.float() - out_w.float()).abs().max().item()
    print(f"[gpu]   split vs whole {d_out:.3e}", flush=True)
    assert d_out <= 1e-2
    assert torch.equal(torch.isneginf(lse_s), torch.isneginf(lse_w))
    _check(out_s, lse_s, o_ref, lse_ref, "split")
