"""GPU parity at batch 2, the batch HY-WorldPlay's decode call runs with.

HY concatenates the RoPE and ProPE query branches (and their keys and values)
on the batch dimension and repeats the cached text K/V to that batch
(hy-worldplay/patches/0001-integrate-acceleration.patch:637-640, 687-691),
with tile (4, 8, 4), ratio 0.175 and recent_protect 4 (patch:600-604,
621-626).  Every check here compares against the float64 oracle: the whole
call on sampled tiles of both batch entries (the last (b, h) included), and
each attention kernel (tiled, token-order, e4m3 tiled and e4m3 token-order)
on random lists, so the batch stride of every kernel's addressing is pinned
independently of the others.
"""
import math

import numpy as np
import pytest
import torch

from helpers import bits, oracle_pipeline
from li_sparse import _core, _pipeline
from li_sparse.hy.ar_sparse_operation import run_sparse_attention
from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import tile as otile
from oracle.bf16 import bf16_to_f32
from oracle.geometry import tile_permutation

pytestmark = pytest.mark.gpu
TOL = 2e-2  # max abs error of the bf16 output against the float64 oracle
HW = (30, 52)
DECODE = {"tile_size": (4, 8, 4), "topk_ratio": 0.175, "recent_protect": 4, "sim_metric": "scaled_dot_product"}


def _blhd(x):
    """(B, H, L, D) view of (B, L, H, D) storage, as the HY call site passes q, k_vis and v_vis."""
    return x.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)


def _hy_batch2_inputs(seed, H=4, fq=4, fk=12, text=200, D=128):
    g = torch.Generator().manual_seed(seed)
    L = HW[0] * HW[1]
    # Smooth-ish fields so the selection has structure: a low-rank part plus noise.
    def field(frames, scale):
        base = torch.randn(2, H, 1, D, generator=g)
        t = torch.linspace(0, 1, frames * L).view(1, 1, -1, 1)
        x = base * torch.cos(6.28 * t * torch.randn(2, H, 1, 1, generator=g)) + 0.5 * torch.randn(2, H, frames * L, D,
                                                                                                   generator=g)
        return _blhd((x * scale).to(torch.bfloat16))
    q = field(fq, 1.0 / math.sqrt(D))
    k, v = field(fk, 1.0), field(fk, 1.0)
    kt1 = torch.randn(1, H, text, D, generator=g).to(torch.bfloat16)
    vt1 = torch.randn(1, H, text, D, generator=g).to(torch.bfloat16)
    # einops.repeat('B H S D -> (B R) H S D', R=2) of the cached text K/V
    return q, k, v, kt1.repeat(2, 1, 1, 1), vt1.repeat(2, 1, 1, 1)


def _sampled_err(got, ref, tiles):
    bs, perm = ref["geo"]["BS"], ref["perm"]
    err = 0.0
    for b, h, m in tiles:
        rows = perm[m * bs:(m + 1) * bs]
        rows = rows[rows >= 0]
        err = max(err, float(np.abs(got[b, h, rows] - ref["out"][b, h, rows]).max()))
    return err


@pytest.mark.parametrize("qk_fp8", [False, True])
def test_hy_decode_call_batch2_vs_oracle(dev, qk_fp8):
    H = 4
    print(f"[gpu] run_sparse_attention B=2 (RoPE+ProPE) H={H} 30x52, 4/12 frames, 200 text tokens, "
          f"tile (4,8,4), qk_fp8={qk_fp8}", flush=True)
    q, k, v, kt, vt = _hy_batch2_inputs(3)
    params = dict(DECODE, qk_fp8=qk_fp8)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    assert _pipeline.uses_fused(qd, kd, vd, params["tile_size"], HW)
    out = run_sparse_attention(qd, kt.to(dev), vt.to(dev), kd, vd, 2, HW, params)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.stride() == qd.stride()
    nq = 1 * math.ceil(HW[0] / 8) * math.ceil(HW[1] / 4)   # one 4-frame slab of 4 x 13 tiles
    rng = np.random.default_rng(1)
    tiles = [(0, 0, 0), (1, 0, 0), (1, H - 1, nq - 1), (0, H - 1, nq - 1)]
    tiles += [(int(b), int(h), int(m)) for b, h, m in
              zip(rng.integers(0, 2, 12), rng.integers(0, H, 12), rng.integers(0, nq, 12))]
    ref = oracle_pipeline(q, k, v, HW, params, text=(kt, vt), heads=tiles)
    assert ref["geo"]["nq_blk"] == nq and ref["geo"]["num_txt_blk"] == 2
    # The two batch entries select differently (different queries and keys).
    assert not np.array_equal(ref["indices"][0], ref["indices"][1])
    err = _sampled_err(out.float().cpu().numpy(), ref, tiles)
    print(f"[gpu]   max abs err over {len(tiles)} tiles of both batch entries {err:.3e}", flush=True)
    assert err <= TOL


def _lists(rng, B, H, nq, nkb, kmax, sort):
    ind = np.zeros((B, H, nq, kmax), np.int32)
    cnt = np.zeros((B, H, nq), np.int32)
    for b in range(B):
        for h in range(H):
            for r in range(nq):
                n = int(rng.integers(1, min(kmax, nkb) + 1))
                sel = rng.choice(nkb, size=n, replace=False)
                ind[b, h, r, :n] = np.sort(sel) if sort else sel
                cnt[b, h, r] = n
    return ind, cnt


def _f64(t):
    return bf16_to_f32(bits(t)).astype(np.float64)


def test_tiled_kernel_batch2_random_lists(dev):
    bs, D, B, H, nq, nkb = 128, 128, 2, 3, 9, 14
    Lq, Lk = nq * bs - 50, nkb * bs
    print(f"[gpu] li_bsa_fwd B={B} H={H} Lq={Lq} Lk={Lk} random lists, whole and split", flush=True)
    g = torch.Generator().manual_seed(71)
    q = (torch.randn(B, H, Lq, D, generator=g) * 0.2).to(torch.bfloat16)
    k = torch.randn(B, H, Lk, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Lk, D, generator=g).to(torch.bfloat16)
    ind, cnt = _lists(np.random.default_rng(71), B, H, nq, nkb, 8, sort=False)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    o_ref, lse_ref = oatt.bsa_forward(_f64(q), _f64(k), _f64(v), ind, cnt, 1.0 / math.sqrt(D), bs)
    for split in (False, True):
        out, lse = _core.bsa_forward(q.to(dev), k.to(dev), v.to(dev), ii, cc, 1.0 / math.sqrt(D), bs,
                                     return_lse=True, split=split)
        torch.cuda.synchronize()
        err = np.abs(out.float().cpu().numpy() - o_ref).max()
        lerr = np.abs(lse.cpu().numpy() - lse_ref).max()
        print(f"[gpu]   split={split}: max abs err {err:.3e}, lse {lerr:.3e}", flush=True)
        assert err <= TOL and lerr < 1e-3


def _tiled_oracle(q, k, v, kt, vt, T_q, T_k, tile, ind, cnt, q_deq=None, k_deq=None):
    """float64 oracle of the token-order kernels: tiles of Q, K, V (text blocks first), attention over the
    lists on the tiled layout, output scattered back to token order (padding rows dropped)."""
    H, W = HW
    B, NH, _, D = q.shape
    bs = tile[0] * tile[1] * tile[2]
    qt = otile.tile_gather(bits(q), T_q, H, W, tile).reshape(B, NH, -1, D)
    kt_ = otile.tile_gather(bits(k), T_k, H, W, tile).reshape(B, NH, -1, D)
    vt_ = otile.tile_gather(bits(v), T_k, H, W, tile).reshape(B, NH, -1, D)
    kf, vf = bf16_to_f32(kt_), bf16_to_f32(vt_)
    if kt is not None:
        kf = np.concatenate([bf16_to_f32(bits(kt)), kf], axis=2)
        vf = np.concatenate([bf16_to_f32(bits(vt)), vf], axis=2)
    qf = bf16_to_f32(qt)
    if q_deq is not None:
        qf, kf = q_deq, k_deq
    o, _ = oatt.bsa_forward(qf.astype(np.float64), kf.astype(np.float64), vf.astype(np.float64), ind, cnt,
                            1.0 / math.sqrt(D), bs)
    perm = tile_permutation(T_q, H, W, tile)
    valid = perm >= 0
    out = np.zeros((B, NH, T_q * H * W, D))
    out[:, :, perm[valid], :] = o[:, :, valid, :]
    return out, qt, kt_


@pytest.mark.parametrize("sort", [True, False])
def test_token_order_kernel_batch2_random_lists(dev, sort):
    tile, T_q, T_k, B, NH, D, ntxt = (4, 8, 4), 4, 12, 2, 2, 128, 2
    H, W = HW
    nh, nw = math.ceil(H / 8), math.ceil(W / 4)
    nq, nk = nh * nw, 3 * nh * nw
    print(f"[gpu] li_bsa_fwd_gather B={B} H={NH} 30x52 tile (4,8,4), {ntxt} text blocks, random lists "
          f"(sorted={sort})", flush=True)
    g = torch.Generator().manual_seed(72)
    q = _blhd((torch.randn(B, NH, T_q * H * W, D, generator=g) * 0.2).to(torch.bfloat16))
    k = _blhd(torch.randn(B, NH, T_k * H * W, D, generator=g).to(torch.bfloat16))
    v = _blhd(torch.randn(B, NH, T_k * H * W, D, generator=g).to(torch.bfloat16))
    kt = torch.randn(B, NH, ntxt * 128, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(B, NH, ntxt * 128, D, generator=g).to(torch.bfloat16)
    ind, cnt = _lists(np.random.default_rng(72), B, NH, nq, ntxt + nk, 12, sort=sort)
    o_ref, _, _ = _tiled_oracle(q, k, v, kt, vt, T_q, T_k, tile, ind, cnt)
    out = torch.empty_like(q.to(dev))
    _core.bsa_forward_gather(q.to(dev), k.to(dev), v.to(dev), kt.to(dev), vt.to(dev), ntxt, T_q, T_k, H, W, *tile,
                             nh, nw, torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev), 1.0 / math.sqrt(D),
                             out, sorted_lists=sort)
    torch.cuda.synchronize()
    err = np.abs(out.float().cpu().numpy() - o_ref).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL


@pytest.mark.parametrize("token_order", [False, True])
def test_e4m3_kernels_batch2_random_lists(dev, token_order):
    tile, T_q, T_k, B, NH, D, ntxt = (2, 8, 8), 4, 8, 2, 2, 128, 1
    H, W = HW
    nh, nw = math.ceil(H / 8), math.ceil(W / 8)
    nq, nk = 2 * nh * nw, 4 * nh * nw
    print(f"[gpu] e4m3 attention B={B} H={NH} (token order: {token_order}), {ntxt} text block, random lists",
          flush=True)
    g = torch.Generator().manual_seed(73)
    q = _blhd((torch.randn(B, NH, T_q * H * W, D, generator=g) * 0.2).to(torch.bfloat16))
    k = _blhd(torch.randn(B, NH, T_k * H * W, D, generator=g).to(torch.bfloat16))
    v = _blhd(torch.randn(B, NH, T_k * H * W, D, generator=g).to(torch.bfloat16))
    kt = torch.randn(B, NH, ntxt * 128, D, generator=g).to(torch.bfloat16)
    vt = torch.randn(B, NH, ntxt * 128, D, generator=g).to(torch.bfloat16)
    ind, cnt = _lists(np.random.default_rng(73), B, NH, nq, ntxt + nk, 10, sort=True)
    # e4m3 tiles and per-block scales from the oracle's quantizer (text blocks first, as the call lays them out)
    qb = otile.tile_gather(bits(q), T_q, H, W, tile)
    kb = np.concatenate([bits(kt).reshape(B, NH, ntxt, 128, D), otile.tile_gather(bits(k), T_k, H, W, tile)], axis=2)
    q8, qs = ofp8.quantize_blocks(bf16_to_f32(qb))
    k8, ks = ofp8.quantize_blocks(bf16_to_f32(kb))
    q_deq = ofp8.dequantize_blocks(q8, qs).reshape(B, NH, -1, D)
    k_deq = ofp8.dequantize_blocks(k8, ks).reshape(B, NH, -1, D)
    o_ref, _, _ = _tiled_oracle(q, k, v, kt, vt, T_q, T_k, tile, ind, cnt, q_deq=q_deq, k_deq=k_deq)
    to_dev = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dev).view(dt)  # noqa: E731
    q8d = to_dev(q8.reshape(B, NH, -1, D), torch.float8_e4m3fn)
    k8d = to_dev(k8.reshape(B, NH, -1, D), torch.float8_e4m3fn)
    qsd, ksd = torch.from_numpy(qs).to(dev), torch.from_numpy(ks).to(dev)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    if token_order:
        out = torch.empty_like(q.to(dev))
        _core.bsa_forward_fp8_gather(q8d, qsd, k8d, ksd, v.to(dev), vt.to(dev), ntxt, T_q, T_k, H, W, *tile, nh, nw,
                                     ii, cc, 1.0 / math.sqrt(D), out, sorted_lists=True)
        got = out.float().cpu().numpy()
    else:
        vb = np.concatenate([bits(vt).reshape(B, NH, ntxt, 128, D), otile.tile_gather(bits(v), T_k, H, W, tile)],
                            axis=2)
        v_tiles = torch.from_numpy(vb.reshape(B, NH, -1, D).view(np.int16)).view(torch.bfloat16).to(dev)
        o_t = _core.bsa_forward_fp8(q8d, qsd, k8d, ksd, v_tiles, ii, cc, 1.0 / math.sqrt(D), 128)
        o_t = o_t.float().cpu().numpy()
        perm = tile_permutation(T_q, H, W, tile)
        valid = perm >= 0
        got = np.zeros_like(o_ref)
        got[:, :, perm[valid], :] = o_t[:, :, valid, :]
    torch.cuda.synchronize()
    err = np.abs(got - o_ref).max()
    print(f"[gpu]   max abs err vs the float64 oracle on the dequantized Q/K {err:.3e}", flush=True)
    assert err <= TOL
