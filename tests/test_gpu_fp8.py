"""GPU parity of the e4m3 (qk_fp8) path.

* quantizing gathers: codes, scales, pools and V tiles bit-exact against the
  oracle (oracle.fp8.quantize_blocks over oracle.tile.tile_gather);
* attention on e4m3 Q/K: against the float64 oracle on the dequantized Q/K
  (max abs error <= 2e-2, LSE within 1e-3), whole / split / balanced;
* the whole call: against the oracle pipeline with ``qk_fp8``, against the
  bf16 call on the same inputs (FP8_VS_BF16) and against the bf16 reference
  output, the float64 oracle on the unquantized bf16 inputs (FP8_VS_BF16_REF).
"""
import math

import numpy as np
import pytest
import torch

from helpers import bits, oracle_pipeline
from li_sparse import _core
from li_sparse._lib import LiError
from li_sparse.hy.ar_sparse_operation import run_sparse_attention
from li_sparse.workloads import WORKLOADS, Workload, make_qkv
from oracle import attention as oatt
from oracle import fp8 as ofp8
from oracle import tile as otile
from oracle.bf16 import bf16_to_f32
from oracle.geometry import block_geometry

pytestmark = pytest.mark.gpu
TOL = 2e-2          # bf16 output vs the float64 oracle on the same (dequantized) Q/K
FP8_VS_BF16 = 1e-2  # e4m3 call vs bf16 call, max abs, HY shape (measured 3.9e-3; mean abs 6.9e-5)
# e4m3 call vs the bf16 reference output (the float64 oracle on the bf16 Q/K/V), max abs, HY shape
FP8_VS_BF16_REF = 1e-2


def _codes(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def _f32_bits(t):
    return t.detach().cpu().contiguous().numpy().view(np.uint32)


@pytest.mark.parametrize("name,layout", [("toy", "blhd"), ("hy", "bhld"), ("mg", "blhd")])
def test_prep_fp8_bit_exact(dev, name, layout):
    wl = WORKLOADS[name]
    print(f"[gpu] fp8 tile prep {name} layout={layout}", flush=True)
    q, k, v = make_qkv(wl, seed=3, layout=layout)
    g = block_geometry(wl.lq, wl.lk, wl.latent_hw, wl.tile)
    H, W = wl.latent_hw
    tt, th, tw = wl.tile
    B, NH, D, bs = wl.batch, wl.heads, wl.head_dim, g["BS"]
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    q8 = torch.empty((B, NH, g["nq_blk"], bs, D), dtype=_core.FP8, device=dev)
    qs = torch.empty((B, NH, g["nq_blk"]), dtype=torch.float32, device=dev)
    qp = torch.empty((B, NH, g["nq_blk"], D), dtype=torch.bfloat16, device=dev)
    _core.tile_prep_fp8(qd, q8, qs, qp, 0, 0, g["T_q"], H, W, tt, th, tw, g["nh"], g["nw"])
    ntxt = 2
    k8 = torch.full((B, NH, ntxt + g["nk_blk"], bs, D), 0x30, dtype=torch.uint8).view(_core.FP8).to(dev)  # 0.5
    ks = torch.full((B, NH, ntxt + g["nk_blk"]), -1.0, dtype=torch.float32, device=dev)
    v_all = torch.full((B, NH, ntxt + g["nk_blk"], bs, D), 7.0, dtype=torch.bfloat16, device=dev)
    kp = torch.empty((B, NH, g["nk_blk"], D), dtype=torch.bfloat16, device=dev)
    _core.kv_prep_fp8(kd, vd, k8, ks, v_all, kp, ntxt, 0, g["T_k"], H, W, tt, th, tw, g["nh"], g["nw"])
    torch.cuda.synchronize()
    oq = otile.tile_gather(bits(q), g["T_q"], H, W, wl.tile)
    oq_c, oq_s = ofp8.quantize_blocks(bf16_to_f32(oq))
    assert np.array_equal(_codes(q8), oq_c)
    assert np.array_equal(_f32_bits(qs), oq_s.view(np.uint32))
    assert np.array_equal(bits(qp), otile.pool_mean(oq))          # the bf16 path's pool, bit for bit
    ok_ = otile.tile_gather(bits(k), g["T_k"], H, W, wl.tile)
    ok_c, ok_s = ofp8.quantize_blocks(bf16_to_f32(ok_))
    assert np.array_equal(_codes(k8[:, :, ntxt:]), ok_c)
    assert np.array_equal(_f32_bits(ks[:, :, ntxt:]), ok_s.view(np.uint32))
    assert np.array_equal(bits(v_all[:, :, ntxt:]), otile.tile_gather(bits(v), g["T_k"], H, W, wl.tile))
    assert np.array_equal(bits(kp), otile.pool_mean(ok_))
    # blocks before dst_off untouched
    assert (_codes(k8[:, :, :ntxt]) == 0x30).all() and (ks[:, :, :ntxt] == -1.0).all().item()
    assert (v_all[:, :, :ntxt] == 7.0).all().item()


def test_text_blocks_with_the_trivial_grid(dev):
    print("[gpu] fp8 quantization of contiguous text blocks (T=n, H=1, W=BS, tile (1,1,BS))", flush=True)
    B, NH, D, bs, n = 1, 3, 128, 128, 3
    g = torch.Generator().manual_seed(2)
    kt = (torch.randn(B, NH, n * bs, D, generator=g) * 3).to(torch.bfloat16)
    kt[:, :, -70:] = 0                     # zero padding of the last block
    kt[:, 1, bs:2 * bs] = 0                # an all-zero block: scale 1, zero codes
    k8 = torch.empty((B, NH, n, bs, D), dtype=_core.FP8, device=dev)
    ks = torch.empty((B, NH, n), dtype=torch.float32, device=dev)
    _core.tile_prep_fp8(kt.to(dev), k8, ks, None, 0, 0, n, 1, bs, 1, 1, bs, 1, 1)
    torch.cuda.synchronize()
    c, s = ofp8.quantize_blocks(bf16_to_f32(bits(kt)).reshape(B, NH, n, bs, D))
    assert np.array_equal(_codes(k8), c)
    assert np.array_equal(_f32_bits(ks), s.view(np.uint32))
    assert ks[0, 1, 1].item() == 1.0 and not _codes(k8[0, 1, 1]).any()


def _quantized_inputs(seed, B, H, Lq, Lk, D, bs=128, zero_tail=0):
    """Random bf16 Q/K/V, Q and K quantized per 128-row block by the oracle (rows past Lq are zeros)."""
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, Lq, D, generator=g) / math.sqrt(D) * 2).to(torch.bfloat16)
    k = torch.randn(B, H, Lk, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Lk, D, generator=g).to(torch.bfloat16)
    if zero_tail:
        k[:, :, -zero_tail:] = 0
        v[:, :, -zero_tail:] = 0
    nq = (Lq + bs - 1) // bs
    qf = np.zeros((B, H, nq * bs, D), np.float32)
    qf[:, :, :Lq] = bf16_to_f32(bits(q))
    qc, qs = ofp8.quantize_blocks(qf.reshape(B, H, nq, bs, D))
    kc, ks = ofp8.quantize_blocks(bf16_to_f32(bits(k)).reshape(B, H, Lk // bs, bs, D))
    q_deq = ofp8.dequantize_blocks(qc, qs).reshape(B, H, nq * bs, D)[:, :, :Lq]
    k_deq = ofp8.dequantize_blocks(kc, ks).reshape(B, H, Lk, D)
    q8 = torch.from_numpy(np.ascontiguousarray(qc.reshape(B, H, nq * bs, D)[:, :, :Lq])).view(_core.FP8)
    k8 = torch.from_numpy(np.ascontiguousarray(kc.reshape(B, H, Lk, D))).view(_core.FP8)
    return dict(q8=q8, qs=torch.from_numpy(qs), k8=k8, ks=torch.from_numpy(ks), v=v, q_deq=q_deq, k_deq=k_deq,
                v64=bf16_to_f32(bits(v)).astype(np.float64))


def _random_lists(rng, B, H, nq, nkb, kmax, allow_empty=True):
    ind = np.zeros((B, H, nq, kmax), np.int32)
    cnt = np.zeros((B, H, nq), np.int32)
    for b in range(B):
        for h in range(H):
            for r in range(nq):
                n = int(rng.integers(0 if allow_empty else 1, min(kmax, nkb) + 1))
                ind[b, h, r, :n] = rng.choice(nkb, size=n, replace=False)
                cnt[b, h, r] = n
    return ind, cnt


def _run(x, dev, ind, cnt, **kw):
    return _core.bsa_forward_fp8(x["q8"].to(dev), x["qs"].to(dev), x["k8"].to(dev), x["ks"].to(dev),
                                 x["v"].to(dev), torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev),
                                 1.0 / math.sqrt(128), 128, return_lse=True, **kw)


def test_fp8_attention_random_lists_vs_oracle(dev):
    B, H, nq, nkb, bs, D = 1, 3, 5, 9, 128, 128
    Lq, Lk = nq * bs - 17, nkb * bs
    print(f"[gpu] fp8 bsa B={B} H={H} Lq={Lq} Lk={Lk} random lists (empty rows, zero tail)", flush=True)
    x = _quantized_inputs(7, B, H, Lq, Lk, D, zero_tail=bs // 2)
    ind, cnt = _random_lists(np.random.default_rng(3), B, H, nq, nkb, 6)
    out, lse = _run(x, dev, ind, cnt)
    torch.cuda.synchronize()
    o_ref, lse_ref = oatt.bsa_forward(x["q_deq"], x["k_deq"], x["v64"], ind, cnt, 1.0 / math.sqrt(D), bs)
    err = np.abs(out.float().cpu().numpy() - o_ref).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL
    lse_g = lse.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isneginf(lse_g), ~fin)
    assert np.abs(lse_g[fin] - lse_ref[fin]).max() < 1e-3


def test_fp8_split_and_balance(dev):
    """Tail split within fp32 rounding of whole tiles; the balanced order gives the same bits as whole tiles."""
    B, H, nq, nkb, bs, D = 1, 8, 44, 12, 128, 128  # 352 tiles: 12 of each XCD's 44 split on 256 CUs
    Lq, Lk = nq * bs - 40, nkb * bs
    print(f"[gpu] fp8 bsa split/balance B={B} H={H} Lq={Lq} Lk={Lk}", flush=True)
    x = _quantized_inputs(9, B, H, Lq, Lk, D)
    ind, cnt = _random_lists(np.random.default_rng(8), B, H, nq, nkb, 12)
    out_s, lse_s = _run(x, dev, ind, cnt, split=True)
    out_w, lse_w = _run(x, dev, ind, cnt, split=False)
    out_b, lse_b = _run(x, dev, ind, cnt, balance=True)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), out_w.view(torch.int16))
    fin = torch.isfinite(lse_w)
    assert torch.equal(torch.isneginf(lse_b), torch.isneginf(lse_w)) and torch.equal(lse_b[fin], lse_w[fin])
    assert torch.equal(torch.isneginf(lse_s), torch.isneginf(lse_w))
    d_out = (out_s.float() - out_w.float()).abs().max().item()
    d_lse = (lse_s[fin] - lse_w[fin]).abs().max().item()
    print(f"[gpu]   split vs whole: out {d_out:.3e} lse {d_lse:.3e}", flush=True)
    assert d_out <= 1e-2 and d_lse <= 1e-4
    o_ref, _ = oatt.bsa_forward(x["q_deq"], x["k_deq"], x["v64"], ind, cnt, 1.0 / math.sqrt(D), bs)
    err = np.abs(out_s.float().cpu().numpy() - o_ref).max()
    print(f"[gpu]   vs oracle: max abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_fp8_full_hy_shape_sampled_tiles(dev):
    print("[gpu] fp8 bsa full HY shape (B=1, H=16, Lq=7168, Lk=21504, 51 blocks/row)", flush=True)
    bs, D, H, nq, nkb, kk = 128, 128, 16, 56, 168, 51
    rng = np.random.default_rng(12)
    x = _quantized_inputs(6, 1, H, nq * bs, nkb * bs, D)
    ind = np.stack([np.stack([np.sort(rng.choice(nkb, kk, replace=False)) for _ in range(nq)])
                    for _ in range(H)])[None].astype(np.int32)
    cnt = np.full((1, H, nq), kk, np.int32)
    out, _ = _run(x, dev, ind, cnt)
    torch.cuda.synchronize()
    tiles = [(0, int(h), int(m)) for h, m in zip(rng.integers(0, H, 24), rng.integers(0, nq, 24))]
    o_ref, _ = oatt.bsa_forward(x["q_deq"], x["k_deq"], x["v64"], ind, cnt, 1.0 / math.sqrt(D), bs, heads=tiles)
    got = out.float().cpu().numpy()
    err = max(np.abs(got[b, h, m * bs:(m + 1) * bs] - o_ref[b, h, m * bs:(m + 1) * bs]).max() for b, h, m in tiles)
    print(f"[gpu]   max abs err over 24 sampled tiles {err:.3e}", flush=True)
    assert err <= TOL


def test_fp8_pipeline_with_text_vs_oracle(dev):
    wl = Workload("hy_fp8_small", 2, 128, (30, 52), 4, 8, (2, 8, 8), 0.3, "scaled_dot_product", qk_fp8=True)
    print("[gpu] run_sparse_attention qk_fp8, 2 heads + 200 text tokens, vs the oracle pipeline", flush=True)
    q, k, v = make_qkv(wl, seed=4, layout="blhd")
    g = torch.Generator().manual_seed(9)
    kt = torch.randn(1, 2, 200, 128, generator=g).to(torch.bfloat16)
    vt = torch.randn(1, 2, 200, 128, generator=g).to(torch.bfloat16)
    params = wl.sparse_params()
    out = run_sparse_attention(q.to(dev), kt.to(dev), vt.to(dev), k.to(dev), v.to(dev), 3, wl.latent_hw, params)
    torch.cuda.synchronize()
    ref = oracle_pipeline(q, k, v, wl.latent_hw, params, text=(kt, vt))
    err = np.abs(out.float().cpu().numpy() - ref["out"]).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_fp8_call_vs_bf16_call_hy_shape(dev):
    """The e4m3 call against the bf16 call at the HY shape: same selection, output within FP8_VS_BF16."""
    wl = WORKLOADS["hy_fp8"]
    print("[gpu] run_sparse_attention hy_fp8 vs hy (bf16), full shape", flush=True)
    q, k, v = make_qkv(wl, seed=0, layout="blhd")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    e = torch.empty((1, wl.heads, 0, wl.head_dim), dtype=torch.bfloat16, device=dev)
    out8 = run_sparse_attention(qd, e, e, kd, vd, 1, wl.latent_hw, wl.sparse_params())
    out16 = run_sparse_attention(qd, e, e, kd, vd, 1, wl.latent_hw, WORKLOADS["hy"].sparse_params())
    torch.cuda.synchronize()
    d = (out8.float() - out16.float()).abs()
    ref_scale = out16.float().abs().max().item()
    print(f"[gpu]   fp8 vs bf16: max abs {d.max().item():.3e} mean abs {d.mean().item():.3e} "
          f"(max |out| {ref_scale:.3f})", flush=True)
    assert d.max().item() <= FP8_VS_BF16
    # sampled tiles against the oracle pipeline on the quantized values
    rng = np.random.default_rng(1)
    nq = math.ceil(wl.frames_q / wl.tile[0]) * math.ceil(wl.latent_hw[0] / wl.tile[1]) * \
        math.ceil(wl.latent_hw[1] / wl.tile[2])
    tiles = [(0, int(h), int(m)) for h, m in zip(rng.integers(0, wl.heads, 12), rng.integers(0, nq, 12))]
    ref = oracle_pipeline(q, k, v, wl.latent_hw, wl.sparse_params(), heads=tiles)
    got = out8.float().cpu().numpy()
    bs = ref["geo"]["BS"]
    err = 0.0
    for b, h, m in tiles:
        rows = ref["perm"][m * bs:(m + 1) * bs]
        rows = rows[rows >= 0]
        err = max(err, np.abs(got[b, h, rows] - ref["out"][b, h, rows]).max())
    print(f"[gpu]   vs oracle over {len(tiles)} sampled tiles {err:.3e}", flush=True)
    assert err <= TOL
    # The e4m3 call against the bf16 reference output: the float64 oracle on the bf16 inputs (qk_fp8 off,
    # so Q and K are not quantized), on more sampled tiles.
    tiles16 = tiles + [(0, int(h), int(m)) for h, m in zip(rng.integers(0, wl.heads, 12), rng.integers(0, nq, 12))]
    ref16 = oracle_pipeline(q, k, v, wl.latent_hw, WORKLOADS["hy"].sparse_params(), heads=tiles16)
    assert np.array_equal(ref16["indices"], ref["indices"])   # the selection does not see the quantization
    err16 = mean16 = 0.0
    n16 = 0
    for b, h, m in tiles16:
        rows = ref16["perm"][m * bs:(m + 1) * bs]
        rows = rows[rows >= 0]
        dd = np.abs(got[b, h, rows] - ref16["out"][b, h, rows])
        err16 = max(err16, dd.max())
        mean16 += dd.sum()
        n16 += dd.size
    print(f"[gpu]   vs the bf16 reference output over {len(tiles16)} sampled tiles: max abs {err16:.3e}, "
          f"mean abs {mean16 / n16:.3e}", flush=True)
    assert err16 <= FP8_VS_BF16_REF


def test_fp8_rejects_unsupported(dev):
    x = _quantized_inputs(1, 1, 1, 128, 256, 128)
    ind = np.zeros((1, 1, 1, 1), np.int32)
    cnt = np.ones((1, 1, 1), np.int32)
    with pytest.raises(TypeError):
        _core.bsa_forward_fp8(x["q8"].to(dev), x["qs"].to(dev), x["k8"].to(dev), x["ks"].to(dev),
                              x["v"].to(dev).half(), torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev),
                              0.1, 128)
    with pytest.raises(LiError, match="UNSUPPORTED|unsupported"):   # built for 128-token blocks only
        _core.bsa_forward_fp8(x["q8"].to(dev), torch.ones((1, 1, 2), device=dev), x["k8"].to(dev),
                              torch.ones((1, 1, 4), device=dev), x["v"].to(dev),
                              torch.zeros((1, 1, 2, 1), dtype=torch.int32, device=dev),
                              torch.ones((1, 1, 2), dtype=torch.int32, device=dev), 0.1, 64)


@pytest.mark.parametrize("latent_hw,tile,frames_k,text,layout", [((30, 52), (2, 8, 8), 8, 200, "blhd"),
                                                                  ((22, 40), (4, 4, 8), 8, 0, "bhld"),
                                                                  ((30, 52), (2, 8, 8), 12, 130, "bhld")])
def test_fp8_fused_equals_tiled(dev, latent_hw, tile, frames_k, text, layout):
    """The fused e4m3 call (V read, O written in token order) gives the bits of the tiled e4m3 sequence."""
    from li_sparse import _pipeline
    from li_sparse.hy.ar_sparse_operation import fast_generate_indices

    wl = Workload("fp8_fused", 2, 128, latent_hw, 4, frames_k, tile, 0.3, "scaled_dot_product", qk_fp8=True)
    print(f"[gpu] fp8 fused vs tiled {latent_hw} tile={tile} text={text} {layout}", flush=True)
    q, k, v = make_qkv(wl, seed=11, layout=layout)
    g = torch.Generator().manual_seed(12)
    kt = torch.randn(1, 2, text, 128, generator=g).to(torch.bfloat16).to(dev) if text else None
    vt = torch.randn(1, 2, text, 128, generator=g).to(torch.bfloat16).to(dev) if text else None
    params = dict(wl.sparse_params(), tile_size=tile)

    def select(q_pool, k_pool, tl, grid_q, grid_k):
        return fast_generate_indices(q_pool, k_pool, tl, grid_q, grid_k, params, dev)

    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    assert _pipeline.uses_fused(qd, kd, vd, tile, latent_hw)
    out_f = _pipeline.sparse_attention(qd, kt, vt, kd, vd, latent_hw, tile, select, qk_fp8=True, fused=True)
    out_t = _pipeline.sparse_attention(qd, kt, vt, kd, vd, latent_hw, tile, select, qk_fp8=True, fused=False)
    torch.cuda.synchronize()
    assert out_f.stride() == qd.stride()
    assert torch.equal(out_f.view(torch.int16), out_t.view(torch.int16))
