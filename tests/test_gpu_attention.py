"""GPU parity: block-sparse attention forward vs the float64 oracle (max abs error <= 2e-2 in bf16)."""
import math

import numpy as np
import pytest
import torch

from helpers import bits
from li_sparse import _core
from li_sparse.hy.longcat_kernel import longcat_flash_attn
from li_sparse.mg.longcat_kernel import longcat_flash_attn as mg_longcat_flash_attn
from oracle import attention as oatt
from oracle.bf16 import bf16_to_f32

pytestmark = pytest.mark.gpu
TOL = 2e-2  # max-abs error of the bf16 output against the float64 reference


def _inputs(seed, B, H, Lq, Lk, D, dtype=torch.bfloat16, zero_tail=0):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, Lq, D, generator=g) / math.sqrt(D) * 2).to(dtype)
    k = torch.randn(B, H, Lk, D, generator=g).to(dtype)
    v = torch.randn(B, H, Lk, D, generator=g).to(dtype)
    if zero_tail:
        k[:, :, -zero_tail:] = 0
        v[:, :, -zero_tail:] = 0
    return q, k, v


def _random_lists(rng, B, H, nq, nkb, kmax, allow_empty=True, shuffle=True):
    ind = np.zeros((B, H, nq, kmax), np.int32)
    cnt = np.zeros((B, H, nq), np.int32)
    for b in range(B):
        for h in range(H):
            for r in range(nq):
                n = int(rng.integers(0 if allow_empty else 1, min(kmax, nkb) + 1))
                sel = rng.choice(nkb, size=n, replace=False)
                if not shuffle:
                    sel = np.sort(sel)
                ind[b, h, r, :n] = sel
                cnt[b, h, r] = n
    return ind, cnt


def _f64(t):
    return t.double().numpy() if t.dtype != torch.bfloat16 else bf16_to_f32(bits(t)).astype(np.float64)


@pytest.mark.parametrize("bs,D", [(128, 128), (128, 64), (64, 128), (64, 64)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_random_lists_vs_oracle(dev, bs, D, dtype):
    print(f"[gpu] bsa bs={bs} D={D} {dtype}", flush=True)
    rng = np.random.default_rng(bs + D)
    B, H, nq, nkb = 1, 3, 5, 9
    Lq, Lk = nq * bs - 17, nkb * bs          # ragged last query tile
    q, k, v = _inputs(bs * 7 + D, B, H, Lq, Lk, D, dtype, zero_tail=bs // 2)
    ind, cnt = _random_lists(rng, B, H, nq, nkb, 6)
    scale = 1.0 / math.sqrt(D)
    out, lse = _core.bsa_forward(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(ind).to(dev),
                                 torch.from_numpy(cnt).to(dev), scale, bs, return_lse=True)
    torch.cuda.synchronize()
    o_ref, lse_ref = oatt.bsa_forward(_f64(q), _f64(k), _f64(v), ind, cnt, scale, bs)
    err = np.abs(out.float().cpu().numpy() - o_ref).max()
    print(f"[gpu]   max abs err {err:.3e}", flush=True)
    assert err <= TOL
    lse_g = lse.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isneginf(lse_g), ~fin)
    assert np.abs(lse_g[fin] - lse_ref[fin]).max() < 1e-3


def test_full_hy_shape_sampled_tiles(dev):
    print("[gpu] bsa full HY shape (B=1, H=16, Lq=7168, Lk=21504, 51 blocks/row)", flush=True)
    bs, D, H = 128, 128, 16
    nq, nkb, kk = 56, 168, 51
    rng = np.random.default_rng(11)
    q, k, v = _inputs(5, 1, H, nq * bs, nkb * bs, D)
    ind = np.stack([np.stack([np.stack([np.sort(rng.choice(nkb, kk, replace=False)) for _ in range(nq)])
                              for _ in range(H)])])[None][0].astype(np.int32)
    cnt = np.full((1, H, nq), kk, np.int32)
    out = _core.bsa_forward(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(ind).to(dev),
                            torch.from_numpy(cnt).to(dev), 1.0 / math.sqrt(D), bs)
    torch.cuda.synchronize()
    tiles = [(0, int(h), int(m)) for h, m in zip(rng.integers(0, H, 24), rng.integers(0, nq, 24))]
    o_ref, _ = oatt.bsa_forward(_f64(q), _f64(k), _f64(v), ind, cnt, 1.0 / math.sqrt(D), bs, heads=tiles)
    got = out.float().cpu().numpy()
    err = max(np.abs(got[b, h, m * bs:(m + 1) * bs] - o_ref[b, h, m * bs:(m + 1) * bs]).max() for b, h, m in tiles)
    print(f"[gpu]   max abs err over 24 sampled tiles {err:.3e}", flush=True)
    assert err <= TOL


def split_per_xcd(tiles, cus):
    """Tail-split tiles per XCD, restated from the rule the library documents: n = tiles / 8 tiles per XCD
    on c = cus / 8 CUs; its last round's r = n % c tiles are split in halves when r <= c / 2."""
    if cus % 8 or tiles % 8:
        return 0
    n, c = tiles // 8, cus // 8
    r = n % c if n > c else 0
    return r if 2 * r <= c else 0


@pytest.mark.parametrize("H,nq", [(8, 44), (8, 58)])
def test_tail_split_matches_whole_tiles_and_oracle(dev, H, nq):
    """Each XCD's tiles of a partial last round run as two halves of their block list plus a merge kernel
    when the round is at most half full (8 x 44 tiles on 256 CUs: 12 of each XCD's 44); a fuller last round
    (8 x 58: 26 of 58) runs whole.  Both against whole tiles and the oracle."""
    from li_sparse import _lib

    bs, D, B, nkb = 128, 128, 1, 12
    Lq, Lk = nq * bs - 40, nkb * bs
    print(f"[gpu] bsa tail split B={B} H={H} Lq={Lq} Lk={Lk}", flush=True)
    tiles = B * H * nq
    with torch.cuda.device(dev):
        ws = _lib.lib.li_bsa_fwd_workspace_size(B, H, Lq, D, bs)
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
    r = split_per_xcd(tiles, cus)
    nsplit = 8 * r
    print(f"[gpu]   {r} split tiles per XCD", flush=True)
    # room for the split partials, or for the tile order of the balanced mode
    assert ws == max(nsplit * 2 * 128 * 130 * 4, (tiles * 4 + 15) // 16 * 16)
    rng = np.random.default_rng(5)
    q, k, v = _inputs(41, B, H, Lq, Lk, D)
    ind, cnt = _random_lists(rng, B, H, nq, nkb, 7)
    # empty, single-block and two-block lists among the split tiles (the last r tiles of each XCD's range)
    flat = cnt.reshape(-1)
    for j, n in enumerate([0, 1, 2, 0, 1]):
        if r > 0:
            flat[(j % 8 + 1) * (tiles // 8) - 1 - (j // 8) % r] = n
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    scale = 1.0 / math.sqrt(D)
    out_s, lse_s = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, return_lse=True, split=True)
    out_w, lse_w = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, return_lse=True, split=False)
    torch.cuda.synchronize()
    d_out = (out_s.float() - out_w.float()).abs().max().item()
    fin = torch.isfinite(lse_w)
    assert torch.equal(torch.isneginf(lse_s), torch.isneginf(lse_w))
    d_lse = (lse_s[fin] - lse_w[fin]).abs().max().item()
    print(f"[gpu]   split vs whole: out {d_out:.3e} lse {d_lse:.3e} ({nsplit} split tiles)", flush=True)
    assert d_out <= 1e-2 and d_lse <= 1e-4
    o_ref, lse_ref = oatt.bsa_forward(_f64(q), _f64(k), _f64(v), ind, cnt, scale, bs)
    err = np.abs(out_s.float().cpu().numpy() - o_ref).max()
    lse_g = lse_s.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isneginf(lse_g), ~fin)
    print(f"[gpu]   vs oracle: max abs err {err:.3e}", flush=True)
    assert err <= TOL
    assert np.abs(lse_g[fin] - lse_ref[fin]).max() < 1e-3


def test_all_blocks_equals_dense_sdpa(dev):
    print("[gpu] bsa all blocks kept vs torch SDPA (fp32)", flush=True)
    bs, D, H, nq, nkb = 128, 128, 4, 6, 12
    q, k, v = _inputs(21, 1, H, nq * bs, nkb * bs, D)
    ind = np.broadcast_to(np.arange(nkb, dtype=np.int32), (1, H, nq, nkb)).copy()
    cnt = np.full((1, H, nq), nkb, np.int32)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = _core.bsa_forward(qd, kd, vd, torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev),
                            1.0 / math.sqrt(D), bs)
    ref = torch.nn.functional.scaled_dot_product_attention(qd.float(), kd.float(), vd.float())
    torch.cuda.synchronize()
    err = (out.float() - ref).abs().max().item()
    assert err <= TOL


def test_out_of_range_ids_are_skipped_and_wrapper_raises(dev):
    print("[gpu] bsa out-of-range ids", flush=True)
    bs, D = 128, 64
    q, k, v = _inputs(31, 1, 1, 2 * bs, 4 * bs, D)
    ind = np.array([[[[1, 9, 2], [-3, 0, 3]]]], np.int32)
    cnt = np.array([[[3, 3]]], np.int32)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = _core.bsa_forward(qd, kd, vd, torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev), 0.125, bs)
    torch.cuda.synchronize()
    ok_ind = np.array([[[[1, 2], [0, 3]]]], np.int32)
    o_ref, _ = oatt.bsa_forward(_f64(q), _f64(k), _f64(v), ok_ind, np.array([[[2, 2]]], np.int32), 0.125, bs)
    assert np.abs(out.float().cpu().numpy() - o_ref).max() <= TOL
    with pytest.raises(ValueError, match="Sparse indices out of bounds."):
        longcat_flash_attn(qd, kd, vd, torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev))
    with pytest.raises(ValueError, match=r"K Length \(320\) must be divisible by logical_block_size \(128\)"):
        longcat_flash_attn(qd, kd[:, :, :320], vd[:, :, :320], torch.from_numpy(ok_ind).to(dev),
                           torch.from_numpy(cnt).to(dev))
    with pytest.raises(AssertionError):
        mg_longcat_flash_attn(qd, kd[:, :, :320], vd[:, :, :320], torch.from_numpy(ok_ind).to(dev),
                              torch.from_numpy(cnt).to(dev))


def test_longcat_entry_fp32_inputs_and_strided_indices(dev):
    """float32 q/k/v through both entry points: the HY entry returns q's dtype (its reference allocates the
    output with torch.empty_like(q), longcat_kernel.py:198), the MG entry bf16 (its reference casts non-half
    inputs to bf16 first, matrix-game-3.0 longcat_kernel.py:139-147).  Both compute in bf16; the oracle runs
    in float64 on the float32 inputs themselves, so the tolerance also covers the bf16 input rounding."""
    print("[gpu] longcat_flash_attn fp32 inputs, non-contiguous indices", flush=True)
    bs, D = 128, 128
    g = torch.Generator().manual_seed(41)
    q = torch.randn(1, 2, 3 * bs - 30, D, generator=g) / math.sqrt(D) * 2
    k = torch.randn(1, 2, 5 * bs, D, generator=g)
    v = torch.randn(1, 2, 5 * bs, D, generator=g)
    rng = np.random.default_rng(4)
    ind, cnt = _random_lists(rng, 1, 2, 3, 5, 4, allow_empty=False)
    wide = np.zeros((1, 2, 3, 8), np.int32)
    wide[..., ::2] = ind
    ind_view = torch.from_numpy(wide).to(dev)[..., ::2]
    o_ref, _ = oatt.bsa_forward(q.double().numpy(), k.double().numpy(), v.double().numpy(), ind, cnt,
                                1.0 / math.sqrt(D), bs)
    for name, entry, want in (("hy", longcat_flash_attn, torch.float32),
                              ("mg", mg_longcat_flash_attn, torch.bfloat16)):
        out = entry(q.to(dev), k.to(dev), v.to(dev), ind_view, torch.from_numpy(cnt).to(dev))
        torch.cuda.synchronize()
        err = np.abs(out.float().cpu().numpy() - o_ref).max()
        print(f"[gpu]   {name}: dtype {out.dtype}, max abs err vs float64 {err:.3e}", flush=True)
        assert out.dtype == want
        assert out.shape == q.shape and out.is_contiguous()
        assert err <= TOL


def test_balanced_order_gives_the_same_bits(dev):
    """LI_BSA_BALANCE only reorders the query tiles: the same bits as whole tiles in natural order."""
    bs, D, B, H, nq, nkb = 128, 128, 2, 3, 37, 40
    Lq, Lk = nq * bs - 5, nkb * bs
    print(f"[gpu] bsa balanced order B={B} H={H} nq={nq} ragged 0..{nkb}", flush=True)
    rng = np.random.default_rng(17)
    q, k, v = _inputs(43, B, H, Lq, Lk, D)
    ind, cnt = _random_lists(rng, B, H, nq, nkb, nkb)   # row lengths 0..40, empty rows included
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    scale = 1.0 / math.sqrt(D)
    out_b, lse_b = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, return_lse=True, balance=True)
    out_w, lse_w = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, return_lse=True, split=False)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), out_w.view(torch.int16))
    assert torch.equal(torch.isneginf(lse_b), torch.isneginf(lse_w))
    fin = torch.isfinite(lse_w)
    assert torch.equal(lse_b[fin], lse_w[fin])
    o_ref, _ = oatt.bsa_forward(_f64(q), _f64(k), _f64(v), ind, cnt, scale, bs)
    err = np.abs(out_b.float().cpu().numpy() - o_ref).max()
    print(f"[gpu]   balanced vs oracle: max abs err {err:.3e}", flush=True)
    assert err <= TOL


def test_balanced_order_per_head_chunks(dev):
    """With B*H a multiple of the 8 XCDs the balanced order sorts and dispatches one head's tiles per chunk: still
    the same bits as whole tiles in natural order."""
    bs, D, B, H, nq, nkb = 128, 128, 2, 4, 21, 30
    Lq, Lk = nq * bs, nkb * bs
    print(f"[gpu] bsa balanced order, per-head chunks B={B} H={H} nq={nq}", flush=True)
    rng = np.random.default_rng(23)
    q, k, v = _inputs(47, B, H, Lq, Lk, D)
    ind, cnt = _random_lists(rng, B, H, nq, nkb, nkb)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    ii, cc = torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)
    scale = 1.0 / math.sqrt(D)
    out_b = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, balance=True)
    out_w = _core.bsa_forward(qd, kd, vd, ii, cc, scale, bs, split=False)
    torch.cuda.synchronize()
    assert torch.equal(out_b.view(torch.int16), out_w.view(torch.int16))
