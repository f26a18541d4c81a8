"""Pins oracle.fp8 against torch's float8_e4m3fn casts and the mathematics of block scaling."""
import numpy as np
import torch

from oracle.fp8 import dequantize_blocks, e4m3_decode, e4m3_encode, quantize_blocks


def _torch_codes(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(
        torch.uint8).numpy()


def test_decode_all_codes_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    got = e4m3_decode(codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))  # signed zeros too
    assert e4m3_decode(np.uint8(0x7E)) == 448.0 and e4m3_decode(np.uint8(0x01)) == 2.0 ** -9


def test_encode_every_bf16_pattern_matches_torch():
    b = np.arange(0, 0x10000, dtype=np.uint32)
    x = (b << 16).view(np.float32)
    x = x[~np.isnan(x)]
    assert np.array_equal(e4m3_encode(x), _torch_codes(x))


def test_encode_midpoints_and_neighbours_match_torch():
    mags = e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float32)
    mids = ((mags[:-1].astype(np.float64) + mags[1:]) / 2).astype(np.float32)
    pts = np.concatenate([mags, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                          np.float32([448, 450, 463.99, 464, 464.00003, 470, 480, 1e30, np.inf, 2.0 ** -10,
                                      2.0 ** -10 * 1.0000001, 3 * 2.0 ** -11])])
    pts = np.concatenate([pts, -pts]).astype(np.float32)
    got = e4m3_encode(pts)
    assert np.array_equal(got, _torch_codes(pts))
    # The documented overflow rule: 464 ties down to 448, anything above is NaN.
    assert e4m3_encode(np.float32(464.0)) == 0x7E
    assert e4m3_encode(np.float32(464.00003)) == 0x7F
    assert e4m3_encode(np.float32(-np.inf)) == 0xFF


def test_encode_random_matches_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(300000) * np.exp(rng.uniform(-14, 7, 300000))).astype(np.float32)
    assert np.array_equal(e4m3_encode(x), _torch_codes(x))


def test_block_quantizer_bounds_and_exact_cases():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((3, 5, 128, 64)) * np.exp(rng.uniform(-6, 6, (3, 5, 1, 1)))).astype(np.float32)
    x[1, 2] = 0.0  # an all-zero block
    codes, scales = quantize_blocks(x)
    assert codes.shape == x.shape and scales.shape == (3, 5)
    assert not np.isnan(e4m3_decode(codes)).any()
    assert scales[1, 2] == 1.0 and not codes[1, 2].any()
    # Each block's largest magnitude maps to 448 (the code 0x7E).
    nz = np.abs(x).max(axis=(-2, -1)) > 0
    assert ((codes & 0x7F).max(axis=(-2, -1))[nz] == 0x7E).all()
    # Within half an e4m3 step: relative 2^-4 for normals, 2^-10 scale units below.
    deq = dequantize_blocks(codes, scales)
    err = np.abs(deq - x)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, 2.0 ** -10 * scales[..., None, None]) * (1 + 1e-6)
    assert (err <= bound).all()
    # Inputs that are e4m3 values times 2^k with the block max at 448 * 2^k are exact.
    c = rng.integers(0, 0x7F, (2, 128, 64)).astype(np.uint8) | (rng.integers(0, 2, (2, 128, 64)) << 7).astype(
        np.uint8)
    c[:, 0, 0] = 0x7E
    y = (e4m3_decode(c).astype(np.float64) * np.array([2.0 ** -5, 2.0 ** 3])[:, None, None]).astype(np.float32)
    codes2, scales2 = quantize_blocks(y)
    assert np.array_equal(codes2 & 0x7F, c & 0x7F)
    assert np.array_equal(dequantize_blocks(codes2, scales2), y.astype(np.float64))


def test_scale_is_amax_over_448():
    x = np.zeros((1, 128, 128), dtype=np.float32)
    x[0, 5, 7] = -3.0
    x[0, 9, 1] = 1.5
    codes, scales = quantize_blocks(x)
    assert scales[0] == np.float32(3.0) / np.float32(448.0)
    assert codes[0, 5, 7] == 0xFE and e4m3_decode(codes[0, 9, 1]) == 224.0
