"""Pins oracle.bf16 against torch's own float32 -> bfloat16 conversion."""
import numpy as np
import torch

from oracle.bf16 import bf16_order_key, bf16_to_f32, f32_to_bf16


def _torch_bits(x):
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_random_values_match_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200000) * np.exp(rng.uniform(-30, 30, 200000))).astype(np.float32)
    assert np.array_equal(f32_to_bf16(x), _torch_bits(x))


def test_ties_overflow_denormals_specials():
    u = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF, 0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF,
                  0x00008000, 0x00018000, 0x00000001, 0x80000000, 0xBF808000, 0xFF7FFFFF, 0x7F800000,
                  0xFF800000, 0x00000000], dtype=np.uint32)
    x = u.view(np.float32)
    assert np.array_equal(f32_to_bf16(x), _torch_bits(x))
    nan = np.array([np.nan], dtype=np.float32)
    assert np.isnan(bf16_to_f32(f32_to_bf16(nan)))[0]


def test_roundtrip_exact_and_order_key():
    b = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    f = bf16_to_f32(b)
    finite = np.isfinite(f)
    assert np.array_equal(f32_to_bf16(f[finite]), b[finite])
    # keys are distinct and increase with value (-0 sorts just below +0)
    ks = bf16_order_key(b[finite])
    assert np.unique(ks).size == ks.size
    vals = f[finite]
    i, j = np.random.default_rng(1).integers(0, vals.size, (2, 100000))
    lt = vals[i] < vals[j]
    assert np.all(ks[i][lt] < ks[j][lt])
