"""Pins oracle.tile: gather/untile round trip, zero padding, pool = exact mean to within rounding."""
import numpy as np
import pytest

from oracle.bf16 import bf16_to_f32, f32_to_bf16
from oracle.tile import pool_mean, tile_gather, untile


def _rand_bits(rng, shape, scale=1.0):
    return f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("T,H,W,tile,D", [(2, 32, 32, (4, 4, 4), 64), (3, 10, 13, (2, 8, 8), 128),
                                          (4, 30, 52, (2, 8, 8), 128), (5, 6, 7, (4, 4, 8), 64)])
def test_roundtrip_and_padding(T, H, W, tile, D):
    rng = np.random.default_rng(T * 100 + H)
    x = _rand_bits(rng, (1, 2, T * H * W, D))
    tiles = tile_gather(x, T, H, W, tile)
    back = untile(tiles, T * H * W, T, H, W, tile)
    assert np.array_equal(back, x)
    # number of nonzero rows equals the number of valid tokens (random data has no zero rows)
    nz = (tiles.reshape(1, 2, -1, D) != 0).any(axis=-1).sum(axis=-1)
    assert np.all(nz == T * H * W)


def test_pool_equals_exact_mean_within_rounding():
    rng = np.random.default_rng(3)
    for D, tile in ((128, (2, 8, 8)), (64, (4, 4, 4))):
        x = _rand_bits(rng, (1, 3, 4 * 24 * 40, D), scale=3.0)
        tiles = tile_gather(x, 4, 24, 40, tile)
        pool = pool_mean(tiles)
        exact = bf16_to_f32(tiles).astype(np.float64).mean(axis=3)
        ref = f32_to_bf16(exact.astype(np.float32))
        diff = np.abs(pool.astype(np.int32) - ref.astype(np.int32))
        assert diff.max() <= 1
        assert (diff == 0).mean() > 0.99


def test_pool_exact_on_integers_and_padding_counts():
    # small integers sum exactly in fp32 in any order: the pool is the exact mean incl. padding rows
    rng = np.random.default_rng(4)
    x = f32_to_bf16(rng.integers(-8, 9, size=(1, 1, 2 * 5 * 6, 64)).astype(np.float32))
    tiles = tile_gather(x, 2, 5, 6, (4, 4, 4))   # every tile has padding (T=2 < 4, H, W ragged)
    pool = pool_mean(tiles)
    s = bf16_to_f32(tiles).astype(np.float64).sum(axis=3) / 64.0
    assert np.array_equal(pool, f32_to_bf16(s.astype(np.float32)))
