"""Pins oracle.geometry: brute-force inverse maps and hand-computed block counts."""
import numpy as np
import pytest

from oracle.geometry import block_geometry, pad_blocks, tile_permutation


@pytest.mark.parametrize("T,H,W,tile", [(2, 32, 32, (4, 4, 4)), (5, 7, 9, (2, 3, 4)), (4, 30, 52, (2, 8, 8)),
                                        (3, 22, 40, (4, 4, 8)), (1, 1, 1, (1, 1, 1)), (6, 8, 8, (4, 8, 4))])
def test_permutation_is_inverse_of_token_to_slot(T, H, W, tile):
    tt, th, tw = tile
    perm = tile_permutation(T, H, W, tile)
    nh, nw = -(-H // th), -(-W // tw)
    bs = tt * th * tw
    # valid slots are a permutation of all tokens
    valid = perm[perm >= 0]
    assert np.array_equal(np.sort(valid), np.arange(T * H * W))
    # brute force from the token side: token (t,h,w) lives in block (t//tt, h//th, w//tw) at row
    # ((t%tt)*th + h%th)*tw + w%tw
    for t in range(T):
        for h in range(H):
            for w in range(W):
                blk = ((t // tt) * nh + h // th) * nw + w // tw
                f = ((t % tt) * th + h % th) * tw + w % tw
                assert perm[blk * bs + f] == (t * H + h) * W + w


def test_block_counts_for_workload_shapes():
    hy = block_geometry(6240, 18720, (30, 52), (2, 8, 8))
    assert (hy["nh"], hy["nw"], hy["nq_blk"], hy["nk_blk"], hy["lq_pad"], hy["lk_pad"]) == (4, 7, 56, 168, 7168, 21504)
    mg = block_geometry(3520, 17600, (22, 40), (2, 8, 8))
    assert (mg["nh"], mg["nw"], mg["nq_blk"], mg["nk_blk"], mg["lq_pad"], mg["lk_pad"]) == (3, 5, 30, 150, 3840, 19200)
    toy = block_geometry(2048, 2048, (32, 32), (4, 4, 4))
    assert (toy["BS"], toy["nq_blk"], toy["nk_blk"], toy["lq_pad"]) == (64, 64, 64, 4096)
    long = block_geometry(6240, 99840, (30, 52), (2, 8, 8))
    assert (long["nk_blk"], long["lk_pad"]) == (896, 114688)
    txt = block_geometry(6240, 18720, (30, 52), (4, 8, 4), text_len=300)
    assert txt["num_txt_blk"] == 3 and txt["BS"] == 128


def test_reference_padding_formula():
    for x in range(0, 200):
        for t in range(1, 9):
            assert pad_blocks(x, t) == -(-x // t)
