"""Pins oracle.attention against torch's own SDPA (float64, CPU), closed forms and invariants."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt


def _rand(rng, *shape, scale=1.0):
    return rng.standard_normal(shape) * scale


def test_single_block_is_dense_softmax():
    rng = np.random.default_rng(0)
    q, k, v = _rand(rng, 1, 2, 128, 64), _rand(rng, 1, 2, 384, 64), _rand(rng, 1, 2, 384, 64)
    ind = np.array([[[[1]], [[2]]]], dtype=np.int32)
    cnt = np.ones((1, 2, 1), np.int32)
    o, lse = oatt.bsa_forward(q, k, v, ind, cnt, 0.125, 128)
    for h, j in ((0, 1), (1, 2)):
        ref = F.scaled_dot_product_attention(torch.tensor(q[:, h]), torch.tensor(k[:, h, j * 128:(j + 1) * 128]),
                                             torch.tensor(v[:, h, j * 128:(j + 1) * 128]), scale=0.125)
        assert np.allclose(o[:, h], ref.numpy(), atol=1e-12)
        s = torch.tensor(q[0, h]) @ torch.tensor(k[0, h, j * 128:(j + 1) * 128]).T * 0.125
        assert np.allclose(lse[0, h], (torch.logsumexp(s, -1) / math.log(2)).numpy(), atol=1e-12)


def test_all_blocks_is_dense_over_padded_keys_and_order_invariant():
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 1, 1, 256, 32), _rand(rng, 1, 1, 512, 32), _rand(rng, 1, 1, 512, 32)
    k[:, :, 300:] = 0.0   # zero-padded key rows take part in the softmax
    v[:, :, 300:] = 0.0
    ind = np.array([[[[0, 1, 2, 3], [0, 1, 2, 3]]]], dtype=np.int32)
    cnt = np.full((1, 1, 2), 4, np.int32)
    o, _ = oatt.bsa_forward(q, k, v, ind, cnt, 0.2, 128)
    ref = F.scaled_dot_product_attention(torch.tensor(q), torch.tensor(k), torch.tensor(v), scale=0.2).numpy()
    assert np.allclose(o, ref, atol=1e-12)
    o_rev, _ = oatt.bsa_forward(q, k, v, ind[..., ::-1].copy(), cnt, 0.2, 128)
    assert np.allclose(o, o_rev, atol=1e-12)


def test_identical_keys_closed_form_with_padding():
    # every valid key is the same vector kk, so s = q.kk for each valid key and 0 for padded keys:
    # out = sum_valid v / (n_valid + n_pad * exp(-s*scale))
    rng = np.random.default_rng(2)
    D, n_valid = 16, 100
    kk = rng.standard_normal(D)
    q = rng.standard_normal((1, 1, 64, D))
    k = np.zeros((1, 1, 128, D))
    v = np.zeros((1, 1, 128, D))
    k[0, 0, :n_valid] = kk
    v[0, 0, :n_valid] = rng.standard_normal((n_valid, D))
    o, _ = oatt.bsa_forward(q, k, v, np.zeros((1, 1, 1, 1), np.int32), np.ones((1, 1, 1), np.int32), 0.3, 128,
                            block_m=64)
    s = (q[0, 0] @ kk) * 0.3
    expect = v[0, 0, :n_valid].sum(0)[None, :] / (n_valid + 28 * np.exp(-s))[:, None]
    assert np.allclose(o[0, 0], expect, atol=1e-12)


def test_empty_rows_are_zero():
    rng = np.random.default_rng(3)
    q, k, v = _rand(rng, 1, 1, 128, 16), _rand(rng, 1, 1, 128, 16), _rand(rng, 1, 1, 128, 16)
    o, lse = oatt.bsa_forward(q, k, v, np.zeros((1, 1, 1, 1), np.int32), np.zeros((1, 1, 1), np.int32), 0.25, 128)
    assert np.all(o == 0) and np.all(np.isneginf(lse))


@pytest.mark.parametrize("bs", [64, 128])
def test_dense_masked_cpu_baseline_matches(bs):
    rng = np.random.default_rng(4)
    nq, nk, D = 3, 5, 64
    q = torch.tensor(rng.standard_normal((1, 2, nq * bs, D)), dtype=torch.bfloat16)
    k = torch.tensor(rng.standard_normal((1, 2, nk * bs, D)), dtype=torch.bfloat16)
    v = torch.tensor(rng.standard_normal((1, 2, nk * bs, D)), dtype=torch.bfloat16)
    ind = np.zeros((1, 2, nq, 3), np.int32)
    cnt = np.zeros((1, 2, nq), np.int32)
    for h in range(2):
        for r in range(nq):
            sel = np.sort(rng.choice(nk, size=r, replace=False))
            ind[0, h, r, :r] = sel
            cnt[0, h, r] = r
    o, _ = oatt.bsa_forward(q.double().numpy(), k.double().numpy(), v.double().numpy(), ind, cnt, 0.125, bs)
    base = oatt.dense_masked_cpu(q, k, v, ind, cnt, 0.125, bs).numpy()
    assert np.allclose(base, o[0], atol=2e-5)
