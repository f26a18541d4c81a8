"""GPU: the torch.ops.li operators pass torch.library.opcheck and trace under torch.compile.

opcheck runs each operator for real on the GPU and checks its schema
(mutated arguments are the annotated ones), its fake implementation against
the real outputs, and its behaviour under AOT dispatch with dynamic shapes.
"""
import math

import numpy as np
import pytest
import torch

from li_sparse._ops import ops

pytestmark = pytest.mark.gpu


def _tokens(dev, B=1, H=2, frames=2, hw=(16, 16), scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    L = frames * hw[0] * hw[1]
    return (torch.randn(B, L, H, 128, generator=g) * scale).to(torch.bfloat16).to(dev).permute(0, 2, 1, 3)


def _lists(dev, H, nq, nk, kmax, seed=1):
    rng = np.random.default_rng(seed)
    ind = np.zeros((1, H, nq, kmax), np.int32)
    cnt = np.zeros((1, H, nq), np.int32)
    for h in range(H):
        for r in range(nq):
            n = int(rng.integers(1, kmax + 1))
            ind[0, h, r, :n] = np.sort(rng.choice(nk, n, replace=False))
            cnt[0, h, r] = n
    return torch.from_numpy(ind).to(dev), torch.from_numpy(cnt).to(dev)


def test_opcheck_attention_ops(dev):
    print("[gpu] opcheck bsa_fwd_gather / bsa_fwd / attn_dense", flush=True)
    q, k, v = _tokens(dev, scale=0.3, seed=1), _tokens(dev, frames=4, seed=2), _tokens(dev, frames=4, seed=3)
    gq, gk = [2, 16, 16, 2, 8, 8, 2, 2], [4, 16, 16, 2, 8, 8, 2, 2]
    ind, cnt = _lists(dev, 2, 4, 8, 5)
    scale = 1.0 / math.sqrt(128)
    torch.library.opcheck(ops.bsa_fwd_gather.default,
                          (q, k, v, None, None, 0, gq, gk, ind, cnt, scale, torch.empty_like(q), True, True, False))
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    torch.library.opcheck(ops.bsa_fwd.default,
                          (qc, kc, vc, ind, cnt, scale, 128, torch.empty_like(qc), True, True, False))
    torch.library.opcheck(ops.attn_dense.default, (q, k, v, None, None, 0, scale, torch.empty_like(q), True, True))


def test_opcheck_prep_and_mask_ops(dev):
    print("[gpu] opcheck pool_pair / q_prep / kv_prep / untile / block_mask", flush=True)
    q, k = _tokens(dev, seed=4), _tokens(dev, frames=4, seed=5)
    gq, gk = [2, 16, 16, 2, 8, 8, 2, 2], [4, 16, 16, 2, 8, 8, 2, 2]
    qp = torch.empty((1, 2, 4, 128), dtype=torch.bfloat16, device=dev)
    kp = torch.empty((1, 2, 8, 128), dtype=torch.bfloat16, device=dev)
    torch.library.opcheck(ops.pool_pair.default, (q, qp, 0, gq, k, kp, 0, gk))
    torch.library.opcheck(ops.pool_pair.default, (q, qp, 0, gq, k, kp, 0, gk, torch.empty_like(kp)))
    qt = torch.empty((1, 2, 4, 128, 128), dtype=torch.bfloat16, device=dev)
    torch.library.opcheck(ops.q_prep.default, (q, qt, qp, gq))
    kt, vt = (torch.empty((1, 2, 8, 128, 128), dtype=torch.bfloat16, device=dev) for _ in range(2))
    torch.library.opcheck(ops.kv_prep.default, (k, k, kt, vt, kp, 0, 0, gk))
    torch.library.opcheck(ops.untile.default, (qt, torch.empty_like(q), gq))
    # opcheck runs the ops above on copies, so qp / kp still hold whatever the allocator gave: fill them.
    g = torch.Generator().manual_seed(9)
    qp.copy_(torch.randn(qp.shape, generator=g).to(qp.dtype))
    kp.copy_(torch.randn(kp.shape, generator=g).to(kp.dtype))
    torch.library.opcheck(ops.block_mask.default,
                          (qp, kp, 1, 0, 0.5, 7, 0, True, True, False, 2, 2, 0, 8, None, True))
    torch.library.opcheck(ops.block_mask.default,
                          (qp, kp, 0, 0, 0.5, 7, 0, True, True, False, 2, 2, 0, 8, None, True, True))


def test_compiled_graph_calls_the_ops(dev):
    """torch.compile(fullgraph=True) traces the pools, the mask and the fused attention through their fakes."""
    print("[gpu] torch.compile fullgraph over torch.ops.li", flush=True)
    q, k, v = _tokens(dev, scale=0.3, seed=6), _tokens(dev, frames=4, seed=7), _tokens(dev, frames=4, seed=8)
    gq, gk = [2, 16, 16, 2, 8, 8, 2, 2], [4, 16, 16, 2, 8, 8, 2, 2]

    def call(q, k, v):
        qp = q.new_empty((1, 2, 4, 128))
        kp = q.new_empty((1, 2, 8, 128))
        torch.ops.li.pool_pair(q, qp, 0, gq, k, kp, 0, gk)
        ind, cnt, _ = torch.ops.li.block_mask(qp, kp, 1, 0, 0.5, 7, 0, True, True, False, 2, 2, 0, 8, None, False)
        out = torch.empty_like(q)
        torch.ops.li.bsa_fwd_gather(q, k, v, None, None, 0, gq, gk, ind, cnt, 1.0 / math.sqrt(128), out, False,
                                    True, False)
        return out

    eager = call(q, k, v)
    compiled = torch.compile(call, fullgraph=True, backend="aot_eager")(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(eager.view(torch.int16), compiled.view(torch.int16))


def test_direct_calls_check_extents(dev):
    """The operators reject tensors shorter than the geometry or lists index them, before any launch."""
    print("[gpu] direct operator calls with short tensors raise", flush=True)
    q, k, v = _tokens(dev, seed=10), _tokens(dev, frames=4, seed=11), _tokens(dev, frames=4, seed=12)
    gq, gk = [2, 16, 16, 2, 8, 8, 2, 2], [4, 16, 16, 2, 8, 8, 2, 2]
    short_k = k[:, :, :-1]
    qp = torch.zeros((1, 2, 4, 128), dtype=torch.bfloat16, device=dev)
    kp = torch.zeros((1, 2, 8, 128), dtype=torch.bfloat16, device=dev)
    ind, cnt = _lists(dev, 2, 4, 8, 5)
    scale = 1.0 / math.sqrt(128)
    txt = torch.zeros((1, 2, 128, 128), dtype=torch.bfloat16, device=dev)
    txt_long = torch.zeros((1, 2, 256, 128), dtype=torch.bfloat16, device=dev)
    q8 = torch.zeros((1, 2, 512, 128), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    k8 = torch.zeros((1, 2, 1024, 128), dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    qs_long = torch.ones((1, 2, 5), dtype=torch.float32, device=dev)
    ks = torch.ones((1, 2, 8), dtype=torch.float32, device=dev)
    vt = torch.zeros((1, 2, 1024, 128), dtype=torch.bfloat16, device=dev)
    cases = [
        ("src must", lambda: torch.ops.li.pool(short_k, kp, 0, gk)),
        ("mean must", lambda: torch.ops.li.pool(k, kp[:, :, :7], 0, gk)),
        ("mean must", lambda: torch.ops.li.pool(k, kp, 1, gk)),
        ("src1 must", lambda: torch.ops.li.pool_pair(q, qp, 0, gq, short_k, kp, 0, gk)),
        ("dst must", lambda: torch.ops.li.q_prep(q, torch.empty((1, 2, 3, 128, 128), dtype=torch.bfloat16, device=dev),
                                            qp, gq)),
        ("dst must", lambda: torch.ops.li.untile(torch.empty((1, 2, 4, 128, 128), dtype=torch.bfloat16, device=dev),
                                            q[:, :, :-1], gq)),
        ("k_pool must", lambda: torch.ops.li.block_mask(qp, kp[..., :64], 1, 0, 0.5, 7, 0, True, True, False, 2, 2, 0, 8,
                                                   None, False)),
        ("k must", lambda: torch.ops.li.bsa_fwd_gather(q, short_k, v, None, None, 0, gq, gk, ind, cnt, scale,
                                                  torch.empty_like(q), False, True, False)),
        ("block_indices must", lambda: torch.ops.li.bsa_fwd_gather(q, k, v, None, None, 0, gq, gk, ind[:, :, :3], cnt,
                                                              scale, torch.empty_like(q), False, True, False)),
        ("k_txt is required", lambda: torch.ops.li.bsa_fwd_gather(q, k, v, None, None, 1, gq, gk, ind, cnt, scale,
                                                      torch.empty_like(q), False, True, False)),
        ("block_counts must", lambda: torch.ops.li.bsa_fwd(q.contiguous(), k.contiguous(), v.contiguous(), ind,
                                                      cnt[:, :, :2], scale, 128, torch.empty_like(q.contiguous()),
                                                      False, True, False)),
        ("v must", lambda: torch.ops.li.attn_dense(q, k, v[:, :, :-128], None, None, 0, scale, torch.empty_like(q),
                                              False, True)),
        # Over-long contiguous tensors the kernels index at a per-head pitch: exact extents only.
        ("k_txt must", lambda: torch.ops.li.bsa_fwd_gather(q, k, v, txt_long, txt, 1, gq, gk, ind, cnt, scale,
                                                      torch.empty_like(q), False, True, False)),
        ("v_txt must", lambda: torch.ops.li.attn_dense(q, k, v, txt, txt_long, 100, scale, torch.empty_like(q),
                                                  False, True)),
        ("q_scale must", lambda: torch.ops.li.bsa_fwd_fp8(q8, qs_long, k8, ks, vt, ind, cnt, scale, 128,
                                                     torch.empty_like(vt[:, :, :512]), False, True, False)),
    ]
    for what, call in cases:
        with pytest.raises(RuntimeError, match=what):
            call()
    torch.cuda.synchronize()
    # The valid calls still run.
    torch.ops.li.pool_pair(q, qp, 0, gq, k, kp, 0, gk)
    torch.ops.li.bsa_fwd_gather(q, k, v, None, None, 0, gq, gk, ind, cnt, scale, torch.empty_like(q), False, True,
                                False)
    torch.cuda.synchronize()
