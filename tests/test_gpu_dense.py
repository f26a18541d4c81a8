"""GPU parity of the dense attention kernel (li_attn_fwd_dense) against softmax attention in float64 / fp32.

The reference's dense fallback is ``F.scaled_dot_product_attention(q, cat(k_txt, k_vis), cat(v_txt, v_vis))``;
the kernel computes it without the concatenation, with the keys past each sequence's end masked out.
"""
import math

import numpy as np
import pytest
import torch

from li_sparse import _core, _pipeline
from li_sparse._lib import LiError
from li_sparse.hy import bi_sparse_operation_for_KV_cache as hykv
from li_sparse.hy.ar_sparse_operation import run_sparse_attention
from li_sparse.hy.infer_state import get_infer_state
from li_sparse.workloads import WORKLOADS, Workload, make_qkv

pytestmark = pytest.mark.gpu
TOL = 2e-2  # max-abs error of the bf16/f16 output


def _ref64(q, k, v, k_txt=None, v_txt=None, scale=None):
    """softmax(scale q K^T) V in float64 on the CPU, K/V = cat(text, visual); also lse in log2 units."""
    if k_txt is not None:
        k, v = torch.cat([k_txt, k], dim=2), torch.cat([v_txt, v], dim=2)
    q, k, v = q.double().cpu(), k.double().cpu(), v.double().cpu()
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    lse = torch.logsumexp(s, dim=-1) / math.log(2.0)
    return torch.matmul(torch.softmax(s, dim=-1), v), lse


def _rand(g, B, H, L, D, dtype, layout):
    x = torch.randn(B, H, L, D, generator=g).to(dtype)
    if layout == "blhd":
        x = x.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    return x


@pytest.mark.parametrize("Lq,Lk,txt", [(300, 520, 0), (300, 520, 77), (128, 256, 128), (50, 36, 0), (200, 0, 90),
                                       (777, 1024, 300)])
@pytest.mark.parametrize("dtype,layout", [(torch.bfloat16, "bhld"), (torch.bfloat16, "blhd"), (torch.float16, "blhd")])
def test_dense_vs_float64(dev, Lq, Lk, txt, dtype, layout):
    print(f"[gpu] dense Lq={Lq} Lk={Lk} txt={txt} {dtype} {layout}", flush=True)
    B, H, D = 1, 3, 128
    g = torch.Generator().manual_seed(Lq * 7 + Lk + txt)
    q = _rand(g, B, H, Lq, D, dtype, layout) * 0.3
    k, v = _rand(g, B, H, Lk, D, dtype, layout), _rand(g, B, H, Lk, D, dtype, layout)
    kt = vt = None
    if txt:
        kt, vt = _rand(g, B, H, txt, D, dtype, "bhld"), _rand(g, B, H, txt, D, dtype, "bhld")
    out, lse = _core.attn_dense(q.to(dev), k.to(dev), v.to(dev), kt.to(dev) if txt else None,
                                vt.to(dev) if txt else None, return_lse=True)
    torch.cuda.synchronize()
    assert out.stride() == q.to(dev).stride()
    ref, lse_ref = _ref64(q, k, v, kt, vt)
    err = (out.double().cpu() - ref).abs().max().item()
    d_lse = (lse[:, :, :Lq].double().cpu() - lse_ref).abs().max().item()
    print(f"[gpu]   max abs err {err:.3e}, lse {d_lse:.3e}", flush=True)
    assert err <= TOL and d_lse < 1e-3


def test_dense_hy_shape_two_heads(dev):
    """Full HY shape (16 heads, Lq=6240, Lk=18720, BLHD views); two heads checked against fp32 SDPA."""
    wl = WORKLOADS["hy"]
    print("[gpu] dense HY shape (16 heads, Lq=6240, Lk=18720)", flush=True)
    q, k, v = make_qkv(wl, seed=2, layout="blhd")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    out = _core.attn_dense(qd, kd, vd)
    heads = [0, 11]
    ref = torch.nn.functional.scaled_dot_product_attention(qd[:, heads].float(), kd[:, heads].float(),
                                                           vd[:, heads].float())
    torch.cuda.synchronize()
    err = (out[:, heads].float() - ref).abs().max().item()
    print(f"[gpu]   max abs err (heads {heads}) {err:.3e}", flush=True)
    assert err <= TOL


def test_entry_points_take_the_dense_kernel(dev, monkeypatch):
    """Untileable decode shapes and prefill chunks < 3 go through li_attn_fwd_dense and match the reference's SDPA."""
    calls = []
    real = _core.attn_dense
    monkeypatch.setattr(_core, "attn_dense", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    wl = Workload("hy_small", 2, 128, (30, 52), 4, 4, (2, 8, 8), 0.3, "scaled_dot_product")
    q, k, v = make_qkv(wl, seed=8, layout="blhd")
    g = torch.Generator().manual_seed(3)
    kt = torch.randn(1, 2, 77, 128, generator=g).to(torch.bfloat16)
    vt = torch.randn(1, 2, 77, 128, generator=g).to(torch.bfloat16)
    qd, kd, vd, ktd, vtd = q.to(dev), k.to(dev), v.to(dev), kt.to(dev), vt.to(dev)
    params = {"tile_size": (2, 8, 8), "topk_ratio": 0.3, "sim_metric": "scaled_dot_product"}
    print("[gpu] dense fallback: untileable decode shape, prefill chunk 1", flush=True)
    out_a = run_sparse_attention(qd[:, :, :1000], ktd, vtd, kd, vd, 0, wl.latent_hw, params)   # 1000 % 1560 != 0
    state = get_infer_state()
    state.current_chunk_index = 1
    try:
        out_b = hykv.run_sparse_prefill_attention(qd, ktd, vtd, kd, vd, 0, wl.latent_hw, params)
    finally:
        state.current_chunk_index = 0
    ref_a = torch.nn.functional.scaled_dot_product_attention(qd[:, :, :1000].float(), torch.cat([ktd, kd], 2).float(),
                                                             torch.cat([vtd, vd], 2).float())
    ref_b = torch.nn.functional.scaled_dot_product_attention(qd.float(), torch.cat([ktd, kd], 2).float(),
                                                             torch.cat([vtd, vd], 2).float())
    torch.cuda.synchronize()
    assert len(calls) == 2
    assert (out_a.float() - ref_a).abs().max().item() <= TOL
    assert (out_b.float() - ref_b).abs().max().item() <= TOL


def test_unsupported_shapes(dev):
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 2, 100, 128, generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn(1, 2, 130, 128, generator=g).to(torch.bfloat16).to(dev)   # 130 % 4 != 0
    v = torch.randn(1, 2, 130, 128, generator=g).to(torch.bfloat16).to(dev)
    assert not _core.dense_supported(q, k, v)
    with pytest.raises(LiError, match="UNSUPPORTED|unsupported"):
        _core.attn_dense(q, k, v)
    # the pipeline takes the reference's torch call for it
    out = _pipeline.dense_attention(q, None, None, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    torch.cuda.synchronize()
    assert (out.float() - ref).abs().max().item() <= TOL
