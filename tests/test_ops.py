"""The torch.ops.li custom operators: registration, schemas and fake (meta) implementations (no GPU needed)."""
import pytest
import torch

from li_sparse._ops import ops

OPS = ["pool", "pool_pair", "q_prep", "kv_prep", "untile", "block_mask", "bsa_fwd", "bsa_fwd_gather", "attn_dense",
       "tile_prep_fp8", "kv_prep_fp8", "bsa_fwd_fp8", "bsa_fwd_fp8_gather"]
META = torch.device("meta")


@pytest.mark.parametrize("name", OPS)
def test_registered_with_gpu_kernel_and_fake(name):
    op = getattr(ops, name).default
    assert op._schema.name == f"li::{name}"
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "CUDA")
    assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), "Meta")


def test_mutation_annotations():
    """Tiles, pools and attention outputs are declared as written (Tensor(a!)); sources are not."""
    def written(name):
        return [a.name for a in getattr(ops, name).default._schema.arguments
                if a.alias_info is not None and a.alias_info.is_write]
    assert written("q_prep") == ["dst", "mean"]
    assert written("kv_prep") == ["k_dst", "v_dst", "k_mean"]
    assert written("pool_pair") == ["mean0", "mean1", "mean1_normalized"]
    assert written("untile") == ["dst"]
    assert written("bsa_fwd") == written("bsa_fwd_gather") == written("attn_dense") == ["out"]
    assert written("block_mask") == []


def _t(shape, dtype=torch.bfloat16):
    return torch.empty(shape, dtype=dtype, device=META)


def test_fake_block_mask_shapes():
    qp, kp = _t((2, 3, 56, 128)), _t((2, 3, 168, 128))
    ind, cnt, sc = ops.block_mask(qp, kp, 1, 0, 0.3, 7, 0, True, True, False, 4, 7, 2, 55, None, True)
    assert ind.shape == (2, 3, 56, 55) and ind.dtype == torch.int32
    assert cnt.shape == (2, 3, 56) and cnt.dtype == torch.int32
    assert sc.shape == (2, 3, 56, 168) and sc.dtype == torch.bfloat16
    _, _, sc = ops.block_mask(qp, kp, 1, 0, 0.3, 7, 0, True, True, False, 4, 7, 2, 55, None, False)
    assert sc.numel() == 0


def test_fake_attention_shapes():
    # HY grid: 4 query frames of 30 x 52 in 2x8x8 tiles -> 56 tiles of 128 rows; BLHD views.
    q = _t((1, 6240, 16, 128)).permute(0, 2, 1, 3)
    k = _t((1, 18720, 16, 128)).permute(0, 2, 1, 3)
    ind, cnt = _t((1, 16, 56, 51), torch.int32), _t((1, 16, 56), torch.int32)
    out = torch.empty_like(q)
    geo_q, geo_k = [4, 30, 52, 2, 8, 8, 4, 7], [12, 30, 52, 2, 8, 8, 4, 7]
    lse = ops.bsa_fwd_gather(q, k, k, None, None, 0, geo_q, geo_k, ind, cnt, 0.088, out, True, True, False)
    assert lse.shape == (1, 16, 56 * 128) and lse.dtype == torch.float32
    lse = ops.bsa_fwd_gather(q, k, k, None, None, 0, geo_q, geo_k, ind, cnt, 0.088, out, False, True, False)
    assert lse.numel() == 0
    qc = _t((1, 16, 7168, 128))
    lse = ops.bsa_fwd(qc, _t((1, 16, 21504, 128)), _t((1, 16, 21504, 128)), ind, cnt, 0.088, 128,
                      torch.empty_like(qc), True, True, False)
    assert lse.shape == (1, 16, 7168)
    lse = ops.attn_dense(q, k, k, None, None, 0, 0.088, out, True, True)
    assert lse.shape == (1, 16, 49 * 128)
    q8 = _t((1, 16, 7168, 128), torch.float8_e4m3fn)
    lse = ops.bsa_fwd_fp8(q8, _t((1, 16, 56), torch.float32), _t((1, 16, 21504, 128), torch.float8_e4m3fn),
                          _t((1, 16, 168), torch.float32), _t((1, 16, 21504, 128)), ind, cnt, 0.088, 128,
                          _t((1, 16, 7168, 128)), True, True, False)
    assert lse.shape == (1, 16, 7168)


def test_ops_trace_under_fake_tensor_mode():
    """The fake implementations are what torch.compile / torch.export trace through."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        qp, kp = torch.empty(1, 2, 8, 64, dtype=torch.bfloat16), torch.empty(1, 2, 16, 64, dtype=torch.bfloat16)
        ind, cnt, _ = torch.ops.li.block_mask.default(qp.to("meta"), kp.to("meta"), 0, 1, 0.5, 7, 0, False, False,
                                                      True, 2, 2, 0, 9, None, False)
        assert ind.shape == (1, 2, 8, 9)


def test_fake_rejects_over_long_pitch_indexed_tensors():
    """Tensors the kernels index at a per-head pitch implied by the geometry (contiguous padded text K/V, e4m3
    tiles and scales) must have exactly that extent: a longer contiguous tensor would make every head after the
    first read another head's rows.  The operators raise for it before tracing (meta tensors, no GPU)."""
    q = _t((1, 6240, 16, 128)).permute(0, 2, 1, 3)
    k = _t((1, 18720, 16, 128)).permute(0, 2, 1, 3)
    ind, cnt = _t((1, 16, 56, 53), torch.int32), _t((1, 16, 56), torch.int32)
    out = torch.empty_like(q)
    geo_q, geo_k = [4, 30, 52, 2, 8, 8, 4, 7], [12, 30, 52, 2, 8, 8, 4, 7]
    txt = _t((1, 16, 256, 128))
    ops.bsa_fwd_gather(q, k, k, txt, txt, 2, geo_q, geo_k, ind, cnt, 0.088, out, False, True, False)
    for bad in (_t((1, 16, 384, 128)), _t((1, 16, 128, 128))):
        with pytest.raises(RuntimeError, match="k_txt must be"):
            ops.bsa_fwd_gather(q, k, k, bad, txt, 2, geo_q, geo_k, ind, cnt, 0.088, out, False, True, False)
        with pytest.raises(RuntimeError, match="v_txt must be"):
            ops.bsa_fwd_gather(q, k, k, txt, bad, 2, geo_q, geo_k, ind, cnt, 0.088, out, False, True, False)
    with pytest.raises(RuntimeError, match="k_txt must be"):
        ops.attn_dense(q, k, k, _t((1, 16, 384, 128)), txt, 200, 0.088, out, False, True)
    q8, k8 = _t((1, 16, 7168, 128), torch.float8_e4m3fn), _t((1, 16, 21504, 128), torch.float8_e4m3fn)
    qs, ks, v = _t((1, 16, 56), torch.float32), _t((1, 16, 168), torch.float32), _t((1, 16, 21504, 128))
    o = _t((1, 16, 7168, 128))
    ops.bsa_fwd_fp8(q8, qs, k8, ks, v, ind, cnt, 0.088, 128, o, False, True, False)
    with pytest.raises(RuntimeError, match="q_scale must be"):
        ops.bsa_fwd_fp8(q8, _t((1, 16, 57), torch.float32), k8, ks, v, ind, cnt, 0.088, 128, o, False, True, False)
    with pytest.raises(RuntimeError, match="k_scale must be"):
        ops.bsa_fwd_fp8(q8, qs, k8, _t((1, 16, 170), torch.float32), v, ind, cnt, 0.088, 128, o, False, True, False)
    # token-order e4m3: V and O in token order, tiles and scales with two text blocks
    k8t, kst = _t((1, 16, 170 * 128, 128), torch.float8_e4m3fn), _t((1, 16, 170), torch.float32)
    ops.bsa_fwd_fp8_gather(q8, qs, k8t, kst, k, txt, 2, geo_q, geo_k, ind, cnt, 0.088, out, False, False, False)
    for args, what in (((_t((1, 16, 7296, 128), torch.float8_e4m3fn), qs, k8t, kst), "q8 must be"),
                       ((q8, qs, _t((1, 16, 171 * 128, 128), torch.float8_e4m3fn), kst), "k8 must be"),
                       ((q8, _t((1, 16, 60), torch.float32), k8t, kst), "q_scale must be"),
                       ((q8, qs, k8t, _t((1, 16, 171), torch.float32)), "k_scale must be")):
        with pytest.raises(RuntimeError, match=what):
            ops.bsa_fwd_fp8_gather(*args, k, txt, 2, geo_q, geo_k, ind, cnt, 0.088, out, False, False, False)
