"""PyTorch custom operators ``torch.ops.li.*`` over the C ABI, and their fake (meta) implementations.

The operators are defined and implemented for ROCm ("cuda") tensors in
``libli_torch_ops.so`` (csrc/li_torch_ops.cpp), a thin C++ layer over
``libli_sparse_attn.so``: each one writes the tensors its schema marks as
mutated (tiles, pools, the attention output ``out``), allocates what it
returns (index lists, LSE) through torch's caching allocator, and enqueues
the C-ABI call on the current stream.  The fake implementations below give
the returned shapes, strides and dtypes without running anything, so the
operators trace under FakeTensor / meta tensors (torch.compile,
torch.export).  Loading fails loudly when either library is missing.

Operators (schemas in csrc/li_torch_ops.cpp): ``pool``, ``pool_pair``,
``q_prep``, ``kv_prep``, ``untile`` (tile gather / pool / scatter,
ar_sparse_operation.py:166-218), ``block_mask`` (fast_generate_indices /
generate_prefill_indices, ar_sparse_operation.py:223-284,
bi_sparse_operation_for_KV_cache.py:220-296), ``bsa_fwd`` (longcat_flash_attn,
longcat_kernel.py:158-233), ``bsa_fwd_gather`` (the fused tile / attend /
untile of run_sparse_attention, ar_sparse_operation.py:330-361),
``attn_dense`` (the dense fallback, ar_sparse_operation.py:316-317) and the
e4m3 variants ``tile_prep_fp8``, ``kv_prep_fp8``, ``bsa_fwd_fp8``,
``bsa_fwd_fp8_gather``.
"""
import os

import torch

from . import _lib  # noqa: F401  (loads libli_sparse_attn.so first; the op library links against it)

OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libli_torch_ops.so")


def _load():
    if not os.path.exists(OPS_PATH):
        raise ImportError(f"{OPS_PATH} is not built; run `python light-interaction-project_amd/build_lib.py` "
                          "(or __graft_entry__.build()) first")
    torch.ops.load_library(OPS_PATH)


_load()
ops = torch.ops.li


def _lse(like, want, B, NH, rows):
    return like.new_empty((B, NH, rows) if want else (0,), dtype=torch.float32)


def _nblk(geom):
    T, _, _, tt, _, _, nh, nw = geom
    return -(-T // tt) * nh * nw


def _exact(t, shape, name):
    """The checks of the operator library for tensors its kernels index at a per-head pitch implied by the
    geometry (contiguous padded text K/V, e4m3 tiles and scales): exactly ``shape``, so that a longer tensor
    cannot make heads after the first read another head's rows."""
    if t is not None and tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")


def _text(t, rows, like, name):
    if rows > 0:
        if t is None:
            raise RuntimeError(f"{name} is required with text blocks")
        B, NH, _, D = like.shape
        _exact(t, (B, NH, rows, D), name)


@torch.library.register_fake("li::pool")
def _pool_fake(src, mean, pool_off, geom):
    return None


@torch.library.register_fake("li::pool_pair")
def _pool_pair_fake(src0, mean0, pool_off0, geom0, src1, mean1, pool_off1, geom1, mean1_normalized=None):
    return None


@torch.library.register_fake("li::q_prep")
def _q_prep_fake(src, dst, mean, geom):
    return None


@torch.library.register_fake("li::kv_prep")
def _kv_prep_fake(k_src, v_src, k_dst, v_dst, k_mean, dst_off, pool_off, geom):
    return None


@torch.library.register_fake("li::untile")
def _untile_fake(src, dst, geom):
    return None


@torch.library.register_fake("li::block_mask")
def _block_mask_fake(q_pool, k_pool, metric, budget_mode, ratio, min_budget, n_recent, force_diag, force_sink,
                     force_neighbors, nh, nw, num_txt_blk, kmax, row_budget, return_scores, k_normalized=False):
    B, NH, nq, _ = q_pool.shape
    nk = k_pool.shape[2]
    indices = q_pool.new_empty((B, NH, nq, kmax), dtype=torch.int32)
    counts = q_pool.new_empty((B, NH, nq), dtype=torch.int32)
    scores = q_pool.new_empty((B, NH, nq, nk) if return_scores else (0,))
    return indices, counts, scores


@torch.library.register_fake("li::bsa_fwd")
def _bsa_fwd_fake(q, k, v, indices, counts, sm_scale, block_size, out, return_lse, split, balance):
    B, NH, Lq, _ = q.shape
    return _lse(q, return_lse, B, NH, Lq)


@torch.library.register_fake("li::bsa_fwd_gather")
def _bsa_fwd_gather_fake(q, k, v, k_txt, v_txt, num_txt_blk, q_geom, k_geom, indices, counts, sm_scale, out,
                         return_lse, split, balance, sorted=False):
    B, NH = q.shape[:2]
    bs = q_geom[3] * q_geom[4] * q_geom[5]
    _text(k_txt, num_txt_blk * bs, q, "k_txt")
    _text(v_txt, num_txt_blk * bs, q, "v_txt")
    return _lse(q, return_lse, B, NH, _nblk(q_geom) * bs)


@torch.library.register_fake("li::attn_dense")
def _attn_dense_fake(q, k, v, k_txt, v_txt, txt_len, sm_scale, out, return_lse, split):
    B, NH, Lq, _ = q.shape
    _text(k_txt, -(-txt_len // 128) * 128, q, "k_txt")
    _text(v_txt, -(-txt_len // 128) * 128, q, "v_txt")
    return _lse(q, return_lse, B, NH, -(-Lq // 128) * 128)


@torch.library.register_fake("li::tile_prep_fp8")
def _tile_prep_fp8_fake(src, dst, scales, mean, dst_off, pool_off, geom):
    return None


@torch.library.register_fake("li::kv_prep_fp8")
def _kv_prep_fp8_fake(k_src, v_src, k_dst, k_scales, v_dst, k_mean, dst_off, pool_off, geom):
    return None


@torch.library.register_fake("li::bsa_fwd_fp8")
def _bsa_fwd_fp8_fake(q8, q_scale, k8, k_scale, v, indices, counts, sm_scale, block_size, out, return_lse, split,
                      balance):
    B, NH, Lq, _ = q8.shape
    _exact(q_scale, (B, NH, -(-Lq // block_size)), "q_scale")
    _exact(k_scale, (B, NH, k8.shape[2] // block_size), "k_scale")
    return _lse(v, return_lse, B, NH, Lq)


@torch.library.register_fake("li::bsa_fwd_fp8_gather")
def _bsa_fwd_fp8_gather_fake(q8, q_scale, k8, k_scale, v, v_txt, num_txt_blk, q_geom, k_geom, indices, counts,
                             sm_scale, out, return_lse, balance, sorted=False):
    B, NH, _, D = v.shape
    nq, nkb = _nblk(q_geom), num_txt_blk + _nblk(k_geom)
    _exact(q8, (B, NH, nq * 128, D), "q8")
    _exact(k8, (B, NH, nkb * 128, D), "k8")
    _exact(q_scale, (B, NH, nq), "q_scale")
    _exact(k_scale, (B, NH, nkb), "k_scale")
    _text(v_txt, num_txt_blk * 128, v, "v_txt")
    return _lse(v, return_lse, B, NH, nq * 128)
