"""GPU: the context cache reuses the key-side preparation of fixed context frames without changing any bit."""
import pytest
import torch

from li_sparse import ContextCache, _pipeline
from li_sparse.hy.ar_sparse_operation import fast_generate_indices, run_sparse_attention
from li_sparse.workloads import Workload, make_qkv

pytestmark = pytest.mark.gpu


def _wl():
    # 8 context frames + a 4-frame chunk, HY latent grid, 2 heads
    return Workload("ctx", 2, 128, (30, 52), 4, 12, (2, 8, 8), 0.3, "scaled_dot_product")


def _inputs(dev, seed, text):
    wl = _wl()
    q, k, v = make_qkv(wl, seed=seed, layout="blhd")
    g = torch.Generator().manual_seed(seed + 100)
    kt = torch.randn(1, 2, text, 128, generator=g).to(torch.bfloat16).to(dev) if text else None
    vt = torch.randn(1, 2, text, 128, generator=g).to(torch.bfloat16).to(dev) if text else None
    return q.to(dev), k.to(dev), v.to(dev), kt, vt


def _new_chunk(q, k, v, seed):
    """The same context frames, new chunk frames (the last 4 frames of K/V) and a new query."""
    wl = _wl()
    q2, k2, v2 = make_qkv(wl, seed=seed, layout="blhd")
    n_ctx = 8 * 30 * 52
    k = k.clone()
    v = v.clone()
    k[:, :, n_ctx:] = k2[:, :, n_ctx:].to(k.device)
    v[:, :, n_ctx:] = v2[:, :, n_ctx:].to(v.device)
    return q2.to(q.device), k, v


@pytest.mark.parametrize("fused,fp8", [(True, False), (True, True), (False, False), (False, True)])
@pytest.mark.parametrize("text", [0, 200])
def test_cached_calls_give_the_uncached_bits(dev, fused, fp8, text):
    print(f"[gpu] context cache fused={fused} fp8={fp8} text={text}", flush=True)
    wl = _wl()
    params = dict(wl.sparse_params(), tile_size=wl.tile)

    def select(q_pool, k_pool, tl, grid_q, grid_k):
        return fast_generate_indices(q_pool, k_pool, tl, grid_q, grid_k, params, dev)

    def call(q, k, v, kt, vt, context):
        return _pipeline.sparse_attention(q, kt, vt, k, v, wl.latent_hw, wl.tile, select, fused=fused, qk_fp8=fp8,
                                          context=context)

    q, k, v, kt, vt = _inputs(dev, 1, text)
    cache = ContextCache()
    ref1 = call(q, k, v, kt, vt, None)
    out1 = call(q, k, v, kt, vt, (cache, 5, 8))          # fills the cache
    q2, k2, v2 = _new_chunk(q, k, v, 2)
    ref2 = call(q2, k2, v2, kt, vt, None)
    out2 = call(q2, k2, v2, kt, vt, (cache, 5, 8))        # context blocks from the cache
    out3 = call(q2, k2, v2, kt, vt, (cache, 5, 8))
    torch.cuda.synchronize()
    assert len(cache) == 1
    assert torch.equal(out1.view(torch.int16), ref1.view(torch.int16))
    assert torch.equal(out2.view(torch.int16), ref2.view(torch.int16))
    assert torch.equal(out3.view(torch.int16), ref2.view(torch.int16))
    assert not torch.equal(ref1, ref2)
    cache.reset()
    assert len(cache) == 0


@pytest.mark.parametrize("text", [0, 200])
def test_cached_cosine_calls_with_the_normalised_key_pool(dev, text):
    """Cosine selection: the key pool's normalised copy is cached with the pool and kept in step with it."""
    print(f"[gpu] context cache, cosine selection through the normalised key pool, text={text}", flush=True)
    wl = _wl()
    params = dict(wl.sparse_params(), tile_size=wl.tile, sim_metric="cosine")

    def select(q_pool, k_pool, tl, grid_q, grid_k, k_pool_normalized=None):
        return fast_generate_indices(q_pool, k_pool, tl, grid_q, grid_k, params, dev,
                                     k_pool_normalized=k_pool_normalized)

    def call(q, k, v, kt, vt, context, norm):
        return _pipeline.sparse_attention(q, kt, vt, k, v, wl.latent_hw, wl.tile, select, context=context,
                                          normalize_k_pool=norm)

    q, k, v, kt, vt = _inputs(dev, 3, text)
    cache = ContextCache()
    ref1 = call(q, k, v, kt, vt, None, False)             # the mask normalises the raw pool itself
    out1 = call(q, k, v, kt, vt, (cache, 2, 8), True)     # fills the cache (pool + normalised copy)
    q2, k2, v2 = _new_chunk(q, k, v, 4)
    ref2 = call(q2, k2, v2, kt, vt, None, False)
    out2 = call(q2, k2, v2, kt, vt, (cache, 2, 8), True)  # context rows of both from the cache
    raw2 = call(q2, k2, v2, kt, vt, (cache, 2, 8), False)  # a raw-pool entry of its own
    torch.cuda.synchronize()
    assert len(cache) == 2
    for out, ref in ((out1, ref1), (out2, ref2), (raw2, ref2)):
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert not torch.equal(ref1, ref2)


def test_entry_point_keys_and_layers(dev):
    """Through run_sparse_attention: one entry per layer (block_idx); an odd context is rounded down to whole slabs."""
    print("[gpu] context cache through run_sparse_attention", flush=True)
    wl = _wl()
    q, k, v, kt, vt = _inputs(dev, 3, 77)
    cache = ContextCache()
    base = dict(wl.sparse_params(), tile_size=wl.tile)
    ref = run_sparse_attention(q, kt, vt, k, v, 0, wl.latent_hw, base)
    params = dict(base, context_cache=cache, context_frames=7)   # 7 frames -> 3 whole 2-frame slabs
    outs = [run_sparse_attention(q, kt, vt, k, v, layer, wl.latent_hw, params) for layer in (0, 1, 0, 1)]
    q2, k2, v2 = _new_chunk(q, k, v, 4)
    ref2 = run_sparse_attention(q2, kt, vt, k2, v2, 0, wl.latent_hw, base)
    out2 = run_sparse_attention(q2, kt, vt, k2, v2, 1, wl.latent_hw, params)
    torch.cuda.synchronize()
    assert len(cache) == 2
    for o in outs:
        assert torch.equal(o.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(out2.view(torch.int16), ref2.view(torch.int16))
    with pytest.raises(TypeError):
        run_sparse_attention(q, kt, vt, k, v, 0, wl.latent_hw, dict(base, context_cache={}))
