"""Matrix-Game-3.0 sparse self-attention (drop-in).

Mirrors matrix-game-3.0/files/wan/modules/bi_sparse_operation.py:
``launch_q_prep`` / ``launch_kv_prep`` / ``launch_untile`` (:142-177),
``generate_prefill_indices`` (:179-234, default ratio 0.25) and
``run_sparse_attention(q, k, v, text_len, ...)`` (:236-348) on a combined
text+visual K/V, tile default (4, 4, 8), with the optional per-stage event
timing of the reference (``ENABLE_SPARSE_PROFILING``, :13, 237-346).  The
extension keys of the HY module (``force_diag``, ``force_sink``,
``row_budget``, ``qk_fp8``) apply here too.
"""
import torch

from .. import _pipeline
from ..hy.ar_sparse_operation import launch_kv_prep, launch_q_prep, launch_untile  # noqa: F401
from ..hy.bi_sparse_operation_for_KV_cache import generate_prefill_indices as _prefill_indices

ENABLE_SPARSE_PROFILING = False


def generate_prefill_indices(q_in, k_in, text_len, grid_thw, params, device, *, k_pool_normalized=None):
    return _prefill_indices(q_in, k_in, text_len, grid_thw, params, device, default_ratio=0.25,
                            k_pool_normalized=k_pool_normalized)


def run_sparse_attention(q, k, v, text_len, block_idx, latent_hw, sparse_params):
    """Sparse self-attention over ``k``/``v`` = text tokens (first ``text_len``) + visual tokens."""
    import torch

    LATENT_H, LATENT_W = latent_hw
    if q.shape[2] % (LATENT_H * LATENT_W) != 0:
        return _pipeline.dense_attention(q, None, None, k, v)
    tile = tuple(sparse_params.get("tile_size", (4, 4, 8)))
    events = {} if ENABLE_SPARSE_PROFILING else None
    if events is not None:
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        events["start"] = e
    k_txt = k[:, :, :text_len] if text_len > 0 else None
    v_txt = v[:, :, :text_len] if text_len > 0 else None

    def select(q_pool, k_pool, tl, grid_q, grid_k, k_pool_normalized=None):
        return generate_prefill_indices(q_pool, k_pool, tl, grid_k, dict(sparse_params, tile_size=tile), q.device,
                                        k_pool_normalized=k_pool_normalized)

    # The block mask lists every row's text blocks first (ascending ids).
    o = _pipeline.sparse_attention(q, k_txt, v_txt, k[:, :, text_len:], v[:, :, text_len:], latent_hw, tile,
                                   select, events, sorted_lists=True, balance=_pipeline.ragged(sparse_params),
                                   qk_fp8=_pipeline.qk_fp8(sparse_params),
                                   context=_pipeline.context_of(sparse_params, block_idx),
                                   normalize_k_pool=_pipeline.cosine(sparse_params))
    if events is not None:
        torch.cuda.synchronize()
        t = lambda a, b: events[a].elapsed_time(events[b])  # noqa: E731
        print(f"[Block {block_idx:2d}] Sparse Workflow: Total {t('start', 'untile_end'):>5.2f}ms | "
              f"Alloc {t('alloc_start', 'alloc_end'):>4.2f}ms | Tiling {t('prep_start', 'prep_end'):>4.2f}ms | "
              f"Index {t('index_start', 'index_end'):>4.2f}ms | SparseAttn {t('attn_start', 'attn_end'):>4.2f}ms | "
              f"Untile {t('untile_start', 'untile_end'):>4.2f}ms")
    return o
