"""HY-WorldPlay KV-recompute (prefill) sparse attention (drop-in).

Mirrors hy-worldplay/files/hyvideo/models/transformers/modules/bi_sparse_operation_for_KV_cache.py:
``generate_prefill_indices`` (:220-296) and ``run_sparse_prefill_attention``
(:301-395): dense SDPA for the first three chunks or untileable shapes
(:329-343), otherwise the sparse pipeline with the 3D-neighbour forced set
and the ``min(max(int(Nk*ratio), 7), Nk)`` budget.  The extension keys of
ar_sparse_operation (``force_diag``, ``force_sink``, ``row_budget``,
``qk_fp8``) apply here too.
"""
from .. import _core, _lib, _pipeline
from .ar_sparse_operation import launch_kv_prep, launch_q_prep, launch_untile  # noqa: F401
from .infer_state import get_infer_state


def _pool(x):
    return x.mean(dim=-2) if x.dim() == 5 else x


def generate_prefill_indices(q_in, k_in, text_len, grid_thw, params, device, default_ratio=None, *,
                             k_pool_normalized=None):
    """Block-sparse indices for the bidirectional prefill phase.

    ``q_in`` / ``k_in`` are pooled ``(B, H, N, D)`` or tiled ``(B, H, N, Bs, D)``
    (mean-pooled here, bi_sparse_operation_for_KV_cache.py:239-250).  Key blocks
    at 3D Manhattan distance <= 1 from the query's block are always kept.
    ``params['topk_ratio']`` is required (``default_ratio`` is the MG entry's 0.25).  ``k_pool_normalized``
    (extension, keyword only, pooled ``k_in`` only): the key pool's rows normalised for the cosine metric,
    see ``_core.block_mask``.
    """
    if q_in.dim() == 5:
        bs = q_in.shape[-2]
    else:
        tt, th, tw = params["tile_size"]
        bs = tt * th * tw
    q_pool, k_pool = _pool(q_in), _pool(k_in)
    _, nh, nw = grid_thw
    ratio = params["topk_ratio"] if default_ratio is None else params.get("topk_ratio", default_ratio)
    num_txt_blk = (text_len + bs - 1) // bs
    return _core.block_mask(q_pool, k_pool, metric=params.get("sim_metric", "cosine"),
                            budget_mode=_lib.LI_BUDGET_TOTAL, ratio=ratio, nh=nh, nw=nw, num_txt_blk=num_txt_blk,
                            force_neighbors=True, min_budget=7,
                            k_pool_normalized=k_pool_normalized if k_in.dim() == 4 else None,
                            **_pipeline.extras(params))


def run_sparse_prefill_attention(q, k_txt, v_txt, k_vis, v_vis, block_idx, latent_hw, sparse_params):
    """One bidirectional (prefill) sparse-attention forward; same signature as the decode entry."""
    current_global_chunk = getattr(get_infer_state(), "current_chunk_index", 0)
    LATENT_H, LATENT_W = latent_hw
    if current_global_chunk < 3 or q.shape[2] % (LATENT_H * LATENT_W) != 0:
        return _pipeline.dense_attention(q, k_txt, v_txt, k_vis, v_vis)
    tile = tuple(sparse_params.get("tile_size", (4, 8, 4)))

    def select(q_pool, k_pool, text_len, grid_q, grid_k, k_pool_normalized=None):
        return generate_prefill_indices(q_pool, k_pool, text_len, grid_k, dict(sparse_params, tile_size=tile),
                                        q.device, k_pool_normalized=k_pool_normalized)

    # The block mask lists every row's text blocks first (ascending ids).
    return _pipeline.sparse_attention(q, k_txt, v_txt, k_vis, v_vis, latent_hw, tile, select, sorted_lists=True,
                                      balance=_pipeline.ragged(sparse_params),
                                      qk_fp8=_pipeline.qk_fp8(sparse_params),
                                      context=_pipeline.context_of(sparse_params, block_idx),
                                      normalize_k_pool=_pipeline.cosine(sparse_params))
