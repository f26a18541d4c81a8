"""HY-WorldPlay autoregressive-decode sparse attention (drop-in).

Mirrors hy-worldplay/files/hyvideo/models/transformers/modules/ar_sparse_operation.py:
``launch_q_prep`` / ``launch_kv_prep`` / ``launch_untile`` (:166-218),
``fast_generate_indices`` (:223-284) and ``run_sparse_attention`` (:289-362),
with every kernel a gfx950 HIP kernel of this package.

``sparse_params`` keys: ``tile_size`` (default (4, 8, 4)), ``topk_ratio``,
``recent_protect``, ``sim_metric`` as in the reference; optional extensions
``force_diag`` / ``force_sink`` (keep the query's own key block and the
t-slab-0 block at its (h, w)), ``row_budget`` (explicit per-row totals) and
``qk_fp8`` (Q K^T on e4m3 codes with one fp32 scale per tile block; the
selection is unchanged).  Unset, they leave the reference's behaviour
unchanged.
"""
from .. import _core, _lib, _pipeline


def launch_q_prep(src, dst, mean, T, H, W, tt, th, tw, nh, nw):
    _core.q_prep(src, dst, mean, T, H, W, tt, th, tw, nh, nw)


def launch_kv_prep(k_src, v_src, k_dst, v_dst, k_mean, dst_off, pool_off, T, H, W, tt, th, tw, nh, nw):
    _core.kv_prep(k_src, v_src, k_dst, v_dst, k_mean, dst_off, pool_off, T, H, W, tt, th, tw, nh, nw)


def launch_untile(src, dst, T, H, W, tt, th, tw, nh, nw):
    _core.untile(src, dst, T, H, W, tt, th, tw, nh, nw)


def fast_generate_indices(q_pool, k_pool, text_len, grid_thw_q, grid_thw_k, params, device, *,
                          k_pool_normalized=None):
    """Block-sparse indices for the AR decode path (ar_sparse_operation.py:223-284).

    Returns ``(final_indices (B, H, Nq_blk, K) int32, final_counts (B, H, Nq_blk) int32)``:
    text blocks first, then the selected visual blocks ascending.  ``k_pool_normalized`` (extension,
    keyword only): the key pool's rows normalised for the cosine metric, see ``_core.block_mask``.
    """
    tt, th, tw = params["tile_size"]
    bs = tt * th * tw
    nq, nk = q_pool.shape[2], k_pool.shape[2]
    nh, nw = grid_thw_q[1], grid_thw_q[2]
    n_prot = _pipeline.recent_blocks(params, tt, nh, nw, nk)
    num_txt_blk = (text_len + bs - 1) // bs
    return _core.block_mask(q_pool, k_pool, metric=params.get("sim_metric", "cosine"),
                            budget_mode=_lib.LI_BUDGET_HISTORY, ratio=params.get("topk_ratio", 1.0), nh=nh, nw=nw,
                            num_txt_blk=num_txt_blk, n_recent=n_prot, k_pool_normalized=k_pool_normalized,
                            **_pipeline.extras(params))


def run_sparse_attention(q, k_txt, v_txt, k_vis, v_vis, block_idx, latent_hw, sparse_params):
    """One autoregressive sparse-attention forward (ar_sparse_operation.py:289-362).

    Args:
        q: ``(B, H, Nq, D)`` (any strides); k_txt, v_txt: ``(B, H, N_txt, D)``;
        k_vis, v_vis: ``(B, H, N_vis, D)``; block_idx: layer index (informational);
        latent_hw: ``(H_lat, W_lat)``; sparse_params: see the module docstring.

    Returns:
        ``(B, H, Nq, D)``.  Shapes that cannot be tiled (``Nq % (H_lat*W_lat) != 0``)
        take the reference's dense SDPA path.
    """
    LATENT_H, LATENT_W = latent_hw
    if q.shape[2] % (LATENT_H * LATENT_W) != 0:
        return _pipeline.dense_attention(q, k_txt, v_txt, k_vis, v_vis)
    tile = tuple(sparse_params.get("tile_size", (4, 8, 4)))

    def select(q_pool, k_pool, text_len, grid_q, grid_k, k_pool_normalized=None):
        return fast_generate_indices(q_pool, k_pool, text_len, grid_q, grid_k, dict(sparse_params, tile_size=tile),
                                     q.device, k_pool_normalized=k_pool_normalized)

    # The block mask lists every row's text blocks first (ascending ids).
    return _pipeline.sparse_attention(q, k_txt, v_txt, k_vis, v_vis, latent_hw, tile, select, sorted_lists=True,
                                      balance=_pipeline.ragged(sparse_params),
                                      qk_fp8=_pipeline.qk_fp8(sparse_params),
                                      context=_pipeline.context_of(sparse_params, block_idx),
                                      normalize_k_pool=_pipeline.cosine(sparse_params))
