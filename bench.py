"""Benchmark: AR-aware 3D block-sparse attention forward on one MI355X.

A step is one ``run_sparse_attention`` call of the HY-WorldPlay decode entry
point on resident bf16 inputs: Q and K block pools, block mask, then one
block-sparse attention kernel that gathers Q/K/V tiles from token order and
writes the output in token order (shapes the fused kernel does not take run the
tiled sequence: tile gather + pool, mask, attention, untile).  Default workload
(``--workload hy``): B=1, 16 heads, D=128, 30x52 latent, Lq = 4 frames (6240
tokens), Lk = 12 frames (18720 tokens), 2x8x8 tiles, 30% keep ratio plus the
forced diagonal and sink blocks.

Prints one JSON line.  ``value`` is TFLOP/s over the retained blocks for the
whole call; the attention kernel's own rate, its share of the bf16 MFMA peak,
a dense GPU comparator (torch SDPA at the same shape) and a CPU baseline (the
reference's dense-masked torch semantics on the host, on a bounded sample of
heads) are reported beside it.
"""
import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "light-interaction-project_amd"))
sys.path.insert(0, REPO)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
# The e4m3 path does half of its FLOPs (Q K^T) at the fp8 peak and half (P V)
# at the bf16 peak: its MFMA-bound time is F/2/P8 + F/2/P16.
PEAK_MIXED_TFLOPS = 1.0 / (0.5 / PEAK_FP8_TFLOPS + 0.5 / PEAK_BF16_TFLOPS)
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="hy")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=16, help="heads timed for the CPU baseline sample")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--compare-dense", action="store_true",
                    help="also time this kernel with every block kept (same kernel symbol as the sparse "
                         "launches, so it is off by default to keep per-kernel profiles clean)")
    ap.add_argument("--profile", action="store_true",
                    help="launch each kernel of the call --steps times (and a 256 MiB copy for counter "
                         "calibration) for rocprofv3, then print per-launch algorithmic bytes/FLOPs")
    return ap.parse_args()


def event_loop(fn, iters, stream):
    """Times ``iters`` back-to-back calls of ``fn``.

    Returns (wall ms per call over the whole loop, bracketed by device
    synchronisation on both sides; per-call GPU ms from events recorded on
    ``stream``, the stream the library launches on).
    """
    import torch

    starts = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(iters):
        starts[i].record(stream)
        fn()
        ends[i].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / iters
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return wall, per


def wall_loop(fn, iters, stream=None):
    """Times ``iters`` back-to-back calls, bracketed by device synchronisation on both sides.

    Returns (wall ms per call; host ms per call to enqueue them, i.e. until the
    last call returned, before the closing synchronisation; GPU ms per call
    between one event recorded before the first call and one after the last on
    ``stream``, or None).  Host time well below the wall time means the loop is
    bound by the GPU, not by the host's submission.
    """
    import torch

    e0 = e1 = None
    if stream is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if e0 is not None:
        e0.record(stream)
    for _ in range(iters):
        fn()
    if e1 is not None:
        e1.record(stream)
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    gpu = e0.elapsed_time(e1) / iters if e0 is not None else None
    return (t2 - t0) * 1e3 / iters, (t1 - t0) * 1e3 / iters, gpu


def interleaved(fns, iters, stream):
    """Times the functions in ``fns`` alternately, ``iters`` rounds of one call each, with events on ``stream``.

    Returns the per-call GPU ms of each function.  Alternating puts every
    function in the same clock and power state, which back-to-back loops
    measured minutes apart do not (the MI355X clock dips for some tens of
    calls after a heavy load starts, then settles).
    """
    import torch

    per = [[] for _ in fns]
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in fns]
          for _ in range(iters)]
    torch.cuda.synchronize()
    for i in range(iters):
        for j, fn in enumerate(fns):
            ev[i][j][0].record(stream)
            fn()
            ev[i][j][1].record(stream)
    torch.cuda.synchronize()
    for i in range(iters):
        for j in range(len(fns)):
            per[j].append(ev[i][j][0].elapsed_time(ev[i][j][1]))
    return per


def mean(xs):
    return sum(xs) / len(xs)


TRAFFIC_SUMMARIES = {"hy": "bsa_fwd_hy_traffic.md", "hy_fp8": "bsa_fwd_e4m3_hy_traffic.md"}


def valid_rows(T, H, W, tile, nh, nw):
    """Valid (in-grid) token count of every block of a (T, H, W) grid in block order."""
    import numpy as np

    tt, th, tw = tile
    nt = -(-T // tt)
    ct, ch, cw = np.meshgrid(np.arange(nt), np.arange(nh), np.arange(nw), indexing="ij")
    n = (np.minimum(tt, T - ct * tt) * np.minimum(th, H - ch * th) * np.minimum(tw, W - cw * tw))
    return n.reshape(-1).astype(np.float64)


def valid_token_flops(ind, cnt, g, D, num_txt_blk=0):
    """4 * D * (valid query rows) * (valid key rows) summed over every kept (query tile, key block) pair."""
    import numpy as np

    vq = valid_rows(g.T_q, g.H, g.W, (g.tt, g.th, g.tw), g.nh, g.nw)
    vk = np.concatenate([np.full(num_txt_blk, float(g.bs)), valid_rows(g.T_k, g.H, g.W, (g.tt, g.th, g.tw), g.nh,
                                                                       g.nw)])
    kmax = ind.shape[-1]
    keep = np.arange(kmax)[None, None, None, :] < cnt[..., None]
    rows_k = np.where(keep, vk[np.clip(ind, 0, vk.size - 1)], 0.0).sum(axis=-1)   # (B, H, nq)
    return float((rows_k * vq[None, None, :]).sum()) * 4.0 * D


def load_traffic(kernel, workload):
    """HBM bytes per launch of ``kernel`` from the committed counter summary of ``workload``, or None.

    The summaries (profiles/bsa_fwd_*hy_traffic.md) hold rocprofv3 FETCH_SIZE and
    WRITE_SIZE per dispatch, each scaled by the factor the same counter reads
    for a copy kernel of known size in the same run.
    """
    if workload not in TRAFFIC_SUMMARIES:
        return None
    path = os.path.join(REPO, "profiles", TRAFFIC_SUMMARIES[workload])
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch") and kernel in line:
                    return float(line.split("=")[1].split()[0])
    except OSError:
        return None
    return None


def pct(xs, p):
    xs = sorted(xs)
    return xs[min(len(xs) - 1, max(0, int(round(p / 100.0 * (len(xs) - 1)))))]


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}): the sparse-attention path is "
              "single-GPU; head sharding over several GPUs is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from li_sparse import _core, _lib, _pipeline
    from li_sparse.hy.ar_sparse_operation import fast_generate_indices, run_sparse_attention
    from li_sparse.workloads import WORKLOADS, make_qkv

    wl = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    q, k, v = make_qkv(wl, seed=args.seed, layout="blhd")
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    empty = torch.empty((wl.batch, wl.heads, 0, wl.head_dim), dtype=torch.bfloat16, device=dev)
    g = _pipeline.geometry(wl.latent_hw, wl.tile, wl.lq, wl.lk, 0)
    params = wl.sparse_params(g.nq_blk)
    stream = torch.cuda.current_stream(dev)

    def step():
        return run_sparse_attention(qd, empty, empty, kd, vd, 1, wl.latent_hw, params)

    def warm(fn):
        # The same --warmup count of untimed calls before every timed loop.
        for _ in range(args.warmup):
            fn()

    # Work actually retained: counts from the emitted block lists.
    B, H, D, bs = wl.batch, wl.heads, wl.head_dim, g.bs
    q_t = torch.empty((B, H, g.nq_blk, bs, D), dtype=torch.bfloat16, device=dev)
    q_p = torch.empty((B, H, g.nq_blk, D), dtype=torch.bfloat16, device=dev)
    k_all = torch.empty((B, H, g.nk_blk, bs, D), dtype=torch.bfloat16, device=dev)
    v_all = torch.empty_like(k_all)
    k_p = torch.empty((B, H, g.nk_blk, D), dtype=torch.bfloat16, device=dev)
    _core.q_prep(qd, q_t, q_p, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    _core.kv_prep(kd, vd, k_all, v_all, k_p, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
    ind, cnt = fast_generate_indices(q_p, k_p, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
    # Rows whose selection cannot change with the score sum order (k-th and (k+1)-th non-forced scores two
    # ulps apart or more): the same selection again with its scores, and the forced set of the same rules.
    n_recent = _pipeline.recent_blocks(params, g.tt, g.nh, g.nw, g.nk_blk)
    ex = _pipeline.extras(params)
    _, _, sc = _core.block_mask(q_p, k_p, metric=params.get("sim_metric", "cosine"), budget_mode=_lib.LI_BUDGET_HISTORY,
                                ratio=params.get("topk_ratio", 1.0), nh=g.nh, nw=g.nw, n_recent=n_recent,
                                return_scores=True, **ex)
    forced = _core.forced_blocks(g.nq_blk, g.nk_blk, g.nh, g.nw, n_recent, ex["force_diag"], ex["force_sink"])
    torch.cuda.synchronize()
    counts = cnt.cpu().numpy()
    flops = float(counts.sum()) * 4.0 * bs * bs * D
    flops_valid = valid_token_flops(ind.cpu().numpy(), counts, g, D)
    qf, kf, vf = q_t.flatten(2, 3), k_all.flatten(2, 3), v_all.flatten(2, 3)
    scale = 1.0 / math.sqrt(D)
    fp8 = bool(params.get("qk_fp8", False))
    fused = _pipeline.uses_fused(qd, kd, vd, wl.tile, wl.latent_hw)
    o_tok = torch.empty_like(qd)
    # The attention launches as the call makes them (ragged rows: longest tiles first).
    balance = _pipeline.ragged(params)
    tiled_attn = lambda: _core.bsa_forward(qf, kf, vf, ind, cnt, scale, bs, balance=balance)  # noqa: E731
    fused_attn = lambda: _core.bsa_forward_gather(  # noqa: E731
        qd, kd, vd, None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt, scale, o_tok,
        balance=balance, sorted_lists=True)
    # The roofline kernel is the attention kernel the call launches.
    attn = fused_attn if fused else tiled_attn
    if fp8:
        q8 = torch.empty((B, H, g.nq_blk, bs, D), dtype=_core.FP8, device=dev)
        qs = torch.empty((B, H, g.nq_blk), dtype=torch.float32, device=dev)
        k8 = torch.empty((B, H, g.nk_blk, bs, D), dtype=_core.FP8, device=dev)
        ks = torch.empty((B, H, g.nk_blk), dtype=torch.float32, device=dev)
        _core.tile_prep_fp8(qd, q8, qs, None, 0, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
        _core.kv_prep_fp8(kd, vd, k8, ks, v_all, k_p, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
        q8f, k8f = q8.flatten(2, 3), k8.flatten(2, 3)
        tiled_fp8 = lambda: _core.bsa_forward_fp8(q8f, qs, k8f, ks, vf, ind, cnt, scale, bs,  # noqa: E731
                                                  balance=balance)
        fused_fp8 = lambda: _core.bsa_forward_fp8_gather(  # noqa: E731
            q8f, qs, k8f, ks, vd, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt, scale,
            o_tok, balance=balance, sorted_lists=True)
        attn = fused_fp8 if fused else tiled_fp8

    if args.profile:
        profile_kernels(args, wl, g, qd, kd, vd, q_t, q_p, k_all, v_all, k_p, params, ind, cnt, flops, dev,
                        fp8_tiles=(q8, qs, k8, ks) if fp8 else None)
        return

    # All host-side set-up is done above, so the GPU loops below run back to back
    # with no idle stretch between them.  The first loop after the set-up is
    # timed like the headline and reported as first_loop_after_idle: the GPU
    # clock dips for some tens of calls after a heavy load starts on an idle
    # GPU, then settles.
    warm(step)
    first_ms, _, first_gpu_ms = wall_loop(step, args.steps, stream)
    # Per-call GPU times from events around each call, in a loop of their own:
    # the event records add a few microseconds per call to the wall clock.
    warm(step)
    _, per_step = event_loop(step, args.steps, stream)

    # The same call with the key side of the fixed context frames (all K frames
    # before the query chunk) kept in a ContextCache: steps 2.. of a chunk's
    # denoising loop.  Reported beside the uncached step, which is the headline.
    cached = None
    ctx_frames = wl.frames_k - wl.frames_q
    if ctx_frames > 0:
        from li_sparse import ContextCache

        cache = ContextCache()
        cparams = dict(params, context_cache=cache, context_frames=ctx_frames)
        cstep = lambda: run_sparse_attention(qd, empty, empty, kd, vd, 1, wl.latent_hw, cparams)  # noqa: E731
        warm(cstep)
        c_ms, _, _ = wall_loop(cstep, args.steps)
        cached = {"ms_per_call": round(c_ms, 4), "context_frames": ctx_frames,
                  "note": "wall clock per call with the key side of the first context_frames K frames taken from "
                          "a warm ContextCache (the chunk frames are prepared every call)"}

    warm(attn)
    _, attn_per = event_loop(attn, args.steps, stream)
    # Average launch duration: one event before the first launch and one after
    # the last (events over the timed region, on the launch stream), so the
    # per-call event records of the loop above do not add to it; that loop
    # gives the per-call spread.
    _, _, attn_ms = wall_loop(attn, args.steps, stream)
    attn_tflops = flops / (attn_ms * 1e-3) / 1e12
    tiled_info = None
    if fused or fp8:
        warm(tiled_attn)
        _, tiled_per = event_loop(tiled_attn, max(5, args.steps // 5), stream)
        tiled_ms = mean(tiled_per)
        tiled_info = {"ms": round(tiled_ms, 4), "tflops": round(flops / (tiled_ms * 1e-3) / 1e12, 2),
                      "note": "the bf16 attention on bf16 tiles of the same inputs and lists" if fp8 else
                              "the same attention on pre-gathered tiles (the unfused sequence's kernel)"}
    tiled_fp8_info = None
    if fp8 and fused:
        warm(tiled_fp8)
        _, t8_per = event_loop(tiled_fp8, max(5, args.steps // 5), stream)
        t8_ms = mean(t8_per)
        tiled_fp8_info = {"ms": round(t8_ms, 4), "tflops": round(flops / (t8_ms * 1e-3) / 1e12, 2),
                          "note": "the e4m3 attention on V tiles (the tiled e4m3 sequence's kernel)"}

    # Dense comparators: torch SDPA (valid tokens) and this kernel with every block kept.
    sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)  # noqa: E731
    warm(sdpa)
    _, dense_per = event_loop(sdpa, max(5, args.steps // 5), stream)
    dense_ms = mean(dense_per)
    dense_flops = 4.0 * wl.lq * wl.lk * D * H * B
    # The same dense attention over the tiled, padded layout (every block of the padded grids).
    dense_flops_padded = 4.0 * g.nq_blk * bs * g.nk_blk * bs * D * H * B
    dense = {"gflop_valid_tokens": round(dense_flops / 1e9, 1), "gflop_padded_tiles": round(dense_flops_padded / 1e9, 1),
             "torch_sdpa_ms": round(dense_ms, 4),
             "torch_sdpa_tflops": round(dense_flops / (dense_ms * 1e-3) / 1e12, 2),
             "speedup_attention_vs_sdpa": round(dense_ms / attn_ms, 3)}
    if _core.dense_supported(qd, kd, vd):
        # This library's dense kernel (li_attn_fwd_dense) on the same valid tokens.
        own = lambda: _core.attn_dense(qd, kd, vd)  # noqa: E731
        warm(own)
        _, own_per = event_loop(own, max(5, args.steps // 5), stream)
        own_ms = mean(own_per)
        dense.update({"own_dense_kernel_ms": round(own_ms, 4),
                      "own_dense_kernel_tflops": round(dense_flops / (own_ms * 1e-3) / 1e12, 2),
                      "speedup_attention_vs_own_dense": round(own_ms / attn_ms, 3)})
        # The call, its attention kernel and the dense kernel alternated call by
        # call, so that all three see the same clock state.
        c_per, a_per, d_per = interleaved([step, attn, own], args.steps, stream)
        c_ms, a_ms, d_ms = mean(c_per), mean(a_per), mean(d_per)
        dense["interleaved"] = {
            "call_ms": round(c_ms, 4), "attention_ms": round(a_ms, 4), "own_dense_kernel_ms": round(d_ms, 4),
            "speedup_call_vs_own_dense": round(d_ms / c_ms, 3),
            "speedup_attention_vs_own_dense": round(d_ms / a_ms, 3),
            "note": "the call, its attention kernel and the dense kernel timed alternately, one call each per "
                    "round for --steps rounds (events on the launch stream), so the three ratios share one "
                    "clock state; speedup_call_vs_own_dense above divides the dense kernel's event time by the "
                    "headline loop's wall time"}
    if args.compare_dense:
        all_ind = torch.arange(g.nk_blk, dtype=torch.int32, device=dev).expand(B, H, g.nq_blk, g.nk_blk).contiguous()
        all_cnt = torch.full((B, H, g.nq_blk), g.nk_blk, dtype=torch.int32, device=dev)
        full = lambda: _core.bsa_forward(qf, kf, vf, all_ind, all_cnt, scale, bs)  # noqa: E731
        warm(full)
        _, full_per = event_loop(full, max(5, args.steps // 5), stream)
        full_ms = mean(full_per)
        full_flops = float(B * H * g.nq_blk * g.nk_blk) * 4.0 * bs * bs * D
        dense["own_kernel_all_blocks_ms"] = round(full_ms, 4)
        dense["own_kernel_all_blocks_tflops"] = round(full_flops / (full_ms * 1e-3) / 1e12, 2)
    # Timed region (the headline): --warmup untimed calls, then exactly --steps
    # calls bracketed by device synchronisation, with nothing else enqueued
    # between them (one event before and one after the loop give the GPU's own
    # time for it).  It runs last of the GPU loops, in the clock state of a GPU
    # that has been running this work, as in a rollout that calls it layer after
    # layer.
    warm(step)
    step_ms, submit_ms, step_gpu_ms = wall_loop(step, args.steps, stream)
    dense["speedup_call_vs_sdpa"] = round(dense_ms / step_ms, 3)
    if "own_dense_kernel_ms" in dense:
        dense["speedup_call_vs_own_dense"] = round(dense["own_dense_kernel_ms"] / step_ms, 3)

    if fp8:
        kname = "bsa_fwd_dma_kernel<bf16,128,gather,e4m3,zero-region>" if fused else "bsa_fwd_dma_kernel<bf16,128,e4m3>"
    elif fused:
        kname = "bsa_fwd_dma_kernel<bf16,128,gather,zero-region>"
    elif D == 128 and bs in (64, 128):
        kname = "bsa_fwd_dma_kernel<bf16,128>"
    else:
        kname = f"bsa_fwd_kernel<bf16,{bs},{D}>"

    # Bytes the call moves outside attention: the pools read Q and K once
    # (fused); the tiled sequence also writes and re-reads the tiles and untiles.
    if fused and not fp8:
        prep_bytes = 2.0 * (wl.lq + wl.lk) * H * D * B
    elif fp8 and fused:
        # Q, K read as bf16 and written as e4m3 tiles (V and O stay in token order).
        prep_bytes = (2.0 * (wl.lq + wl.lk) + 1.0 * (g.nq_blk + g.nk_blk) * bs) * H * D * B
    elif fp8:
        # Q, K read as bf16 and written as e4m3 tiles; V gathered; output untiled.
        prep_bytes = (2.0 * (wl.lq + 2 * wl.lk) + 1.0 * (g.nq_blk + g.nk_blk) * bs + 2.0 * g.nk_blk * bs
                      + 2.0 * (g.nq_blk * bs + wl.lq)) * H * D * B
    else:
        prep_bytes = 2.0 * (wl.lq + 2 * wl.lk) * H * D * B + 2.0 * (g.nq_blk + 2 * g.nk_blk) * bs * H * D * B

    peak = PEAK_MIXED_TFLOPS if fp8 else PEAK_BF16_TFLOPS
    # Host-side work after the timed loops, so that no loop starts on an idle (down-clocked) GPU.
    tie_free = _core.tie_free_fraction(sc, cnt, forced)
    result = {
        "metric": "sparse-attn fwd ms/call + TFLOPS (% MFMA peak) at HY shape, 30% keep",
        "value": round(flops / (step_ms * 1e-3) / 1e12, 2),
        "value_valid_tokens": round(flops_valid / (step_ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "timed_loop": {"host_submit_ms_per_step": round(submit_ms, 4), "gpu_ms_per_step": round(step_gpu_ms, 4),
                       "warmup_calls_before_every_timed_loop": args.warmup,
                       "note": "host_submit = host time to enqueue the K timed calls (until the last call "
                               "returned, before the closing synchronisation); gpu = one event before and one "
                               "after the K calls on the launch stream; the loop runs after the other GPU loops "
                               "of this run"},
        "first_loop_after_idle": {"ms_per_step": round(first_ms, 4), "gpu_ms_per_step": round(first_gpu_ms, 4),
                                  "tflops": round(flops / (first_ms * 1e-3) / 1e12, 2),
                                  "note": "the same --warmup calls and --steps timed calls, run first, right after "
                                          "the set-up left the GPU idle: the MI355X clock dips for some tens of "
                                          "calls after a heavy load starts on an idle GPU"},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 Q K^T (fp32 accumulate) + bf16 P V" if fp8 else "bf16",
        "data": "synthetic (seeded smooth (t,h,w) field + 0.5*N(0,1), bf16, Q pre-scaled by 1/sqrt(D))",
        "config": {"workload": wl.note, "batch": B, "heads": H, "head_dim": D, "lq": wl.lq, "lk": wl.lk,
                   "tile": list(wl.tile), "keep_ratio": wl.ratio, "block_size": bs, "nq_blocks": g.nq_blk,
                   "nk_blocks": g.nk_blk, "kept_blocks_per_row_mean": round(float(counts.mean()), 2),
                   "tie_free_rows": round(tie_free, 4), "parallelism": "single GPU"},
        "context_cached": cached,
        "ms_per_call_gpu": {"mean": round(mean(per_step), 4), "median": round(pct(per_step, 50), 4),
                            "p10": round(pct(per_step, 10), 4), "p90": round(pct(per_step, 90), 4),
                            "note": "events around each call on the launch stream; ms_per_step is wall clock"},
        "attention_kernel": {"kernel": kname, "ms": round(attn_ms, 4),
                             "ms_per_call_events": round(mean(attn_per), 4),
                             "median_ms": round(pct(attn_per, 50), 4),
                             "tflops": round(attn_tflops, 2),
                             "pct_bf16_peak": round(100.0 * attn_tflops / PEAK_BF16_TFLOPS, 2),
                             "retained_gflop": round(flops / 1e9, 2),
                             "retained_gflop_valid_tokens": round(flops_valid / 1e9, 2),
                             "tflops_valid_tokens": round(flops_valid / (attn_ms * 1e-3) / 1e12, 2),
                             "flop_bases": "retained_gflop (value, roofline) counts every row of each kept 128x128 "
                                           "tile pair, padding rows included (the kernel computes them); "
                                           "*_valid_tokens counts valid query rows x valid key rows only, the "
                                           "basis of the dense comparators' gflop_valid_tokens"},
        ("attention_kernel_bf16" if fp8 else "attention_kernel_tiled"): tiled_info,
        "attention_kernel_e4m3_tiled": tiled_fp8_info,
        "dense_comparator": dense,
        "roofline": {"bound": "mfma", "kernel": kname,
                     "achieved": round(attn_tflops, 2), "peak": round(peak, 1), "unit": "TFLOP/s",
                     "frac": round(attn_tflops / peak, 4),
                     "peak_note": ("half the FLOPs (Q K^T) at the 5.0 PFLOP/s fp8 peak, half (P V) at the "
                                   "2.5 PFLOP/s bf16 peak") if fp8 else "dense bf16 MFMA peak",
                     "traffic": load_traffic(kname, args.workload),
                     "traffic_unit": "bytes per launch (HBM/MALL side, rocprofv3 FETCH_SIZE + WRITE_SIZE)",
                     "traffic_source": (f"read from profiles/{TRAFFIC_SUMMARIES[args.workload]} (committed "
                                        "rocprofv3 --pmc summary of `bench.py --profile`), not measured in this "
                                        "run") if args.workload in TRAFFIC_SUMMARIES else None},
        "fused_path": fused,
        "prep_bytes_per_call": prep_bytes,
    }

    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(wl, q, k, v, counts, ind.cpu().numpy(), g, args.cpu_heads, flops)
    print(json.dumps(result), flush=True)


def profile_kernels(args, wl, g, qd, kd, vd, q_t, q_p, k_all, v_all, k_p, params, ind, cnt, flops, dev,
                    fp8_tiles=None):
    """Each kernel of one call, --steps launches apiece, for rocprofv3 kernel traces and counters."""
    import torch

    from li_sparse import _core, _pipeline
    from li_sparse.hy.ar_sparse_operation import fast_generate_indices

    B, H, D, bs = wl.batch, wl.heads, wl.head_dim, g.bs
    qf, kf, vf = q_t.flatten(2, 3), k_all.flatten(2, 3), v_all.flatten(2, 3)
    scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(qf)
    o_lin = torch.empty_like(qd)
    o_tok = torch.empty_like(qd)
    src = torch.empty(1 << 27, dtype=torch.bfloat16, device=dev).fill_(1.0)   # 256 MiB
    dst = torch.empty_like(src)
    fp8 = fp8_tiles is not None
    fused = _pipeline.uses_fused(qd, kd, vd, wl.tile, wl.latent_hw)
    balance = _pipeline.ragged(params)
    q_pool = torch.empty_like(q_p)
    k_pool = torch.empty_like(k_p)
    for _ in range(args.steps):
        if fp8:
            # The fused e4m3 call's kernels: quantizing Q gather + pool,
            # quantizing K gather + pool, block mask, e4m3 attention reading V
            # and writing O in token order (+ merge); then, on the same lists,
            # the tiled e4m3 attention (V tiles from a K/V gather) and the bf16
            # tiled attention.
            q8, qs, k8, ks = fp8_tiles
            _core.tile_prep_fp8(qd, q8, qs, q_pool, 0, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            _core.tile_prep_fp8(kd, k8, ks, k_pool, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            fast_generate_indices(q_pool, k_pool, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
            _core.bsa_forward_fp8_gather(q8.flatten(2, 3), qs, k8.flatten(2, 3), ks, vd, None, 0, g.T_q, g.T_k, g.H,
                                         g.W, g.tt, g.th, g.tw, g.nh, g.nw, ind, cnt, scale, o_tok, balance=balance,
                                         sorted_lists=True)
            _core.kv_prep_fp8(kd, vd, k8, ks, v_all, k_pool, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            _core.bsa_forward_fp8(q8.flatten(2, 3), qs, k8.flatten(2, 3), ks, vf, ind, cnt, scale, bs, out=out,
                                  balance=balance)
            _core.bsa_forward(qf, kf, vf, ind, cnt, scale, bs, out=out, balance=balance)
        elif fused:
            # The call's own kernels: Q pool, K pool, block mask, fused
            # attention (+ its tail merge); then the tiled attention kernel on
            # the same lists, for comparison.
            _core.pool(qd, q_pool, 0, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            _core.pool(kd, k_pool, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            fast_generate_indices(q_pool, k_pool, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
            _core.bsa_forward_gather(qd, kd, vd, None, None, 0, g.T_q, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh,
                                     g.nw, ind, cnt, scale, o_tok, balance=balance, sorted_lists=True)
            _core.bsa_forward(qf, kf, vf, ind, cnt, scale, bs, out=out, balance=balance)
        else:
            _core.q_prep(qd, q_t, q_p, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            _core.kv_prep(kd, vd, k_all, v_all, k_p, 0, 0, g.T_k, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
            fast_generate_indices(q_p, k_p, 0, (g.nt_q, g.nh, g.nw), (g.nt_k, g.nh, g.nw), params, dev)
            _core.bsa_forward(qf, kf, vf, ind, cnt, scale, bs, out=out, balance=balance)
            _core.untile(out.view(B, H, g.nq_blk, bs, D), o_lin, g.T_q, g.H, g.W, g.tt, g.th, g.tw, g.nh, g.nw)
        dst.copy_(src)
    torch.cuda.synchronize()
    e = 2  # bytes per element
    alg = {
        "bsa_fwd_kernel": {"flop": flops,
                           "bytes_min": e * (wl.lq + 2 * wl.lk) * H * D * B,
                           "note": "FLOPs = sum(counts) * 4 * BS^2 * D; bytes_min = Q + K + V read once and O "
                                   "written once for the fused kernel (Q + K + V tiles read once for the tiled one)"},
        "copy (calibration)": {"bytes_read": src.numel() * e, "bytes_written": dst.numel() * e},
    }
    if fp8:
        alg["bsa_fwd_kernel"]["bytes_min_e4m3"] = (1 * (g.nq_blk + g.nk_blk) + 2 * g.nk_blk + 2 * g.nq_blk) * bs * H * D * B
        alg["bsa_fwd_kernel"]["bytes_min_e4m3_fused"] = ((g.nq_blk + g.nk_blk) * bs + 2 * (wl.lk + wl.lq)) * H * D * B
        alg["gather_fp8_kernel<1> (Q)"] = {"bytes": H * D * B * (e * wl.lq + g.nq_blk * bs) + e * H * D * g.nq_blk}
        alg["gather_fp8_kernel<1> (K)"] = {"bytes": H * D * B * (e * wl.lk + g.nk_blk * bs) + e * H * D * g.nk_blk}
        alg["gather_fp8_kernel<2> (K e4m3, V)"] = {"bytes": H * D * B * (2 * e * wl.lk + (1 + e) * g.nk_blk * bs)
                                                   + e * H * D * g.nk_blk}
    elif fused:
        alg["bsa_fwd_kernel"]["bytes_min_fused"] = e * (2 * wl.lq + 2 * wl.lk) * H * D * B
        alg["pool (Q)"] = {"bytes": e * H * D * B * wl.lq + e * H * D * g.nq_blk, "grid_blocks": g.nq_blk}
        alg["pool (K)"] = {"bytes": e * H * D * B * wl.lk + e * H * D * g.nk_blk, "grid_blocks": g.nk_blk}
    else:
        alg["gather_pool_kernel<1> (Q)"] = {"bytes": e * H * D * B * (wl.lq + g.nq_blk * bs) + e * H * D * g.nq_blk}
        alg["gather_pool_kernel<2> (K,V)"] = {"bytes": e * H * D * B * 2 * (wl.lk + g.nk_blk * bs)
                                              + e * H * D * g.nk_blk}
        alg["untile_kernel"] = {"bytes": e * H * D * B * 2 * wl.lq}
    print(json.dumps({"profile": wl.name, "fused": fused, "e4m3": fp8, "launches_per_kernel": args.steps,
                      "algorithmic_per_launch": alg}), flush=True)


def cpu_baseline(wl, q, k, v, counts, ind, g, n_heads, flops, min_seconds=10.0):
    """The reference's dense-masked torch semantics on the host CPU, on a bounded sample of heads."""
    import numpy as np
    import torch

    from li_sparse.workloads import WORKLOADS  # noqa: F401
    from oracle import attention as oatt
    from oracle import tile as otile

    cores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(cores)
    H, W = wl.latent_hw
    n_heads = max(1, min(n_heads, wl.heads))
    heads = [(0, h) for h in range(n_heads)]

    def tiles(x, frames):
        b = x.contiguous().view(torch.int16).numpy().view(np.uint16)[:, :n_heads]
        t = otile.tile_gather(b, frames, H, W, wl.tile)
        return torch.from_numpy(t.reshape(t.shape[0], t.shape[1], -1, t.shape[-1]).view(np.int16)).view(torch.bfloat16)

    qt, kt, vt = tiles(q, wl.frames_q), tiles(k, wl.frames_k), tiles(v, wl.frames_k)
    # Repeat the head sample until about 10 s of CPU work (at most 5 passes).
    reps, sec = 0, 0.0
    while reps < 5 and (reps == 0 or sec < min_seconds):
        t0 = time.perf_counter()
        oatt.dense_masked_cpu(qt, kt, vt, ind[:, :n_heads], counts[:, :n_heads], 1.0 / math.sqrt(wl.head_dim),
                              g.bs, head_list=heads)
        sec += time.perf_counter() - t0
        reps += 1
    per_pass = sec / reps
    sample_flops = float(counts[:, :n_heads].sum()) * 4.0 * g.bs * g.bs * wl.head_dim
    ms_full = per_pass * 1e3 * wl.heads / n_heads
    return {"value": round(sample_flops / per_pass / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "ms_per_call_scaled": round(ms_full, 1),
            "sample": f"{n_heads} of {wl.heads} heads of the same call, {reps} passes, {sec:.1f} s in total "
                      f"(torch CPU SDPA, fp32 from bf16, boolean mask expanded from the kept blocks over the "
                      f"tiled/padded layout); ms_per_call_scaled = time per pass x {wl.heads}/{n_heads}"}


if __name__ == "__main__":
    main()
