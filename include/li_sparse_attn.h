/*
 * li_sparse_attn.h -- C ABI of the MI355X (gfx950) AR-aware 3D block-sparse
 * attention forward.
 *
 * Plain C: pointers, sizes and strides only.  Every buffer is allocated by the
 * caller (device memory); no entry point allocates device memory, keeps a
 * pointer after it returns, or synchronises the stream.  Strides are in
 * elements.  Each entry point validates its arguments on the host and returns
 * LI_OK or a negative status without touching the GPU when they are invalid;
 * kernels are enqueued on `stream` (a hipStream_t, NULL = default stream).
 *
 * Element types: LI_DTYPE_BF16 (default) or LI_DTYPE_F16 for Q/K/V, tiles,
 * pools and outputs.  Index lists are int32.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   HYAR = hy-worldplay/files/hyvideo/models/transformers/modules/ar_sparse_operation.py
 *   HYKV = hy-worldplay/files/hyvideo/models/transformers/modules/bi_sparse_operation_for_KV_cache.py
 *   HYK  = hy-worldplay/files/hyvideo/models/transformers/modules/longcat_kernel.py
 *   MGS  = matrix-game-3.0/files/wan/modules/bi_sparse_operation.py
 */
#ifndef LI_SPARSE_ATTN_H
#define LI_SPARSE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum li_status {
  LI_OK = 0,
  LI_ERR_INVALID_ARG = -1,   /* null pointer, negative or zero size */
  LI_ERR_SHAPE = -2,         /* inconsistent shapes / geometry */
  LI_ERR_K_LEN = -3,         /* K length not a multiple of the logical block size (HYK:192-193) */
  LI_ERR_INDEX_RANGE = -4,   /* block index out of range (HYK:194-195) */
  LI_ERR_UNSUPPORTED = -5,   /* head_dim / block size / dtype not built */
  LI_ERR_LAUNCH = -6,        /* HIP launch error */
  LI_ERR_TOO_LARGE = -7      /* above a built-in limit: mask builder key blocks, noalloc scratch */
};

enum li_dtype { LI_DTYPE_BF16 = 0, LI_DTYPE_F16 = 1 };

/* Latent grid and tile: frames T, height H, width W; tile (tt, th, tw);
 * nh = ceil(H/th), nw = ceil(W/tw) tiles per t-slab (HYAR:322). */
typedef struct li_tile_geom {
  int32_t T, H, W;
  int32_t tt, th, tw;
  int32_t nh, nw;
} li_tile_geom;

/* ABI version (bumped on any signature change). */
int li_abi_version(void);
/* Static text for a status code. */
const char* li_status_string(int status);
/* HIP error name and text of the calling thread's last failed launch (LI_ERR_LAUNCH). */
const char* li_last_error(void);

/*
 * Q tile gather + mean pool.  Replaces launch_q_prep(src, dst, mean, T, H, W,
 * tt, th, tw, nh, nw) and _fused_q_prep_kernel (HYAR:26-70, 166-181; HYKV:27-73,
 * 168-181; MGS:25-64, 142-152).
 *   src  (B, NH, L, D), any strides, L >= T*H*W
 *   dst  (B, NH, nblk, BS, D) tiles, any strides (nblk = ceil(T/tt)*nh*nw, BS = tt*th*tw)
 *   mean (B, NH, nblk, D) pooled means: bf16/f16( fp32 sum over BS rows / BS ), padding included
 * Rows outside the (T, H, W) grid are written as zeros.
 */
int li_q_prep(int dtype, int32_t B, int32_t NH, int32_t D,
              const void* src, const int64_t src_strides[4],
              void* dst, const int64_t dst_strides[5],
              void* mean, const int64_t mean_strides[4],
              const li_tile_geom* geom, void* stream);

/*
 * K/V tile gather + K mean pool.  Replaces launch_kv_prep(k_src, v_src, k_dst,
 * v_dst, k_mean, dst_off, pool_off, T, H, W, tt, th, tw, nh, nw) and
 * _fused_kv_prep_kernel (HYAR:75-122, 183-202; HYKV:78-126; MGS:66-107, 154-166).
 * Tiles are written at block (blk + dst_off), pools at (blk + pool_off).
 */
int li_kv_prep(int dtype, int32_t B, int32_t NH, int32_t D,
               const void* k_src, const int64_t k_src_strides[4],
               const void* v_src, const int64_t v_src_strides[4],
               void* k_dst, const int64_t k_dst_strides[5],
               void* v_dst, const int64_t v_dst_strides[5],
               void* k_mean, const int64_t mean_strides[4],
               int64_t dst_off, int64_t pool_off,
               const li_tile_geom* geom, void* stream);

/*
 * Tile mean pool without writing tiles: the pooling half of launch_q_prep /
 * launch_kv_prep (HYAR:58-70, 110-122) for the fused attention path, whose
 * kernel reads tokens in tile order straight from the untiled tensors.
 *   src (B, NH, L, D) any strides; mean (B, NH, nblk, D), written at block (blk + pool_off);
 *   same values, bit for bit, as the mean written by li_q_prep / li_kv_prep.
 */
int li_pool(int dtype, int32_t B, int32_t NH, int32_t D,
            const void* src, const int64_t src_strides[4],
            void* mean, const int64_t mean_strides[4], int64_t pool_off,
            const li_tile_geom* geom, void* stream);

/*
 * The query pool and the key pool of one attention call in a single launch:
 * job 0 (src0, mean0, pool_off0, geom0) and job 1 (src1, ...) as li_pool each,
 * same bits.  Replaces the two pool calls the reference makes per call, the
 * launch_q_prep and launch_kv_prep means (HYAR:58-70, 110-122, called at
 * HYAR:330-361), for the fused path.  When one job has no blocks or their
 * sources differ in vector access (16-byte aligned unit-stride rows), the
 * jobs are launched one after the other.
 *   mean1_normalized: optional (NULL), same shape and strides as mean1: each
 *     pooled row of job 1 divided by its L2 norm as the cosine metric of
 *     li_block_mask normalises a key pool row (HYAR:250-252), same bits; the
 *     block mask takes it with li_mask_params.k_normalized set, so the
 *     normalisation runs once per key block rather than once per workgroup
 *     of query rows.
 */
int li_pool_pair(int dtype, int32_t B, int32_t NH, int32_t D,
                 const void* src0, const int64_t src0_strides[4],
                 void* mean0, const int64_t mean0_strides[4], int64_t pool_off0,
                 const li_tile_geom* geom0,
                 const void* src1, const int64_t src1_strides[4],
                 void* mean1, const int64_t mean1_strides[4], int64_t pool_off1,
                 const li_tile_geom* geom1, void* mean1_normalized, void* stream);

/*
 * Untile scatter.  Replaces launch_untile(src, dst, T, H, W, tt, th, tw, nh, nw)
 * and _fused_untile_kernel (HYAR:127-161, 204-218; MGS:109-140, 168-177).
 *   src (B, NH, nblk, BS, D) tiles, any strides; dst (B, NH, L, D), any strides.
 * Only slots inside the (T, H, W) grid are stored (padding dropped).
 */
int li_untile(int dtype, int32_t B, int32_t NH, int32_t D,
              const void* src, const int64_t src_strides[5],
              void* dst, const int64_t dst_strides[4],
              const li_tile_geom* geom, void* stream);

/* Similarity metric of the block-mask builder (HYAR:250-256). */
enum li_metric { LI_METRIC_COSINE = 0, LI_METRIC_SCALED_DOT = 1, LI_METRIC_DOT = 2 };
/* Budget rule: HISTORY = nf + int((nk - nf) * ratio), clamped to [1, nk] (HYAR:268-272);
 * TOTAL = min(max(int(nk * ratio), min_budget), nk) (HYKV:282-285). */
enum li_budget_mode { LI_BUDGET_HISTORY = 0, LI_BUDGET_TOTAL = 1 };

typedef struct li_mask_params {
  int32_t metric;           /* li_metric */
  int32_t budget_mode;      /* li_budget_mode */
  double topk_ratio;        /* Python float semantics: int() truncation of a double product */
  int32_t min_budget;       /* TOTAL mode floor (7 in the reference) */
  int32_t n_recent;         /* trailing key blocks always kept (recent_protect slabs) */
  int32_t force_diag;       /* keep the key block at the query's key-grid position */
  int32_t force_sink;       /* keep the t-slab-0 key block at the query's (h, w) */
  int32_t force_neighbors;  /* keep key blocks at 3D Manhattan distance <= 1 (HYKV:268-280) */
  int32_t nq, nk;           /* query / key visual block counts */
  int32_t nh, nw;           /* tiles per slab (key grid) */
  int32_t num_txt_blk;      /* text blocks prepended to every row (HYAR:277-281) */
  int32_t kmax;             /* row length of `indices` (>= num_txt_blk + largest budget) */
  const int32_t* row_budget;/* optional device (nq,) per-row visual totals (ragged rows); NULL = rule */
  float scale;              /* 1/sqrt(D) for LI_METRIC_SCALED_DOT, as fp32 */
  int32_t k_normalized;     /* LI_METRIC_COSINE: k_pool rows are already normalised
                               (li_pool_pair's mean1_normalized); 0 = raw pooled means */
} li_mask_params;

/*
 * Block-mask builder.  Replaces fast_generate_indices (HYAR:223-284) and
 * generate_prefill_indices (HYKV:220-296; MGS:179-234).
 *   q_pool (B, NH, nq, D), k_pool (B, NH, nk, D): pooled means, any strides
 *   indices (B, NH, nq, kmax) int32 contiguous: text blocks, then the selected
 *     visual blocks ascending (+num_txt_blk); unused tail entries are 0
 *   counts (B, NH, nq) int32 contiguous
 *   scores (B, NH, nq, nk) optional (NULL): the bf16/f16 similarity scores
 * Selection: every forced block, then the top (k - n_forced) non-forced blocks by
 * score, ties to the lower block index.  nk <= 12288.
 */
int li_block_mask(int dtype, int32_t B, int32_t NH, int32_t D,
                  const void* q_pool, const int64_t q_pool_strides[4],
                  const void* k_pool, const int64_t k_pool_strides[4],
                  const li_mask_params* params,
                  int32_t* indices, int32_t* counts, void* scores, void* stream);

/*
 * Block-sparse flash-attention forward.  Replaces longcat_flash_attn(q, k, v,
 * block_indices, block_counts, sm_scale, logical_block_size) and
 * _attn_fwd_bsa_align (HYK:27-155, 158-233; MG longcat_kernel.py:28-134, 137-190).
 *   q (B, NH, Lq, D), k / v (B, NH, Lk, D): contiguous; Lk % block_size == 0
 *   block_indices (B, NH, ceil(Lq/block_size), n_cols) int32, any strides
 *   block_counts (B, NH, ceil(Lq/block_size)) int32, any strides
 *   out (B, NH, Lq, D) contiguous; lse (B, NH, Lq) fp32 log2-domain LSE or NULL
 * Query tile m (block_size rows) attends to key blocks
 * block_indices[b,h,m,:block_counts[b,h,m]] (each block_size rows of K/V).
 * Zero rows inside kept blocks take part in the softmax, as in the reference.
 * Out-of-range ids add nothing and access nothing out of bounds (callers
 * validate beforehand): the D=64 kernel skips them; the D=128 kernel fetches
 * block 0 in their place and gives it zero probability (the same result when
 * block 0 holds finite values).  Lk = 0 (no key block at all) is
 * LI_ERR_SHAPE, here and on every attention entry point below.
 * Built for block_size in {64, 128} and D in {64, 128}.
 *
 * workspace (optional, device, 16-byte aligned, NULL allowed): scratch of
 * li_bsa_fwd_workspace_size() bytes.  With it, when the query tiles fill the
 * device's CUs unevenly, the tiles of the last partial round are each split
 * into two halves of their block list that run on different CUs and are
 * combined by a second kernel on the same stream.  Without it (or when it is
 * smaller than required) every tile runs whole.  Results are the same up to
 * fp32 rounding of the combination.
 *
 * flags: a combination of
 *  LI_BSA_BALANCE for rows of unequal length (ragged budgets): with the
 *    workspace, a small kernel first sorts the query tiles by their
 *    kept-block counts and the tiles start longest first (no tail split
 *    then).  It changes the order of work only; results are identical to
 *    flags = 0 without a tail split.  Used by the D = 128 kernels; ignored
 *    for D = 64.
 *  LI_BSA_SORTED (token-order entry points only, li_bsa_fwd_gather and its
 *    variants; ignored here): every row lists its text blocks (ids below
 *    num_txt_blk) before its visual blocks, as the mask builder's ascending
 *    lists do.  The kernel then reads the out-of-grid chunks of visual
 *    blocks from a zero region at the visual chunks' own offsets, which
 *    saves a vector select per load; same results, bit for bit.  A text
 *    block listed after a visual block reads as zeros under this flag.
 *    No counterpart in the reference (its lists are always ascending).
 */
enum li_bsa_flags { LI_BSA_BALANCE = 1, LI_BSA_SORTED = 2 };
int li_bsa_fwd(int dtype, int32_t B, int32_t NH, int32_t Lq, int32_t Lk, int32_t D,
               const void* q, const void* k, const void* v,
               const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
               const int32_t* block_counts, const int64_t cnt_strides[3],
               float sm_scale, int32_t block_size,
               void* out, float* lse, void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

/*
 * Block-sparse attention with the tile gather and untile fused into the
 * kernel: the whole of run_sparse_attention's tile / attend / untile
 * sequence (HYAR:330-361; the tiles of HYAR:26-161 are never written).
 *   q (B, NH, Lq, D), k / v (B, NH, Lk, D), out (B, NH, Lq, D): untiled
 *     tokens, any batch/head/token strides (multiples of 8 elements, unit d
 *     stride, 16-byte aligned); token t*H*W + h*W + w of the grids in
 *     q_geom / k_geom (T = frames of each, other fields equal).  Tokens
 *     outside the grid read as zeros; out is written at valid tokens only.
 *   k_txt / v_txt: (B, NH, num_txt_blk*BS, D) contiguous zero-padded text
 *     keys/values (block ids < num_txt_blk), or NULL when num_txt_blk = 0;
 *     visual block vb has id num_txt_blk + vb.
 *   block_indices / block_counts as for li_bsa_fwd, over the q_geom tiles.
 *   lse (B, NH, nq_blk*BS) fp32 per tiled query row, or NULL.
 *   workspace and flags as for li_bsa_fwd (same size function with Lq = nq_blk*BS).
 * Same results as li_q_prep + li_kv_prep + li_bsa_fwd + li_untile, bit for
 * bit.  Built for D = 128, BS = tt*th*tw = 128, tw and W multiples of 4, a
 * grid at least one tile high and wide (H >= th, W >= tw) and K/V token
 * strides of at least D (LI_ERR_UNSUPPORTED otherwise); the byte offset of a
 * K/V row from its tile's first token must fit 32 bits (LI_ERR_SHAPE).  No
 * counterpart in the reference as one call.
 */
int li_bsa_fwd_gather(int dtype, int32_t B, int32_t NH, int32_t D,
                      const void* q, const int64_t q_strides[4],
                      const void* k, const int64_t k_strides[4],
                      const void* v, const int64_t v_strides[4],
                      const void* k_txt, const void* v_txt, int32_t num_txt_blk,
                      const li_tile_geom* q_geom, const li_tile_geom* k_geom,
                      const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
                      const int32_t* block_counts, const int64_t cnt_strides[3],
                      float sm_scale, void* out, const int64_t out_strides[4], float* lse,
                      void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

/*
 * li_bsa_fwd_gather without a workspace argument and without any device
 * allocation: the tail split's partials and the LI_BSA_BALANCE tile order go
 * to a scratch array of li_bsa_fwd_noalloc_scratch_bytes() bytes (32 MiB)
 * that the library holds on each device it runs on until the process ends.
 * Same kernels, same split and order decisions and same results, bit for
 * bit, as li_bsa_fwd_gather given a workspace of li_bsa_fwd_workspace_size()
 * bytes.  LI_ERR_TOO_LARGE when that workspace would exceed the scratch.
 * Every call on a device shares that device's scratch: calls that overlap
 * on one GPU (other streams, other threads) race and must be serialised by
 * the caller.  No counterpart in the reference: for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 */
int li_bsa_fwd_gather_noalloc(int dtype, int32_t B, int32_t NH, int32_t D,
                              const void* q, const int64_t q_strides[4],
                              const void* k, const int64_t k_strides[4],
                              const void* v, const int64_t v_strides[4],
                              const void* k_txt, const void* v_txt, int32_t num_txt_blk,
                              const li_tile_geom* q_geom, const li_tile_geom* k_geom,
                              const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
                              const int32_t* block_counts, const int64_t cnt_strides[3],
                              float sm_scale, void* out, const int64_t out_strides[4], float* lse,
                              int32_t flags, void* stream);
/* Size of the per-device scratch of li_bsa_fwd_gather_noalloc (no counterpart in the reference). */
int64_t li_bsa_fwd_noalloc_scratch_bytes(void);

/*
 * Workspace bytes li_bsa_fwd / li_bsa_fwd_gather can use for these sizes on
 * the current device: room for the tail split's partials or for the tile
 * order of LI_BSA_BALANCE, whichever is larger (0 for D != 128).  Depends on
 * the device's CU count.  No counterpart in the reference (its Triton launch
 * has neither).
 */
int64_t li_bsa_fwd_workspace_size(int32_t B, int32_t NH, int32_t Lq, int32_t D, int32_t block_size);

/*
 * Dense attention over all keys: the reference's dense fallback
 * F.scaled_dot_product_attention(q, cat(k_txt, k_vis), cat(v_txt, v_vis))
 * (HYAR:316-317; HYKV:331-343; MGS:246-248), with the concatenation never
 * formed.  out = softmax(sm_scale q K^T) V over the txt_len text keys and the
 * Lk visual keys, no padding key taking part; P is rounded to the element
 * type before P V, as on the sparse path.
 *   q (B, NH, Lq, D), k / v (B, NH, Lk, D), out (B, NH, Lq, D): token views,
 *     any batch/head/token strides (multiples of 8 elements, unit d stride,
 *     16-byte aligned), K/V token strides >= D.
 *   k_txt / v_txt: (B, NH, ceil(txt_len/128)*128, D) contiguous text keys/values
 *     (rows past txt_len are ignored), or NULL when txt_len = 0.
 *   lse: (B, NH, ceil(Lq/128)*128) fp32 (log2 units; rows past Lq belong to zero
 *     queries), or NULL.  workspace as for li_bsa_fwd (size function with
 *     Lq = ceil(Lq/128)*128).
 * Built for D = 128 and Lk a multiple of 4 (LI_ERR_UNSUPPORTED otherwise).
 */
int li_attn_fwd_dense(int dtype, int32_t B, int32_t NH, int32_t D, int32_t Lq, int32_t Lk,
                      const void* q, const int64_t q_strides[4],
                      const void* k, const int64_t k_strides[4],
                      const void* v, const int64_t v_strides[4],
                      const void* k_txt, const void* v_txt, int32_t txt_len,
                      float sm_scale, void* out, const int64_t out_strides[4], float* lse,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * fp8 variant of the tiled path: Q and K as OCP e4m3 (float8_e4m3fn) codes
 * with one fp32 scale per tile block, V bf16.  The reference has no fp8
 * path; these mirror li_q_prep / li_kv_prep / li_bsa_fwd (HYAR:166-202,
 * HYK:158-216) with the score product Q K^T taken on e4m3 codes.
 *
 * Quantization of one tile block x (BS x D values, padding rows included):
 * amax = max |x|, scale = amax / 448, codes = e4m3(x * (448 / amax)) rounded
 * to nearest even (both quotients correctly rounded fp32); scale 1 and zero
 * codes for an all-zero block.  Finite inputs never give a NaN code.
 *
 * li_tile_prep_fp8: li_q_prep's gather (dtype = the 16-bit type of src) with
 * the tiles written as codes: dst (B, NH, nblk, BS, D) bytes, unit d stride,
 * other strides multiples of 8, 8-byte aligned; scales (B, NH, nblk) fp32 at
 * block (blk + dst_off).  mean (optional, NULL allowed) is li_q_prep's pool
 * of the unquantized values, bit for bit, at block (blk + pool_off).  Built
 * for BS <= 128 (D = 128) or BS <= 256 (D = 64).  Zero-padded contiguous
 * text blocks (B, NH, n*BS, D) are quantized with the trivial geometry
 * T = n, H = 1, W = BS, tile (1, 1, BS).
 */
int li_tile_prep_fp8(int dtype, int32_t B, int32_t NH, int32_t D,
                     const void* src, const int64_t src_strides[4],
                     void* dst, const int64_t dst_strides[5],
                     float* scales, const int64_t scale_strides[3],
                     void* mean, const int64_t mean_strides[4],
                     int64_t dst_off, int64_t pool_off,
                     const li_tile_geom* geom, void* stream);

/*
 * li_kv_prep with K written as codes and scales (as li_tile_prep_fp8) and V
 * gathered unchanged; the K pool is li_kv_prep's, bit for bit.
 */
int li_kv_prep_fp8(int dtype, int32_t B, int32_t NH, int32_t D,
                   const void* k_src, const int64_t k_src_strides[4],
                   const void* v_src, const int64_t v_src_strides[4],
                   void* k_dst, const int64_t k_dst_strides[5],
                   float* k_scales, const int64_t k_scale_strides[3],
                   void* v_dst, const int64_t v_dst_strides[5],
                   void* k_mean, const int64_t mean_strides[4],
                   int64_t dst_off, int64_t pool_off,
                   const li_tile_geom* geom, void* stream);

/*
 * li_bsa_fwd with e4m3 Q and K: S = (q_scale[tile] * k_scale[block]) *
 * (Q8 K8^T) from the codes on the fp8 MFMA (fp32 accumulation), then the
 * same online softmax, P V in bf16 and outputs as li_bsa_fwd.
 *   q8 (B, NH, Lq, D) codes, contiguous; q_scale (B, NH, ceil(Lq/128)) fp32, contiguous
 *   k8 (B, NH, Lk, D) codes, contiguous; k_scale (B, NH, Lk/128) fp32, contiguous
 *   v (B, NH, Lk, D) bf16, contiguous; out (B, NH, Lq, D) bf16
 * Built for D = 128, block_size = 128 (LI_ERR_UNSUPPORTED otherwise);
 * workspace and flags as for li_bsa_fwd (same size function).
 */
int li_bsa_fwd_fp8(int32_t B, int32_t NH, int32_t Lq, int32_t Lk, int32_t D,
                   const void* q8, const float* q_scale, const void* k8, const float* k_scale,
                   const void* v,
                   const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
                   const int32_t* block_counts, const int64_t cnt_strides[3],
                   float sm_scale, int32_t block_size,
                   void* out, float* lse, void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

/*
 * li_bsa_fwd_fp8 with V read and O written in token order, as
 * li_bsa_fwd_gather does (the fused call of the e4m3 variant):
 *   q8 (B, NH, nq_blk*128, D) e4m3 tiles, q_scale (B, NH, nq_blk) fp32
 *   k8 (B, NH, (num_txt_blk + nk_blk)*128, D) e4m3 tiles (text blocks
 *     first), k_scale (B, NH, num_txt_blk + nk_blk) fp32; all contiguous
 *   v (B, NH, Lk, D) bf16 token view and v_txt / num_txt_blk, the q_geom /
 *     k_geom grids, the lists, out (B, NH, Lq, D) bf16 token view, lse,
 *     workspace and flags: as for li_bsa_fwd_gather (the same shape limits).
 * Same results as li_bsa_fwd_fp8 on the V tiles followed by li_untile.
 */
int li_bsa_fwd_fp8_gather(int32_t B, int32_t NH, int32_t D,
                          const void* q8, const float* q_scale, const void* k8, const float* k_scale,
                          const void* v, const int64_t v_strides[4], const void* v_txt, int32_t num_txt_blk,
                          const li_tile_geom* q_geom, const li_tile_geom* k_geom,
                          const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
                          const int32_t* block_counts, const int64_t cnt_strides[3],
                          float sm_scale, void* out, const int64_t out_strides[4], float* lse,
                          void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LI_SPARSE_ATTN_H */
