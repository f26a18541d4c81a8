// Block-mask builder for gfx950: pooled block similarity, forced AR blocks,
// per-query-block top-k and ascending block lists.
//
// Replaces fast_generate_indices (hy-worldplay/.../ar_sparse_operation.py:223-284)
// and generate_prefill_indices (bi_sparse_operation_for_KV_cache.py:220-296,
// matrix-game-3.0/.../bi_sparse_operation.py:179-234), which run normalize /
// matmul / +1e6 bias / topk / sort / cat as a chain of torch launches.  Here one
// 256-thread workgroup per (query block, batch*head) does all of it:
//
// 1. score[j] for every key block j, with the reference's rounding points:
//    cosine  xn = E(x / max(E(sqrt(sum x^2)), E(1e-12))), sim = E(sum qn*kn);
//    scaled  sim = E(f32(E(sum q*k)) * scale);  dot  sim = E(sum q*k)
//    (E = round to the element type).  Every fp32 sum over d runs sequentially
//    from +0.0; element products are exact in fp32.
// 2. forced blocks (recent slabs, diagonal, sink, 3D neighbours) are kept
//    unconditionally -- the reference's +1e6 bias has the same effect;
// 3. the budget k follows the reference's integer arithmetic (int() truncation
//    of a double product) and the remaining k - n_forced blocks are the
//    largest non-forced scores, ties to the lower index: every key block gets
//    the unique 32-bit key (order-preserving score bits << 16 | 0xFFFF - j) and
//    a 32-step bitwise search finds the exact (k - n_forced)-th largest key;
// 4. the selected blocks are written in ascending order by a ballot/prefix
//    compaction over j, which replaces the reference's topk + sort.
#include "li_common.hpp"

namespace li {
namespace {

constexpr int kMaxNk = 12288;

struct MaskArgs {
  const uint16_t* qp;
  int64_t qs[4];
  const uint16_t* kp;
  int64_t ks[4];
  li_mask_params p;
  int32_t* indices;
  int32_t* counts;
  uint16_t* scores;
  int32_t NH;
};

__device__ __forceinline__ uint32_t order16(uint16_t bits) {
  return (bits & 0x8000u) ? (uint32_t)(~bits & 0xFFFFu) : (uint32_t)(bits | 0x8000u);
}

__device__ __forceinline__ int block_sum(int v, int* scratch) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  return scratch[0] + scratch[1] + scratch[2] + scratch[3];
}

template <typename E, int D>
__device__ __forceinline__ void load_row(const uint16_t* p, int64_t stride, bool vec, float* x) {
  if (vec) {
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      u32x4 w = *reinterpret_cast<const u32x4*>(p + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[8 * c + 2 * i] = E::to_f32(uint16_t(w[i] & 0xFFFFu));
        x[8 * c + 2 * i + 1] = E::to_f32(uint16_t(w[i] >> 16));
      }
    }
  } else {
#pragma unroll
    for (int d = 0; d < D; ++d) x[d] = E::to_f32(p[d * stride]);
  }
}

template <typename E, int D>
__global__ __launch_bounds__(256) void block_mask_kernel(MaskArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  const li_mask_params& p = a.p;
  const int nk = p.nk;
  uint32_t* keys = smem;                                        // nk
  uint8_t* forced = reinterpret_cast<uint8_t*>(smem + nk);       // nk
  __shared__ float qv[D];
  __shared__ float qden;
  __shared__ int scratch[4];
  __shared__ int wave_cnt[4];

  const int qb = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.NH, h = bh % a.NH;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool cosine = p.metric == LI_METRIC_COSINE;

  // 1a. query pool row (normalised for cosine).
  const uint16_t* qrow = a.qp + b * a.qs[0] + h * a.qs[1] + (int64_t)qb * a.qs[2];
  if (tid < D) qv[tid] = E::to_f32(qrow[(int64_t)tid * a.qs[3]]);
  __syncthreads();
  if (cosine) {
    if (tid == 0) {
      float ss = 0.0f;
      for (int d = 0; d < D; ++d) ss = ss + qv[d] * qv[d];
      const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss)));
      const float eps = E::to_f32(E::from_f32(1e-12f));
      qden = nrm > eps ? nrm : eps;
    }
    __syncthreads();
    if (tid < D) qv[tid] = E::to_f32(E::from_f32(qv[tid] / qden));
    __syncthreads();
  }

  // 1b/2. scores, forced flags, order keys.
  const int pos = nk - p.nq + qb;  // query block's position in the key grid
  const int hw = p.nh * p.nw;
  const int pt = pos / hw, ph = (pos % hw) / p.nw, pw = pos % p.nw;
  const bool vec = a.ks[3] == 1 && (reinterpret_cast<uintptr_t>(a.kp) & 15u) == 0 && a.ks[0] % 8 == 0 &&
                   a.ks[1] % 8 == 0 && a.ks[2] % 8 == 0;
  const uint16_t* kbase = a.kp + b * a.ks[0] + h * a.ks[1];
  uint16_t* srow = a.scores ? a.scores + ((int64_t)bh * p.nq + qb) * nk : nullptr;
  int nf_local = 0;
  for (int j = tid; j < nk; j += 256) {
    float x[D];
    load_row<E, D>(kbase + (int64_t)j * a.ks[2], a.ks[3], vec, x);
    float dot = 0.0f;
    if (cosine) {
      float ss = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) ss = ss + x[d] * x[d];
      const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss)));
      const float eps = E::to_f32(E::from_f32(1e-12f));
      const float den = nrm > eps ? nrm : eps;
#pragma unroll
      for (int d = 0; d < D; ++d) dot = dot + qv[d] * E::to_f32(E::from_f32(x[d] / den));
    } else {
#pragma unroll
      for (int d = 0; d < D; ++d) dot = dot + qv[d] * x[d];
    }
    uint16_t s = E::from_f32(dot);
    if (p.metric == LI_METRIC_SCALED_DOT) s = E::from_f32(E::to_f32(s) * p.scale);
    if (srow) srow[j] = s;

    bool f = (p.n_recent > 0) && (j >= nk - p.n_recent);
    if (p.force_diag && j == pos) f = true;
    if (p.force_sink && j == qb % hw) f = true;
    if (p.force_neighbors && pos >= 0 && pos < nk) {
      const int jt = j / hw, jh = (j % hw) / p.nw, jw = j % p.nw;
      const int dist = abs(jt - pt) + abs(jh - ph) + abs(jw - pw);
      if (dist <= 1) f = true;
    }
    forced[j] = f ? 1 : 0;
    keys[j] = f ? 0u : ((order16(s) << 16) | (0xFFFFu - (uint32_t)j));
    nf_local += f ? 1 : 0;
  }
  const int nf = block_sum(nf_local, scratch);  // also orders the LDS writes above

  // 3. budget.
  int k;
  if (p.row_budget) {
    k = p.row_budget[qb];
    k = k < nf ? nf : k;
    k = k > nk ? nk : k;
  } else if (p.budget_mode == LI_BUDGET_HISTORY) {
    k = nf + (int)((double)(nk - nf) * p.topk_ratio);
    const int lo = nk > 0 ? 1 : 0;
    k = k < lo ? lo : k;
    k = k > nk ? nk : k;
    k = k < nf ? nf : k;
  } else {
    k = (int)((double)nk * p.topk_ratio);
    k = k < p.min_budget ? p.min_budget : k;
    k = k > nk ? nk : k;
    k = k < nf ? nf : k;
  }
  const int kk = k - nf;       // non-forced blocks to keep
  const int nfree = nk - nf;

  // Exact kk-th largest key among non-forced blocks.
  uint32_t thr = 0;
  if (kk > 0 && kk < nfree) {
    uint32_t prefix = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = prefix | (1u << bit);
      int c = 0;
      for (int j = tid; j < nk; j += 256) c += (!forced[j] && keys[j] >= cand) ? 1 : 0;
      c = block_sum(c, scratch);
      if (c >= kk) prefix = cand;
    }
    thr = prefix;
  }

  // 4. ascending compaction.
  const int64_t row = (int64_t)bh * p.nq + qb;
  int32_t* irow = a.indices + row * p.kmax;
  const int ntxt = p.num_txt_blk;
  for (int i = tid; i < ntxt && i < p.kmax; i += 256) irow[i] = i;
  int base = 0;
  for (int c0 = 0; c0 < nk; c0 += 256) {
    const int j = c0 + tid;
    bool sel = false;
    if (j < nk) sel = forced[j] || (kk > 0 && (kk >= nfree || keys[j] >= thr));
    const uint64_t m = __ballot(sel);
    const int lp = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[wave] = __popcll(m);
    __syncthreads();
    int off = base;
    for (int w = 0; w < wave; ++w) off += wave_cnt[w];
    const int dst = ntxt + off + lp;
    if (sel && dst < p.kmax) irow[dst] = j + ntxt;
    base += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
  }
  for (int i = ntxt + k + tid; i < p.kmax; i += 256) irow[i] = 0;
  if (tid == 0) a.counts[row] = ntxt + k;
}

}  // namespace
}  // namespace li

using namespace li;

extern "C" int li_block_mask(int dtype, int32_t B, int32_t NH, int32_t D, const void* q_pool,
                             const int64_t q_pool_strides[4], const void* k_pool, const int64_t k_pool_strides[4],
                             const li_mask_params* params, int32_t* indices, int32_t* counts, void* scores,
                             void* stream) {
  if (!q_pool || !k_pool || !q_pool_strides || !k_pool_strides || !params || !indices || !counts)
    return LI_ERR_INVALID_ARG;
  if (B <= 0 || NH <= 0) return LI_ERR_INVALID_ARG;
  const li_mask_params& p = *params;
  if (p.nq < 0 || p.nk < 0 || p.nh <= 0 || p.nw <= 0 || p.num_txt_blk < 0 || p.kmax < 0 || p.n_recent < 0)
    return LI_ERR_SHAPE;
  if (p.metric < LI_METRIC_COSINE || p.metric > LI_METRIC_DOT) return LI_ERR_INVALID_ARG;
  if (p.budget_mode != LI_BUDGET_HISTORY && p.budget_mode != LI_BUDGET_TOTAL) return LI_ERR_INVALID_ARG;
  if (!(p.topk_ratio >= 0.0) || p.topk_ratio > 1e6) return LI_ERR_INVALID_ARG;
  if (p.nk > kMaxNk) return LI_ERR_TOO_LARGE;
  if (p.kmax < p.num_txt_blk) return LI_ERR_SHAPE;
  if (p.nq == 0) return LI_OK;
  if ((int64_t)B * NH > 65535) return LI_ERR_SHAPE;
  MaskArgs a = {};
  a.qp = static_cast<const uint16_t*>(q_pool);
  a.kp = static_cast<const uint16_t*>(k_pool);
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_pool_strides[i];
    a.ks[i] = k_pool_strides[i];
  }
  a.p = p;
  a.indices = indices;
  a.counts = counts;
  a.scores = static_cast<uint16_t*>(scores);
  a.NH = NH;
  const size_t lds = (size_t)p.nk * 4 + (size_t)p.nk + 16;
  dim3 grid((unsigned)p.nq, (unsigned)(B * NH));
  hipStream_t s = static_cast<hipStream_t>(stream);
  clear_launch_error();
  if (dtype == LI_DTYPE_BF16 && D == 128)
    hipLaunchKernelGGL((block_mask_kernel<Bf16, 128>), grid, dim3(256), lds, s, a);
  else if (dtype == LI_DTYPE_BF16 && D == 64)
    hipLaunchKernelGGL((block_mask_kernel<Bf16, 64>), grid, dim3(256), lds, s, a);
  else if (dtype == LI_DTYPE_F16 && D == 128)
    hipLaunchKernelGGL((block_mask_kernel<F16, 128>), grid, dim3(256), lds, s, a);
  else if (dtype == LI_DTYPE_F16 && D == 64)
    hipLaunchKernelGGL((block_mask_kernel<F16, 64>), grid, dim3(256), lds, s, a);
  else
    return LI_ERR_UNSUPPORTED;
  return launch_status();
}
