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
//    the unique 32-bit key (order-preserving score bits << 16 | 0xFFFF - j;
//    0 marks a forced block) and a 32-step bitwise search finds the exact
//    (k - n_forced)-th largest key;
// 4. the selected blocks are written in ascending order by a ballot/prefix
//    compaction over j, which replaces the reference's topk + sort.
//
// One wave per query row, WAVES rows per workgroup: every reduction is a
// ballot + popcount inside the wave, so the kernel has no workgroup barrier.
// The wave's keys live in its own LDS slice (4 bytes per key block).
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

// Sequential fp32 sum of squares from +0.0, then the reference's normaliser
// max(E(sqrt(.)), E(1e-12)).
template <typename E, int D>
__device__ __forceinline__ float norm_den(const float* x) {
  float ss = 0.0f;
#pragma unroll
  for (int d = 0; d < D; ++d) ss = ss + x[d] * x[d];
  const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss)));
  const float eps = E::to_f32(E::from_f32(1e-12f));
  return nrm > eps ? nrm : eps;
}

__device__ __forceinline__ int wave_count(bool pred) { return __popcll(__ballot(pred)); }

#define LI_MASK_INLINE __attribute__((always_inline))

// KR > 0: nk <= 64 KR and contiguous pool rows; a lane keeps the keys of
// blocks lane, lane + 64, ... in registers and computes their dot products
// side by side (each still summed over d in order).  KR = 0: any nk, keys
// in the wave's LDS slice.
template <typename E, int D, int KR>
__global__ __launch_bounds__(256) void block_mask_kernel(MaskArgs a, int waves) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  const li_mask_params& p = a.p;
  const int nk = p.nk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int qb = blockIdx.x * waves + wave;
  const int bh = blockIdx.y;
  if (qb >= p.nq) return;  // whole wave leaves; no workgroup barrier follows
  const int b = bh / a.NH, h = bh % a.NH;
  const bool cosine = p.metric == LI_METRIC_COSINE;
  uint32_t* keys = smem + (size_t)wave * (nk + D);
  float* qv = reinterpret_cast<float*>(keys + nk);

  // 1a. query pool row, normalised for cosine (every lane computes the same
  // sequential normaliser; lanes then own elements lane, lane + 64, ...).
  const uint16_t* qrow = a.qp + b * a.qs[0] + h * a.qs[1] + (int64_t)qb * a.qs[2];
  for (int d = lane; d < D; d += 64) qv[d] = E::to_f32(qrow[(int64_t)d * a.qs[3]]);
  __builtin_amdgcn_wave_barrier();
  if (cosine) {
    float ss = 0.0f;
    for (int d = 0; d < D; ++d) ss = ss + qv[d] * qv[d];
    const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss)));
    const float eps = E::to_f32(E::from_f32(1e-12f));
    const float den = nrm > eps ? nrm : eps;
    __builtin_amdgcn_wave_barrier();
    for (int d = lane; d < D; d += 64) qv[d] = E::to_f32(E::from_f32(qv[d] / den));
    __builtin_amdgcn_wave_barrier();
  }

  // 1b/2. scores, forced flags, order keys.
  const int pos = nk - p.nq + qb;  // query block's position in the key grid
  const int hw = p.nh * p.nw;
  const int pt = pos / hw, ph = (pos % hw) / p.nw, pw = pos % p.nw;
  const bool vec = a.ks[3] == 1 && (reinterpret_cast<uintptr_t>(a.kp) & 15u) == 0 && a.ks[0] % 8 == 0 &&
                   a.ks[1] % 8 == 0 && a.ks[2] % 8 == 0;
  const uint16_t* kbase = a.kp + b * a.ks[0] + h * a.ks[1];
  uint16_t* srow = a.scores ? a.scores + ((int64_t)bh * p.nq + qb) * nk : nullptr;
  // Score bits of block j -> forced flag and order key.
  auto finish = [&](int j, float dot, bool& f) {
    uint16_t s = E::from_f32(dot);
    if (p.metric == LI_METRIC_SCALED_DOT) s = E::from_f32(E::to_f32(s) * p.scale);
    if (srow) srow[j] = s;
    f = (p.n_recent > 0) && (j >= nk - p.n_recent);
    if (p.force_diag && j == pos) f = true;
    if (p.force_sink && j == qb % hw) f = true;
    if (p.force_neighbors && pos >= 0 && pos < nk) {
      const int jt = j / hw, jh = (j % hw) / p.nw, jw = j % p.nw;
      if (abs(jt - pt) + abs(jh - ph) + abs(jw - pw) <= 1) f = true;
    }
    return f ? 0u : ((order16(s) << 16) | (0xFFFFu - (uint32_t)j));
  };
  int nf = 0;
  uint32_t kr[KR > 0 ? KR : 1];
  if constexpr (KR > 0) {
    // Dot products of this lane's KR blocks, 8 dimensions at a time.
    float dot[KR], den[KR];
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      dot[r] = 0.0f;
      den[r] = 1.0f;
    }
    if (cosine) {
      float ss[KR];
#pragma unroll
      for (int r = 0; r < KR; ++r) ss[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < D / 8; ++c)
#pragma unroll
        for (int r = 0; r < KR; ++r) {
          const int j = r * 64 + lane;
          if (j < nk) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(kbase + (int64_t)j * a.ks[2] + 8 * c);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float x = E::to_f32(uint16_t((w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu));
              ss[r] = ss[r] + x * x;
            }
          }
        }
      const float eps = E::to_f32(E::from_f32(1e-12f));
#pragma unroll
      for (int r = 0; r < KR; ++r) {
        const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss[r])));
        den[r] = nrm > eps ? nrm : eps;
      }
    }
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      float q8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) q8[i] = qv[8 * c + i];
#pragma unroll
      for (int r = 0; r < KR; ++r) {
        const int j = r * 64 + lane;
        if (j < nk) {
          const u32x4 w = *reinterpret_cast<const u32x4*>(kbase + (int64_t)j * a.ks[2] + 8 * c);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float x = E::to_f32(uint16_t((w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu));
            if (cosine) x = E::to_f32(E::from_f32(x / den[r]));
            dot[r] = dot[r] + q8[i] * x;
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < KR; ++r) {
      const int j = r * 64 + lane;
      bool f = false;
      kr[r] = 0u;
      if (j < nk) kr[r] = finish(j, dot[r], f);
      nf += wave_count(f);
    }
  } else {
    for (int j0 = 0; j0 < nk; j0 += 64) {
      const int j = j0 + lane;
      bool f = false;
      if (j < nk) {
        float x[D];
        load_row<E, D>(kbase + (int64_t)j * a.ks[2], a.ks[3], vec, x);
        float dot = 0.0f;
        if (cosine) {
          const float den = norm_den<E, D>(x);
#pragma unroll
          for (int d = 0; d < D; ++d) dot = dot + qv[d] * E::to_f32(E::from_f32(x[d] / den));
        } else {
#pragma unroll
          for (int d = 0; d < D; ++d) dot = dot + qv[d] * x[d];
        }
        keys[j] = finish(j, dot, f);
      }
      nf += wave_count(f);
    }
  }
  __builtin_amdgcn_wave_barrier();
  // Key of block r * 64 + lane (0 past nk: never selected, never counted).
  auto key_at = [&](int r) LI_MASK_INLINE {
    if constexpr (KR > 0) {
      return kr[r];
    } else {
      const int j = r * 64 + lane;
      return j < nk ? keys[j] : 0u;
    }
  };
  const int nchunk = KR > 0 ? KR : (nk + 63) / 64;
  constexpr int KUNROLL = KR > 0 ? KR : 1;

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
  const int kk = k - nf;  // non-forced blocks to keep
  const int nfree = nk - nf;

  // Exact kk-th largest key among non-forced blocks (forced keys are 0 and
  // never reach a candidate, which is always >= 1 here).
  uint32_t thr = 1u;
  if (kk > 0 && kk < nfree) {
    uint32_t prefix = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = prefix | (1u << bit);
      int c = 0;
#pragma unroll KUNROLL
      for (int r = 0; r < nchunk; ++r) c += wave_count(key_at(r) >= cand);
      if (c >= kk) prefix = cand;
    }
    thr = prefix;
  }

  // 4. ascending compaction.
  const int64_t row = (int64_t)bh * p.nq + qb;
  int32_t* irow = a.indices + row * p.kmax;
  const int ntxt = p.num_txt_blk;
  for (int i = lane; i < ntxt && i < p.kmax; i += 64) irow[i] = i;
  int base = ntxt;
#pragma unroll KUNROLL
  for (int r = 0; r < nchunk; ++r) {
    const int j = r * 64 + lane;
    bool sel = false;
    if (j < nk) {
      const uint32_t key = key_at(r);
      sel = key == 0u || (kk > 0 && key >= thr);
    }
    const uint64_t m = __ballot(sel);
    const int dst = base + __popcll(m & ((1ull << lane) - 1ull));
    if (sel && dst < p.kmax) irow[dst] = j + ntxt;
    base += __popcll(m);
  }
  for (int i = ntxt + k + lane; i < p.kmax; i += 64) irow[i] = 0;
  if (lane == 0) a.counts[row] = ntxt + k;
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
  // Per-wave LDS slice: nk keys (LDS path only) + the query row; up to 4
  // waves (rows) per workgroup.
  const bool vec_k = k_pool_strides[3] == 1 && (reinterpret_cast<uintptr_t>(k_pool) & 15u) == 0 &&
                     k_pool_strides[0] % 8 == 0 && k_pool_strides[1] % 8 == 0 && k_pool_strides[2] % 8 == 0;
  const int kr = !vec_k ? 0 : (p.nk <= 256 ? 4 : (p.nk <= 1024 ? 16 : 0));
  const size_t per_wave = ((size_t)p.nk + D) * 4;
  int waves = (int)(65536 / per_wave);
  waves = waves < 1 ? 1 : (waves > 4 ? 4 : waves);
  const size_t lds = per_wave * waves;
  dim3 grid((unsigned)((p.nq + waves - 1) / waves), (unsigned)(B * NH));
  dim3 block((unsigned)(64 * waves));
  hipStream_t s = static_cast<hipStream_t>(stream);
  clear_launch_error();
#define LI_MASK_LAUNCH(E_, D_)                                                                          \
  do {                                                                                                  \
    if (kr == 4)                                                                                        \
      hipLaunchKernelGGL((block_mask_kernel<E_, D_, 4>), grid, block, lds, s, a, waves);              \
    else if (kr == 16)                                                                                  \
      hipLaunchKernelGGL((block_mask_kernel<E_, D_, 16>), grid, block, lds, s, a, waves);             \
    else                                                                                                \
      hipLaunchKernelGGL((block_mask_kernel<E_, D_, 0>), grid, block, lds, s, a, waves);              \
  } while (0)
  if (dtype == LI_DTYPE_BF16 && D == 128)
    LI_MASK_LAUNCH(Bf16, 128);
  else if (dtype == LI_DTYPE_BF16 && D == 64)
    LI_MASK_LAUNCH(Bf16, 64);
  else if (dtype == LI_DTYPE_F16 && D == 128)
    LI_MASK_LAUNCH(F16, 128);
  else if (dtype == LI_DTYPE_F16 && D == 64)
    LI_MASK_LAUNCH(F16, 64);
  else
    return LI_ERR_UNSUPPORTED;
#undef LI_MASK_LAUNCH
  return launch_status();
}
