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
//    (E = round to the element type).  Element products are exact in fp32.
//    A dot product over d takes eight fp32 partial sums, partial i over
//    d = i, i+8, ... sequentially from +0.0, combined as
//    ((s0+s1)+(s2+s3))+((s4+s5)+(s6+s7)) (eight short chains instead of one
//    of D dependent multiply-adds); a sum of squares runs sequentially.
// 2. forced blocks (recent slabs, diagonal, sink, 3D neighbours) are kept
//    unconditionally -- the reference's +1e6 bias has the same effect;
// 3. the budget k follows the reference's integer arithmetic (int() truncation
//    of a double product) and the remaining k - n_forced blocks are the
//    largest non-forced scores, ties to the lower index: every key block gets
//    the unique 32-bit key (order-preserving score bits << 16 | 0xFFFF - j;
//    0 marks a forced block) and a search two bits at a time finds a
//    threshold with exactly k - n_forced non-forced keys at or above it;
// 4. the selected blocks are written in ascending order by a ballot/prefix
//    compaction over j, which replaces the reference's topk + sort.
//
// One wave selects each query row: every per-row reduction is a ballot +
// popcount inside that wave, and the row's 32-bit keys live in LDS (4 bytes
// per key block).  Aligned pools with a unit d stride take the shared-pool
// kernel (4 rows of one head per workgroup, two waves scoring each row, the
// head's pool streamed once through LDS tiles); other pools and very long key
// grids take the generic kernel, in which each wave scores its row by reading
// the pool rows itself.
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

// The dot product's combination of its eight partial sums.
__device__ __forceinline__ float sum8(const float* s) {
  return ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
}

#define LI_SEL_INLINE __attribute__((always_inline))

// Steps 3 and 4 for query row qb of (b, h) = bh, run by one wave: key_at(r)
// is the key of block 64 r + lane (0 for forced blocks and past nk), nchunk =
// ceil(nk / 64), nf the number of forced blocks.
template <int KUNROLL, typename KeyAt>
__device__ __forceinline__ void select_row(const MaskArgs& a, KeyAt&& key_at, int nchunk, int nf, int qb, int bh,
                                           int lane) {
  const li_mask_params& p = a.p;
  const int nk = p.nk;

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
  // Wave-uniform, so the search below runs on scalar registers.
  const int kk = __builtin_amdgcn_readfirstlane(k - nf);  // non-forced blocks to keep
  const int nfree = nk - nf;

  // Threshold thr with exactly kk non-forced keys >= thr, found from the top
  // two bits per step: with the bits above settled in `prefix`, the three
  // candidates prefix|11, prefix|10 and prefix|01 are counted together (their
  // ballots are independent), and the largest one with at least kk keys at
  // or above it is kept -- what two single-bit steps would keep.  Forced keys
  // are 0 and never reach a candidate, which is always >= 1 here.  The search
  // stops as soon as a kept candidate has exactly kk keys at or above it, the
  // same set as the kk-th largest key selects; for distinct scores that
  // happens within the 16 score bits.  Index bits 15 .. L-1 of the low half
  // are 1 in every key (0xFFFF - j with j < nk <= 2^L): they are set in the
  // prefix from the start (no key's count changes) and not searched.
  uint32_t thr = 1u;
  if (kk > 0 && kk < nfree) {
    const int L = nk > 1 ? 32 - __builtin_clz((uint32_t)(nk - 1)) : 0;
    // The searched bit below b, or -1.
    auto below = [&](int b) LI_SEL_INLINE { return b - 1 >= 16 || b - 1 < L ? b - 1 : L - 1; };
    uint32_t prefix = 0xFFFFu & ~((1u << L) - 1u);
    int b1 = 31;
    while (b1 >= 0) {
      const int b0 = below(b1);
      const uint32_t m1 = 1u << b1, m0 = b0 >= 0 ? 1u << b0 : 0u;
      const uint32_t c3 = prefix | m1 | m0, c2 = prefix | m1, c1 = prefix | m0;
      int n3 = 0, n2 = 0, n1 = 0;
#pragma unroll KUNROLL
      for (int r = 0; r < nchunk; ++r) {
        const uint32_t key = key_at(r);
        n3 += wave_count(key >= c3);
        n2 += wave_count(key >= c2);
        n1 += wave_count(key >= c1);
      }
      if (n3 >= kk) {
        prefix = c3;
        if (n3 == kk) break;
      } else if (n2 >= kk) {
        prefix = c2;
        if (n2 == kk) break;
      } else if (m0 != 0u && n1 >= kk) {
        prefix = c1;
        if (n1 == kk) break;
      }
      b1 = b0 >= 0 ? below(b0) : -1;
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

#define LI_MASK_INLINE __attribute__((always_inline))

// Query row qb of (b, h) into qv (fp32, D values), normalised for cosine: every
// lane computes the same sequential normaliser; lanes own d = lane, lane + 64, ...
template <typename E, int D>
__device__ __forceinline__ void load_query(const MaskArgs& a, int b, int h, int qb, bool cosine, float* qv,
                                           int lane) {
  const uint16_t* qrow = a.qp + b * a.qs[0] + h * a.qs[1] + (int64_t)qb * a.qs[2];
  // All of the lane's loads are issued before the first is used.
  constexpr int PER = (D + 63) / 64;
  uint16_t x[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane + 64 * i;
    x[i] = d < D ? qrow[(int64_t)d * a.qs[3]] : uint16_t(0);
  }
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < D) qv[lane + 64 * i] = E::to_f32(x[i]);
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
}

// A query row's position in the key grid, for the forced-block tests.
struct RowGeom {
  int nk, qb, pos, hw, pt, ph, pw;
  __device__ RowGeom(const li_mask_params& p, int qb_) : nk(p.nk), qb(qb_) {
    pos = p.nk - p.nq + qb;  // query block's position in the key grid
    hw = p.nh * p.nw;
    pt = pos / hw;
    ph = (pos % hw) / p.nw;
    pw = pos % p.nw;
  }
};

// Step 1b/2 for one (row, block): score bits from the fp32 dot product, the
// forced flag, and the order key (0 for a forced block).
template <typename E>
__device__ __forceinline__ uint32_t finish_key(const li_mask_params& p, const RowGeom& g, uint16_t* srow, int j,
                                               float dot, bool& f) {
  uint16_t s = E::from_f32(dot);
  if (p.metric == LI_METRIC_SCALED_DOT) s = E::from_f32(E::to_f32(s) * p.scale);
  if (srow) srow[j] = s;
  f = (p.n_recent > 0) && (j >= g.nk - p.n_recent);
  if (p.force_diag && j == g.pos) f = true;
  if (p.force_sink && j == g.qb % g.hw) f = true;
  if (p.force_neighbors && g.pos >= 0 && g.pos < g.nk) {
    const int jt = j / g.hw, jh = (j % g.hw) / p.nw, jw = j % p.nw;
    if (abs(jt - g.pt) + abs(jh - g.ph) + abs(jw - g.pw) <= 1) f = true;
  }
  return f ? 0u : ((order16(s) << 16) | (0xFFFFu - (uint32_t)j));
}

// Generic path (any pool strides, any nk <= kMaxNk): one wave per query row,
// `waves` rows per workgroup, each wave reading its head's pool rows itself;
// the keys live in the wave's LDS slice (nk + D words).
template <typename E, int D>
__global__ __launch_bounds__(256) void block_mask_kernel(MaskArgs a, int waves) {
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  const li_mask_params& p = a.p;
  const int nk = p.nk;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qb = blockIdx.x * waves + wave;
  const int bh = blockIdx.y;
  if (qb >= p.nq) return;  // whole wave leaves; no workgroup barrier follows
  const int b = bh / a.NH, h = bh % a.NH;
  const bool cosine = p.metric == LI_METRIC_COSINE;
  uint32_t* keys = smem + (size_t)wave * (nk + D);
  float* qv = reinterpret_cast<float*>(keys + nk);
  load_query<E, D>(a, b, h, qb, cosine, qv, lane);

  const RowGeom g(p, qb);
  const bool vec = a.ks[3] == 1 && (reinterpret_cast<uintptr_t>(a.kp) & 15u) == 0 && a.ks[0] % 8 == 0 &&
                   a.ks[1] % 8 == 0 && a.ks[2] % 8 == 0;
  const uint16_t* kbase = a.kp + b * a.ks[0] + h * a.ks[1];
  uint16_t* srow = a.scores ? a.scores + ((int64_t)bh * p.nq + qb) * nk : nullptr;
  int nf = 0;
  for (int j0 = 0; j0 < nk; j0 += 64) {
    const int j = j0 + lane;
    bool f = false;
    if (j < nk) {
      float x[D];
      load_row<E, D>(kbase + (int64_t)j * a.ks[2], a.ks[3], vec, x);
      float ps[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
      if (cosine && !p.k_normalized) {
        const float den = norm_den<E, D>(x);
#pragma unroll
        for (int d = 0; d < D; ++d) ps[d & 7] = ps[d & 7] + qv[d] * E::to_f32(E::from_f32(x[d] / den));
      } else {
#pragma unroll
        for (int d = 0; d < D; ++d) ps[d & 7] = ps[d & 7] + qv[d] * x[d];
      }
      const float dot = sum8(ps);
      keys[j] = finish_key<E>(p, g, srow, j, dot, f);
    }
    nf += wave_count(f);
  }
  __builtin_amdgcn_wave_barrier();
  auto key_at = [&](int r) LI_MASK_INLINE {
    const int j = r * 64 + lane;
    return j < nk ? keys[j] : 0u;
  };
  select_row<1>(a, key_at, (nk + 63) / 64, nf, qb, bh, lane);
}

// Shared-pool path (16-byte aligned pools with unit d stride): a workgroup
// holds 4 query rows of one (b, h), two waves per row, and streams the head's
// pool through LDS in tiles of 128 blocks, so each pool row is read from
// memory once per 4 query rows.  Wave (row, half) scores blocks 64 half +
// lane of every tile against its row's query vector, held in registers.
// Rows are padded by 16 bytes in LDS so that lanes reading consecutive
// blocks hit distinct banks.  For cosine, thread t computes the normaliser of
// block t of the tile and the whole workgroup then divides the tile in place
// before the dot products.  Per (row, block) the arithmetic is the generic
// path's: the same fp32 sums over d of the same operands.  The next
// tile's loads are in flight while the current one is scored, and the first
// wave of each row then selects with the row's keys in registers
// (nk <= 64 KS).
template <typename E, int D, int KS>
__global__ __launch_bounds__(512) void block_mask_tiled_kernel(MaskArgs a) {
  constexpr int NT = 128;          // blocks per tile: one per lane of a row's two waves
  constexpr int NTHR = 512;
  constexpr int RS = 2 * D + 16;   // LDS row stride in bytes
  constexpr int CH = D / 8;        // 16-byte chunks per pool row
  constexpr int PF = NT * CH / NTHR;  // 16-byte chunks per thread per tile
  static_assert(PF * NTHR == NT * CH, "tile must split evenly over the workgroup");
  extern __shared__ __attribute__((aligned(16))) uint32_t smem[];
  const li_mask_params& p = a.p;
  const int nk = p.nk;
  uint8_t* ktile = reinterpret_cast<uint8_t*>(smem);
  float* qall = reinterpret_cast<float*>(ktile + NT * RS);
  float* dn = qall + 4 * D;  // cosine normalisers of the tile's blocks
  uint32_t* kall = reinterpret_cast<uint32_t*>(dn + NT);
  int* nf2 = reinterpret_cast<int*>(kall + (size_t)4 * nk);  // forced counts of the second waves
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = wave & 3, half = wave >> 2;
  const int qb = blockIdx.x * 4 + row;
  const bool live = qb < p.nq;  // dead waves still take part in the tile loads and barriers
  const int bh = blockIdx.y, b = bh / a.NH, h = bh % a.NH;
  const bool cosine = p.metric == LI_METRIC_COSINE;
  float* qv = qall + row * D;
  uint32_t* keys = kall + (size_t)row * nk;
  if (live && half == 0) load_query<E, D>(a, b, h, qb, cosine, qv, lane);

  const RowGeom g(p, qb);
  const uint16_t* kbase = a.kp + b * a.ks[0] + h * a.ks[1];
  uint16_t* srow = (a.scores && live) ? a.scores + ((int64_t)bh * p.nq + qb) * nk : nullptr;
  // Chunk i of this thread: tile row tid / CH + i * (NTHR / CH), column tid % CH.
  const int r0 = tid / CH, cc = tid % CH;
  u32x4 pf[PF];
  // The chunks of tile rows past nt repeat the last row: every load is
  // issued unconditionally, so they all go out together, and only rows below
  // nt are stored.  A tile is fetched only at j0 < nk, so nt >= 1.
  auto fetch = [&](int j0) LI_MASK_INLINE {
    const int nt = nk - j0 < NT ? nk - j0 : NT;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int r = r0 + i * (NTHR / CH);
      const int rr = r < nt ? r : nt - 1;
      pf[i] = *reinterpret_cast<const u32x4*>(kbase + (int64_t)(j0 + rr) * a.ks[2] + 8 * cc);
    }
  };
  if (nk > 0) fetch(0);  // no key blocks: nothing to read
  __syncthreads();  // the query rows are visible to both waves of their row
  // The query row in registers for the dot products (wave-uniform values;
  // stale on dead waves, never used there).
  float qr[D];
#pragma unroll
  for (int d = 0; d < D; ++d) qr[d] = qv[d];
  int nf = 0;
  for (int j0 = 0; j0 < nk; j0 += NT) {
    const int nt = nk - j0 < NT ? nk - j0 : NT;
    __syncthreads();  // the previous tile is consumed
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int r = r0 + i * (NTHR / CH);
      if (r < nt) *reinterpret_cast<u32x4*>(ktile + r * RS + 16 * cc) = pf[i];
    }
    __syncthreads();
    if (j0 + NT < nk) fetch(j0 + NT);
    if (cosine && !p.k_normalized) {
      if (tid < nt) {
        uint8_t* krow = ktile + tid * RS;
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const u32x4 w = *reinterpret_cast<const u32x4*>(krow + 16 * c);
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float x = E::to_f32(uint16_t((w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu));
            ss = ss + x * x;
          }
        }
        const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss)));
        const float eps = E::to_f32(E::from_f32(1e-12f));
        dn[tid] = nrm > eps ? nrm : eps;
      }
      __syncthreads();
      // The divisions, spread over the whole workgroup: each thread rewrites
      // the chunks it stored.
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int r = r0 + i * (NTHR / CH);
        if (r < nt) {
          u32x4* at = reinterpret_cast<u32x4*>(ktile + r * RS + 16 * cc);
          u32x4 w = *at;
          const float den = dn[r];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t lo = E::from_f32(E::to_f32(uint16_t(w[e] & 0xFFFFu)) / den);
            const uint32_t hi = E::from_f32(E::to_f32(uint16_t(w[e] >> 16)) / den);
            w[e] = lo | (hi << 16);
          }
          *at = w;
        }
      }
      __syncthreads();
    }
    if (live) {
      // Tile rows past nt hold stale data; their sums are computed and
      // dropped, so the LDS reads carry no branch and can be issued ahead.
      const int jl = lane + 64 * half;
      float ps[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(ktile + jl * RS + 16 * c);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          ps[e] = ps[e] + qr[8 * c + e] * E::to_f32(uint16_t((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu));
      }
      const float dot = sum8(ps);
      bool f = false;
      if (jl < nt) keys[j0 + jl] = finish_key<E>(p, g, srow, j0 + jl, dot, f);
      nf += wave_count(f);
    }
  }
  if (half == 1 && lane == 0) nf2[row] = nf;
  __syncthreads();  // both halves' keys and the second halves' counts are in LDS
  if (!live || half == 1) return;
  nf += nf2[row];
  uint32_t kr[KS];
#pragma unroll
  for (int r = 0; r < KS; ++r) {
    const int j = r * 64 + lane;
    kr[r] = j < nk ? keys[j] : 0u;
  }
  select_row<KS>(a, [&](int r) LI_MASK_INLINE { return kr[r]; }, KS, nf, qb, bh, lane);
}

constexpr int kTiledMaxNk = 64 * 28;

// LDS bytes of the shared-pool path, or 0 when it does not apply.
size_t tiled_lds(int D, int nk, bool vec_k) {
  if (!vec_k || nk > kTiledMaxNk) return 0;
  const size_t bytes = (size_t)128 * (2 * D + 16 + 4) + (size_t)4 * D * 4 + (size_t)4 * nk * 4 + 4 * 4;
  return bytes <= 65536 ? bytes : 0;
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
  const bool vec_k = k_pool_strides[3] == 1 && (reinterpret_cast<uintptr_t>(k_pool) & 15u) == 0 &&
                     k_pool_strides[0] % 8 == 0 && k_pool_strides[1] % 8 == 0 && k_pool_strides[2] % 8 == 0;
  const size_t tiled = tiled_lds(D, p.nk, vec_k);
  // Generic path: per-wave LDS slice of nk keys + the query row, up to 4
  // waves (rows) per workgroup.
  const size_t per_wave = ((size_t)p.nk + D) * 4;
  int waves = (int)(65536 / per_wave);
  waves = waves < 1 ? 1 : (waves > 4 ? 4 : waves);
  const int rows = tiled ? 4 : waves;
  const size_t lds = tiled ? tiled : per_wave * waves;
  dim3 grid((unsigned)((p.nq + rows - 1) / rows), (unsigned)(B * NH));
  dim3 block((unsigned)(tiled ? 512 : 64 * waves));
  hipStream_t s = static_cast<hipStream_t>(stream);
  clear_launch_error();
#define LI_MASK_LAUNCH(E_, D_)                                                                          \
  do {                                                                                                  \
    if (tiled && p.nk <= 256)                                                                           \
      hipLaunchKernelGGL((block_mask_tiled_kernel<E_, D_, 4>), grid, block, lds, s, a);                 \
    else if (tiled && p.nk <= 1024)                                                                     \
      hipLaunchKernelGGL((block_mask_tiled_kernel<E_, D_, 16>), grid, block, lds, s, a);                \
    else if (tiled)                                                                                     \
      hipLaunchKernelGGL((block_mask_tiled_kernel<E_, D_, 28>), grid, block, lds, s, a);                \
    else                                                                                                \
      hipLaunchKernelGGL((block_mask_kernel<E_, D_>), grid, block, lds, s, a, waves);                 \
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
