// Block-sparse flash-attention forward for gfx950 (MI355X), bf16/f16 MFMA.
//
// Replaces _attn_fwd_bsa_align (hy-worldplay/.../longcat_kernel.py:27-155;
// matrix-game-3.0/.../longcat_kernel.py:28-134).  Semantics kept from the
// reference: for query tile m (BS rows) and each kept key block j in stored
// order, S = Q K_j^T in fp32; online softmax in base 2 with
// qk_scale = sm_scale * 1.44269504 (longcat_kernel.py:107, 128-138); P is
// rounded to the element type before P V (longcat_kernel.py:141); zero key
// rows of a kept block are not masked; output acc / l, and the log2-domain
// LSE m + log2(l) (longcat_kernel.py:146-155).  A row with no kept block
// yields zeros and lse = -inf.
//
// Design (one workgroup = 2*BS/32 waves = one BS-row query tile; at BS = 128
// that is 8 waves, two per SIMD, so one wave's softmax overlaps the other's
// MFMAs):
//  * wave w owns the 32 query rows [32*qq, +32) with qq = w >> 1 and the key
//    rows [kh*BS/2, +BS/2) of every kept block with kh = w & 1.  Each wave
//    runs its own online softmax over its key half; the two halves are
//    merged once at the end through LDS.
//  * The transposed score tile S^T = K Q^T is computed with
//    v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q^T held in registers for
//    the whole tile).  Its accumulator layout puts one query per lane
//    column, so the softmax row statistics need a single cross-half
//    exchange, and the probabilities feed O^T = V^T P^T directly as the MFMA
//    B operand without an LDS round trip.
//  * K and V tiles are double-buffered in LDS: block i+1 is fetched into
//    registers while block i is computed, then written to the other stage.
//    K keeps its row layout with a 16-byte-granule XOR swizzle; V is written
//    transposed (V^T, keys contiguous) with an 8-byte-granule XOR swizzle, so
//    both MFMA operand reads are bank-conflict free.
//  * Workgroup ids are remapped so that each XCD (ids are dealt round-robin
//    over the 8 XCDs) processes a contiguous range of (head, tile) work and
//    the tiles of one head share that XCD's L2 for their K/V blocks.
#include "li_common.hpp"

namespace li {
namespace {

struct BsaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* idx;
  int64_t is[4];
  const int32_t* cnt;
  int64_t cs[3];
  uint16_t* out;
  float* lse;
  int32_t NH, Lq, nkb, nqt, n_cols;
  float qk_scale;
};

template <int BS, int D>
struct Cfg {
  static constexpr int WAVES = 2 * (BS / 32);
  static constexpr int NTHR = 64 * WAVES;
  static constexpr int QW = 32;           // query rows per wave
  static constexpr int KW = BS / 2;       // keys per wave per block
  static constexpr int NQT = QW / 32;     // 32-query sub-tiles per wave
  static constexpr int NKT = KW / 32;     // 32-key sub-tiles per wave
  static constexpr int DS = D / 16;       // MFMA k-steps of S (over d)
  static constexpr int NDT = D / 32;      // 32-wide d tiles of O
  static constexpr int PST = KW / 16;     // MFMA k-steps of P V (over keys)
  static constexpr int KGR = D / 8;       // 16-byte granules per K row
  static constexpr int KSW = (KGR < 16 ? KGR : 16) - 1;  // K swizzle mask
  static constexpr int VGR = BS / 4;      // 8-byte granules (4 keys) per V^T row
  static constexpr int K_UNITS = BS * KGR;          // 16-byte K loads per block
  static constexpr int V_UNITS = (BS / 4) * KGR;    // (4 keys x 8 d) V units per block
  static constexpr int K_IT = (K_UNITS + NTHR - 1) / NTHR;
  static constexpr int V_IT = (V_UNITS + NTHR - 1) / NTHR;
  static constexpr int STAGE_ELEMS = BS * D;        // per K or V^T stage
  static constexpr int KV_BYTES = 2 * 2 * STAGE_ELEMS * 2;
  static constexpr int NQW = WAVES / 2;                         // query groups
  static constexpr int X_FLOATS = NQW * NDT * NQT * 16 * 64;     // epilogue O exchange
  static constexpr int X_BYTES = X_FLOATS * 4 + NQW * 2 * NQT * 64 * 4;
  static constexpr int LDS_BYTES = KV_BYTES > X_BYTES ? KV_BYTES : X_BYTES;
};

__device__ __forceinline__ int vswz(int d, int vgr) { return ((d & (vgr - 1)) ^ (d / vgr)) & (vgr - 1); }

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);  // {a.lo16, b.lo16}
}
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);  // {a.hi16, b.hi16}
}

template <typename E, int BS, int D>
__global__ __launch_bounds__(4 * BS) void bsa_fwd_kernel(BsaArgs a) {
  using C = Cfg<BS, D>;
  typedef typename E::vec8 vec8;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  uint16_t* kbuf = reinterpret_cast<uint16_t*>(smem);               // [2][BS][D] swizzled
  uint16_t* vbuf = kbuf + 2 * C::STAGE_ELEMS;                        // [2][D][BS] transposed, swizzled

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qh = wave >> 1, kh = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;

  // XCD-aware remap: hardware deals workgroup ids round-robin over 8 XCDs;
  // give each XCD a contiguous slice of the head-major work list.
  const int nwg = gridDim.x, id = blockIdx.x;
  const int xcd = id & 7, slot = id >> 3;
  const int per = nwg >> 3, rem = nwg & 7;
  const int w = xcd * per + (xcd < rem ? xcd : rem) + slot;
  const int bh = w / a.nqt, m = w % a.nqt;
  const int b = bh / a.NH, h = bh % a.NH;

  const uint16_t* qhead = a.q + (int64_t)bh * a.Lq * D;
  const uint16_t* khead = a.k + (int64_t)bh * a.nkb * BS * D;
  const uint16_t* vhead = a.v + (int64_t)bh * a.nkb * BS * D;
  uint16_t* ohead = a.out + (int64_t)bh * a.Lq * D;
  const int32_t* irow = a.idx + b * a.is[0] + h * a.is[1] + (int64_t)m * a.is[2];
  int count = a.cnt[b * a.cs[0] + h * a.cs[1] + (int64_t)m * a.cs[2]];
  count = count < 0 ? 0 : (count > a.n_cols ? a.n_cols : count);
  count = __builtin_amdgcn_readfirstlane(count);
  const int row0 = m * BS;

  if (count == 0) {
    // No kept block: zeros (and lse = -inf), as the reference's l_i = 1, acc = 0.
    for (int u = tid; u < BS * (D / 8); u += C::NTHR) {
      const int r = row0 + u / (D / 8);
      if (r < a.Lq) *reinterpret_cast<u32x4*>(ohead + (int64_t)r * D + 8 * (u % (D / 8))) = u32x4{0u, 0u, 0u, 0u};
    }
    if (a.lse)
      for (int r = tid; r < BS; r += C::NTHR)
        if (row0 + r < a.Lq) a.lse[(int64_t)bh * a.Lq + row0 + r] = -__builtin_inff();
    return;
  }

  // Q^T fragments (MFMA B operand): lane holds query row (l32) and d = 16 s + 8 hl .. +7.
  vec8 qf[C::NQT][C::DS];
#pragma unroll
  for (int qt = 0; qt < C::NQT; ++qt) {
    const int r = row0 + C::QW * qh + 32 * qt + l32;
#pragma unroll
    for (int s = 0; s < C::DS; ++s) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (r < a.Lq) x = *reinterpret_cast<const u32x4*>(qhead + (int64_t)r * D + 16 * s + 8 * hl);
      qf[qt][s] = __builtin_bit_cast(vec8, x);
    }
  }

  u32x4 kst[C::K_IT];
  u32x4 vst[C::V_IT][4];
  auto fetch = [&](int blk) {
    const uint16_t* kb = khead + (int64_t)blk * BS * D;
    const uint16_t* vb = vhead + (int64_t)blk * BS * D;
#pragma unroll
    for (int it = 0; it < C::K_IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::K_UNITS % C::NTHR == 0 || u < C::K_UNITS)
        kst[it] = *reinterpret_cast<const u32x4*>(kb + (u / C::KGR) * D + 8 * (u % C::KGR));
    }
#pragma unroll
    for (int it = 0; it < C::V_IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::V_UNITS % C::NTHR == 0 || u < C::V_UNITS) {
        const int q4 = u / C::KGR, c = u % C::KGR;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          vst[it][e] = *reinterpret_cast<const u32x4*>(vb + (4 * q4 + e) * D + 8 * c);
      }
    }
  };
  auto stash = [&](int stage) {
    uint16_t* kd = kbuf + stage * C::STAGE_ELEMS;
    uint16_t* vd = vbuf + stage * C::STAGE_ELEMS;
#pragma unroll
    for (int it = 0; it < C::K_IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::K_UNITS % C::NTHR == 0 || u < C::K_UNITS) {
        const int key = u / C::KGR, g = u % C::KGR;
        *reinterpret_cast<u32x4*>(kd + key * D + 8 * (g ^ (key & C::KSW))) = kst[it];
      }
    }
#pragma unroll
    for (int it = 0; it < C::V_IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::V_UNITS % C::NTHR == 0 || u < C::V_UNITS) {
        const int q4 = u / C::KGR, c = u % C::KGR;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int d = 8 * c + i;
          const int wd = i >> 1;
          u32x2 word;
          if (i & 1) {
            word[0] = hi_pair(vst[it][0][wd], vst[it][1][wd]);
            word[1] = hi_pair(vst[it][2][wd], vst[it][3][wd]);
          } else {
            word[0] = lo_pair(vst[it][0][wd], vst[it][1][wd]);
            word[1] = lo_pair(vst[it][2][wd], vst[it][3][wd]);
          }
          *reinterpret_cast<u32x2*>(vd + d * BS + 4 * (q4 ^ vswz(d, C::VGR))) = word;
        }
      }
    }
  };

  f32x16 o[C::NDT][C::NQT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < C::NQT; ++qt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][qt][r] = 0.0f;
  float mrow[C::NQT], lrow[C::NQT];
#pragma unroll
  for (int qt = 0; qt < C::NQT; ++qt) {
    mrow[qt] = -__builtin_inff();
    lrow[qt] = 0.0f;
  }
  const float qk_scale = a.qk_scale;

  auto block_id = [&](int i) {
    int id = __builtin_amdgcn_readfirstlane(irow[(int64_t)i * a.is[3]]);
    return id;
  };

  int cur = block_id(0);
  fetch(((unsigned)cur < (unsigned)a.nkb) ? cur : 0);
  stash(0);
  __syncthreads();

  for (int i = 0; i < count; ++i) {
    const int stage = i & 1;
    int nxt = 0;
    if (i + 1 < count) {
      nxt = block_id(i + 1);
      fetch(((unsigned)nxt < (unsigned)a.nkb) ? nxt : 0);
    }
    if ((unsigned)cur < (unsigned)a.nkb) {
      const uint16_t* kd = kbuf + stage * C::STAGE_ELEMS;
      const uint16_t* vd = vbuf + stage * C::STAGE_ELEMS;
      // S^T = K Q^T for this wave's key half.
      f32x16 sacc[C::NKT][C::NQT];
#pragma unroll
      for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
        for (int qt = 0; qt < C::NQT; ++qt)
#pragma unroll
          for (int r = 0; r < 16; ++r) sacc[kt][qt][r] = 0.0f;
#pragma unroll
      for (int s = 0; s < C::DS; ++s) {
        vec8 ka[C::NKT];
#pragma unroll
        for (int kt = 0; kt < C::NKT; ++kt) {
          const int key = C::KW * kh + 32 * kt + l32;
          const int g = 2 * s + hl;
          ka[kt] = __builtin_bit_cast(vec8, *reinterpret_cast<const u32x4*>(kd + key * D + 8 * (g ^ (key & C::KSW))));
        }
#pragma unroll
        for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
          for (int qt = 0; qt < C::NQT; ++qt) sacc[kt][qt] = E::mfma32(ka[kt], qf[qt][s], sacc[kt][qt]);
      }
      // Online softmax: lane owns query column l32 of each sub-tile; the other
      // half of the wave's keys for that query sits in lane ^ 32.
#pragma unroll
      for (int qt = 0; qt < C::NQT; ++qt) {
        float mx = sacc[0][qt][0];
#pragma unroll
        for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, sacc[kt][qt][r]);
        mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
        const float mnew = __builtin_fmaxf(mrow[qt], mx * qk_scale);
        const float alpha = __builtin_amdgcn_exp2f(mrow[qt] - mnew);
        mrow[qt] = mnew;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[dt][qt][r] *= alpha;
        float ls = 0.0f;
#pragma unroll
        for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][qt][r], qk_scale, -mnew));
            sacc[kt][qt][r] = pv;
            ls += pv;
          }
        lrow[qt] = lrow[qt] * alpha + ls;
      }
      // O^T += V^T P^T, one 16-key step at a time: the probabilities of a
      // step are packed to the element type right before their MFMAs.
#pragma unroll
      for (int st = 0; st < C::PST; ++st) {
        const int kt = st >> 1, ip = st & 1;
        vec8 pf[C::NQT];
#pragma unroll
        for (int qt = 0; qt < C::NQT; ++qt) {
          u32x4 pk;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            pk[e] = pack2(E::from_f32(sacc[kt][qt][8 * ip + 2 * e]), E::from_f32(sacc[kt][qt][8 * ip + 2 * e + 1]));
          pf[qt] = __builtin_bit_cast(vec8, pk);
        }
        const int ga = (C::KW * kh + 32 * kt + 16 * ip) / 4 + hl;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt) {
          const int d = 32 * dt + l32;
          const int sw = vswz(d, C::VGR);
          const uint16_t* vrow = vd + d * BS;
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + 4 * (ga ^ sw));
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 4 * ((ga + 2) ^ sw));
          const vec8 va = __builtin_bit_cast(vec8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
          for (int qt = 0; qt < C::NQT; ++qt) o[dt][qt] = E::mfma32(va, pf[qt], o[dt][qt]);
        }
      }
    }
    if (i + 1 < count) stash(stage ^ 1);
    __syncthreads();
    cur = nxt;
  }

  // Merge the two key halves (waves kh = 0 and kh = 1 of the same qh).
#pragma unroll
  for (int qt = 0; qt < C::NQT; ++qt) lrow[qt] += __shfl_xor(lrow[qt], 32);
  float* xo = reinterpret_cast<float*>(smem) + qh * (C::NDT * C::NQT * 16 * 64);
  float* xm = reinterpret_cast<float*>(smem) + C::X_FLOATS + qh * (2 * C::NQT * 64);
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int qt = 0; qt < C::NQT; ++qt)
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[((dt * C::NQT + qt) * 16 + r) * 64 + lane] = o[dt][qt][r];
#pragma unroll
    for (int qt = 0; qt < C::NQT; ++qt) {
      xm[(2 * qt) * 64 + lane] = mrow[qt];
      xm[(2 * qt + 1) * 64 + lane] = lrow[qt];
    }
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int qt = 0; qt < C::NQT; ++qt) {
      const float m1 = xm[(2 * qt) * 64 + lane], l1 = xm[(2 * qt + 1) * 64 + lane];
      const float mm = __builtin_fmaxf(mrow[qt], m1);
      const float a0 = __builtin_amdgcn_exp2f(mrow[qt] - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
      const float l = lrow[qt] * a0 + l1 * a1;
      const float inv = 1.0f / l;
      const int r = row0 + C::QW * qh + 32 * qt + l32;
      if (r < a.Lq) {
        uint16_t* orow = ohead + (int64_t)r * D;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            float val[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int rr = 4 * i4 + j;
              const float o1 = xo[((dt * C::NQT + qt) * 16 + rr) * 64 + lane];
              val[j] = (o[dt][qt][rr] * a0 + o1 * a1) * inv;
            }
            const u32x2 pk = {pack2(E::from_f32(val[0]), E::from_f32(val[1])),
                              pack2(E::from_f32(val[2]), E::from_f32(val[3]))};
            *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i4 + 4 * hl) = pk;
          }
        if (a.lse && hl == 0) a.lse[(int64_t)bh * a.Lq + r] = mm + __builtin_log2f(l);
      }
    }
  }
}

template <typename E, int BS, int D>
int launch_bsa(BsaArgs& a, int tiles, hipStream_t s) {
  clear_launch_error();
  hipLaunchKernelGGL((bsa_fwd_kernel<E, BS, D>), dim3(tiles), dim3(Cfg<BS, D>::NTHR), 0, s, a);
  return launch_status();
}

template <typename E>
int dispatch_bsa(BsaArgs& a, int bs, int D, int tiles, hipStream_t s) {
  if (bs == 128 && D == 128) return launch_bsa<E, 128, 128>(a, tiles, s);
  if (bs == 128 && D == 64) return launch_bsa<E, 128, 64>(a, tiles, s);
  if (bs == 64 && D == 128) return launch_bsa<E, 64, 128>(a, tiles, s);
  if (bs == 64 && D == 64) return launch_bsa<E, 64, 64>(a, tiles, s);
  return LI_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace li

using namespace li;

extern "C" int li_bsa_fwd(int dtype, int32_t B, int32_t NH, int32_t Lq, int32_t Lk, int32_t D, const void* q,
                          const void* k, const void* v, const int32_t* block_indices, const int64_t idx_strides[4],
                          int32_t n_cols, const int32_t* block_counts, const int64_t cnt_strides[3], float sm_scale,
                          int32_t block_size, void* out, float* lse, void* stream) {
  if (!q || !k || !v || !block_indices || !idx_strides || !block_counts || !cnt_strides || !out)
    return LI_ERR_INVALID_ARG;
  if (B <= 0 || NH <= 0 || Lq < 0 || Lk < 0 || D <= 0 || n_cols < 0 || block_size <= 0) return LI_ERR_INVALID_ARG;
  if (Lk % block_size != 0) return LI_ERR_K_LEN;
  if (dtype != LI_DTYPE_BF16 && dtype != LI_DTYPE_F16) return LI_ERR_UNSUPPORTED;
  if (!(block_size == 64 || block_size == 128) || !(D == 64 || D == 128)) return LI_ERR_UNSUPPORTED;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
       reinterpret_cast<uintptr_t>(out)) & 15u)
    return LI_ERR_INVALID_ARG;
  if (Lq == 0) return LI_OK;
  const int64_t nqt = (Lq + block_size - 1) / block_size;
  const int64_t tiles = nqt * B * NH;
  if (tiles > 0x7FFFFFFF) return LI_ERR_SHAPE;
  BsaArgs a = {};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.idx = block_indices;
  for (int i = 0; i < 4; ++i) a.is[i] = idx_strides[i];
  a.cnt = block_counts;
  for (int i = 0; i < 3; ++i) a.cs[i] = cnt_strides[i];
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.NH = NH;
  a.Lq = Lq;
  a.nkb = Lk / block_size;
  a.nqt = (int32_t)nqt;
  a.n_cols = n_cols;
  a.qk_scale = sm_scale * 1.44269504f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == LI_DTYPE_BF16) return dispatch_bsa<Bf16>(a, block_size, D, (int)tiles, s);
  return dispatch_bsa<F16>(a, block_size, D, (int)tiles, s);
}
