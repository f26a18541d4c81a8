// Block-sparse flash-attention forward, D = 128, 128-row query tiles, four
// waves per workgroup (one per SIMD), for gfx950.
//
// Same semantics as the 8-wave kernel in li_bsa_fwd.hip (which restates
// _attn_fwd_bsa_align, hy-worldplay/.../longcat_kernel.py:27-155); this file
// only changes how the work is laid out on the chip:
//
//  * wave w owns 64 query rows (qg = w >> 1) and one half of every kept key
//    block (kh = w & 1).  Each K operand of S^T = K Q^T and each V^T operand
//    of O^T = V^T P^T is read from LDS once and used by two MFMAs (the two
//    32-query tiles), which halves LDS reads per MFMA against the 8-wave
//    layout, where a wave owns 32 rows.
//  * with one wave per SIMD the softmax overlaps the MFMAs inside the wave.
//    A block is processed as two regions, one per 32-key tile kt of the
//    wave's key half: region kt issues the P V MFMAs of key tile kt of block
//    i and the S MFMAs of key tile kt of block i+1 (32 MFMAs), interleaved
//    with the exponentials of the other key tile (block i for kt = 0, block
//    i+1 for kt = 1).  Scores and probabilities of the two key tiles live in
//    separate registers, so the MFMA and VALU streams of a region are
//    independent.  Each region is one basic block.
//  * the exponentials use the running max as it stands; when a lane's
//    partial row sum exceeds 2^20 (this includes the first block, whose
//    running max is -inf) the wave raises the max, rescales O and l and redoes
//    that key tile's exponentials, between regions, where no MFMA is writing
//    O.  An out-of-range block id adds -inf to its scores (probability 0).
//  * K and V stages are loaded with direct-to-LDS DMA in the swizzled layouts
//    of the 8-wave kernel; stage i % 2 holds {V(i), K(i+1)}; the loads of the
//    next stage are spread over both regions and published by one barrier
//    per block.
#include "li_bsa_common.hpp"

namespace li {
namespace {

constexpr float kRescaleSum = 1048576.0f;  // 2^20

template <typename E>
__global__ __launch_bounds__(256) void bsa_fwd_w4_kernel(BsaArgs a) {
  constexpr int BS = 128, D = 128;
  constexpr int NQT = 2;     // 32-query MFMA tiles per wave
  constexpr int NKT = 2;     // 32-key tiles per wave per block
  constexpr int DS = 8;      // 16-wide d steps of S
  constexpr int NDT = 4;     // 32-wide d tiles of O
  constexpr int CPW = 8;     // 1 KiB chunks per wave per K or V block
  constexpr int LA = 3;      // operand pairs read ahead
  typedef typename E::vec8 vec8;
  typedef __attribute__((address_space(3))) void lds_void;
  __shared__ __attribute__((aligned(16))) char ks0[32 * 1088];
  __shared__ __attribute__((aligned(16))) char ks1[32 * 1088];
  __shared__ __attribute__((aligned(16))) char vs0[BS * 256];
  __shared__ __attribute__((aligned(16))) char vs1[BS * 256];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qg = wave >> 1, kh = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;

  // Work unit -> query tile, as in the 8-wave kernel.
  const int id = blockIdx.x;
  int tile, half = -1;
  if (id < a.n_full) {
    tile = unit_tile(a, id);
  } else {
    tile = a.n_full + ((id - a.n_full) >> 1);
    half = (id - a.n_full) & 1;
  }
  const int bh = tile / a.nqt, m = tile % a.nqt;
  const int b = bh / a.NH, h = bh % a.NH;
  const uint16_t* qhead = a.q + (int64_t)bh * a.Lq * D;
  const uint16_t* khead = a.k + (int64_t)bh * a.nkb * BS * D;
  const uint16_t* vhead = a.v + (int64_t)bh * a.nkb * BS * D;
  uint16_t* ohead = a.out + (int64_t)bh * a.Lq * D;
  const int32_t* irow = a.idx + b * a.is[0] + h * a.is[1] + (int64_t)m * a.is[2];
  int count = a.cnt[b * a.cs[0] + h * a.cs[1] + (int64_t)m * a.cs[2]];
  count = count < 0 ? 0 : (count > a.n_cols ? a.n_cols : count);
  count = __builtin_amdgcn_readfirstlane(count);
  if (half >= 0) {
    const int h0 = (count + 1) >> 1;
    irow += half ? (int64_t)h0 * a.is[3] : 0;
    count = half ? count - h0 : h0;
  }
  const int row0 = m * BS;
  float* part_o = half >= 0 ? a.part + (int64_t)(2 * (tile - a.n_full) + half) * BS * (D + 2) : nullptr;
  float* part_ml = half >= 0 ? part_o + BS * D : nullptr;

  if (count == 0) {
    if (half >= 0) {
      for (int u = tid; u < BS * D / 4; u += 256) reinterpret_cast<f32x4*>(part_o)[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      for (int r = tid; r < BS; r += 256) {
        part_ml[2 * r] = -__builtin_inff();
        part_ml[2 * r + 1] = 0.0f;
      }
      return;
    }
    for (int u = tid; u < BS * (D / 8); u += 256) {
      const int r = row0 + u / (D / 8);
      if (r < a.Lq) *reinterpret_cast<u32x4*>(ohead + (int64_t)r * D + 8 * (u % (D / 8))) = u32x4{0u, 0u, 0u, 0u};
    }
    if (a.lse)
      for (int r = tid; r < BS; r += 256)
        if (row0 + r < a.Lq) a.lse[(int64_t)bh * a.Lq + row0 + r] = -__builtin_inff();
    return;
  }

  // Q^T fragments of the wave's two query tiles.
  vec8 qf[NQT][DS];
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) {
    const int r = row0 + 64 * qg + 32 * qt + l32;
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (r < a.Lq) x = *reinterpret_cast<const u32x4*>(qhead + (int64_t)r * D + 16 * s + 8 * hl);
      qf[qt][s] = __builtin_bit_cast(vec8, x);
    }
  }

  // DMA lane offsets and LDS operand offsets (layouts of the 8-wave kernel,
  // with 64 keys per wave and block).
  const int rp = lane >> 4;
  const uint32_t k_src = 2u * (rp * D + 8 * ((lane & 15) ^ rp));
  const uint32_t v_src = 2u * (rp * D + 32 * (((lane & 15) >> 2) ^ rp) + 8 * (lane & 3));
  const int R = 64 * kh + kperm(l32);
  const int rc = R & 3;
  const int k_base = (R >> 2) * 1088 + rc * 256 + 16 * (hl ^ (rc & 1));
  const int k_off[2] = {k_base + 32 * (rc >> 1), k_base + 32 * (1 ^ (rc >> 1))};
  const int t16 = lane & 15, g16 = lane >> 4;
  const int v_base = (64 * kh + 8 * hl + (t16 >> 2)) * 256 + 32 * (g16 & 1) + 8 * (t16 & 3);
  int v_off[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) v_off[dt] = v_base + 64 * (dt ^ (t16 >> 2));

  auto lds_addr = [&](char* p) LI_INLINE { return (uint32_t)(uintptr_t)(lds_void*)p; };
  const uint32_t a_ks0 = lds_addr(ks0), a_ks1 = lds_addr(ks1), a_vs0 = lds_addr(vs0), a_vs1 = lds_addr(vs1);
  auto block_ptr = [&](const uint16_t* head, int blk) LI_INLINE {
    return reinterpret_cast<const char*>(head + (int64_t)blk * BS * D);
  };
  auto dma_v = [&](int j, const char* vb, uint32_t vd) LI_INLINE {
    const int c = wave * CPW + j;
    dma16(vb + 8 * c * D, v_src, vd + c * 1024);
  };
  auto dma_k = [&](int j, const char* kb, uint32_t kd) LI_INLINE {
    const int c = wave * CPW + j;
    dma16(kb + 8 * c * D, k_src, kd + c * 1088);
  };

  typedef __attribute__((address_space(4))) const int32_t const_i32;
  const_i32* irow_s = (const_i32*)irow;
  auto block_id = [&](int i) LI_INLINE { return irow_s[(int64_t)(i < count ? i : count - 1) * a.is[3]]; };
  auto valid = [&](int id_) LI_INLINE { return (unsigned)id_ < (unsigned)a.nkb; };
  auto safe = [&](int id_) LI_INLINE { return valid(id_) ? id_ : 0; };

  f32x16 o[NDT][NQT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][qt][r] = 0.0f;
  float mrow[NQT] = {-__builtin_inff(), -__builtin_inff()};
  float lrow[NQT] = {0.0f, 0.0f};
  const float qk_scale = a.qk_scale;
  f32x16 sacc[NKT][NQT];
  u32x4 ppk[NQT][4];  // [qt][st], 16-key step st = 2 kt + ip
  f32x16 zero16;
#pragma unroll
  for (int r = 0; r < 16; ++r) zero16[r] = 0.0f;

  // Operand p (0..15) of a region for key tile kt: p < 8 is the V^T tile
  // (dt, st) = (p & 3, 2 kt + (p >> 2)), p >= 8 the K tile of d step p - 8.
  auto read_op = [&](int p, int kt, const char* vc, const char* kc) LI_INLINE {
    if (p < 8) {
      const int dt = p & 3, st = 2 * kt + (p >> 2);
      const int ktt = st >> 1, ip = st & 1;
      const uint16_t* q = reinterpret_cast<const uint16_t*>(vc + v_off[dt] + (32 * ktt + 16 * ip) * 256);
      const u32x2 lo = lds_read_tr(q), hi = lds_read_tr(q + 4 * 128);
      return __builtin_bit_cast(vec8, u32x4{lo[0], lo[1], hi[0], hi[1]});
    }
    const int s = p - 8;
    return __builtin_bit_cast(vec8, *reinterpret_cast<const u32x4*>(kc + k_off[s & 1] + 8704 * kt + 64 * (s >> 1)));
  };
  // MFMA u (0..31) of a region for key tile kt, operand op = operand u >> 1.
  auto mfma_u = [&](int u, int kt, const vec8& op) LI_INLINE {
    const int p = u >> 1, qt = u & 1;
    if (p < 8) {
      const int dt = p & 3, st = 2 * kt + (p >> 2);
      o[dt][qt] = E::mfma32(op, __builtin_bit_cast(vec8, ppk[qt][st]), o[dt][qt]);
    } else {
      const int s = p - 8;
      sacc[kt][qt] = E::mfma32(op, qf[qt][s], s == 0 ? zero16 : sacc[kt][qt]);
    }
  };
  // Exponential step e (0..31) of key tile kt2: query tile qt = e >> 4,
  // 16-key step ip = (e >> 3) & 1, element e & 7.  Pairs are packed as they
  // complete.
  float pv[NQT][2][8];
  float ls[NQT];
  auto exp_step = [&](int e, int kt2, const float* bias) LI_INLINE {
    const int qt = e >> 4, ip = (e >> 3) & 1, el = e & 7;
    pv[qt][ip][el] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt2][qt][8 * ip + el], qk_scale, bias[qt]));
    if (el & 1) ppk[qt][2 * kt2 + ip][el >> 1] = cvt_pk<E>(pv[qt][ip][el - 1], pv[qt][ip][el]);
    if (el == 7) {
      const float* x = pv[qt][ip];
      const float s2 = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
      ls[qt] = ip == 0 ? s2 : ls[qt] + s2;
    }
  };
  auto exps_all = [&](int kt2, const float* bias) LI_INLINE {
#pragma unroll
    for (int e = 0; e < 32; ++e) exp_step(e, kt2, bias);
  };
  // Rare path for key tile kt2 of a valid block: raise the running max to the
  // tile's max, rescale O and l, redo the exponentials.
  auto rescale_redo = [&](int kt2) LI_INLINE {
    float bias[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      float mx = sacc[kt2][qt][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mx = __builtin_fmaxf(mx, sacc[kt2][qt][r]);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * qk_scale;
      const float mnew = __builtin_fmaxf(mrow[qt], mx);
      const float alpha = __builtin_amdgcn_exp2f(mrow[qt] - mnew);
      mrow[qt] = mnew;
      lrow[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][qt][r] *= alpha;
      bias[qt] = -mnew;
    }
    exps_all(kt2, bias);
  };
  // After the exponentials of key tile kt2 of block blk: rare path if needed,
  // then accumulate the row sums.
  auto finish_exps = [&](int kt2, int blk) LI_INLINE {
    if (valid(blk) && __ballot(!(ls[0] <= kRescaleSum && ls[1] <= kRescaleSum))) rescale_redo(kt2);
    if (valid(blk)) {
      lrow[0] += ls[0];
      lrow[1] += ls[1];
    }
  };
  auto bias_of = [&](int blk, float* bias) LI_INLINE {
    const bool v = valid(blk);
    bias[0] = v ? -mrow[0] : -__builtin_inff();
    bias[1] = v ? -mrow[1] : -__builtin_inff();
  };

  // One region: 32 MFMAs for key tile kt (P V of block i from vc, S of block
  // i+1 from kc) interleaved with the exponentials of key tile 1 - kt and
  // eight stage loads (loads(j), j = 0..7: one 1 KiB chunk per 4 MFMAs).
  auto region = [&](int kt, const char* vc, const char* kc, const float* bias, auto loads) LI_INLINE {
    vec8 ring[LA + 1];
#pragma unroll
    for (int p = 0; p < LA; ++p) ring[p] = read_op(p, kt, vc, kc);
#pragma unroll
    for (int u = 0; u < 32; ++u) {
      const int p = u >> 1;
      if ((u & 1) == 0 && p + LA < 16) ring[(p + LA) % (LA + 1)] = read_op(p + LA, kt, vc, kc);
      mfma_u(u, kt, ring[p % (LA + 1)]);
      exp_step(u, 1 - kt, bias);
      if ((u & 3) == 3) loads(u >> 2);
    }
  };

  // Prologue: K(0) -> ks1, V(0) -> vs0, K(1) -> ks0; S(0); exponentials of
  // key tile 0 of block 0.
  int id_c = block_id(0), id_n = block_id(1), id_nn = block_id(2);
  {
    const char* kb0 = block_ptr(khead, safe(id_c));
    const char* vb0 = block_ptr(vhead, safe(id_c));
    const char* kb1 = block_ptr(khead, safe(id_n));
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
      dma_k(j, kb0, a_ks1);
      dma_v(j, vb0, a_vs0);
      dma_k(j, kb1, a_ks0);
    }
    wait_vm0();
  }
  __syncthreads();
#pragma unroll
  for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
    for (int s = 0; s < DS; ++s) {
      const vec8 ka = __builtin_bit_cast(
          vec8, *reinterpret_cast<const u32x4*>(ks1 + k_off[s & 1] + 8704 * kt + 64 * (s >> 1)));
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) sacc[kt][qt] = E::mfma32(ka, qf[qt][s], s == 0 ? zero16 : sacc[kt][qt]);
    }
  {
    float bias[NQT];
    bias_of(id_c, bias);
    exps_all(0, bias);
    finish_exps(0, id_c);
  }
  // Every wave has read K(0) from ks1 before stage 1 is loaded over it.
  __syncthreads();

  // Block i: stage i % 2 holds {V(i), K(i+1)}; loads {V(i+1), K(i+2)} into the
  // other stage.
  auto cycle = [&](int i, const char* vc, const char* kc, uint32_t vn, uint32_t kn) LI_INLINE {
    const char* vb = block_ptr(vhead, safe(id_n));
    const char* kb = block_ptr(khead, safe(id_nn));
    float bias[NQT];
    bias_of(id_c, bias);
    region(0, vc, kc, bias, [&](int j) LI_INLINE { dma_v(j, vb, vn); });
    finish_exps(1, id_c);
    const bool more = i + 1 < count;
    bias_of(more ? id_n : -1, bias);
    region(1, vc, kc, bias, [&](int j) LI_INLINE { dma_k(j, kb, kn); });
    if (more) finish_exps(0, id_n);
    __builtin_amdgcn_sched_barrier(0);
    wait_vm0();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    id_c = id_n;
    id_n = id_nn;
    id_nn = block_id(i + 3);
  };
  for (int i = 0; i < count; i += 2) {
    cycle(i, vs0, ks0, a_vs1, a_ks1);
    if (i + 1 < count) cycle(i + 1, vs1, ks1, a_vs0, a_ks0);
  }

  // Merge the two key halves (waves kh = 0 and 1 of the same qg) through LDS.
#pragma unroll
  for (int qt = 0; qt < NQT; ++qt) lrow[qt] += __shfl_xor(lrow[qt], 32);
  float* xo = reinterpret_cast<float*>(qg == 0 ? ks0 : ks1);
  float* xm = reinterpret_cast<float*>(vs0) + qg * (4 * 64);
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
        for (int r = 0; r < 16; ++r) xo[((dt * NQT + qt) * 16 + r) * 64 + lane] = o[dt][qt][r];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      xm[(2 * qt) * 64 + lane] = mrow[qt];
      xm[(2 * qt + 1) * 64 + lane] = lrow[qt];
    }
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
      const float m1 = xm[(2 * qt) * 64 + lane], l1 = xm[(2 * qt + 1) * 64 + lane];
      const float mm = __builtin_fmaxf(mrow[qt], m1);
      const bool none = mm == -__builtin_inff();
      const float a0 = none ? 0.0f : __builtin_amdgcn_exp2f(mrow[qt] - mm);
      const float a1 = none ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
      const float l = lrow[qt] * a0 + l1 * a1;
      const int rt = 64 * qg + 32 * qt + l32;
      if (half >= 0) {
        float* prow = part_o + rt * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            f32x4 val;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int rr = 4 * i4 + j;
              val[j] = o[dt][qt][rr] * a0 + xo[((dt * NQT + qt) * 16 + rr) * 64 + lane] * a1;
            }
            *reinterpret_cast<f32x4*>(prow + 32 * dt + 8 * i4 + 4 * hl) = val;
          }
        if (hl == 0) {
          part_ml[2 * rt] = mm;
          part_ml[2 * rt + 1] = l;
        }
      } else if (row0 + rt < a.Lq) {
        const int r = row0 + rt;
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        uint16_t* orow = ohead + (int64_t)r * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            float val[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int rr = 4 * i4 + j;
              val[j] = (o[dt][qt][rr] * a0 + xo[((dt * NQT + qt) * 16 + rr) * 64 + lane] * a1) * inv;
            }
            const u32x2 pk = {cvt_pk<E>(val[0], val[1]), cvt_pk<E>(val[2], val[3])};
            *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i4 + 4 * hl) = pk;
          }
        if (a.lse && hl == 0) a.lse[(int64_t)bh * a.Lq + r] = none ? -__builtin_inff() : mm + __builtin_log2f(l);
      }
    }
  }
}

}  // namespace

int launch_bsa_w4(int dtype, BsaArgs& a, int units, hipStream_t s) {
  if (dtype == LI_DTYPE_BF16)
    hipLaunchKernelGGL(bsa_fwd_w4_kernel<Bf16>, dim3(units), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(bsa_fwd_w4_kernel<F16>, dim3(units), dim3(256), 0, s, a);
  return 0;
}

}  // namespace li
