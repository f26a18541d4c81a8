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
//    B operand without an LDS round trip.  The A operand reads K rows in the
//    order perm(i) (bits 2 and 3 of the row index swapped): the softmax does
//    not care about key order, and with it each lane's 8 probabilities of a
//    16-key MFMA step are 8 consecutive keys, so the matching V^T operand is
//    two transposing LDS reads of 4 consecutive keys each (below).
//  * K and V tiles are double-buffered in LDS in their natural [key][d]
//    layout: block i+1 is fetched into registers while block i is computed,
//    then copied to the other stage with 16-byte stores.  The V^T operand is
//    read with gfx950's transposing LDS load (ds_read_b64_tr_b16): in each
//    16-lane group, lane t supplies V[key0 + t/4][d0 + 4*(t%4) .. +3] and lane
//    u receives V[key0 + j][d0 + u] for j = 0..3, i.e. four consecutive keys
//    of its own d row; two such loads give the 8 keys of one MFMA step.
//    K rows are padded to D+8 elements and V rows to D+32, which makes the K
//    operand reads and the transposing V reads bank-conflict free (LDS serves
//    16 lanes of a 16-byte access, or four 64-byte row segments of a
//    transposing access, per clock) and keeps every LDS address a per-lane
//    base plus a constant offset.
//  * Rescaling is lazy: the running max used for the exponentials is only
//    raised (and O, l rescaled) when a row's block max exceeds it by more
//    than 8 in log2 units, so probabilities stay <= 2^8 and most blocks skip
//    the rescale.  The result is the same softmax.
//  * Workgroup ids are remapped so that each XCD (ids are dealt round-robin
//    over the 8 XCDs) processes a contiguous range of (head, tile) work and
//    the tiles of one head share that XCD's L2 for their K/V blocks.
#include <mutex>

#include "li_bsa_common.hpp"

namespace li {
namespace {

template <int BS, int D>
struct Cfg {
  static constexpr int WAVES = 2 * (BS / 32);
  static constexpr int NTHR = 64 * WAVES;
  static constexpr int KW = BS / 2;       // keys per wave per block
  static constexpr int NKT = KW / 32;     // 32-key sub-tiles per wave
  static constexpr int DS = D / 16;       // MFMA k-steps of S (over d)
  static constexpr int NDT = D / 32;      // 32-wide d tiles of O
  static constexpr int PST = KW / 16;     // MFMA k-steps of P V (over keys)
  static constexpr int KGR = D / 8;       // 16-byte granules per K row
  static constexpr int KP = D + 8;        // K row pitch (elements)
  static constexpr int VP = D + 32;       // V row pitch (elements)
  static constexpr int K_STAGE = BS * KP;
  static constexpr int V_STAGE = BS * VP;
  static constexpr int UNITS = BS * KGR;            // 16-byte loads per K (or V) block
  static constexpr int IT = (UNITS + NTHR - 1) / NTHR;
  static constexpr int KV_BYTES = 2 * (K_STAGE + V_STAGE) * 2;
  static constexpr int NQW = WAVES / 2;                      // query groups
  static constexpr int X_FLOATS = NQW * NDT * 16 * 64;       // epilogue O exchange
  static constexpr int X_BYTES = X_FLOATS * 4 + NQW * 2 * 64 * 4;
  static constexpr int LDS_BYTES = KV_BYTES > X_BYTES ? KV_BYTES : X_BYTES;
};

template <typename E, int BS, int D>
__global__ __launch_bounds__(4 * BS) void bsa_fwd_kernel(BsaArgs a) {
  using C = Cfg<BS, D>;
  typedef typename E::vec8 vec8;
  __shared__ __attribute__((aligned(16))) char smem[C::LDS_BYTES];
  uint16_t* kbuf = reinterpret_cast<uint16_t*>(smem);          // [2][BS][KP]
  uint16_t* vbuf = kbuf + 2 * C::K_STAGE;                       // [2][BS][VP]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qq = wave >> 1, kh = wave & 1;
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
  vec8 qf[C::DS];
  {
    const int r = row0 + 32 * qq + l32;
#pragma unroll
    for (int s = 0; s < C::DS; ++s) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (r < a.Lq) x = *reinterpret_cast<const u32x4*>(qhead + (int64_t)r * D + 16 * s + 8 * hl);
      qf[s] = __builtin_bit_cast(vec8, x);
    }
  }

  // Per-lane LDS element offsets (stage 0); stage 1 adds K_STAGE / V_STAGE.
  int k_rd[C::NKT];
#pragma unroll
  for (int kt = 0; kt < C::NKT; ++kt) k_rd[kt] = (C::KW * kh + 32 * kt + kperm(l32)) * C::KP + 8 * hl;
  // Transposing V read: lane t of each 16-lane group g points at key
  // (KW*kh + 8*hl + t/4) and d = 16*(g&1) + 4*(t%4) of the block.
  const int t16 = lane & 15, g16 = lane >> 4;
  const int v_tr = (C::KW * kh + 8 * hl + (t16 >> 2)) * C::VP + 16 * (g16 & 1) + 4 * (t16 & 3);

  u32x4 kst[C::IT];
  u32x4 vst[C::IT];
  auto fetch_k = [&](int blk) {
    const uint16_t* kb = khead + (int64_t)blk * BS * D;
#pragma unroll
    for (int it = 0; it < C::IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::UNITS % C::NTHR == 0 || u < C::UNITS)
        kst[it] = *reinterpret_cast<const u32x4*>(kb + (u / C::KGR) * D + 8 * (u % C::KGR));
    }
  };
  auto fetch_v = [&](int blk) {
    const uint16_t* vb = vhead + (int64_t)blk * BS * D;
#pragma unroll
    for (int it = 0; it < C::IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::UNITS % C::NTHR == 0 || u < C::UNITS)
        vst[it] = *reinterpret_cast<const u32x4*>(vb + (u / C::KGR) * D + 8 * (u % C::KGR));
    }
  };
  auto stash_k = [&](auto stage) {
    uint16_t* kd = kbuf + decltype(stage)::value * C::K_STAGE;
#pragma unroll
    for (int it = 0; it < C::IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::UNITS % C::NTHR == 0 || u < C::UNITS)
        *reinterpret_cast<u32x4*>(kd + (u / C::KGR) * C::KP + 8 * (u % C::KGR)) = kst[it];
    }
  };
  auto stash_v = [&](auto stage) {
    uint16_t* vd = vbuf + decltype(stage)::value * C::V_STAGE;
#pragma unroll
    for (int it = 0; it < C::IT; ++it) {
      const int u = tid + C::NTHR * it;
      if (C::UNITS % C::NTHR == 0 || u < C::UNITS)
        *reinterpret_cast<u32x4*>(vd + (u / C::KGR) * C::VP + 8 * (u % C::KGR)) = vst[it];
    }
  };

  f32x16 o[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
  float mrow = -__builtin_inff(), lrow = 0.0f;
  const float qk_scale = a.qk_scale;

  // S^T = K Q^T of one block for this wave's key half.
  auto scores = [&](auto stage, f32x16* sacc) {
    const uint16_t* kd = kbuf + decltype(stage)::value * C::K_STAGE;
#pragma unroll
    for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.0f;
#pragma unroll
    for (int s = 0; s < C::DS; ++s) {
#pragma unroll
      for (int kt = 0; kt < C::NKT; ++kt) {
        const vec8 ka = __builtin_bit_cast(vec8, *reinterpret_cast<const u32x4*>(kd + k_rd[kt] + 16 * s));
        sacc[kt] = E::mfma32(ka, qf[s], sacc[kt]);
      }
    }
  };
  // Online softmax of one block, in two parts so that the next block's score
  // MFMAs can be issued between them (same basic block as the exponentials).
  // The lane owns query column l32; the other half of the wave's keys for
  // that query sits in lane ^ 32, reached with v_permlane32_swap.
  auto softmax_max = [&](f32x16* sacc) {
    float mx = sacc[0][0];
#pragma unroll
    for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, sacc[kt][r]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * qk_scale;
    if (__ballot(mx > mrow + 8.0f)) {
      const float mnew = __builtin_fmaxf(mrow, mx);
      const float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
      mrow = mnew;
      lrow *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
    }
  };
  // Probabilities overwrite the scores.  mrow is still -inf only when every
  // block so far was skipped (all scores -inf): the offset 0 keeps exp2 at 0.
  auto softmax_exp = [&](f32x16* sacc) {
    const float moff = mrow == -__builtin_inff() ? 0.0f : mrow;
    float ls = 0.0f;
#pragma unroll
    for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][r], qk_scale, -moff));
        sacc[kt][r] = pv;
        ls += pv;
      }
    lrow += ls;
  };
  // O^T += V^T P^T, one 16-key step at a time.
  auto pv_update = [&](auto stage, f32x16* sacc) {
    const uint16_t* vd = vbuf + decltype(stage)::value * C::V_STAGE;
#pragma unroll
    for (int st = 0; st < C::PST; ++st) {
      const int kt = st >> 1, ip = st & 1;
      u32x4 pk;
#pragma unroll
      for (int e = 0; e < 4; ++e) pk[e] = cvt_pk<E>(sacc[kt][8 * ip + 2 * e], sacc[kt][8 * ip + 2 * e + 1]);
      const vec8 pf = __builtin_bit_cast(vec8, pk);
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        const uint16_t* pv = vd + v_tr + (32 * kt + 16 * ip) * C::VP + 32 * dt;
        const u32x2 lo = lds_read_tr(pv);               // keys +0..3 of the step's 8
        const u32x2 hi = lds_read_tr(pv + 4 * C::VP);   // keys +4..7
        const vec8 va = __builtin_bit_cast(vec8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        o[dt] = E::mfma32(va, pf, o[dt]);
      }
    }
  };

  auto block_id = [&](int i) { return __builtin_amdgcn_readfirstlane(irow[(int64_t)i * a.is[3]]); };
  auto valid = [&](int id_) { return (unsigned)id_ < (unsigned)a.nkb; };
  auto safe = [&](int id_) { return valid(id_) ? id_ : 0; };

  // Software pipeline, one kept block per step i (K runs one block ahead of V):
  //   fetch K(i+2), V(i+1) into registers;
  //   row max of S(i) (and a rare rescale), then S(i+1) = K(i+1) Q^T on the
  //   MFMA pipe interleaved with the exponentials of S(i) on the VALU;
  //   O += V(i)^T P(i);
  //   write K(i+2) into K's stage i%2 and V(i+1) into V's stage (i+1)%2; barrier.
  // Stage i%2 of K held K(i), last read in step i-1 (hence the barrier after
  // the prologue's S(0)); V's stage (i+1)%2 held V(i-1), last read in step i-1.
  // The step has no branch besides the rescale test: past the last block the
  // prefetch repeats the last block (indices stay in range) and S(i+1) is
  // computed on a stale stage and never used.  A block id out of range is
  // loaded as block 0 and skipped through -inf scores.
  f32x16 sa[C::NKT], sb[C::NKT];
  const int id0 = block_id(0);
  const int id1 = block_id(count > 1 ? 1 : 0);
  fetch_k(safe(id0));
  fetch_v(safe(id0));
  stash_k(Stage<0>{});
  stash_v(Stage<0>{});
  fetch_k(safe(id1));
  stash_k(Stage<1>{});
  __syncthreads();
  scores(Stage<0>{}, sa);
  __syncthreads();

  auto step = [&](auto stage, int i, int& cur, int& nxt, f32x16* s_cur, f32x16* s_nxt) {
    constexpr int ST = decltype(stage)::value;
    const int nn = block_id(i + 2 < count ? i + 2 : count - 1);
    fetch_k(safe(nn));
    fetch_v(safe(nxt));
    if (!valid(cur)) {
#pragma unroll
      for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) s_cur[kt][r] = -__builtin_inff();
    }
    softmax_max(s_cur);
    scores(Stage<ST ^ 1>{}, s_nxt);
    softmax_exp(s_cur);
    pv_update(stage, s_cur);
    stash_k(stage);
    stash_v(Stage<ST ^ 1>{});
    __syncthreads();
    cur = nxt;
    nxt = nn;
  };
  int cur = id0, nxt = id1;
  for (int i = 0; i < count; i += 2) {
    step(Stage<0>{}, i, cur, nxt, sa, sb);
    if (i + 1 < count) step(Stage<1>{}, i + 1, cur, nxt, sb, sa);
  }

  // Merge the two key halves (waves kh = 0 and kh = 1 of the same qq).
  lrow += __shfl_xor(lrow, 32);
  float* xo = reinterpret_cast<float*>(smem) + qq * (C::NDT * 16 * 64);
  float* xm = reinterpret_cast<float*>(smem) + C::X_FLOATS + qq * (2 * 64);
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) xo[(dt * 16 + r) * 64 + lane] = o[dt][r];
    xm[lane] = mrow;
    xm[64 + lane] = lrow;
  }
  __syncthreads();
  if (kh == 0) {
    const float m1 = xm[lane], l1 = xm[64 + lane];
    const float mm = __builtin_fmaxf(mrow, m1);
    const float a0 = __builtin_amdgcn_exp2f(mrow - mm), a1 = __builtin_amdgcn_exp2f(m1 - mm);
    const float l = lrow * a0 + l1 * a1;
    const float inv = 1.0f / l;
    const int r = row0 + 32 * qq + l32;
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
            const float o1 = xo[(dt * 16 + rr) * 64 + lane];
            val[j] = (o[dt][rr] * a0 + o1 * a1) * inv;
          }
          const u32x2 pk = {cvt_pk<E>(val[0], val[1]), cvt_pk<E>(val[2], val[3])};
          *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i4 + 4 * hl) = pk;
        }
      if (a.lse && hl == 0) a.lse[(int64_t)bh * a.Lq + r] = mm + __builtin_log2f(l);
    }
  }
}

// ---------------------------------------------------------------------------
// D = 128 variant with direct-to-LDS block loads (global_load_lds_dwordx4).
//
// Each wave-wide DMA instruction writes 1 KiB of LDS at consecutive 16-byte
// slots, one per lane; the layout is chosen through each lane's global
// address:
//  * K stage: 4-row chunks of 1 KiB at a 1088-byte pitch; row r of a chunk
//    at +256 r, its 16-byte granule g at slot g ^ r.  The b128 operand reads
//    of 16 rows kperm(i) then hit 16 distinct bank windows, and a lane's
//    address for MFMA step s is one of two per-lane bases plus 64*(s/2).
//  * V stage: 256-byte rows; the 64-byte granule q of row r at q ^ (r % 4).
//    Each transposing read covers 4 consecutive rows, which then occupy the
//    4 distinct 64-byte bank windows.
// Block i+1 is loaded into the other stage while block i is computed; the
// barrier at the end of a step (which waits for all of the wave's loads)
// publishes it.  No staging registers, no LDS store instructions.
template <int BS>
struct DmaCfg {
  static constexpr int D = 128;
  static constexpr int WAVES = 2 * (BS / 32);
  static constexpr int NTHR = 64 * WAVES;
  static constexpr int KW = BS / 2;
  static constexpr int NKT = KW / 32;
  static constexpr int DS = D / 16;
  static constexpr int NDT = D / 32;
  static constexpr int PST = KW / 16;
  static constexpr int CHUNKS = BS / 4;                // 1 KiB chunks per K (or V) block
  static constexpr int CPW = CHUNKS / WAVES;           // chunks per wave
  static constexpr int K_STAGE_BYTES = CHUNKS * 1088;
  static constexpr int V_STAGE_BYTES = BS * 256;
  static constexpr int NQW = WAVES / 2;
};

// Scheduling pins of an M phase (one basic block): the operand reads of the
// first LA MFMAs, then per MFMA u: the MFMA and the reads of MFMA u + LA (two
// transposing reads for a P V step, RS 16-byte reads for an S step).
template <int NPV, int RS, int U, int END>
__device__ __forceinline__ void sched_first_reads() {
  if constexpr (U < END) {
    __builtin_amdgcn_sched_group_barrier(0x100, U < NPV ? 2 : RS, 0);
    sched_first_reads<NPV, RS, U + 1, END>();
  }
}
template <int NPV, int RS, int NU, int LA, int U>
__device__ __forceinline__ void sched_m_units() {
  if constexpr (U < NU) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (U + LA < NU) __builtin_amdgcn_sched_group_barrier(0x100, U + LA < NPV ? 2 : RS, 0);
    sched_m_units<NPV, RS, NU, LA, U + 1>();
  }
}
// RS: LDS reads per S MFMA (one 16-byte read for 16-bit K, two for e4m3).
template <int NPV, int RS, int NU, int LA>
__device__ __forceinline__ void sched_m_phase() {
  sched_first_reads<NPV, RS, 0, LA>();
  sched_m_units<NPV, RS, NU, LA, 0>();
}

// F8: Q and K are e4m3 codes with one fp32 scale per tile (BsaArgs::q_scale,
// k_scale) and S^T = K Q^T is taken with the 32x32x64 e4m3 MFMA (four per
// block and wave instead of sixteen); the block's score scale
// qk_scale * q_scale * k_scale[blk] enters the softmax, and P V stays in
// 16-bit.  Q and K are always tiled (text blocks included); with G, V is
// read and O written in token order.  The e4m3 K stage has 128-byte rows with no padding: the 16-byte
// granule g of row r sits at slot g ^ ((r >> 1) & 7), so the 16 rows a
// 16-lane group reads (any 16 aligned rows) fall in 16 distinct bank windows.
// DN (dense calls, token-order addressing only): no index lists, every tile
// keeps blocks 0 .. n_cols - 1; queries and keys past the token bounds are
// skipped, and the padding rows of the last text and visual blocks score -inf.
// ZR (with G): the zero-region load path (BsaArgs::zero_region, gen_pairs).
template <typename E, int BS, bool G = false, bool F8 = false, bool DN = false, bool ZR = false>
__global__ __launch_bounds__(4 * BS) void bsa_fwd_dma_kernel(BsaArgs a) {
  using C = DmaCfg<BS>;
  static_assert(!G || BS == 128, "token-order addressing is built for 128-row tiles");
  static_assert(!F8 || BS == 128, "the e4m3 kernel is built for 128-row blocks");
  static_assert(!DN || (G && !F8), "dense calls use token-order addressing and 16-bit keys");
  constexpr int D = 128;
  typedef typename E::vec8 vec8;
  typedef __attribute__((address_space(3))) void lds_void;
  constexpr int KSB = F8 ? BS * D : C::K_STAGE_BYTES;  // bytes of a K stage
  // Separate arrays per stage let the compiler see that a load into one stage
  // never aliases the reads of the other.
  __shared__ __attribute__((aligned(16))) char ks0[KSB];
  __shared__ __attribute__((aligned(16))) char ks1[KSB];
  __shared__ __attribute__((aligned(16))) char vs0[C::V_STAGE_BYTES];
  __shared__ __attribute__((aligned(16))) char vs1[C::V_STAGE_BYTES];
  // The epilogue's O exchange goes to the K stages, or to the V stages for F8.
  static_assert(F8 || C::NQW / 2 * C::NDT * 16 * 64 * 4 <= C::K_STAGE_BYTES, "epilogue exchange must fit a K stage");
  static_assert(!F8 || C::NQW / 2 * C::NDT * 16 * 64 * 4 <= C::V_STAGE_BYTES, "epilogue exchange must fit a V stage");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int qq = wave >> 1, kh = wave & 1;
  const int l32 = lane & 31, hl = lane >> 5;

  // Work unit -> query tile: unit_tile gives each XCD (ids are dealt
  // round-robin over the 8 XCDs) a contiguous range of tiles; with the tail
  // split, the last slots of an XCD run the halves of its split tiles
  // (`half` = which half, `pslot` = its partial slot).
  const int id = blockIdx.x;
  int tile, half = -1, pslot = 0;
  if (a.xsplit == 0 || (id >> 3) < a.xtiles - a.xsplit) {
    tile = unit_tile(a, id);
  } else {
    const int x = id & 7;
    int j = (id >> 3) - (a.xtiles - a.xsplit);
    half = j >= a.xsplit ? 1 : 0;
    j -= half ? a.xsplit : 0;
    tile = x * a.xtiles + (a.xtiles - a.xsplit) + j;
    pslot = 2 * (x * a.xsplit + j) + half;
  }
  const int bh = tile / a.nqt, m = tile % a.nqt;
  const int b = bh / a.NH, h = bh % a.NH;

  const uint16_t* qhead = a.q + (int64_t)bh * a.Lq * D;
  const uint16_t* vhead = a.v + (int64_t)bh * a.nkb * BS * D;
  uint16_t* ohead = a.out + (int64_t)bh * a.Lq * D;
  constexpr int KEB = F8 ? 1 : 2;  // bytes per K element
  const char* kbytes = reinterpret_cast<const char*>(a.k) + (int64_t)bh * a.nkb * BS * D * KEB;
  const int row0 = m * BS;

  // Q^T fragments first: their loads depend on the tile alone, so they go
  // out together with the loads of the count and the first block ids below.
  // Lanes without a query row read row 0 of the head and keep zeros, which
  // keeps the loads free of branches.
  vec8 qf[C::DS];
  // e4m3 Q^T fragments: lane holds query row l32 and bytes 64 s + 32 hl .. +31.
  i32x8 qf8[2];
  float qk_scale = a.qk_scale;
  if constexpr (F8) {
    const int r = row0 + 32 * qq + l32;
    const bool ok = r < a.Lq;
    const char* qrow8 = reinterpret_cast<const char*>(a.q) + ((int64_t)bh * a.Lq + (ok ? r : 0)) * D;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u32x4 lo = *reinterpret_cast<const u32x4*>(qrow8 + 64 * s + 32 * hl);
      u32x4 hi = *reinterpret_cast<const u32x4*>(qrow8 + 64 * s + 32 * hl + 16);
      if (!ok) lo = hi = u32x4{0u, 0u, 0u, 0u};
      qf8[s] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
    typedef __attribute__((address_space(4))) const float const_f32;
    qk_scale *= ((const_f32*)a.q_scale)[(int64_t)bh * a.nqt + m];
  } else {
    const uint16_t* qrow;
    bool ok;
    if constexpr (G) {
      const int32_t l = tile_token(a.g, a.g.Tq, m, 32 * qq + l32, ok);
      ok = ok && (!DN || l < a.g.q_tokens);
      qrow = a.q + b * a.g.qs[0] + h * a.g.qs[1] + (int64_t)(ok ? l : 0) * a.g.qs[2];
    } else {
      const int r = row0 + 32 * qq + l32;
      ok = r < a.Lq;
      qrow = qhead + (int64_t)(ok ? r : 0) * D;
    }
#pragma unroll
    for (int s = 0; s < C::DS; ++s) {
      u32x4 x = *reinterpret_cast<const u32x4*>(qrow + 16 * s + 8 * hl);
      if (!ok) x = u32x4{0u, 0u, 0u, 0u};
      qf[s] = __builtin_bit_cast(vec8, x);
    }
  }

  // Dense calls: tile m keeps blocks 0 .. n_cols - 1, ids id_base + i.
  typedef __attribute__((address_space(4))) const int32_t const_i32;
  const int32_t* irow = DN ? nullptr : a.idx + b * a.is[0] + h * a.is[1] + (int64_t)m * a.is[2];
  // The first four entries of the row (clamped to its columns), read through
  // the scalar cache without waiting for the count, which picks among them;
  // the second half of a split tile reads its own after the count.
  int r0 = -1, r1 = -1, r2 = -1, r3 = -1;
  auto read_first = [&](const int32_t* row, int ncols) LI_INLINE {
    const const_i32* rs = (const const_i32*)row;
    const int64_t is3 = a.is[3];
    r0 = rs[0];
    r1 = rs[(int64_t)(1 < ncols ? 1 : ncols - 1) * is3];
    r2 = rs[(int64_t)(2 < ncols ? 2 : ncols - 1) * is3];
    r3 = rs[(int64_t)(3 < ncols ? 3 : ncols - 1) * is3];
  };
  if (!DN && half != 1 && a.n_cols > 0) read_first(irow, a.n_cols);
  const int32_t* cnt_at = DN ? nullptr : a.cnt + b * a.cs[0] + h * a.cs[1] + (int64_t)m * a.cs[2];
  int count = DN ? a.n_cols : *cnt_at;
  count = count < 0 ? 0 : (count > a.n_cols ? a.n_cols : count);
  count = __builtin_amdgcn_readfirstlane(count);
  int id_base = 0;
  if (half >= 0) {
    const int h0 = (count + 1) >> 1;
    if constexpr (!DN) irow += half ? (int64_t)h0 * a.is[3] : 0;
    id_base = half ? h0 : 0;
    count = half ? count - h0 : h0;
    if (!DN && half == 1 && a.n_cols - h0 > 0) read_first(irow, a.n_cols - h0);
  }
  // An empty list (or an empty half of a split tile) runs as one block with
  // an out-of-range id, which gets all-zero probabilities: the epilogue then
  // writes zero rows and an LSE of -inf (zero partials and (m, l) = (-inf, 0)
  // for a half), with no early exit to hold back the loads above.
  const bool empty = count == 0;
  count = empty ? 1 : count;
  // Partial rows of a split unit: O as [128 rows][128 d] fp32, then (m, l).
  float* part_o = half >= 0 ? a.part + (int64_t)pslot * BS * (D + 2) : nullptr;
  float* part_ml = half >= 0 ? part_o + BS * D : nullptr;

  // Output row of tile row rt, or null when it is not stored (past Lq, or
  // outside the token grid on the fused path).
  auto out_row = [&](int rt) LI_INLINE -> uint16_t* {
    if constexpr (G) {
      bool ok;
      const int32_t l = tile_token(a.g, a.g.Tq, m, rt, ok);
      return ok && (!DN || l < a.g.q_tokens) ? a.out + b * a.g.os[0] + h * a.g.os[1] + (int64_t)l * a.g.os[2]
                                             : nullptr;
    } else {
      return row0 + rt < a.Lq ? ohead + (int64_t)(row0 + rt) * D : nullptr;
    }
  };

  // DMA source byte offsets of this lane within a chunk; the chunk base is
  // wave-uniform (scalar registers), so each load is base + constant lane
  // offset with no per-load vector address arithmetic.
  const int rp = lane >> 4;
  const uint32_t k_src = 2u * (rp * D + 8 * ((lane & 15) ^ rp));
  const uint32_t v_src = 2u * (rp * D + 32 * (((lane & 15) >> 2) ^ rp) + 8 * (lane & 3));
  // Fused path: the same granules, with the rows of a chunk one token stride
  // apart in the untiled visual K / V.
  uint32_t k_src_vis = 0, v_src_vis = 0;
  if constexpr (G) {
    k_src_vis = (uint32_t)(rp * a.g.ks[2] * 2) + 16u * ((lane & 15) ^ rp);
    v_src_vis = (uint32_t)(rp * a.g.vs[2] * 2) + 2u * (32 * (((lane & 15) >> 2) ^ rp) + 8 * (lane & 3));
  }
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  // e4m3 K: a 1 KiB chunk is 8 rows of 128 bytes; lane t fills slot t % 8 of
  // row t / 8 with the row's granule (t % 8) ^ ((row >> 1) & 7), which for
  // chunk c is (t % 8) ^ (t / 16) ^ 4 (c % 2).
  uint32_t k8_src[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) k8_src[p] = (lane >> 3) * 128 + 16 * ((lane & 7) ^ (lane >> 4) ^ (4 * p));

  // K operand byte offsets: row R = KW*kh + kperm(l32) (+32 kt), granule 2s+hl.
  const int R = C::KW * kh + kperm(l32);
  const int rc = R & 3;
  const int k_base = (R >> 2) * 1088 + rc * 256 + 16 * (hl ^ (rc & 1));
  const int k_off[2] = {k_base + 32 * (rc >> 1), k_base + 32 * (1 ^ (rc >> 1))};
  // e4m3 K operand of step s (64 deep): granules 4 s + 2 hl and +1 of row R
  // (+32 kt rows = 4096 bytes).
  int k8_off[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int e = 0; e < 2; ++e) k8_off[s][e] = R * 128 + 16 * ((4 * s + 2 * hl + e) ^ ((R >> 1) & 7));
  // V^T operand byte offsets for the transposing reads, one per 32-wide d tile.
  const int t16 = lane & 15, g16 = lane >> 4;
  const int v_base = (C::KW * kh + 8 * hl + (t16 >> 2)) * 256 + 32 * (g16 & 1) + 8 * (t16 & 3);
  int v_off[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt) v_off[dt] = v_base + 64 * (dt ^ (t16 >> 2));

  f32x16 o[C::NDT];
#pragma unroll
  for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.0f;
  float mrow = -__builtin_inff(), lrow = 0.0f;
  // Score scale of the current block: qk_scale (times the tile's Q scale for
  // F8); for F8 also times the block's K scale, set before each softmax.
  const float qk_base = qk_scale;

  // Score tile S^T = K Q^T of one block (this wave's key half).
  f32x16 sacc[C::NKT];
  auto read_k8 = [&](const char* kd, int s, int kt) LI_INLINE {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(kd + k8_off[s][0] + 4096 * kt);
    const u32x4 hi = *reinterpret_cast<const u32x4*>(kd + k8_off[s][1] + 4096 * kt);
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  auto scores = [&](const char* kd) LI_INLINE {
    f32x16 z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.0f;
    if constexpr (F8) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int kt = 0; kt < C::NKT; ++kt) sacc[kt] = mfma_e4m3(read_k8(kd, s, kt), qf8[s], s == 0 ? z : sacc[kt]);
      return;
    }
#pragma unroll
    for (int s = 0; s < C::DS; ++s) {
#pragma unroll
      for (int kt = 0; kt < C::NKT; ++kt) {
        const vec8 ka = __builtin_bit_cast(
            vec8, *reinterpret_cast<const u32x4*>(kd + k_off[s & 1] + 8704 * kt + 64 * (s >> 1)));
        sacc[kt] = E::mfma32(ka, qf[s], s == 0 ? z : sacc[kt]);
      }
    }
  };
  // Online softmax of the scores in sacc; the probabilities are packed to the
  // element type into ppk (one u32x4 per 16-key MFMA step).
  //
  // The exponentials are taken against the running max mrow as it stands.
  // Only when a lane's partial row sum exceeds 2^20 (some score above mrow + 20
  // in log2 units; this includes the first block, where mrow = -inf, and
  // non-finite scores) does the wave take the slow path: block max across
  // both half-waves, raise mrow, rescale O and l, redo the exponentials.  So
  // probabilities stay below 2^20 (O, l and the bf16 P far from overflow) and
  // the block max is not computed at all on the common path; the result is
  // the same softmax.
  u32x4 ppk[C::PST];
  auto exps = [&](float off) LI_INLINE {
    float ls = 0.0f;
#pragma unroll
    for (int st = 0; st < C::PST; ++st) {
      const int kt = st >> 1, ip = st & 1;
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][8 * ip + e], qk_scale, -off));
      float s2 = (pv[0] + pv[1]) + (pv[2] + pv[3]);
      float s3 = (pv[4] + pv[5]) + (pv[6] + pv[7]);
      ls += s2 + s3;
#pragma unroll
      for (int e = 0; e < 4; ++e) ppk[st][e] = cvt_pk<E>(pv[2 * e], pv[2 * e + 1]);
    }
    return ls;
  };
  // A lane whose keys so far all scored -inf (keys masked on dense calls)
  // keeps mrow = -inf, l = 0 and O = 0: the slow path then takes its
  // exponentials against 0 instead (all zero), never against -inf.
  auto softmax = [&]() LI_INLINE {
    float ls = exps(mrow);
    if (__ballot(!(ls <= 1048576.0f))) {
      float mx = sacc[0][0];
#pragma unroll
      for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, sacc[kt][r]);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * qk_scale;
      const float mnew = __builtin_fmaxf(mrow, mx);
      const float msafe = mnew == -__builtin_inff() ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(mrow - msafe);
      mrow = mnew;
      lrow *= alpha;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
      ls = exps(msafe);
    }
    lrow += ls;
  };
  // The softmax of a tile's first block (mrow = -inf, l = 0, O = 0), which
  // always takes the slow path above: the block max first, then one set of
  // exponentials; O and l need no rescale.  The same values as softmax().
  auto softmax_first = [&]() LI_INLINE {
    float mx = sacc[0][0];
#pragma unroll
    for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, sacc[kt][r]);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = __builtin_fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * qk_scale;
    const float mnew = __builtin_fmaxf(mrow, mx);
    const float msafe = mnew == -__builtin_inff() ? 0.0f : mnew;
    mrow = mnew;
    lrow = exps(msafe);
  };
  // O^T += V^T P^T.
  auto pv_update = [&](const char* vd) LI_INLINE {
#pragma unroll
    for (int st = 0; st < C::PST; ++st) {
      const int kt = st >> 1, ip = st & 1;
      const vec8 pf = __builtin_bit_cast(vec8, ppk[st]);
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt) {
        const uint16_t* pv = reinterpret_cast<const uint16_t*>(vd + v_off[dt] + (32 * kt + 16 * ip) * 256);
        const u32x2 lo = lds_read_tr(pv);
        const u32x2 hi = lds_read_tr(pv + 4 * 128);
        o[dt] = E::mfma32(__builtin_bit_cast(vec8, u32x4{lo[0], lo[1], hi[0], hi[1]}), pf, o[dt]);
      }
    }
  };

  // Block ids are wave-uniform: read them through the scalar cache.
  const_i32* irow_s = (const_i32*)irow;
  auto block_id = [&](int i) LI_INLINE {
    const int j = i < count ? i : count - 1;
    if constexpr (DN)
      return empty ? -1 : id_base + j;
    else
      return empty ? -1 : (int)irow_s[(int64_t)j * a.is[3]];
  };
  auto valid = [&](int id_) LI_INLINE { return (unsigned)id_ < (unsigned)a.nkb; };
  auto safe = [&](int id_) LI_INLINE { return valid(id_) ? id_ : 0; };

  if constexpr (C::WAVES == 8) {
    // Ping-pong schedule.  Waves 0-3 (group 0) and 4-7 (group 1) share the
    // four SIMDs pairwise (wave w and w+4 on one SIMD), and group 1 runs one
    // phase behind group 0.  Phases alternate between an MFMA phase
    // M(i) = {O += V(i)^T P(i); S(i+1) = K(i+1) Q^T} and a VALU phase
    // X(i) = softmax(i) -> P(i), so in every slot one wave of a SIMD issues
    // MFMAs while the other runs its softmax:
    //   slot 0      : g0 S(0) X(0)      | g1 S(0)
    //   slot 2i+1   : g0 M(i)           | g1 X(i)
    //   slot 2i+2   : g0 X(i+1)         | g1 M(i)
    // Every wave runs the same sequence S(0) X(0) | M(0) | X(1) | M(1) | ...
    // with a barrier between phases; group 1 takes one extra barrier before
    // X(0) and group 0 one after its last phase, which sets the offset.
    //
    // LDS stage j (= i % 2) holds {V(i), K(i+1)}; K(0) sits in ks1 until
    // slot 1.  Group 0 alone loads the stages: during its M(i) (slot 2i+1,
    // after every read of the stage being replaced completed in slot 2i) it
    // issues one 1 KiB DMA per two MFMAs for {V(i+1), K(i+2)}, and waits for
    // them at the end of its X(i+1), so a load has the rest of its slot plus
    // one more to land.  No other barrier waits for memory.
    //
    // An M phase is one basic block: its 32 MFMAs take their LDS operands
    // four MFMAs ahead, pinned by sched_group_barrier.  A block id that is
    // out of range is fetched as block 0 and gets all-zero probabilities, so
    // it adds nothing (for finite block-0 data) and needs no branch.
    const int grp = wave_s >> 2;
    const int gw = wave_s & 3;          // wave within group 0
    constexpr int LPW = 2 * C::CPW;     // chunks of one V block per group-0 wave
    constexpr int KPW = F8 ? LPW / 2 : LPW;  // chunks of one K block per group-0 wave
    constexpr int NL = LPW + KPW;       // loads per M phase and group-0 wave
    constexpr int NPV = C::PST * C::NDT;
    constexpr int NU = NPV + (F8 ? 2 * C::NKT : C::DS * C::NKT);
    constexpr int LA = 4;
    static_assert(NL <= NU, "an M phase issues at most one load per MFMA");
    auto barrier = [&]() LI_INLINE {
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    };
    auto wait_loads = [&]() LI_INLINE {
      __builtin_amdgcn_sched_barrier(0);
      wait_vm0();
      __builtin_amdgcn_sched_barrier(0);
    };
    auto lds_addr = [&](char* p) LI_INLINE { return (uint32_t)(uintptr_t)(lds_void*)p; };
    const uint32_t a_ks0 = lds_addr(ks0), a_ks1 = lds_addr(ks1), a_vs0 = lds_addr(vs0), a_vs1 = lds_addr(vs1);
    // A group-0 wave loads chunks c = gw * LPW + j (j < LPW) of every V and
    // 16-bit K block (1 KiB each, block rows 4c..4c+3), and chunks
    // c = gw * KPW + j (j < KPW, rows 8c..8c+7) of an e4m3 K block.  Each load
    // is one instruction: scalar base + lane offset + instruction offset
    // (j & 3) * 1024.
    //
    // Tiled blocks, text blocks (contiguous in the padded text buffer) and
    // out-of-grid chunks (read from g_zero_rows) have contiguous rows: the
    // base is alt (j < 4) or alt + 4096, the lane offset k_src/v_src.
    // A visual chunk on the fused path is 4 consecutive tokens along w (tw and
    // W are multiples of 4), all inside the grid or all outside it.  Its
    // offset from the block's origin token does not depend on the block, so
    // each lane keeps the byte offsets of its wave's chunks, less the
    // instruction offset, in kvo/vvo; a block costs one origin computation and
    // one ballot for the in-grid mask.  The offsets stay non-negative because
    // a chunk's token offset is at least 4c when the grid is at least one tile
    // in each dimension, and a token is at least 256 bytes.
    static_assert(LPW == 8, "two scalar bases of four chunks each");
    struct Blk {
      const char* vis;  // fused path: origin token of a visual block
      const char* alt;  // contiguous source at this wave's first chunk
      uint32_t mask;    // bit j: chunk j of this wave is an in-grid visual chunk
    };

    uint32_t kvo[LPW], vvo[LPW];
    uint32_t lane_ft = 0, lane_fh = 0, lane_fw = 0;
    int32_t lane_coff = 0;  // token offset of chunk lane % 32 from its block's first token
    const char* vis_k = nullptr;
    const char* vis_v = nullptr;
    const char* txt_k = nullptr;
    const char* txt_v = nullptr;
    const char* zero_rows = reinterpret_cast<const char*>(g_zero_rows);
    if constexpr (G) {
      vis_k = reinterpret_cast<const char*>(a.k + b * a.g.ks[0] + h * a.g.ks[1]);
      vis_v = reinterpret_cast<const char*>(a.v + b * a.g.vs[0] + h * a.g.vs[1]);
      txt_k = reinterpret_cast<const char*>(a.g.ktxt + (int64_t)bh * a.g.ntxt * BS * D) + gw * LPW * 1024;
      txt_v = reinterpret_cast<const char*>(a.g.vtxt + (int64_t)bh * a.g.ntxt * BS * D) + gw * LPW * 1024;
      const uint32_t thtw = a.g.th * a.g.tw;
      auto coords = [&](uint32_t c, uint32_t& ft, uint32_t& fh, uint32_t& fw) LI_INLINE {
        ft = udiv16(4 * c, a.g.mg_thtw);
        const uint32_t r = 4 * c - ft * thtw;
        fh = udiv16(r, a.g.mg_tw);
        fw = r - fh * (uint32_t)a.g.tw;
      };
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        uint32_t ft, fh, fw;
        coords(gw * LPW + j, ft, fh, fw);
        const uint32_t coff = (ft * a.g.H + fh) * a.g.W + fw;
        if constexpr (!F8) kvo[j] = coff * (uint32_t)(2 * a.g.ks[2]) + k_src_vis - (j & 3) * 1024;
        vvo[j] = coff * (uint32_t)(2 * a.g.vs[2]) + v_src_vis - (j & 3) * 1024;
      }
      coords(lane & 31, lane_ft, lane_fh, lane_fw);
      if constexpr (DN) lane_coff = (int32_t)((lane_ft * a.g.H + lane_fh) * a.g.W + lane_fw);
    }
    // A key block's geometry, shared by its K and V loads: its first token
    // and this wave's in-grid chunk mask (0 for text blocks).  A block is a
    // K block in one M phase and the V block of the next, so each M phase
    // works out one new geometry.
    struct Geo {
      int32_t blk, l0;
      uint32_t mask;
      bool txt;
    };
    auto geo_of = [&](int blk) LI_INLINE {
      Geo g_{blk, 0, 0u, false};
      if constexpr (G) {
        // Straight-line scalar code: both sides of each choice are computed;
        // the text test is skipped when there are no text blocks.
        bool txt = false;
        uint32_t vb = (uint32_t)blk;
        if (a.g.ntxt > 0) {
          txt = blk < a.g.ntxt;
          const int32_t vbs = blk - a.g.ntxt;
          vb = (uint32_t)(vbs > 0 ? vbs : 0);
        }
        const uint32_t ct = udiv16m(vb, a.g.mg_nhnw, a.g.id_nhnw), rem = vb - ct * (uint32_t)(a.g.nh * a.g.nw);
        const uint32_t ch = udiv16m(rem, a.g.mg_nw, a.g.id_nw), cw = rem - ch * (uint32_t)a.g.nw;
        const uint32_t t0 = ct * a.g.tt, h0 = ch * a.g.th, w0 = cw * a.g.tw;
        g_.l0 = (int32_t)((t0 * a.g.H + h0) * a.g.W + w0);
        const bool inside = (lane_ft < a.g.Tk - t0) & (lane_fh < a.g.H - h0) & (lane_fw < a.g.W - w0) &
                            (!DN || (int32_t)g_.l0 + lane_coff < a.g.k_tokens);
        const uint32_t in_grid = (uint32_t)__ballot(inside);
        g_.mask = (in_grid >> (gw * LPW)) & (txt ? 0u : (1u << LPW) - 1u);
        g_.txt = txt;
      }
      return g_;
    };
    // Byte strides between K / V tokens (below 2^32: the host bounds the
    // largest row offset of a tile).
    const uint32_t kst = G ? (uint32_t)(2 * a.g.ks[2]) : 0u, vst = G ? (uint32_t)(2 * a.g.vs[2]) : 0u;
    auto blk_src = [&](const Geo& g_, bool is_v) LI_INLINE {
      Blk s_{nullptr, nullptr, 0u};
      if constexpr (!G) {
        s_.alt = is_v ? reinterpret_cast<const char*>(vhead + (int64_t)g_.blk * BS * D) + gw * LPW * 1024
                      : kbytes + (int64_t)g_.blk * BS * D * KEB + gw * KPW * 1024;
      } else {
        if (F8 && !is_v) {
          s_.alt = kbytes + (int64_t)g_.blk * BS * D + gw * KPW * 1024;
          return s_;
        }
        s_.vis = (is_v ? vis_v : vis_k) + (uint64_t)(uint32_t)g_.l0 * (is_v ? vst : kst);
        s_.mask = g_.mask;
        const char* tb = (is_v ? txt_v : txt_k) + (int64_t)g_.blk * (BS * D * 2);
        s_.alt = g_.txt ? tb : zero_rows;
      }
      return s_;
    };
    // Chunk n of a group-0 wave's share of a stage: n < LPW is V, else K.
    // src_n gives its global source, issue_n loads it into the stage.
    // zr = Stage<1>: the zero-region source (visual or zero base, visual lane
    // offset); text blocks, whose mask is 0, then read as zeros, so these
    // phases come after a row's text blocks.  Stage<0>: base and lane offset
    // per chunk (visual, text or the small zero buffer).
    auto src_n = [&](int n, const Blk& sv, const Blk& sk, auto zr) LI_INLINE {
      const bool isv = n < LPW;
      const int j = isv ? n : n - LPW;
      const Blk& s_ = isv ? sv : sk;
      const uint32_t lin = isv ? v_src : (F8 ? k8_src[j & 1] : k_src);
      const char* alt = j < 4 ? s_.alt : s_.alt + 4096;
      if (!G || (F8 && !isv))
        return DmaSrc{alt, lin};
      else if constexpr (decltype(zr)::value == 1)
        return dma_sel_base(s_.mask, j, s_.vis, a.zero_region, isv ? vvo[j] : kvo[j]);
      else
        return dma_sel(s_.mask, j, s_.vis, isv ? vvo[j] : kvo[j], alt, lin);
    };
    auto issue_n = [&](int n, const DmaSrc& src, uint32_t vn, uint32_t kn) LI_INLINE {
      const bool isv = n < LPW;
      const int j = isv ? n : n - LPW;
      const int c = gw * (isv ? LPW : KPW) + j;
      const int imm = (j & 3) * 1024;
      dma16_imm(src.base, src.voff, (isv ? vn + c * 1024 : kn + c * (F8 ? 1024 : 1088)) - imm, imm);
    };
    auto dma = [&](int n, const Blk& sv, const Blk& sk, uint32_t vn, uint32_t kn) LI_INLINE {
      issue_n(n, src_n(n, sv, sk, Stage<0>{}), vn, kn);
    };
    // A operand of MFMA u of an M phase: the V^T tile of P V step
    // (st, dt) = (u / NDT, u % NDT) for u < NPV, else the K tile of S step
    // (s, kt) = ((u - NPV) / NKT, (u - NPV) % NKT).  An operand is 16 bytes
    // (p), or 32 bytes (k) for an e4m3 S step.
    struct Op {
      vec8 p;
      i32x8 k;
    };
    auto read_op = [&](int u, const char* vc, const char* kc) LI_INLINE {
      Op r;
      if (u < NPV) {
        const int st = u / C::NDT, dt = u % C::NDT, kt = st >> 1, ip = st & 1;
        const uint16_t* p = reinterpret_cast<const uint16_t*>(vc + v_off[dt] + (32 * kt + 16 * ip) * 256);
        const u32x2 lo = lds_read_tr(p), hi = lds_read_tr(p + 4 * 128);
        r.p = __builtin_bit_cast(vec8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        return r;
      }
      const int w = u - NPV, s = w / C::NKT, kt = w % C::NKT;
      if constexpr (F8)
        r.k = read_k8(kc, s, kt);
      else
        r.p = __builtin_bit_cast(vec8,
                                 *reinterpret_cast<const u32x4*>(kc + k_off[s & 1] + 8704 * kt + 64 * (s >> 1)));
      return r;
    };
    f32x16 zero16;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero16[r] = 0.0f;
    auto mfma_u = [&](int u, const Op& op) LI_INLINE {
      if (u < NPV) {
        const int st = u / C::NDT, dt = u % C::NDT;
        o[dt] = E::mfma32(op.p, __builtin_bit_cast(vec8, ppk[st]), o[dt]);
      } else {
        const int w = u - NPV, s = w / C::NKT, kt = w % C::NKT;
        if constexpr (F8)
          sacc[kt] = mfma_e4m3(op.k, qf8[s], s == 0 ? zero16 : sacc[kt]);
        else
          sacc[kt] = E::mfma32(op.p, qf[s], s == 0 ? zero16 : sacc[kt]);
      }
    };
    // M phase; group 0 (load = true) also issues the stage DMAs, group 1
    // runs the same MFMAs and reads without them.  Each is one basic block.
    // vb / kb: load sources of the V and K blocks the phase fetches, worked
    // out during the preceding softmax phase.
    auto m_phase = [&](const char* vc, const char* kc, uint32_t vn, uint32_t kn, const Blk& vb, const Blk& kb,
                       bool load, auto zr) LI_INLINE {
      Op opb[LA];
#pragma unroll
      for (int u = 0; u < LA; ++u) opb[u] = read_op(u, vc, kc);
      // The source of each load is worked out one load ahead, off the path
      // between the MFMAs.  The NL loads are spread evenly: load n follows
      // MFMA u when floor(u NL / NU) = n < floor((u + 1) NL / NU).
      DmaSrc nxt{nullptr, 0u};
      if (load) nxt = src_n(0, vb, kb, zr);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const Op op = opb[u % LA];
        if (u + LA < NU) opb[u % LA] = read_op(u + LA, vc, kc);
        mfma_u(u, op);
        const int n = u * NL / NU;
        if (load && (u + 1) * NL / NU > n) {
          issue_n(n, nxt, vn, kn);
          if (n + 1 < NL) nxt = src_n(n + 1, vb, kb, zr);
        }
      }
      sched_m_phase<NPV, F8 ? 2 : 1, NU, LA>();
    };
    // Dense calls: the keys past the end of the last text block and of the
    // last visual block get score -inf.  Element r of sacc[kt] holds key
    // KW*kh + 32*kt + kperm(8*(r/4) + 4*hl + r%4) of the block.
    auto mask_tail = [&](int blk) LI_INLINE {
      if constexpr (DN) {
        int nv = BS;
        if (a.g.txt_tail > 0 && blk == a.g.ntxt - 1) nv = a.g.txt_tail;
        if (a.g.vis_tail > 0 && blk == a.nkb - 1) nv = a.g.vis_tail;
        if (nv < BS) {
#pragma unroll
          for (int kt = 0; kt < C::NKT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              if (C::KW * kh + 32 * kt + kperm(8 * (r >> 2) + 4 * hl + (r & 3)) >= nv) sacc[kt][r] = -__builtin_inff();
        }
      }
    };
    // pre() runs at the head of either branch, where its scalar work can
    // interleave with the softmax's vector work.
    auto x_phase = [&](int blk, auto&& pre) LI_INLINE {
      if (valid(blk)) {
        pre();
        mask_tail(blk);
        softmax();
      } else {
        pre();
#pragma unroll
        for (int st = 0; st < C::PST; ++st) ppk[st] = u32x4{0u, 0u, 0u, 0u};
      }
    };
    // Block ids i+1 .. i+3 are kept ahead of block i, so the sources of the
    // next M phase can be worked out before it starts.
    int id_c, id_n, id_nn, id_n3;
    if constexpr (DN) {
      id_c = block_id(0), id_n = block_id(1), id_nn = block_id(2), id_n3 = block_id(3);
    } else {
      id_c = empty ? -1 : r0;
      id_n = count > 1 ? r1 : id_c;
      id_nn = count > 2 ? r2 : id_n;
      id_n3 = count > 3 ? r3 : id_nn;
    }
    // The next id to read, stepped along the row and held at its last entry
    // (the same clamp as block_id), so a read costs no index arithmetic.
    const int64_t ist = a.is[3];
    // An empty unit's row may have no entry to read (no columns, or the
    // second half of a one-block list): its pointer is the count it was
    // given, which is readable, and the value read is never used.
    const_i32* idp = DN ? nullptr
                        : empty ? (const_i32*)cnt_at
                                : irow_s + (int64_t)(count > 4 ? 4 : (count > 0 ? count - 1 : 0)) * ist;
    Blk dv{nullptr, nullptr, 0u}, dk{nullptr, nullptr, 0u};
    Geo geo_k{0, 0, 0u, false};  // geometry of the K block of the next M phase
    // F8: K scales of blocks id_n and id_nn, read one pair ahead of their
    // softmax through the scalar cache.
    typedef __attribute__((address_space(4))) const float const_f32;
    const_f32* ksc = (const_f32*)a.k_scale + (int64_t)bh * a.nkb;
    float sk_n = 0.0f, sk_nn = 0.0f;
    if constexpr (F8) {
      sk_n = ksc[safe(id_n)];
      sk_nn = ksc[safe(id_nn)];
    }
    // The prologue waits only for K(0) (with the Q fragments); group 0 issues
    // the loads of V(0) and K(1) at the head of its S(0) and waits for them
    // at the end of its X(0), so they land while S(0) and X(0) run.
    Blk vb0{nullptr, nullptr, 0u}, kb1{nullptr, nullptr, 0u};
    if (grp == 0) {
      const Geo g0 = geo_of(safe(id_c)), g1 = geo_of(safe(id_n));
      vb0 = blk_src(g0, true);
      const Blk kb0 = blk_src(g0, false);
      kb1 = blk_src(g1, false);
#pragma unroll
      for (int n = 0; n < KPW; ++n) dma(n + LPW, vb0, kb0, a_vs0, a_ks1);
      geo_k = geo_of(safe(id_nn));
      dv = blk_src(g1, true);
      dk = blk_src(geo_k, false);
      wait_vm0();
    }
    __syncthreads();
    // Each group runs its own copy of the block loop (group 0's with the
    // stage loads), so neither carries the other's load code and the copies
    // meet only after the loop.
    auto pair = [&](int i, const char* vc, const char* kc, uint32_t vn, uint32_t kn, bool load,
                    auto zr) LI_INLINE {
      barrier();
      m_phase(vc, kc, vn, kn, dv, dk, load, zr);
      barrier();
      const int id_x = id_n;
      id_c = id_n;
      id_n = id_nn;
      id_nn = id_n3;
      if constexpr (DN) {
        id_n3 = id_base + (i + 4 < count ? i + 4 : count - 1);
      } else {
        id_n3 = *idp;
        idp = i + 5 < count ? idp + ist : idp;
      }
      if constexpr (F8) {
        qk_scale = qk_base * sk_n;
        sk_n = sk_nn;
        sk_nn = ksc[safe(id_nn)];
      }
      auto next_sources = [&]() LI_INLINE {
        if (load) {
          dv = blk_src(geo_k, true);
          geo_k = geo_of(safe(id_nn));
          dk = blk_src(geo_k, false);
        }
      };
      if (i + 1 < count) x_phase(id_x, next_sources);
      if (load) wait_loads();
      // The scalar loads of this phase (the next block id, and for F8 a K
      // scale) complete here, before the next M phase: one still in flight
      // there would make its first operand wait cover all LA MFMAs' LDS reads
      // (lgkmcnt counts both, and scalar loads return out of order).
      if constexpr (F8)
        __asm__ volatile("" ::"s"(id_n3), "s"(sk_nn));
      else
        __asm__ volatile("" ::"s"(id_n3));
    };
    auto run = [&](bool load) LI_INLINE {
      if (load) {
#pragma unroll
        for (int n = 0; n < LPW; ++n) dma(n, vb0, kb1, a_vs0, a_ks0);
#pragma unroll
        for (int n = 0; n < KPW; ++n) dma(n + LPW, vb0, kb1, a_vs0, a_ks0);
      }
      scores(ks1);
      if (!load) barrier();
      if constexpr (F8) qk_scale = qk_base * ksc[safe(id_c)];
      if (valid(id_c)) {
        mask_tail(id_c);
        softmax_first();
      } else {
#pragma unroll
        for (int st = 0; st < C::PST; ++st) ppk[st] = u32x4{0u, 0u, 0u, 0u};
      }
      if (load) wait_loads();
      if (!load) {
        for (int i = 0; i < count; i += 2) {
          pair(i, vs0, ks0, a_vs1, a_ks1, false, Stage<0>{});
          if (i + 1 < count) pair(i + 1, vs1, ks1, a_vs0, a_ks0, false, Stage<0>{});
        }
      } else {
        // The last block's phase loads nothing, since its V(i + 1) and
        // K(i + 2) lie past the row: a separate copy of that phase skips the
        // loads and the wait for them (one memory round trip per tile).  On
        // the zero-region path the phases after the first gen_pairs load with
        // the zero-region sources; the others (the row's text blocks, and the
        // last loading phase, which may still reach a short row's text
        // blocks) pick their sources per chunk.
        int i = 0;
        if constexpr (ZR) {
          for (; i < a.gen_pairs && i + 2 < count; i += 2) {
            pair(i, vs0, ks0, a_vs1, a_ks1, true, Stage<0>{});
            pair(i + 1, vs1, ks1, a_vs0, a_ks0, true, Stage<0>{});
          }
          for (; i + 2 < count; i += 2) {
            pair(i, vs0, ks0, a_vs1, a_ks1, true, Stage<1>{});
            pair(i + 1, vs1, ks1, a_vs0, a_ks0, true, Stage<1>{});
          }
        } else {
          for (; i + 2 < count; i += 2) {
            pair(i, vs0, ks0, a_vs1, a_ks1, true, Stage<0>{});
            pair(i + 1, vs1, ks1, a_vs0, a_ks0, true, Stage<0>{});
          }
        }
        if (i + 1 < count) {
          pair(i, vs0, ks0, a_vs1, a_ks1, true, Stage<0>{});
          pair(i + 1, vs1, ks1, a_vs0, a_ks0, false, Stage<0>{});
        } else {
          pair(i, vs0, ks0, a_vs1, a_ks1, false, Stage<0>{});
        }
      }
      if (load) barrier();
    };
    if (grp == 0)
      run(true);
    else
      run(false);
  } else {
    // One wave per SIMD: plain double buffering, block i+1 loaded while
    // block i is computed.
    auto load_block = [&](int blk, char* kd, char* vd) LI_INLINE {
      const char* kb = kbytes + (int64_t)blk * BS * D * 2;
      const char* vb = reinterpret_cast<const char*>(vhead + (int64_t)blk * BS * D);
#pragma unroll
      for (int j = 0; j < C::CPW; ++j) {
        const int c = wave_s * C::CPW + j;
        __builtin_amdgcn_global_load_lds(kb + 8 * c * D + k_src, (lds_void*)(kd + c * 1088), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vb + 8 * c * D + v_src, (lds_void*)(vd + c * 1024), 16, 0, 0);
      }
    };
    int cur = block_id(0);
    load_block(safe(cur), ks0, vs0);
    int nxt = block_id(1);
    __syncthreads();
    auto step = [&](char* kc, char* vc, char* kn, char* vn, int i) LI_INLINE {
      const int nn = block_id(i + 2);
      if (i + 1 < count) load_block(safe(nxt), kn, vn);
      if (valid(cur)) {
        scores(kc);
        softmax();
        pv_update(vc);
      }
      __syncthreads();
      cur = nxt;
      nxt = nn;
    };
    for (int i = 0; i < count; i += 2) {
      step(ks0, vs0, ks1, vs1, i);
      if (i + 1 < count) step(ks1, vs1, ks0, vs0, i + 1);
    }
  }

  // Merge the two key halves (waves kh = 0 and kh = 1 of the same qq).  The
  // exchanged O of a wave is stored as 16-byte runs: element (dt, 4 i4 + j)
  // of lane l at ((dt * 4 + i4) * 64 + l) * 4 + j.
  {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(lrow), __float_as_uint(lrow), false, false);
    lrow = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
  }
  char* xo_st = F8 ? (qq < C::NQW / 2 || C::NQW == 1 ? vs0 : vs1) : (qq < C::NQW / 2 || C::NQW == 1 ? ks0 : ks1);
  float* xo = reinterpret_cast<float*>(xo_st) + (qq % (C::NQW > 1 ? C::NQW / 2 : 1)) * (C::NDT * 16 * 64);
  float* xm = reinterpret_cast<float*>(F8 ? ks0 : vs0) + qq * (2 * 64);
  if (kh == 1) {
#pragma unroll
    for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
        *reinterpret_cast<f32x4*>(xo + ((dt * 4 + i4) * 64 + lane) * 4) =
            f32x4{o[dt][4 * i4], o[dt][4 * i4 + 1], o[dt][4 * i4 + 2], o[dt][4 * i4 + 3]};
    xm[lane] = mrow;
    xm[64 + lane] = lrow;
  }
  __syncthreads();
  if (kh == 0) {
    const float m1 = xm[lane], l1 = xm[64 + lane];
    const float mm = __builtin_fmaxf(mrow, m1);
    // A row whose blocks were all out of range has mm = -inf: it gets zeros.
    const bool none = mm == -__builtin_inff();
    const float a0 = none ? 0.0f : __builtin_amdgcn_exp2f(mrow - mm);
    const float a1 = none ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
    const float l = lrow * a0 + l1 * a1;
    const int rt = 32 * qq + l32;
    if (half >= 0) {
      float* prow = part_o + rt * D;
#pragma unroll
      for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          const f32x4 o1 = *reinterpret_cast<const f32x4*>(xo + ((dt * 4 + i4) * 64 + lane) * 4);
          f32x4 val;
#pragma unroll
          for (int j = 0; j < 4; ++j) val[j] = o[dt][4 * i4 + j] * a0 + o1[j] * a1;
          *reinterpret_cast<f32x4*>(prow + 32 * dt + 8 * i4 + 4 * hl) = val;
        }
      if (hl == 0) {
        part_ml[2 * rt] = mm;
        part_ml[2 * rt + 1] = l;
      }
    } else {
      if (uint16_t* orow = out_row(rt)) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int dt = 0; dt < C::NDT; ++dt)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const f32x4 o1 = *reinterpret_cast<const f32x4*>(xo + ((dt * 4 + i4) * 64 + lane) * 4);
            float val[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) val[j] = (o[dt][4 * i4 + j] * a0 + o1[j] * a1) * inv;
            const u32x2 pk = {cvt_pk<E>(val[0], val[1]), cvt_pk<E>(val[2], val[3])};
            *reinterpret_cast<u32x2*>(orow + 32 * dt + 8 * i4 + 4 * hl) = pk;
          }
      }
      // The LSE is in tile-row order and covers the grid's padding rows too
      // (their queries are zero), whether or not the row has an output token.
      const int r = row0 + rt;
      if (a.lse && hl == 0 && r < a.Lq) a.lse[(int64_t)bh * a.Lq + r] = none ? -__builtin_inff() : mm + __builtin_log2f(l);
    }
  }
}

// Combines the two halves of each split query tile: O = (O0 a0 + O1 a1) /
// (l0 a0 + l1 a1) with a_i = 2^(m_i - max(m0, m1)); lse = max + log2(l).  Four
// workgroups per split tile (32 rows each), eight threads per row (16 d each,
// 64 contiguous bytes of each partial).  Split tile p = x * xsplit + j is
// tile j of the split tiles of XCD x.
template <typename E, bool G = false>
__global__ __launch_bounds__(256) void bsa_merge_kernel(BsaArgs a) {
  constexpr int BS = 128, D = 128;
  const int p = blockIdx.x >> 2;
  const int x = p / a.xsplit, j = p - x * a.xsplit;
  const int tile = x * a.xtiles + (a.xtiles - a.xsplit) + j;
  const int bh = tile / a.nqt, m = tile % a.nqt;
  const int rt = (blockIdx.x & 3) * 32 + (threadIdx.x >> 3), dq = threadIdx.x & 7;
  const int r = m * BS + rt;
  if (r >= a.Lq) return;
  // Padding rows of the grid have no output token but do have an LSE.
  uint16_t* orow = nullptr;
  if constexpr (G) {
    const int b = bh / a.NH, h = bh % a.NH;
    bool ok;
    const int32_t l = tile_token(a.g, a.g.Tq, m, rt, ok);
    if (ok && l < a.g.q_tokens) orow = a.out + b * a.g.os[0] + h * a.g.os[1] + (int64_t)l * a.g.os[2] + 16 * dq;
  } else {
    orow = a.out + ((int64_t)bh * a.Lq + r) * D + 16 * dq;
  }
  const float* p0 = a.part + (int64_t)(2 * p) * BS * (D + 2);
  const float* p1 = p0 + BS * (D + 2);
  const float m0 = p0[BS * D + 2 * rt], l0 = p0[BS * D + 2 * rt + 1];
  const float m1 = p1[BS * D + 2 * rt], l1 = p1[BS * D + 2 * rt + 1];
  const float mm = __builtin_fmaxf(m0, m1);
  const bool none = mm == -__builtin_inff();
  const float a0 = none ? 0.0f : __builtin_amdgcn_exp2f(m0 - mm);
  const float a1 = none ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
  const float l = l0 * a0 + l1 * a1;
  if (orow) {
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const f32x4* o0 = reinterpret_cast<const f32x4*>(p0 + rt * D + 16 * dq);
    const f32x4* o1 = reinterpret_cast<const f32x4*>(p1 + rt * D + 16 * dq);
    f32x4 x0[4], x1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x0[i] = o0[i];
      x1[i] = o1[i];
    }
    u32x4 pk[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pk[i >> 1][2 * (i & 1)] = cvt_pk<E>((x0[i][0] * a0 + x1[i][0] * a1) * inv, (x0[i][1] * a0 + x1[i][1] * a1) * inv);
      pk[i >> 1][2 * (i & 1) + 1] =
          cvt_pk<E>((x0[i][2] * a0 + x1[i][2] * a1) * inv, (x0[i][3] * a0 + x1[i][3] * a1) * inv);
    }
    *reinterpret_cast<u32x4*>(orow) = pk[0];
    *reinterpret_cast<u32x4*>(orow + 8) = pk[1];
  }
  if (a.lse && dq == 0) a.lse[(int64_t)bh * a.Lq + r] = none ? -__builtin_inff() : mm + __builtin_log2f(l);
}

template <typename E, bool DN = false>
int launch_bsa_gather(BsaArgs& a, int tiles, hipStream_t s) {
  const int nsplit = 8 * a.xsplit;
  clear_launch_error();
  if (a.zero_region)
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<E, 128, true, false, DN, true>), dim3(tiles + nsplit),
                       dim3(DmaCfg<128>::NTHR), 0, s, a);
  else
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<E, 128, true, false, DN>), dim3(tiles + nsplit),
                       dim3(DmaCfg<128>::NTHR), 0, s, a);
  if (nsplit > 0) hipLaunchKernelGGL((bsa_merge_kernel<E, true>), dim3(4 * nsplit), dim3(256), 0, s, a);
  return launch_status();
}

template <bool G>
int launch_bsa_fp8(BsaArgs& a, int tiles, hipStream_t s) {
  const int nsplit = 8 * a.xsplit;
  clear_launch_error();
  if (G && a.zero_region)
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<Bf16, 128, G, true, false, G>), dim3(tiles + nsplit),
                       dim3(DmaCfg<128>::NTHR), 0, s, a);
  else
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<Bf16, 128, G, true>), dim3(tiles + nsplit), dim3(DmaCfg<128>::NTHR),
                       0, s, a);
  if (nsplit > 0) hipLaunchKernelGGL((bsa_merge_kernel<Bf16, G>), dim3(4 * nsplit), dim3(256), 0, s, a);
  return launch_status();
}

template <typename E, int BS>
int launch_bsa_dma(BsaArgs& a, int tiles, hipStream_t s) {
  const int nsplit = 8 * a.xsplit;
  clear_launch_error();
  hipLaunchKernelGGL((bsa_fwd_dma_kernel<E, BS>), dim3(tiles + nsplit), dim3(DmaCfg<BS>::NTHR), 0, s, a);
  if constexpr (BS == 128) {
    if (nsplit > 0) hipLaunchKernelGGL(bsa_merge_kernel<E>, dim3(4 * nsplit), dim3(256), 0, s, a);
  }
  return launch_status();
}

template <typename E, int BS, int D>
int launch_bsa(BsaArgs& a, int tiles, hipStream_t s) {
  clear_launch_error();
  hipLaunchKernelGGL((bsa_fwd_kernel<E, BS, D>), dim3(tiles), dim3(Cfg<BS, D>::NTHR), 0, s, a);
  return launch_status();
}

template <typename E>
int dispatch_bsa(BsaArgs& a, int bs, int D, int tiles, hipStream_t s) {
  if (bs == 128 && D == 128) return launch_bsa_dma<E, 128>(a, tiles, s);
  if (bs == 128 && D == 64) return launch_bsa<E, 128, 64>(a, tiles, s);
  if (bs == 64 && D == 128) return launch_bsa_dma<E, 64>(a, tiles, s);
  if (bs == 64 && D == 64) return launch_bsa<E, 64, 64>(a, tiles, s);
  return LI_ERR_UNSUPPORTED;
}

// Compute units of the current device, cached per device.
int device_cus() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    cached[dev] = n > 0 ? n : -1;
  }
  return cached[dev] > 0 ? cached[dev] : 0;
}

// Dispatch order for rows of unequal length: within each range of positions
// that unit_tile gives one XCD (its whole range, or each of its chunks when
// a.xchunk is set), tiles sorted by kept-block count, longest first, so every
// XCD starts its longest work first (longest processing time first).  A
// counting sort over 1024 buckets of the count (exact when n_cols < 1024);
// one workgroup per range.  Any order gives the same results: each tile is
// computed on its own.
__global__ __launch_bounds__(1024) void bsa_order_kernel(BsaArgs a, int32_t* order) {
  __shared__ int hist[1024];
  const int tid = threadIdx.x, x = blockIdx.x;
  const int tiles = a.ntiles;
  const int per = tiles >> 3, rem = tiles & 7;
  int start = x * per + (x < rem ? x : rem), len = per + (x < rem ? 1 : 0);
  if (a.xchunk > 0) {
    start = x * a.xchunk;
    len = a.xchunk;
  }
  const int nc = a.n_cols > 0 ? a.n_cols : 1;
  auto bucket = [&](int tile) {
    const int bh = tile / a.nqt, m = tile % a.nqt;
    const int b = bh / a.NH, h = bh % a.NH;
    int c = a.cnt ? a.cnt[b * a.cs[0] + h * a.cs[1] + (int64_t)m * a.cs[2]] : nc;
    c = c < 0 ? 0 : (c > nc ? nc : c);
    return nc < 1024 ? nc - c : (int)(((int64_t)(nc - c) * 1023) / nc);
  };
  hist[tid] = 0;
  __syncthreads();
  for (int t = tid; t < len; t += 1024) atomicAdd(&hist[bucket(start + t)], 1);
  __syncthreads();
  // Exclusive prefix sum of the bucket sizes (Hillis-Steele, 1024 entries).
  const int own = hist[tid];
  for (int d = 1; d < 1024; d <<= 1) {
    __syncthreads();
    const int add = tid >= d ? hist[tid - d] : 0;
    __syncthreads();
    hist[tid] += add;
  }
  __syncthreads();
  const int incl = hist[tid];
  __syncthreads();
  hist[tid] = incl - own;
  __syncthreads();
  for (int t = tid; t < len; t += 1024) {
    const int p = atomicAdd(&hist[bucket(start + t)], 1);
    order[start + p] = start + t;
  }
}

// Query tiles of each XCD whose block lists are split in halves.  The tiles
// are dealt to the 8 XCDs in contiguous ranges of n = tiles / 8, and with
// one 8-wave workgroup per CU an XCD of c = cus / 8 CUs runs its n tiles in
// ceil(n / c) rounds, the last holding r = n % c tiles.  When r <= c / 2,
// those r tiles run as 2 r halves on their own XCD (so that their key blocks
// stay in its L2), and the last round is half as long (HY shape: 896 tiles,
// n = 112, c = 32, r = 16).  A fuller last round is left whole: at the
// Matrix-Game shape (n = 90, r = 26) uneven pieces (5/6 of a list on 26 CUs,
// the 1/6 pieces on the other 6) ran as long as the whole round, each short
// piece paying ~4 us of prologue and epilogue, and the merge added ~10 us.
// No split when the tiles or the CUs do not divide evenly over the XCDs.
int64_t split_per_xcd(int64_t tiles, int cus) {
  if (cus <= 0 || cus % 8 != 0 || tiles % 8 != 0) return 0;
  const int64_t n = tiles / 8, c = cus / 8;
  if (n <= c) return 0;
  const int64_t r = n % c;
  return 2 * r <= c ? r : 0;
}

constexpr int64_t kPartBytesPerTile = 2 * 128 * (128 + 2) * 4;

int64_t order_bytes(int64_t tiles) { return (tiles * 4 + 15) & ~(int64_t)15; }

// Workspace use of one call: with LI_BSA_BALANCE (D = 128 kernels) the tile
// order, built by bsa_order_kernel and no tail split; otherwise the tail
// split's partials (D = 128, BS = 128).  Returns the launch status of the
// order kernel (LI_OK when none runs).
// XCD chunk of the longest-first order: one head's query tiles (nqt), so that
// each XCD sorts and runs one head at a time and its L2 holds that head's
// K/V blocks (HY long rollout: 0.687 against 0.706 ms with two heads mixed per
// XCD).  0 when the heads do not split evenly over the XCDs.
int xcd_chunk(int64_t tiles, int32_t nqt) {
  return (nqt > 0 && tiles > 0 && tiles % (8 * (int64_t)nqt) == 0) ? nqt : 0;
}

int plan_units(BsaArgs& a, int64_t tiles, int32_t D, int32_t block_size, void* workspace, int64_t workspace_bytes,
               int32_t flags, hipStream_t s) {
  a.ntiles = (int32_t)tiles;
  a.xtiles = (int32_t)(tiles / 8);
  a.xsplit = 0;
  a.part = nullptr;
  a.order = nullptr;
  if (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0 || D != 128) return LI_OK;
  if (flags & LI_BSA_BALANCE) {
    if (workspace_bytes < order_bytes(tiles)) return LI_OK;
    int32_t* order = static_cast<int32_t*>(workspace);
    a.xchunk = xcd_chunk(tiles, a.nqt);
    clear_launch_error();
    hipLaunchKernelGGL(bsa_order_kernel, dim3(a.xchunk > 0 ? (unsigned)(tiles / a.xchunk) : 8u), dim3(1024), 0, s, a,
                       order);
    const int st = launch_status();
    if (st == LI_OK) a.order = order;
    return st;
  }
  if (block_size != 128) return LI_OK;
  const int64_t r = split_per_xcd(tiles, device_cus());
  if (r > 0 && workspace_bytes >= 8 * r * kPartBytesPerTile) {
    a.xsplit = (int32_t)r;
    a.part = static_cast<float*>(workspace);
  }
  return LI_OK;
}

}  // namespace
}  // namespace li

using namespace li;

extern "C" int64_t li_bsa_fwd_workspace_size(int32_t B, int32_t NH, int32_t Lq, int32_t D, int32_t block_size) {
  if (B <= 0 || NH <= 0 || Lq <= 0 || D != 128 || block_size <= 0) return 0;
  const int64_t tiles = (int64_t)((Lq + block_size - 1) / block_size) * B * NH;
  const int64_t split = block_size == 128 ? 8 * split_per_xcd(tiles, device_cus()) * kPartBytesPerTile : 0;
  const int64_t ord = order_bytes(tiles);
  return split > ord ? split : ord;
}

extern "C" int li_bsa_fwd(int dtype, int32_t B, int32_t NH, int32_t Lq, int32_t Lk, int32_t D, const void* q,
                          const void* k, const void* v, const int32_t* block_indices, const int64_t idx_strides[4],
                          int32_t n_cols, const int32_t* block_counts, const int64_t cnt_strides[3], float sm_scale,
                          int32_t block_size, void* out, float* lse, void* workspace, int64_t workspace_bytes,
                          int32_t flags, void* stream) {
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
  // No key block at all: there is nothing to attend to (and no block 0 to
  // stand in for out-of-range ids).
  if (a.nkb <= 0) return LI_ERR_SHAPE;
  a.nqt = (int32_t)nqt;
  a.n_cols = n_cols;
  a.qk_scale = sm_scale * 1.44269504f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int st = plan_units(a, tiles, D, block_size, workspace, workspace_bytes, flags, s);
  if (st != LI_OK) return st;
  if (dtype == LI_DTYPE_BF16) return dispatch_bsa<Bf16>(a, block_size, D, (int)tiles, s);
  return dispatch_bsa<F16>(a, block_size, D, (int)tiles, s);
}

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// (B, NH, L, D) view usable by the fused kernel: unit d stride, 16-byte rows.
bool row_view_ok(const void* p, const int64_t st[4]) {
  return p && aligned16(p) && st[3] == 1 && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0 && st[2] > 0;
}

}  // namespace

// Zero bytes for the zero-region kernels (BsaArgs::zero_region): a static
// array, zero from module load and never written.  Each device holds its own
// copy until the process ends; host code passes zero_region_ptr(), never the
// array's name.
// 32 MiB reaches the largest row offset of the call shapes of both models
// (HY-WorldPlay's (4, 8, 4) tile over a 30 x 52 grid: 5047 tokens of up to
// 24 heads x 128 bf16 = 31 MB); larger calls pick their sources per chunk.
constexpr int64_t kZeroRegionBytes = 32ll << 20;
static __device__ __align__(256) char g_zero_region[kZeroRegionBytes];

namespace {

// Device address of g_zero_region on the current device (looked up once per
// device), or null, in which case the kernels pick their sources per chunk.
const char* zero_region_ptr() {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(g_zero_region)) != hipSuccess) return nullptr;
    ptrs[dev] = p;
  }
  return static_cast<const char*>(ptrs[dev]);
}

// Zero-region set-up of a fused call whose K / V rows lie up to max_row
// tokens of st elements from their tile's origin token (plus one 128-element
// row), with ntxt text blocks at the head of every row: the region when it
// reaches that far, else null; and the leading block phases that still pick
// their sources per chunk (those whose loads can reach a text block, rounded
// up to an even count).
void setup_zero_region(BsaArgs& a, int64_t max_row, int64_t st, int32_t ntxt) {
  a.zero_region = (max_row * st + 128) * 2 <= kZeroRegionBytes ? zero_region_ptr() : nullptr;
  a.gen_pairs = ((ntxt > 1 ? ntxt - 1 : 0) + 1) & ~1;
}


// Checks and BsaArgs of a token-order (fused) call over the q_geom / k_geom
// grids.  With e4m3 keys (k8) only V is read in token order: k / k_strides
// are unused and K comes from the tiles in a.k.  Returns LI_OK with `tiles`
// set, or a status; tiles = 0 means nothing to launch.
int gather_setup(BsaArgs& a, int64_t& tiles, int32_t B, int32_t NH, int32_t D, const void* q,
                 const int64_t q_strides[4], const void* k, const int64_t k_strides[4], const void* v,
                 const int64_t v_strides[4], const void* k_txt, const void* v_txt, int32_t num_txt_blk,
                 const li_tile_geom* q_geom, const li_tile_geom* k_geom, const int32_t* block_indices,
                 const int64_t idx_strides[4], int32_t n_cols, const int32_t* block_counts,
                 const int64_t cnt_strides[3], float sm_scale, void* out, const int64_t out_strides[4], float* lse,
                 bool k8, bool sorted) {
  tiles = 0;
  if (!v_strides || !out_strides || !q_geom || !k_geom || !block_indices || !idx_strides || !block_counts ||
      !cnt_strides || (!k8 && (!q_strides || !k_strides)))
    return LI_ERR_INVALID_ARG;
  if (B <= 0 || NH <= 0 || n_cols < 0 || num_txt_blk < 0) return LI_ERR_INVALID_ARG;
  const li_tile_geom& gq = *q_geom;
  const li_tile_geom& gk = *k_geom;
  if (gq.H != gk.H || gq.W != gk.W || gq.tt != gk.tt || gq.th != gk.th || gq.tw != gk.tw || gq.nh != gk.nh ||
      gq.nw != gk.nw)
    return LI_ERR_SHAPE;
  if (gq.H <= 0 || gq.W <= 0 || gq.tt <= 0 || gq.th <= 0 || gq.tw <= 0 || gq.T < 0 || gk.T < 0)
    return LI_ERR_SHAPE;
  if (gq.nh != (gq.H + gq.th - 1) / gq.th || gq.nw != (gq.W + gq.tw - 1) / gq.tw) return LI_ERR_SHAPE;
  // Built for D = 128, 128-token tiles whose w extent and the grid width are
  // multiples of 4 (a 4-row DMA chunk is 4 consecutive tokens along w).
  if (D != 128 || gq.tt * gq.th * gq.tw != 128 || gq.tw % 4 != 0 || gq.W % 4 != 0) return LI_ERR_UNSUPPORTED;
  // The grid is at least one tile high and wide, and K/V tokens do not
  // overlap, so a chunk's byte offset from its tile's origin is at least
  // 1024 * (chunk index) (the kernel subtracts the instruction offset).
  if (gq.H < gq.th || gq.W < gq.tw) return LI_ERR_UNSUPPORTED;
  if ((!k8 && (!row_view_ok(q, q_strides) || !row_view_ok(k, k_strides))) || !row_view_ok(v, v_strides) ||
      !row_view_ok(out, out_strides))
    return LI_ERR_INVALID_ARG;
  if ((!k8 && k_strides[2] < D) || v_strides[2] < D) return LI_ERR_UNSUPPORTED;
  if (num_txt_blk > 0 && (!v_txt || !aligned16(v_txt) || (!k8 && (!k_txt || !aligned16(k_txt)))))
    return LI_ERR_INVALID_ARG;
  const int64_t nq = (int64_t)((gq.T + gq.tt - 1) / gq.tt) * gq.nh * gq.nw;
  const int64_t nkv = (int64_t)((gk.T + gk.tt - 1) / gk.tt) * gk.nh * gk.nw;
  if ((int64_t)gq.nh * gq.nw >= 65536 || nkv + num_txt_blk >= 65536 || nq >= 65536) return LI_ERR_SHAPE;
  if ((int64_t)gq.T * gq.H * gq.W >= (1ll << 31) || (int64_t)gk.T * gk.H * gk.W >= (1ll << 31)) return LI_ERR_SHAPE;
  // The byte offset of a K/V row from its tile's origin token is held in 32
  // bits: at most max_row tokens, times the token stride, plus one row.
  const int64_t max_row = (int64_t)(gq.tt - 1) * gq.H * gq.W + (int64_t)(gq.th - 1) * gq.W + gq.tw - 1;
  const int64_t kv_st = !k8 && k_strides[2] > v_strides[2] ? k_strides[2] : v_strides[2];
  if ((max_row * kv_st + D) * 2 > (1ll << 32)) return LI_ERR_SHAPE;
  if (sorted) setup_zero_region(a, max_row, kv_st, num_txt_blk);
  if (nq == 0) return LI_OK;
  tiles = nq * B * NH;
  if (tiles > 0x7FFFFFFF) return LI_ERR_SHAPE;
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
  a.Lq = (int32_t)(nq * 128);
  a.nkb = (int32_t)(nkv + num_txt_blk);
  if (a.nkb <= 0) return LI_ERR_SHAPE;  // no key block at all
  a.nqt = (int32_t)nq;
  a.n_cols = n_cols;
  a.qk_scale = sm_scale * 1.44269504f;
  BsaGather& g = a.g;
  for (int i = 0; i < 3; ++i) {
    g.qs[i] = k8 ? 0 : q_strides[i];
    g.ks[i] = k8 ? v_strides[i] : k_strides[i];
    g.vs[i] = v_strides[i];
    g.os[i] = out_strides[i];
  }
  g.ktxt = static_cast<const uint16_t*>(k_txt);
  g.vtxt = static_cast<const uint16_t*>(v_txt);
  g.ntxt = num_txt_blk;
  g.H = gq.H;
  g.W = gq.W;
  g.tt = gq.tt;
  g.th = gq.th;
  g.tw = gq.tw;
  g.nh = gq.nh;
  g.nw = gq.nw;
  g.Tq = gq.T;
  g.Tk = gk.T;
  g.mg_nhnw = magic16(gq.nh * gq.nw);
  g.mg_nw = magic16(gq.nw);
  g.mg_thtw = magic16(gq.th * gq.tw);
  g.mg_tw = magic16(gq.tw);
  g.id_nhnw = gq.nh * gq.nw == 1 ? ~0u : 0u;
  g.id_nw = gq.nw == 1 ? ~0u : 0u;
  g.q_tokens = gq.T * gq.H * gq.W;
  g.k_tokens = gk.T * gk.H * gk.W;
  g.txt_tail = 0;
  g.vis_tail = 0;
  return LI_OK;
}

}  // namespace

extern "C" int li_bsa_fwd_gather(int dtype, int32_t B, int32_t NH, int32_t D, const void* q,
                                 const int64_t q_strides[4], const void* k, const int64_t k_strides[4],
                                 const void* v, const int64_t v_strides[4], const void* k_txt, const void* v_txt,
                                 int32_t num_txt_blk, const li_tile_geom* q_geom, const li_tile_geom* k_geom,
                                 const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
                                 const int32_t* block_counts, const int64_t cnt_strides[3], float sm_scale, void* out,
                                 const int64_t out_strides[4], float* lse, void* workspace, int64_t workspace_bytes,
                                 int32_t flags, void* stream) {
  if (dtype != LI_DTYPE_BF16 && dtype != LI_DTYPE_F16) return LI_ERR_UNSUPPORTED;
  BsaArgs a = {};
  int64_t tiles = 0;
  int st = gather_setup(a, tiles, B, NH, D, q, q_strides, k, k_strides, v, v_strides, k_txt, v_txt, num_txt_blk,
                        q_geom, k_geom, block_indices, idx_strides, n_cols, block_counts, cnt_strides, sm_scale, out,
                        out_strides, lse, false, (flags & LI_BSA_SORTED) != 0);
  if (st != LI_OK || tiles == 0) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = plan_units(a, tiles, D, 128, workspace, workspace_bytes, flags, s);
  if (st != LI_OK) return st;
  if (dtype == LI_DTYPE_BF16) return launch_bsa_gather<Bf16>(a, (int)tiles, s);
  return launch_bsa_gather<F16>(a, (int)tiles, s);
}

// Scratch of li_bsa_fwd_gather_noalloc: the tail split's partials or the
// tile order of LI_BSA_BALANCE (what the workspace of li_bsa_fwd_gather
// holds).  Each device holds its own copy from module load until the process
// ends.  Host code must not pass the array's name to a kernel (it is a
// host-side stand-in); scratch_ptr() gives the device address instead.
constexpr int64_t kScratchBytes = 32ll << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

// Device address of `scratch` on the current device, looked up once per
// device with hipGetSymbolAddress and cached; null (with the error recorded
// for li_last_error) when the lookup fails.
void* scratch_ptr() {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      record_launch_error(e != hipSuccess ? e : hipErrorInvalidSymbol);
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

}  // namespace

extern "C" int li_bsa_fwd_gather_noalloc(int dtype, int32_t B, int32_t NH, int32_t D, const void* q,
                                         const int64_t q_strides[4], const void* k, const int64_t k_strides[4],
                                         const void* v, const int64_t v_strides[4], const void* k_txt,
                                         const void* v_txt, int32_t num_txt_blk, const li_tile_geom* q_geom,
                                         const li_tile_geom* k_geom, const int32_t* block_indices,
                                         const int64_t idx_strides[4], int32_t n_cols, const int32_t* block_counts,
                                         const int64_t cnt_strides[3], float sm_scale, void* out,
                                         const int64_t out_strides[4], float* lse, int32_t flags, void* stream) {
  if (dtype != LI_DTYPE_BF16 && dtype != LI_DTYPE_F16) return LI_ERR_UNSUPPORTED;
  BsaArgs a = {};
  int64_t tiles = 0;
  int st = gather_setup(a, tiles, B, NH, D, q, q_strides, k, k_strides, v, v_strides, k_txt, v_txt, num_txt_blk,
                        q_geom, k_geom, block_indices, idx_strides, n_cols, block_counts, cnt_strides, sm_scale, out,
                        out_strides, lse, false, (flags & LI_BSA_SORTED) != 0);
  if (st != LI_OK || tiles == 0) return st;
  // The workspace li_bsa_fwd_gather would use for this call must fit the scratch.
  const int64_t need = li_bsa_fwd_workspace_size(B, NH, a.nqt * 128, D, 128);
  if (need > kScratchBytes) return LI_ERR_TOO_LARGE;
  void* ws = scratch_ptr();
  if (!ws) return LI_ERR_LAUNCH;
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = plan_units(a, tiles, D, 128, ws, need, flags, s);
  if (st != LI_OK) return st;
  if (dtype == LI_DTYPE_BF16) return launch_bsa_gather<Bf16>(a, (int)tiles, s);
  return launch_bsa_gather<F16>(a, (int)tiles, s);
}

extern "C" int64_t li_bsa_fwd_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int li_bsa_fwd_fp8(int32_t B, int32_t NH, int32_t Lq, int32_t Lk, int32_t D, const void* q8,
                              const float* q_scale, const void* k8, const float* k_scale, const void* v,
                              const int32_t* block_indices, const int64_t idx_strides[4], int32_t n_cols,
                              const int32_t* block_counts, const int64_t cnt_strides[3], float sm_scale,
                              int32_t block_size, void* out, float* lse, void* workspace, int64_t workspace_bytes,
                              int32_t flags, void* stream) {
  if (!q8 || !q_scale || !k8 || !k_scale || !v || !block_indices || !idx_strides || !block_counts || !cnt_strides ||
      !out)
    return LI_ERR_INVALID_ARG;
  if (B <= 0 || NH <= 0 || Lq < 0 || Lk < 0 || D <= 0 || n_cols < 0 || block_size <= 0) return LI_ERR_INVALID_ARG;
  if (Lk % block_size != 0) return LI_ERR_K_LEN;
  if (D != 128 || block_size != 128) return LI_ERR_UNSUPPORTED;
  if (!aligned16(q8) || !aligned16(k8) || !aligned16(v) || !aligned16(out) ||
      ((reinterpret_cast<uintptr_t>(q_scale) | reinterpret_cast<uintptr_t>(k_scale)) & 3u))
    return LI_ERR_INVALID_ARG;
  if (Lq == 0) return LI_OK;
  const int64_t nqt = (Lq + block_size - 1) / block_size;
  const int64_t tiles = nqt * B * NH;
  if (tiles > 0x7FFFFFFF) return LI_ERR_SHAPE;
  BsaArgs a = {};
  a.q = static_cast<const uint16_t*>(q8);
  a.k = static_cast<const uint16_t*>(k8);
  a.v = static_cast<const uint16_t*>(v);
  a.q_scale = q_scale;
  a.k_scale = k_scale;
  a.idx = block_indices;
  for (int i = 0; i < 4; ++i) a.is[i] = idx_strides[i];
  a.cnt = block_counts;
  for (int i = 0; i < 3; ++i) a.cs[i] = cnt_strides[i];
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.NH = NH;
  a.Lq = Lq;
  a.nkb = Lk / block_size;
  // No key block at all: there is nothing to attend to (and no block 0 to
  // stand in for out-of-range ids).
  if (a.nkb <= 0) return LI_ERR_SHAPE;
  a.nqt = (int32_t)nqt;
  a.n_cols = n_cols;
  a.qk_scale = sm_scale * 1.44269504f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int st = plan_units(a, tiles, D, block_size, workspace, workspace_bytes, flags, s);
  if (st != LI_OK) return st;
  return launch_bsa_fp8<false>(a, (int)tiles, s);
}

extern "C" int li_bsa_fwd_fp8_gather(int32_t B, int32_t NH, int32_t D, const void* q8, const float* q_scale,
                                     const void* k8, const float* k_scale, const void* v, const int64_t v_strides[4],
                                     const void* v_txt, int32_t num_txt_blk, const li_tile_geom* q_geom,
                                     const li_tile_geom* k_geom, const int32_t* block_indices,
                                     const int64_t idx_strides[4], int32_t n_cols, const int32_t* block_counts,
                                     const int64_t cnt_strides[3], float sm_scale, void* out,
                                     const int64_t out_strides[4], float* lse, void* workspace,
                                     int64_t workspace_bytes, int32_t flags, void* stream) {
  if (!q8 || !q_scale || !k8 || !k_scale || !aligned16(q8) || !aligned16(k8) ||
      ((reinterpret_cast<uintptr_t>(q_scale) | reinterpret_cast<uintptr_t>(k_scale)) & 3u))
    return LI_ERR_INVALID_ARG;
  BsaArgs a = {};
  int64_t tiles = 0;
  int st = gather_setup(a, tiles, B, NH, D, q8, nullptr, k8, nullptr, v, v_strides, nullptr, v_txt, num_txt_blk,
                        q_geom, k_geom, block_indices, idx_strides, n_cols, block_counts, cnt_strides, sm_scale, out,
                        out_strides, lse, true, (flags & LI_BSA_SORTED) != 0);
  if (st != LI_OK || tiles == 0) return st;
  a.q_scale = q_scale;
  a.k_scale = k_scale;
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = plan_units(a, tiles, D, 128, workspace, workspace_bytes, flags, s);
  if (st != LI_OK) return st;
  return launch_bsa_fp8<true>(a, (int)tiles, s);
}

extern "C" int li_attn_fwd_dense(int dtype, int32_t B, int32_t NH, int32_t D, int32_t Lq, int32_t Lk, const void* q,
                                 const int64_t q_strides[4], const void* k, const int64_t k_strides[4], const void* v,
                                 const int64_t v_strides[4], const void* k_txt, const void* v_txt, int32_t txt_len,
                                 float sm_scale, void* out, const int64_t out_strides[4], float* lse,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!q_strides || !k_strides || !v_strides || !out_strides) return LI_ERR_INVALID_ARG;
  if (B <= 0 || NH <= 0 || Lq < 0 || Lk < 0 || txt_len < 0) return LI_ERR_INVALID_ARG;
  if (dtype != LI_DTYPE_BF16 && dtype != LI_DTYPE_F16) return LI_ERR_UNSUPPORTED;
  // Keys are read in 4-token chunks of 128-token blocks: D = 128, whole chunks.
  if (D != 128 || Lk % 4 != 0) return LI_ERR_UNSUPPORTED;
  if (Lk + txt_len == 0) return LI_ERR_INVALID_ARG;
  if (!row_view_ok(q, q_strides) || !row_view_ok(out, out_strides)) return LI_ERR_INVALID_ARG;
  if (Lk > 0 && (!row_view_ok(k, k_strides) || !row_view_ok(v, v_strides))) return LI_ERR_INVALID_ARG;
  if (Lk > 0 && (k_strides[2] < D || v_strides[2] < D)) return LI_ERR_UNSUPPORTED;
  if (txt_len > 0 && (!k_txt || !v_txt || !aligned16(k_txt) || !aligned16(v_txt))) return LI_ERR_INVALID_ARG;
  const int64_t nq = (Lq + 127) / 128, nvis = (Lk + 127) / 128, ntxt = (txt_len + 127) / 128;
  if (nq >= 65536 || nvis + ntxt >= 65536) return LI_ERR_SHAPE;
  // Byte offset of a key row from its block's first token, held in 32 bits.
  const int64_t kv_st = Lk > 0 ? (k_strides[2] > v_strides[2] ? k_strides[2] : v_strides[2]) : 0;
  if ((127 * kv_st + D) * 2 > (1ll << 32)) return LI_ERR_SHAPE;
  if (Lq == 0) return LI_OK;
  const int64_t tiles = nq * B * NH;
  if (tiles > 0x7FFFFFFF) return LI_ERR_SHAPE;
  BsaArgs a = {};
  // Every tile keeps blocks 0 .. n - 1 in order, text blocks first.
  setup_zero_region(a, 127, kv_st, (int32_t)ntxt);
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.idx = nullptr;   // every tile keeps every block, in order
  a.cnt = nullptr;
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.NH = NH;
  a.Lq = (int32_t)(nq * 128);
  a.nkb = (int32_t)(ntxt + nvis);
  if (a.nkb <= 0) return LI_ERR_SHAPE;  // no key block at all
  a.nqt = (int32_t)nq;
  a.n_cols = a.nkb;
  a.qk_scale = sm_scale * 1.44269504f;
  // The token sequence as a grid of 128-token rows: T = blocks, H = 1,
  // W = 128, tile (1, 1, 128), so block t holds tokens 128 t .. 128 t + 127.
  BsaGather& g = a.g;
  for (int i = 0; i < 3; ++i) {
    g.qs[i] = q_strides[i];
    g.ks[i] = Lk > 0 ? k_strides[i] : 0;
    g.vs[i] = Lk > 0 ? v_strides[i] : 0;
    g.os[i] = out_strides[i];
  }
  g.ktxt = static_cast<const uint16_t*>(k_txt);
  g.vtxt = static_cast<const uint16_t*>(v_txt);
  g.ntxt = (int32_t)ntxt;
  g.H = 1;
  g.W = 128;
  g.tt = 1;
  g.th = 1;
  g.tw = 128;
  g.nh = 1;
  g.nw = 1;
  g.Tq = (int32_t)nq;
  g.Tk = (int32_t)nvis;
  g.mg_nhnw = magic16(1);
  g.mg_nw = magic16(1);
  g.mg_thtw = magic16(128);
  g.mg_tw = magic16(128);
  g.id_nhnw = ~0u;
  g.id_nw = ~0u;
  g.q_tokens = Lq;
  g.k_tokens = Lk;
  g.txt_tail = txt_len % 128;
  g.vis_tail = Lk % 128;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int st = plan_units(a, tiles, D, 128, workspace, workspace_bytes, 0, s);
  if (st != LI_OK) return st;
  if (dtype == LI_DTYPE_BF16) return launch_bsa_gather<Bf16, true>(a, (int)tiles, s);
  return launch_bsa_gather<F16, true>(a, (int)tiles, s);
}
