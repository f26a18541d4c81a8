// Shared pieces of the block-sparse attention kernels (gfx950).
#pragma once

#include "li_common.hpp"

namespace li {

// Token-order addressing of the fused path, in which the tiled Q/K/V/O
// buffers are never materialised: tile row f of block blk of a (t, h, w) grid
// is token l = t*H*W + h*W + w with (t, h, w) = (ct*tt + ft, ch*th + fh,
// cw*tw + fw), (ct, ch, cw) = (blk / (nh*nw), (blk / nw) % nh, blk % nw) and
// (ft, fh, fw) = (f / (th*tw), (f / tw) % th, f % tw) (the tile permutation of
// hy-worldplay/.../ar_sparse_operation.py:42-59); tokens outside the grid
// read as zeros and are not stored.  q, out and the visual k, v are
// (B, NH, L, D) views with element strides (d stride 1); key blocks with ids
// below ntxt are text blocks, read from zero-padded (B, NH, ntxt*BS, D)
// buffers; visual block vb has id ntxt + vb.
struct BsaGather {
  int64_t qs[3], os[3], ks[3], vs[3];  // batch, head, token strides
  const uint16_t* ktxt;
  const uint16_t* vtxt;
  int32_t ntxt;
  int32_t H, W, tt, th, tw, nh, nw, Tq, Tk;
  // ceil(2^32 / d) for d = nh*nw, nw, th*tw, tw (0 for d = 1): x / d ==
  // umulhi(x, magic) exactly for x, d < 2^16.
  uint32_t mg_nhnw, mg_nw, mg_thtw, mg_tw;
  // ~0 where the matching divisor is 1, else 0 (the identity term of udiv16m).
  uint32_t id_nhnw, id_nw;
  // Token bounds: query rows at tokens >= q_tokens are neither read nor
  // stored, and visual K/V chunks starting at tokens >= k_tokens are read as
  // zeros (Tq*H*W and Tk*H*W on the sparse path, where the grid bounds
  // decide).  Dense calls: the last text block keeps txt_tail rows and the
  // last visual block vis_tail rows, the others get score -inf (0 = all
  // rows kept, zero rows included, as on the sparse path).
  int32_t q_tokens, k_tokens;
  int32_t txt_tail, vis_tail;
};

// Kernel arguments of the attention forward (all pointers are device
// pointers; strides in elements).
struct BsaArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  // Kept block ids (B, NH, nqt, n_cols) and their counts (B, NH, nqt), or
  // null for every tile keeping blocks 0 .. n_cols - 1 in order (dense calls).
  const int32_t* idx;
  int64_t is[4];
  const int32_t* cnt;
  int64_t cs[3];
  uint16_t* out;
  float* lse;
  int32_t NH, Lq, nkb, nqt, n_cols;
  float qk_scale;
  // Query tiles of the launch (B * NH * nqt), placed on the XCDs by unit_tile.
  int32_t ntiles;
  // Tail split (D = 128, BS = 128 kernel only; ntiles a multiple of 8): XCD x
  // (unit ids x, x + 8, ...) owns the xtiles = ntiles / 8 tiles from
  // x * xtiles on.  When xsplit > 0, the last xsplit of them run as two
  // halves of their kept-block list, the first ceil(count / 2) blocks and
  // the rest.  Slot s of XCD x (unit 8 s + x) runs whole tile x * xtiles + s
  // for s < xtiles - xsplit, then come the first halves of the split tiles,
  // then their second halves, so a split tile's halves stay on the XCD whose
  // L2 holds its head's keys.  Half e of split tile j of XCD x writes
  // unnormalised fp32 O and (m, l) rows to partial slot 2 (x * xsplit + j) +
  // e of `part` for the merge kernel.
  int32_t xtiles, xsplit;
  float* part;
  // Optional dispatch order of the tiles (a permutation of [0, ntiles);
  // never with the tail split): position p of the XCD-aware unit order runs
  // tile order[p].
  const int32_t* order;
  // XCD chunk: 0 gives each XCD one contiguous range of positions; C > 0
  // (ntiles a multiple of 8 C) deals chunks of C positions round-robin over
  // the XCDs, so the tiles in flight at once span about 8 C positions.
  int32_t xchunk;
  // e4m3 kernel only: q and k hold e4m3 codes (1 byte per element) with one
  // fp32 scale per 128-row tile, (B*NH, nqt) and (B*NH, nkb) contiguous.
  const float* q_scale;
  const float* k_scale;
  // Fused path only (kernel template flag); unused otherwise.
  BsaGather g;
  // Zero-region kernels (fused path, rows listing their text blocks first):
  // zero bytes reaching past the largest K / V row offset of a tile from its
  // origin token.  An out-of-grid chunk of a visual block is read from here
  // at the visual chunk's own lane offsets, so a load picks only its scalar
  // base.  The first gen_pairs block phases of a tile (an even count, enough
  // to cover the text blocks' loads) pick base and lane offset per chunk.
  const char* zero_region;
  int32_t gen_pairs;
};

// Tile of work unit `id` (< a.ntiles): ids are dealt round-robin over
// the 8 XCDs, so they are remapped to give each XCD a contiguous range of
// positions; a.order, when given, names the tile at each position.
__device__ __forceinline__ int unit_tile(const BsaArgs& a, int id) {
  const int xcd = id & 7, slot = id >> 3;
  int pos;
  if (a.xchunk > 0) {
    const int c = a.xchunk;
    pos = ((slot / c) * 8 + xcd) * c + slot % c;
  } else {
    const int per = a.ntiles >> 3, rem = a.ntiles & 7;
    pos = xcd * per + (xcd < rem ? xcd : rem) + slot;
  }
  if (!a.order) return pos;
  const int t = __builtin_amdgcn_readfirstlane(a.order[pos]);
  return t < 0 ? 0 : (t >= a.ntiles ? a.ntiles - 1 : t);
}

namespace {

// MFMA row i of the score tile reads K row perm(i): bits 2 and 3 swapped.
__device__ __forceinline__ int kperm(int i) { return (i & 0x13) | ((i & 4) << 1) | ((i & 8) >> 1); }

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

// 32x32x64 e4m3 MFMA (v_mfma_f32_32x32x64_f8f6f4 with unit scales): lane l
// holds A row l % 32 and B column l % 32, each with the 32 bytes k =
// 32 (l / 32) .. +31 of the 64-deep step; the accumulator layout is that of
// the 32x32x16 16-bit MFMA.
__device__ __forceinline__ f32x16 mfma_e4m3(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Lambdas of the kernels are always inlined: an outlined one would pass the
// accumulators through scratch memory.
#define LI_INLINE __attribute__((always_inline))

// Transposing LDS load (ds_read_b64_tr_b16) of 4 x 16-bit elements.
__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}

template <typename E>
__device__ __forceinline__ uint32_t cvt_pk(float a, float b);
template <>
__device__ __forceinline__ uint32_t cvt_pk<Bf16>(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), h2));
}
template <>
__device__ __forceinline__ uint32_t cvt_pk<F16>(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2{a, b}), h2));
}

template <int N>
struct Stage {
  static constexpr int value = N;
};

// 16 bytes per lane from global memory (wave-uniform base in SGPRs plus a
// per-lane byte offset) straight into LDS at lds_addr + 16 * lane
// (global_load_lds_dwordx4).  Issued as inline assembly so that the
// compiler's wait-count bookkeeping does not see it: the compiler would
// otherwise treat every pending LDS DMA as making the LDS counter unordered
// and drain all operand reads in flight (lgkmcnt(0)) after each one.  Being
// invisible only makes the compiler's own waits stricter (the extra loads
// are counted by the hardware), never weaker; the caller publishes the data
// with wait_vm0() before a barrier.  The s_nop covers the M0-write to LDS-DMA
// hazard.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_addr) : "memory");
}
// The same load with an instruction offset imm (it must fold to a constant in
// [0, 4096)), which the hardware adds to both the global address
// (sbase + voff + imm) and the LDS address (m0 + imm + 16 * lane).
__device__ __forceinline__ void dma16_imm(const void* sbase, uint32_t voff, uint32_t m0_addr, int imm) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 offset:%3" ::"v"(voff), "s"(sbase), "{m0}"(m0_addr),
               "i"(imm)
               : "memory");
}
// The source (sa, va) when bit `bit` of the wave-uniform `mask` is set, else
// (sb, vb): three scalar instructions and one vector select.  Not volatile,
// so the scheduler may compute it well before the load that uses it.
struct DmaSrc {
  const void* base;
  uint32_t voff;
};
__device__ __forceinline__ DmaSrc dma_sel(uint32_t mask, int bit, const void* sa, uint32_t va, const void* sb,
                                         uint32_t vb) {
  DmaSrc r;
  uint64_t lm;
  asm("s_bitcmp1_b32 %[mask], %[bit]\n\t"
      "s_cselect_b64 %[base], %[sa], %[sb]\n\t"
      "s_cselect_b64 %[lm], -1, 0\n\t"
      "v_cndmask_b32_e64 %[voff], %[vb], %[va], %[lm]"
      : [base] "=&s"(r.base), [lm] "=&s"(lm), [voff] "=&v"(r.voff)
      : [mask] "s"(mask), [bit] "i"(bit), [sa] "s"(sa), [sb] "s"(sb), [va] "v"(va), [vb] "v"(vb)
      : "scc");
  return r;
}
// The base sa when bit `bit` of the wave-uniform `mask` is set, else sb,
// with one lane offset for both (two scalar instructions).
__device__ __forceinline__ DmaSrc dma_sel_base(uint32_t mask, int bit, const void* sa, const void* sb, uint32_t voff) {
  DmaSrc r;
  asm("s_bitcmp1_b32 %[mask], %[bit]\n\t"
      "s_cselect_b64 %[base], %[sa], %[sb]"
      : [base] "=&s"(r.base)
      : [mask] "s"(mask), [bit] "i"(bit), [sa] "s"(sa), [sb] "s"(sb)
      : "scc");
  r.voff = voff;
  return r;
}
__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// udiv16 with its identity mask (~0 for magic 0, else 0) passed in.
__device__ __forceinline__ uint32_t udiv16m(uint32_t x, uint32_t magic, uint32_t id) {
  return __umulhi(x, magic) | (x & id);
}

// Token of tile row f of block blk in a grid of T frames; valid = inside.
__device__ __forceinline__ int32_t tile_token(const BsaGather& g, int32_t T, uint32_t blk, uint32_t f, bool& valid) {
  const uint32_t ct = udiv16(blk, g.mg_nhnw), rem = blk - ct * (uint32_t)(g.nh * g.nw);
  const uint32_t ch = udiv16(rem, g.mg_nw), cw = rem - ch * (uint32_t)g.nw;
  const uint32_t ft = udiv16(f, g.mg_thtw), r = f - ft * (uint32_t)(g.th * g.tw);
  const uint32_t fh = udiv16(r, g.mg_tw), fw = r - fh * (uint32_t)g.tw;
  const int32_t t = ct * g.tt + ft, hh = ch * g.th + fh, w = cw * g.tw + fw;
  valid = t < T && hh < g.H && w < g.W;
  return (t * g.H + hh) * g.W + w;
}

// 8 KiB of zeros: the source of DMA chunks that fall outside the grid (chunk
// j < 8 of a wave reads bytes [1024 j, 1024 j + 1024)).
__device__ __attribute__((aligned(16))) const uint32_t g_zero_rows[2048] = {0};

}  // namespace
}  // namespace li
