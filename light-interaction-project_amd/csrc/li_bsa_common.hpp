// Shared pieces of the block-sparse attention kernels (gfx950).
#pragma once

#include "li_common.hpp"

namespace li {

// Kernel arguments of the attention forward (all pointers are device
// pointers; strides in elements).
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
  // Tail split (D = 128, BS = 128 kernel only): work units u < n_full are
  // whole query tiles; unit n_full + 2p + half is half `half` of tile
  // n_full + p (the first or second half of its kept-block list), which
  // writes unnormalised fp32 O and (m, l) rows to `part` for the merge kernel.
  int32_t n_full;
  float* part;
};

// Launches the 4-wave D = 128, BS = 128 kernel for units [0, a.n_full) whole
// tiles plus the split half-units (li_bsa_fwd_w4.hip).
int launch_bsa_w4(int dtype, BsaArgs& a, int units, hipStream_t s);

namespace {

// MFMA row i of the score tile reads K row perm(i): bits 2 and 3 swapped.
__device__ __forceinline__ int kperm(int i) { return (i & 0x13) | ((i & 4) << 1) | ((i & 8) >> 1); }

typedef short s16x4 __attribute__((ext_vector_type(4)));

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
__device__ __forceinline__ void wait_vm0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace
}  // namespace li
