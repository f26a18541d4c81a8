// Shared device helpers for the gfx950 sparse-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "li_sparse_attn.h"

namespace li {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Element-type traits: storage is always 16-bit; conversion to/from fp32 and
// the matching 32x32x16 MFMA differ.
struct Bf16 {
  typedef bf16x8 vec8;
  static __device__ __forceinline__ float to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    __bf16 h = (__bf16)x;  // round to nearest even
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

struct F16 {
  typedef f16x8 vec8;
  static __device__ __forceinline__ float to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
  // The empty asm keeps x an fp32 value: otherwise the compiler may fold the
  // multiply-add that produced x into the conversion (v_fma_mixlo_f16), one
  // rounding of the exact result where the arithmetic asks for two (fp32, then
  // half), which differs at half-way cases.
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    asm("" : "+v"(x));
    _Float16 h = (_Float16)x;
    return __builtin_bit_cast(uint16_t, h);
  }
  static __device__ __forceinline__ f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) { return uint32_t(lo) | (uint32_t(hi) << 16); }

// x / d for x, d < 2^16 without a division: magic = ceil(2^32 / d), and 0
// encodes d = 1.  With magic = (2^32 + e) / d, 0 <= e < d, the quotient
// x * magic / 2^32 = x / d + x e / (d 2^32) exceeds x / d by less than 1 / d,
// so its floor is exact.  Branch-free: umulhi(x, 0) = 0, and the identity term
// is x only for magic 0.
__device__ __forceinline__ uint32_t udiv16(uint32_t x, uint32_t magic) {
  return __umulhi(x, magic) | (x & (0u - (uint32_t)(magic == 0u)));
}
inline uint32_t magic16(int32_t d) {
  return d == 1 ? 0u : (uint32_t)(((1ull << 32) + (uint64_t)d - 1) / (uint64_t)d);
}

// Launch status: call clear_launch_error() right before a kernel launch and
// launch_status() right after it, so an error left by an earlier, unrelated
// runtime call is not attributed to this launch.  The text of a failed
// launch is kept per thread for li_last_error().
void record_launch_error(hipError_t e);

inline void clear_launch_error() { (void)hipGetLastError(); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return LI_OK;
  record_launch_error(e);
  return LI_ERR_LAUNCH;
}

}  // namespace li
