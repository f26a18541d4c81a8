// 3D (t,h,w) tile gather with fixed-order fp32 mean pooling, and its inverse
// scatter, for gfx950.
//
// Replaces the Triton kernels _fused_q_prep_kernel, _fused_kv_prep_kernel and
// _fused_untile_kernel (hy-worldplay/.../ar_sparse_operation.py:26-161; copies in
// bi_sparse_operation_for_KV_cache.py:27-163 and matrix-game-3.0/.../bi_sparse_operation.py:25-140).
//
// Index maps (ar_sparse_operation.py:42-59): block blk -> (ct, ch, cw) =
// (blk / (nh*nw), (blk / nw) % nh, blk % nw); tile row f -> (ft, fh, fw) =
// (f / (tw*th), (f / tw) % th, f % tw); token l = t*H*W + h*W + w.
//
// One 256-thread workgroup per (tile, batch*head).  Thread t owns the 16-byte
// column chunk c = t % (D/8) (8 elements) of tile rows f = g, g+NG, ... with
// g = t / (D/8) and NG = 256 / (D/8): sixteen consecutive threads move one
// 256-byte token row, so every global access is a coalesced 16-byte vector
// access whenever the row is contiguous.  The pool sums each group's rows
// sequentially in fp32 from +0.0, then combines the NG partials with the
// pairwise tree s[g] += s[g + stride], stride = NG/2 .. 1, and divides by BS.
// That order is fixed so the pooled values are reproducible bit for bit.
#include "li_common.hpp"

namespace li {
namespace {

struct GatherArgs {
  const uint16_t* src[2];
  int64_t ss[2][4];
  uint16_t* dst[2];
  int64_t ds[2][5];
  uint16_t* mean;
  int64_t ms[4];
  // Optional second pool output (strides ms): each pooled row divided by its
  // L2 norm as the cosine block-mask metric normalises it.
  uint16_t* mean_n;
  int64_t dst_off, pool_off;
  int32_t NH, bs;
  li_tile_geom g;
  int32_t vec_src, vec_dst;
  uint32_t mg_tw, mg_th;  // udiv16 magics of tw and th
  // e4m3 output of tensor 0 (Q8 kernels): one fp32 scale per tile block.
  float* scale;
  int64_t scs[3];
};

__device__ __forceinline__ u32x4 load8(const uint16_t* p, int64_t stride, bool vec) {
  if (vec) return *reinterpret_cast<const u32x4*>(p);
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack2(p[(2 * i) * stride], p[(2 * i + 1) * stride]);
  return r;
}

__device__ __forceinline__ void store8(uint16_t* p, int64_t stride, bool vec, u32x4 v) {
  if (vec) {
    *reinterpret_cast<u32x4*>(p) = v;
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[(2 * i) * stride] = uint16_t(v[i] & 0xFFFFu);
    p[(2 * i + 1) * stride] = uint16_t(v[i] >> 16);
  }
}

// Workgroup -> (tile block, b*h) for a (blocks, B*NH) grid, heads fastest in
// dispatch order: the workgroups in flight together read the same tokens of
// every head, which with (B, L, H, D) token views is one contiguous span per
// token instead of one head's 2*D bytes of it.
__device__ __forceinline__ void tile_unit(int& blk, int& bh) {
  const uint64_t nbh = gridDim.y;
  const uint64_t lin = blockIdx.x + (uint64_t)gridDim.x * blockIdx.y;
  blk = (int)(lin / nbh);
  bh = (int)(lin - (uint64_t)blk * nbh);
}

// VEC: every row of the source and the tiles is moved with 16-byte vector
// accesses (unit innermost stride, 16-byte aligned rows).  The element-wise
// path for other strides is a separate instantiation, so the vector one does
// not carry its per-element address registers.
template <typename E, int D, int NT, bool VEC>
__device__ __forceinline__ void gather_pool_block(const GatherArgs& a, int blk, int bh) {
  constexpr int CPR = D / 8;
  constexpr int NG = 256 / CPR;
  __shared__ float red[NG][D];

  const int b = bh / a.NH, h = bh % a.NH;
  const int tid = threadIdx.x;
  const int c = tid % CPR, g0 = tid / CPR;
  const li_tile_geom& g = a.g;
  const int cw = blk % g.nw, rem = blk / g.nw;
  const int ch = rem % g.nh, ct = rem / g.nh;
  const bool vs = VEC || a.vec_src != 0, vd = VEC || a.vec_dst != 0;

  // NT tensors gathered into tiles (the first one also pooled); NT = 0 pools
  // tensor 0 without writing tiles.
  constexpr int NS = NT > 0 ? NT : 1;
  const uint16_t* sbase[NS];
  uint16_t* dbase[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    sbase[n] = a.src[n] + b * a.ss[n][0] + h * a.ss[n][1] + (int64_t)(8 * c) * a.ss[n][3];
    dbase[n] = NT > 0 ? a.dst[n] + b * a.ds[n][0] + h * a.ds[n][1] + (blk + a.dst_off) * a.ds[n][2] +
                            (int64_t)(8 * c) * a.ds[n][4]
                      : nullptr;
  }

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;

  // R rows per thread in flight: all loads of a batch are issued before its
  // rows are stored and summed (in row order, so the sums are unchanged).
  constexpr int R = 8;
  for (int f0 = g0; f0 < a.bs; f0 += R * NG) {
    u32x4 v[NS][R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t f = f0 + i * NG;
      const uint32_t r = udiv16(f, a.mg_tw), fw = f - r * (uint32_t)g.tw;
      const uint32_t ft = udiv16(r, a.mg_th), fh = r - ft * (uint32_t)g.th;
      const int t = ct * g.tt + (int)ft, hh = ch * g.th + (int)fh, w = cw * g.tw + (int)fw;
      const bool valid = ((int)f < a.bs) && (t < g.T) && (hh < g.H) && (w < g.W);
      const int64_t l = (int64_t)t * g.H * g.W + (int64_t)hh * g.W + w;
#pragma unroll
      for (int n = 0; n < NS; ++n) {
        v[n][i] = u32x4{0u, 0u, 0u, 0u};
        if (valid) v[n][i] = load8(sbase[n] + l * a.ss[n][2], a.ss[n][3], vs);
      }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int f = f0 + i * NG;
      if (f >= a.bs) break;
#pragma unroll
      for (int n = 0; n < NS; ++n)
        if constexpr (NT > 0) store8(dbase[n] + (int64_t)f * a.ds[n][3], a.ds[n][4], vd, v[n][i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[2 * e] = acc[2 * e] + E::to_f32(uint16_t(v[0][i][e] & 0xFFFFu));
        acc[2 * e + 1] = acc[2 * e + 1] + E::to_f32(uint16_t(v[0][i][e] >> 16));
      }
    }
  }

#pragma unroll
  for (int i = 0; i < 8; ++i) red[g0][8 * c + i] = acc[i];
  __syncthreads();
  float mrow = 0.0f;
  if (tid < D) {
    float s[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) s[i] = red[i][tid];
#pragma unroll
    for (int stride = NG / 2; stride >= 1; stride /= 2) {
#pragma unroll
      for (int i = 0; i < stride; ++i) s[i] = s[i] + s[i + stride];
    }
    const float mean = s[0] / (float)a.bs;
    a.mean[b * a.ms[0] + h * a.ms[1] + (blk + a.pool_off) * a.ms[2] + (int64_t)tid * a.ms[3]] = E::from_f32(mean);
    mrow = E::to_f32(E::from_f32(mean));
  }
  if (a.mean_n) {
    // The cosine metric's normalisation of the rounded row: sequential fp32
    // sum of squares over d from +0.0, x / max(E(sqrt(.)), E(1e-12)), the
    // arithmetic the block mask applies to a raw key pool row.
    __syncthreads();  // the partial sums are read
    if (tid < D) red[0][tid] = mrow;
    __syncthreads();
    // Wave 0 alone finishes the row (every lane runs the same chain over
    // broadcast reads); the other waves end here and free their slots.
    if (tid >= 64) return;
    float ss = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) ss = ss + red[0][d] * red[0][d];
    const float nrm = E::to_f32(E::from_f32(__builtin_sqrtf(ss)));
    const float eps = E::to_f32(E::from_f32(1e-12f));
    const float den = nrm > eps ? nrm : eps;
#pragma unroll
    for (int d = tid; d < D; d += 64)
      a.mean_n[b * a.ms[0] + h * a.ms[1] + (blk + a.pool_off) * a.ms[2] + (int64_t)d * a.ms[3]] =
          E::from_f32(red[0][d] / den);
  }
}

template <typename E, int D, int NT, bool VEC>
__global__ __launch_bounds__(256, VEC ? 4 : 1) void gather_pool_kernel(GatherArgs a) {
  int blk, bh;
  tile_unit(blk, bh);
  gather_pool_block<E, D, NT, VEC>(a, blk, bh);
}

// Two pools in one launch (the query and key pools of one attention call):
// tile blocks 0 .. n0 - 1 of the grid pool job a0, the others pool job a1,
// counted from 0 again.  The jobs share B, NH, D, the element type and the
// vector flag; sources, geometry, pool buffers and offsets are their own.
template <typename E, int D, bool VEC>
__global__ __launch_bounds__(256, VEC ? 4 : 1) void pool_pair_kernel(GatherArgs a0, GatherArgs a1, int32_t n0) {
  int blk, bh;
  tile_unit(blk, bh);
  if (blk < n0)
    gather_pool_block<E, D, 0, VEC>(a0, blk, bh);
  else
    gather_pool_block<E, D, 0, VEC>(a1, blk - n0, bh);
}

// The same gather with tensor 0 written as OCP e4m3 codes (1 byte per
// element, rows of D bytes) plus one fp32 scale per tile block:
// amax = max |x| over the block (padding rows are zeros), scale = amax / 448,
// codes e4m3(x * (448 / amax)), both quotients correctly rounded in fp32;
// scale 1 and zero codes for an all-zero block.  After scaling no finite
// element exceeds 448 (1 + 2^-23), which rounds to 448, so v_cvt_pk_fp8_f32
// (round to nearest even) never saturates or yields NaN.  Its mean pool (of
// the unquantized values, written when a.mean is set) and tensor 1 (NT = 2,
// copied unquantized) are as in gather_pool_kernel.  The whole block is held
// in registers (BS <= 8 NG rows): loads, then the workgroup's amax, then the
// stores.
template <typename E, int D, int NT, bool VEC>
__global__ __launch_bounds__(256, VEC ? 4 : 1) void gather_fp8_kernel(GatherArgs a) {
  constexpr int CPR = D / 8;
  constexpr int NG = 256 / CPR;
  constexpr int R = 8;
  __shared__ float red[NG][D];
  __shared__ uint32_t wmax[4];

  int blk, bh;
  tile_unit(blk, bh);
  const int b = bh / a.NH, h = bh % a.NH;
  const int tid = threadIdx.x;
  const int c = tid % CPR, g0 = tid / CPR;
  const li_tile_geom& g = a.g;
  const int cw = blk % g.nw, rem = blk / g.nw;
  const int ch = rem % g.nh, ct = rem / g.nh;
  const bool vs = VEC || a.vec_src != 0, vd = VEC || a.vec_dst != 0;

  const uint16_t* sbase[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n)
    sbase[n] = a.src[n] + b * a.ss[n][0] + h * a.ss[n][1] + (int64_t)(8 * c) * a.ss[n][3];
  uint8_t* d8 = reinterpret_cast<uint8_t*>(a.dst[0]) + b * a.ds[0][0] + h * a.ds[0][1] +
                (blk + a.dst_off) * a.ds[0][2] + 8 * c;
  uint16_t* d1 = NT > 1 ? a.dst[NT - 1] + b * a.ds[NT - 1][0] + h * a.ds[NT - 1][1] +
                              (blk + a.dst_off) * a.ds[NT - 1][2] + (int64_t)(8 * c) * a.ds[NT - 1][4]
                        : nullptr;

  u32x4 v[NT][R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const uint32_t f = g0 + i * NG;
    const uint32_t r = udiv16(f, a.mg_tw), fw = f - r * (uint32_t)g.tw;
    const uint32_t ft = udiv16(r, a.mg_th), fh = r - ft * (uint32_t)g.th;
    const int t = ct * g.tt + (int)ft, hh = ch * g.th + (int)fh, w = cw * g.tw + (int)fw;
    const bool valid = ((int)f < a.bs) && (t < g.T) && (hh < g.H) && (w < g.W);
    const int64_t l = (int64_t)t * g.H * g.W + (int64_t)hh * g.W + w;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      v[n][i] = u32x4{0u, 0u, 0u, 0u};
      if (valid) v[n][i] = load8(sbase[n] + l * a.ss[n][2], a.ss[n][3], vs);
    }
  }

  // Largest magnitude: for finite 16-bit floats the magnitude bits order as
  // the values do.
  uint32_t mb = 0;
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t x = v[0][i][e];
      mb = __builtin_elementwise_max(mb, __builtin_elementwise_max(x & 0x7FFFu, (x >> 16) & 0x7FFFu));
    }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mb = __builtin_elementwise_max(mb, (uint32_t)__shfl_xor((int)mb, o));
  if ((tid & 63) == 0) wmax[tid >> 6] = mb;
  __syncthreads();
  mb = __builtin_elementwise_max(__builtin_elementwise_max(wmax[0], wmax[1]),
                                 __builtin_elementwise_max(wmax[2], wmax[3]));
  const float amax = E::to_f32((uint16_t)mb);
  const bool zero = !(amax > 0.0f);
  const float scale = zero ? 1.0f : amax / 448.0f;
  const float inv = zero ? 1.0f : 448.0f / amax;
  if (tid == 0) a.scale[b * a.scs[0] + h * a.scs[1] + (blk + a.dst_off) * a.scs[2]] = scale;

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int f = g0 + i * NG;
    if (f >= a.bs) break;
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = E::to_f32(uint16_t(v[0][i][e] & 0xFFFFu));
      x[2 * e + 1] = E::to_f32(uint16_t(v[0][i][e] >> 16));
    }
    u32x2 q;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      int w = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * p] * inv, x[4 * p + 1] * inv, 0, false);
      w = __builtin_amdgcn_cvt_pk_fp8_f32(x[4 * p + 2] * inv, x[4 * p + 3] * inv, w, true);
      q[p] = (uint32_t)w;
    }
    *reinterpret_cast<u32x2*>(d8 + (int64_t)f * a.ds[0][3]) = q;
    if constexpr (NT > 1) store8(d1 + (int64_t)f * a.ds[NT - 1][3], a.ds[NT - 1][4], vd, v[NT - 1][i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = acc[e] + x[e];
  }

  if (!a.mean) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) red[g0][8 * c + i] = acc[i];
  __syncthreads();
  if (tid < D) {
    float s[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) s[i] = red[i][tid];
#pragma unroll
    for (int stride = NG / 2; stride >= 1; stride /= 2) {
#pragma unroll
      for (int i = 0; i < stride; ++i) s[i] = s[i] + s[i + stride];
    }
    const float mean = s[0] / (float)a.bs;
    a.mean[b * a.ms[0] + h * a.ms[1] + (blk + a.pool_off) * a.ms[2] + (int64_t)tid * a.ms[3]] = E::from_f32(mean);
  }
}

struct UntileArgs {
  const uint16_t* src;
  int64_t ss[5];
  uint16_t* dst;
  int64_t ds[4];
  int32_t NH, bs;
  li_tile_geom g;
  int32_t vec_src, vec_dst;
};

template <int D, bool VEC>
__global__ __launch_bounds__(256) void untile_kernel(UntileArgs a) {
  constexpr int CPR = D / 8;
  constexpr int NG = 256 / CPR;
  int blk, bh;
  tile_unit(blk, bh);
  const int b = bh / a.NH, h = bh % a.NH;
  const int tid = threadIdx.x;
  const int c = tid % CPR, g0 = tid / CPR;
  const li_tile_geom& g = a.g;
  const int cw = blk % g.nw, rem = blk / g.nw;
  const int ch = rem % g.nh, ct = rem / g.nh;
  const bool vs = VEC || a.vec_src != 0, vd = VEC || a.vec_dst != 0;
  const uint16_t* sbase = a.src + b * a.ss[0] + h * a.ss[1] + blk * a.ss[2] + (int64_t)(8 * c) * a.ss[4];
  uint16_t* dbase = a.dst + b * a.ds[0] + h * a.ds[1] + (int64_t)(8 * c) * a.ds[3];
  for (int f = g0; f < a.bs; f += NG) {
    const int fw = f % g.tw, r = f / g.tw;
    const int fh = r % g.th, ft = r / g.th;
    const int t = ct * g.tt + ft, hh = ch * g.th + fh, w = cw * g.tw + fw;
    if ((t < g.T) && (hh < g.H) && (w < g.W)) {
      const int64_t l = (int64_t)t * g.H * g.W + (int64_t)hh * g.W + w;
      u32x4 v = load8(sbase + (int64_t)f * a.ss[3], a.ss[4], vs);
      store8(dbase + l * a.ds[2], a.ds[3], vd, v);
    }
  }
}

// 16-byte vector access is legal when the innermost stride is 1 and every row
// start (and the base pointer) is 16-byte aligned.
bool vec_ok(const void* p, const int64_t* strides, int nd) {
  if (strides[nd - 1] != 1) return false;
  if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0) return false;
  for (int i = 0; i < nd - 1; ++i)
    if (strides[i] % 8 != 0) return false;
  return true;
}

int check_geom(const li_tile_geom* g) {
  if (!g) return LI_ERR_INVALID_ARG;
  if (g->T < 0 || g->H <= 0 || g->W <= 0 || g->tt <= 0 || g->th <= 0 || g->tw <= 0) return LI_ERR_SHAPE;
  if (g->nh != (g->H + g->th - 1) / g->th || g->nw != (g->W + g->tw - 1) / g->tw) return LI_ERR_SHAPE;
  return LI_OK;
}

int64_t num_blocks(const li_tile_geom* g) { return (int64_t)((g->T + g->tt - 1) / g->tt) * g->nh * g->nw; }

// Checks the geometry and fills a's launch fields; nblk = tile blocks (0:
// nothing to launch, fields unset).
int gather_setup(int32_t B, int32_t NH, GatherArgs& a, const li_tile_geom* geom, int64_t& nblk) {
  nblk = 0;
  if (B <= 0 || NH <= 0) return LI_ERR_INVALID_ARG;
  int st = check_geom(geom);
  if (st != LI_OK) return st;
  const int64_t n = num_blocks(geom);
  if (n == 0) return LI_OK;
  if (n > 0x7FFFFFFF || (int64_t)B * NH > 65535) return LI_ERR_SHAPE;
  if ((int64_t)geom->tt * geom->th * geom->tw >= 65536) return LI_ERR_SHAPE;
  a.NH = NH;
  a.bs = geom->tt * geom->th * geom->tw;
  a.g = *geom;
  a.mg_tw = magic16(geom->tw);
  a.mg_th = magic16(geom->th);
  nblk = n;
  return LI_OK;
}

template <int NT, bool Q8 = false>
int launch_gather(int dtype, int32_t B, int32_t NH, int32_t D, GatherArgs& a, const li_tile_geom* geom,
                  hipStream_t stream) {
  int64_t nblk = 0;
  const int st = gather_setup(B, NH, a, geom, nblk);
  if (st != LI_OK || nblk == 0) return st;
  dim3 grid((unsigned)nblk, (unsigned)(B * NH));
  if constexpr (Q8) {
    // The block is held in registers: at most 8 rows per thread.
    if (a.bs > 8 * (256 / (D / 8))) return LI_ERR_UNSUPPORTED;
    clear_launch_error();
    const bool vec = a.vec_src && (NT < 2 || a.vec_dst);
#define LI_FP8_LAUNCH(E_, D_)                                                                   \
  do {                                                                                         \
    if (vec)                                                                                   \
      hipLaunchKernelGGL((gather_fp8_kernel<E_, D_, NT, true>), grid, dim3(256), 0, stream, a);  \
    else                                                                                       \
      hipLaunchKernelGGL((gather_fp8_kernel<E_, D_, NT, false>), grid, dim3(256), 0, stream, a); \
  } while (0)
    if (dtype == LI_DTYPE_BF16 && D == 128)
      LI_FP8_LAUNCH(Bf16, 128);
    else if (dtype == LI_DTYPE_BF16 && D == 64)
      LI_FP8_LAUNCH(Bf16, 64);
    else if (dtype == LI_DTYPE_F16 && D == 128)
      LI_FP8_LAUNCH(F16, 128);
    else if (dtype == LI_DTYPE_F16 && D == 64)
      LI_FP8_LAUNCH(F16, 64);
    else
      return LI_ERR_UNSUPPORTED;
#undef LI_FP8_LAUNCH
    return launch_status();
  }
  clear_launch_error();
  const bool vec = a.vec_src && (NT == 0 || a.vec_dst);
#define LI_GATHER_LAUNCH(E_, D_)                                                                 \
  do {                                                                                          \
    if (vec)                                                                                    \
      hipLaunchKernelGGL((gather_pool_kernel<E_, D_, NT, true>), grid, dim3(256), 0, stream, a);  \
    else                                                                                        \
      hipLaunchKernelGGL((gather_pool_kernel<E_, D_, NT, false>), grid, dim3(256), 0, stream, a); \
  } while (0)
  if (dtype == LI_DTYPE_BF16 && D == 128)
    LI_GATHER_LAUNCH(Bf16, 128);
  else if (dtype == LI_DTYPE_BF16 && D == 64)
    LI_GATHER_LAUNCH(Bf16, 64);
  else if (dtype == LI_DTYPE_F16 && D == 128)
    LI_GATHER_LAUNCH(F16, 128);
  else if (dtype == LI_DTYPE_F16 && D == 64)
    LI_GATHER_LAUNCH(F16, 64);
  else
    return LI_ERR_UNSUPPORTED;
#undef LI_GATHER_LAUNCH
  return launch_status();
}

bool pool_supported(int dtype, int32_t D) {
  return (dtype == LI_DTYPE_BF16 || dtype == LI_DTYPE_F16) && (D == 128 || D == 64);
}

// Pools a0 (geometry g0) and a1 (g1) in one launch when both have blocks and
// the same vector flag, else as two launches of the single pool.
int launch_pool_pair(int dtype, int32_t B, int32_t NH, int32_t D, GatherArgs& a0, const li_tile_geom* g0,
                     GatherArgs& a1, const li_tile_geom* g1, hipStream_t stream) {
  int64_t n0 = 0, n1 = 0;
  int st = gather_setup(B, NH, a0, g0, n0);
  if (st == LI_OK) st = gather_setup(B, NH, a1, g1, n1);
  if (st != LI_OK) return st;
  if (!pool_supported(dtype, D)) return LI_ERR_UNSUPPORTED;
  if (n0 == 0 || n1 == 0 || a0.vec_src != a1.vec_src || n0 + n1 > 0x7FFFFFFF) {
    st = launch_gather<0>(dtype, B, NH, D, a0, g0, stream);
    return st != LI_OK ? st : launch_gather<0>(dtype, B, NH, D, a1, g1, stream);
  }
  clear_launch_error();
  const dim3 grid((unsigned)(n0 + n1), (unsigned)(B * NH));
  const int32_t n0i = (int32_t)n0;
#define LI_PAIR_LAUNCH(E_, D_)                                                                   \
  do {                                                                                          \
    if (a0.vec_src)                                                                             \
      hipLaunchKernelGGL((pool_pair_kernel<E_, D_, true>), grid, dim3(256), 0, stream, a0, a1, n0i);  \
    else                                                                                        \
      hipLaunchKernelGGL((pool_pair_kernel<E_, D_, false>), grid, dim3(256), 0, stream, a0, a1, n0i); \
  } while (0)
  if (dtype == LI_DTYPE_BF16 && D == 128)
    LI_PAIR_LAUNCH(Bf16, 128);
  else if (dtype == LI_DTYPE_BF16 && D == 64)
    LI_PAIR_LAUNCH(Bf16, 64);
  else if (dtype == LI_DTYPE_F16 && D == 128)
    LI_PAIR_LAUNCH(F16, 128);
  else
    LI_PAIR_LAUNCH(F16, 64);
#undef LI_PAIR_LAUNCH
  return launch_status();
}

// Fills a pool-only job (no tiles written); false on a null pointer or a negative offset.
bool pool_job(GatherArgs& a, const void* src, const int64_t* ss, void* mean, const int64_t* ms, int64_t pool_off) {
  if (!src || !mean || !ss || !ms || pool_off < 0) return false;
  a = GatherArgs{};
  a.src[0] = static_cast<const uint16_t*>(src);
  a.dst[0] = nullptr;
  for (int i = 0; i < 4; ++i) {
    a.ss[0][i] = ss[i];
    a.ms[i] = ms[i];
  }
  a.mean = static_cast<uint16_t*>(mean);
  a.pool_off = pool_off;
  a.vec_src = vec_ok(src, ss, 4);
  return true;
}

}  // namespace
}  // namespace li

using namespace li;

extern "C" int li_q_prep(int dtype, int32_t B, int32_t NH, int32_t D, const void* src, const int64_t src_strides[4],
                         void* dst, const int64_t dst_strides[5], void* mean, const int64_t mean_strides[4],
                         const li_tile_geom* geom, void* stream) {
  if (!src || !dst || !mean || !src_strides || !dst_strides || !mean_strides) return LI_ERR_INVALID_ARG;
  GatherArgs a = {};
  a.src[0] = static_cast<const uint16_t*>(src);
  a.dst[0] = static_cast<uint16_t*>(dst);
  for (int i = 0; i < 4; ++i) a.ss[0][i] = src_strides[i];
  for (int i = 0; i < 5; ++i) a.ds[0][i] = dst_strides[i];
  a.mean = static_cast<uint16_t*>(mean);
  for (int i = 0; i < 4; ++i) a.ms[i] = mean_strides[i];
  a.dst_off = 0;
  a.pool_off = 0;
  a.vec_src = vec_ok(src, src_strides, 4);
  a.vec_dst = vec_ok(dst, dst_strides, 5);
  return launch_gather<1>(dtype, B, NH, D, a, geom, static_cast<hipStream_t>(stream));
}

extern "C" int li_kv_prep(int dtype, int32_t B, int32_t NH, int32_t D, const void* k_src,
                          const int64_t k_src_strides[4], const void* v_src, const int64_t v_src_strides[4],
                          void* k_dst, const int64_t k_dst_strides[5], void* v_dst, const int64_t v_dst_strides[5],
                          void* k_mean, const int64_t mean_strides[4], int64_t dst_off, int64_t pool_off,
                          const li_tile_geom* geom, void* stream) {
  if (!k_src || !v_src || !k_dst || !v_dst || !k_mean || !k_src_strides || !v_src_strides || !k_dst_strides ||
      !v_dst_strides || !mean_strides)
    return LI_ERR_INVALID_ARG;
  if (dst_off < 0 || pool_off < 0) return LI_ERR_INVALID_ARG;
  GatherArgs a = {};
  a.src[0] = static_cast<const uint16_t*>(k_src);
  a.src[1] = static_cast<const uint16_t*>(v_src);
  a.dst[0] = static_cast<uint16_t*>(k_dst);
  a.dst[1] = static_cast<uint16_t*>(v_dst);
  for (int i = 0; i < 4; ++i) {
    a.ss[0][i] = k_src_strides[i];
    a.ss[1][i] = v_src_strides[i];
    a.ms[i] = mean_strides[i];
  }
  for (int i = 0; i < 5; ++i) {
    a.ds[0][i] = k_dst_strides[i];
    a.ds[1][i] = v_dst_strides[i];
  }
  a.mean = static_cast<uint16_t*>(k_mean);
  a.dst_off = dst_off;
  a.pool_off = pool_off;
  a.vec_src = vec_ok(k_src, k_src_strides, 4) && vec_ok(v_src, v_src_strides, 4);
  a.vec_dst = vec_ok(k_dst, k_dst_strides, 5) && vec_ok(v_dst, v_dst_strides, 5);
  return launch_gather<2>(dtype, B, NH, D, a, geom, static_cast<hipStream_t>(stream));
}

extern "C" int li_pool(int dtype, int32_t B, int32_t NH, int32_t D, const void* src, const int64_t src_strides[4],
                       void* mean, const int64_t mean_strides[4], int64_t pool_off, const li_tile_geom* geom,
                       void* stream) {
  if (!src || !mean || !src_strides || !mean_strides) return LI_ERR_INVALID_ARG;
  if (pool_off < 0) return LI_ERR_INVALID_ARG;
  GatherArgs a = {};
  a.src[0] = static_cast<const uint16_t*>(src);
  a.dst[0] = nullptr;
  for (int i = 0; i < 4; ++i) {
    a.ss[0][i] = src_strides[i];
    a.ms[i] = mean_strides[i];
  }
  a.mean = static_cast<uint16_t*>(mean);
  a.dst_off = 0;
  a.pool_off = pool_off;
  a.vec_src = vec_ok(src, src_strides, 4);
  a.vec_dst = 0;
  return launch_gather<0>(dtype, B, NH, D, a, geom, static_cast<hipStream_t>(stream));
}

extern "C" int li_untile(int dtype, int32_t B, int32_t NH, int32_t D, const void* src, const int64_t src_strides[5],
                         void* dst, const int64_t dst_strides[4], const li_tile_geom* geom, void* stream) {
  if (!src || !dst || !src_strides || !dst_strides) return LI_ERR_INVALID_ARG;
  if (B <= 0 || NH <= 0) return LI_ERR_INVALID_ARG;
  if (dtype != LI_DTYPE_BF16 && dtype != LI_DTYPE_F16) return LI_ERR_UNSUPPORTED;
  int st = check_geom(geom);
  if (st != LI_OK) return st;
  const int64_t nblk = num_blocks(geom);
  if (nblk == 0) return LI_OK;
  if (nblk > 0x7FFFFFFF || (int64_t)B * NH > 65535) return LI_ERR_SHAPE;
  UntileArgs a = {};
  a.src = static_cast<const uint16_t*>(src);
  a.dst = static_cast<uint16_t*>(dst);
  for (int i = 0; i < 5; ++i) a.ss[i] = src_strides[i];
  for (int i = 0; i < 4; ++i) a.ds[i] = dst_strides[i];
  a.NH = NH;
  a.bs = geom->tt * geom->th * geom->tw;
  a.g = *geom;
  a.vec_src = vec_ok(src, src_strides, 5);
  a.vec_dst = vec_ok(dst, dst_strides, 4);
  dim3 grid((unsigned)nblk, (unsigned)(B * NH));
  hipStream_t s = static_cast<hipStream_t>(stream);
  clear_launch_error();
  const bool vec = a.vec_src && a.vec_dst;
  if (D == 128 && vec)
    hipLaunchKernelGGL((untile_kernel<128, true>), grid, dim3(256), 0, s, a);
  else if (D == 128)
    hipLaunchKernelGGL((untile_kernel<128, false>), grid, dim3(256), 0, s, a);
  else if (D == 64 && vec)
    hipLaunchKernelGGL((untile_kernel<64, true>), grid, dim3(256), 0, s, a);
  else if (D == 64)
    hipLaunchKernelGGL((untile_kernel<64, false>), grid, dim3(256), 0, s, a);
  else
    return LI_ERR_UNSUPPORTED;
  return launch_status();
}

namespace {

// e4m3 tile rows: unit d stride, 8-byte aligned rows; one scale per block.
bool fp8_dst_ok(const void* p, const int64_t st[5]) {
  return p && (reinterpret_cast<uintptr_t>(p) & 7u) == 0 && st[4] == 1 && st[0] % 8 == 0 && st[1] % 8 == 0 &&
         st[2] % 8 == 0 && st[3] % 8 == 0;
}

}  // namespace

extern "C" int li_tile_prep_fp8(int dtype, int32_t B, int32_t NH, int32_t D, const void* src,
                                const int64_t src_strides[4], void* dst, const int64_t dst_strides[5],
                                float* scales, const int64_t scale_strides[3], void* mean,
                                const int64_t mean_strides[4], int64_t dst_off, int64_t pool_off,
                                const li_tile_geom* geom, void* stream) {
  if (!src || !src_strides || !dst_strides || !scales || !scale_strides || (mean && !mean_strides))
    return LI_ERR_INVALID_ARG;
  if (dst_off < 0 || pool_off < 0 || !fp8_dst_ok(dst, dst_strides)) return LI_ERR_INVALID_ARG;
  GatherArgs a = {};
  a.src[0] = static_cast<const uint16_t*>(src);
  a.dst[0] = static_cast<uint16_t*>(dst);
  for (int i = 0; i < 4; ++i) a.ss[0][i] = src_strides[i];
  for (int i = 0; i < 5; ++i) a.ds[0][i] = dst_strides[i];
  a.mean = static_cast<uint16_t*>(mean);
  if (mean)
    for (int i = 0; i < 4; ++i) a.ms[i] = mean_strides[i];
  a.scale = scales;
  for (int i = 0; i < 3; ++i) a.scs[i] = scale_strides[i];
  a.dst_off = dst_off;
  a.pool_off = pool_off;
  a.vec_src = vec_ok(src, src_strides, 4);
  a.vec_dst = 1;
  return launch_gather<1, true>(dtype, B, NH, D, a, geom, static_cast<hipStream_t>(stream));
}

extern "C" int li_kv_prep_fp8(int dtype, int32_t B, int32_t NH, int32_t D, const void* k_src,
                              const int64_t k_src_strides[4], const void* v_src, const int64_t v_src_strides[4],
                              void* k_dst, const int64_t k_dst_strides[5], float* k_scales,
                              const int64_t k_scale_strides[3], void* v_dst, const int64_t v_dst_strides[5],
                              void* k_mean, const int64_t mean_strides[4], int64_t dst_off, int64_t pool_off,
                              const li_tile_geom* geom, void* stream) {
  if (!k_src || !v_src || !v_dst || !k_mean || !k_src_strides || !v_src_strides || !k_dst_strides ||
      !v_dst_strides || !mean_strides || !k_scales || !k_scale_strides)
    return LI_ERR_INVALID_ARG;
  if (dst_off < 0 || pool_off < 0 || !fp8_dst_ok(k_dst, k_dst_strides)) return LI_ERR_INVALID_ARG;
  GatherArgs a = {};
  a.src[0] = static_cast<const uint16_t*>(k_src);
  a.src[1] = static_cast<const uint16_t*>(v_src);
  a.dst[0] = static_cast<uint16_t*>(k_dst);
  a.dst[1] = static_cast<uint16_t*>(v_dst);
  for (int i = 0; i < 4; ++i) {
    a.ss[0][i] = k_src_strides[i];
    a.ss[1][i] = v_src_strides[i];
    a.ms[i] = mean_strides[i];
  }
  for (int i = 0; i < 5; ++i) {
    a.ds[0][i] = k_dst_strides[i];
    a.ds[1][i] = v_dst_strides[i];
  }
  a.mean = static_cast<uint16_t*>(k_mean);
  a.scale = k_scales;
  for (int i = 0; i < 3; ++i) a.scs[i] = k_scale_strides[i];
  a.dst_off = dst_off;
  a.pool_off = pool_off;
  a.vec_src = vec_ok(k_src, k_src_strides, 4) && vec_ok(v_src, v_src_strides, 4);
  a.vec_dst = vec_ok(v_dst, v_dst_strides, 5);
  return launch_gather<2, true>(dtype, B, NH, D, a, geom, static_cast<hipStream_t>(stream));
}

extern "C" int li_pool_pair(int dtype, int32_t B, int32_t NH, int32_t D, const void* src0,
                            const int64_t src0_strides[4], void* mean0, const int64_t mean0_strides[4],
                            int64_t pool_off0, const li_tile_geom* geom0, const void* src1,
                            const int64_t src1_strides[4], void* mean1, const int64_t mean1_strides[4],
                            int64_t pool_off1, const li_tile_geom* geom1, void* mean1_normalized,
                            void* stream) {
  GatherArgs a0, a1;
  if (!pool_job(a0, src0, src0_strides, mean0, mean0_strides, pool_off0) ||
      !pool_job(a1, src1, src1_strides, mean1, mean1_strides, pool_off1))
    return LI_ERR_INVALID_ARG;
  a1.mean_n = static_cast<uint16_t*>(mean1_normalized);
  return launch_pool_pair(dtype, B, NH, D, a0, geom0, a1, geom1, static_cast<hipStream_t>(stream));
}
