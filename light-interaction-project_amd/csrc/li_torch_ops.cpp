// PyTorch custom operators torch.ops.li.* over the C ABI of libli_sparse_attn.so.
//
// Each operator checks dtypes and ranks, allocates what it returns (and the
// attention workspace) through the caching allocator, writes the tensors its
// schema marks as mutated (Tensor(a!): tiles, pools, attention outputs), and
// enqueues the C-ABI call on torch's current HIP stream of the tensors' device.  Shape rules and
// the reference's error messages stay in the Python wrappers that call these
// operators (li_sparse/_core.py); the fake (meta) implementations, which give
// output shapes for tracing, are registered in li_sparse/_ops.py.
//
// Reference interfaces replaced (paths relative to the reference repository):
//   hy-worldplay/files/hyvideo/models/transformers/modules/ar_sparse_operation.py:166-218 (launch_q_prep,
//     launch_kv_prep, launch_untile), :223-284 (fast_generate_indices), :289-362 (run_sparse_attention)
//   hy-worldplay/.../longcat_kernel.py:158-233 (longcat_flash_attn)
//   hy-worldplay/.../bi_sparse_operation_for_KV_cache.py:220-296 (generate_prefill_indices)
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <array>
#include <cmath>
#include <string>

#include "li_sparse_attn.h"

namespace {

void check(const char* fn, int st) {
  TORCH_CHECK(st == LI_OK, fn, " failed: ", li_status_string(st), " (status ", st, ")",
              st == LI_ERR_LAUNCH ? std::string(": ") + li_last_error() : std::string());
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

int dtype_code(const at::Tensor& t) {
  if (t.scalar_type() == at::kBFloat16) return LI_DTYPE_BF16;
  if (t.scalar_type() == at::kHalf) return LI_DTYPE_F16;
  TORCH_CHECK(false, "unsupported dtype ", t.scalar_type(), "; expected bfloat16 or float16");
}

void gpu(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be on a ROCm (cuda) device");
}

void rank(const at::Tensor& t, int64_t r, const char* name) {
  TORCH_CHECK(t.dim() == r, name, " must have ", r, " dimensions, got ", t.dim());
}

li_tile_geom geom_of(c10::IntArrayRef g) {
  TORCH_CHECK(g.size() == 8, "geometry must be (T, H, W, tt, th, tw, nh, nw)");
  li_tile_geom r;
  r.T = (int32_t)g[0];
  r.H = (int32_t)g[1];
  r.W = (int32_t)g[2];
  r.tt = (int32_t)g[3];
  r.th = (int32_t)g[4];
  r.tw = (int32_t)g[5];
  r.nh = (int32_t)g[6];
  r.nw = (int32_t)g[7];
  return r;
}

template <size_t N>
std::array<int64_t, N> strides(const at::Tensor& t) {
  std::array<int64_t, N> s{};
  for (size_t i = 0; i < N; ++i) s[i] = t.stride((int64_t)i);
  return s;
}

// Workspace of the attention launches: a caching-allocator buffer of the size
// the library asks for on this device (tail split partials or tile order).
at::Tensor workspace(const at::Tensor& like, int64_t B, int64_t NH, int64_t Lq, int64_t D, int64_t bs, bool want) {
  if (!want) return at::Tensor();
  const int64_t bytes = li_bsa_fwd_workspace_size((int32_t)B, (int32_t)NH, (int32_t)Lq, (int32_t)D, (int32_t)bs);
  if (bytes <= 0) return at::Tensor();
  return at::empty({(bytes + 3) / 4}, like.options().dtype(at::kFloat));
}

void* ptr(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

at::Tensor lse_or_empty(const at::Tensor& like, bool want, int64_t B, int64_t NH, int64_t rows) {
  return at::empty(want ? c10::IntArrayRef({B, NH, rows}) : c10::IntArrayRef({0}), like.options().dtype(at::kFloat));
}

// ---------------------------------------------------------------------------

void pool(const at::Tensor& src, at::Tensor& mean, int64_t pool_off, c10::IntArrayRef geom) {
  gpu(src, "src");
  rank(src, 4, "src");
  rank(mean, 4, "mean");
  c10::DeviceGuard guard(src.device());
  const li_tile_geom g = geom_of(geom);
  const auto ss = strides<4>(src);
  const auto ms = strides<4>(mean);
  check("li_pool", li_pool(dtype_code(src), (int32_t)src.size(0), (int32_t)src.size(1), (int32_t)src.size(3),
                           src.data_ptr(), ss.data(), mean.data_ptr(), ms.data(), pool_off, &g, stream_of(src)));
}

void pool_pair(const at::Tensor& src0, at::Tensor& mean0, int64_t off0, c10::IntArrayRef geom0,
               const at::Tensor& src1, at::Tensor& mean1, int64_t off1, c10::IntArrayRef geom1,
               const c10::optional<at::Tensor>& mean1_normalized) {
  gpu(src0, "src0");
  rank(src0, 4, "src0");
  rank(src1, 4, "src1");
  rank(mean0, 4, "mean0");
  rank(mean1, 4, "mean1");
  void* mean1_n = nullptr;
  if (mean1_normalized.has_value() && mean1_normalized->defined()) {
    const at::Tensor& t = *mean1_normalized;
    TORCH_CHECK(t.sizes() == mean1.sizes() && t.strides() == mean1.strides() && t.scalar_type() == mean1.scalar_type() &&
                    t.device() == mean1.device(),
                "mean1_normalized must match mean1 in shape, strides, dtype and device");
    mean1_n = t.data_ptr();
  }
  c10::DeviceGuard guard(src0.device());
  const li_tile_geom g0 = geom_of(geom0), g1 = geom_of(geom1);
  const auto s0 = strides<4>(src0);
  const auto m0 = strides<4>(mean0);
  const auto s1 = strides<4>(src1);
  const auto m1 = strides<4>(mean1);
  check("li_pool_pair",
        li_pool_pair(dtype_code(src0), (int32_t)src0.size(0), (int32_t)src0.size(1), (int32_t)src0.size(3),
                     src0.data_ptr(), s0.data(), mean0.data_ptr(), m0.data(), off0, &g0, src1.data_ptr(), s1.data(),
                     mean1.data_ptr(), m1.data(), off1, &g1, mean1_n, stream_of(src0)));
}

void q_prep(const at::Tensor& src, at::Tensor& dst, at::Tensor& mean, c10::IntArrayRef geom) {
  gpu(src, "src");
  rank(src, 4, "src");
  rank(dst, 5, "dst");
  rank(mean, 4, "mean");
  c10::DeviceGuard guard(src.device());
  const li_tile_geom g = geom_of(geom);
  const auto ss = strides<4>(src);
  const auto ds = strides<5>(dst);
  const auto ms = strides<4>(mean);
  check("li_q_prep", li_q_prep(dtype_code(src), (int32_t)src.size(0), (int32_t)src.size(1), (int32_t)src.size(3),
                               src.data_ptr(), ss.data(), dst.data_ptr(), ds.data(), mean.data_ptr(), ms.data(), &g,
                               stream_of(src)));
}

void kv_prep(const at::Tensor& k_src, const at::Tensor& v_src, at::Tensor& k_dst, at::Tensor& v_dst,
             at::Tensor& k_mean, int64_t dst_off, int64_t pool_off, c10::IntArrayRef geom) {
  gpu(k_src, "k_src");
  rank(k_src, 4, "k_src");
  rank(v_src, 4, "v_src");
  rank(k_dst, 5, "k_dst");
  rank(v_dst, 5, "v_dst");
  rank(k_mean, 4, "k_mean");
  c10::DeviceGuard guard(k_src.device());
  const li_tile_geom g = geom_of(geom);
  const auto ks = strides<4>(k_src);
  const auto vs = strides<4>(v_src);
  const auto kd = strides<5>(k_dst);
  const auto vd = strides<5>(v_dst);
  auto ms = strides<4>(k_mean);
  check("li_kv_prep", li_kv_prep(dtype_code(k_src), (int32_t)k_src.size(0), (int32_t)k_src.size(1),
                                 (int32_t)k_src.size(3), k_src.data_ptr(), ks.data(), v_src.data_ptr(), vs.data(),
                                 k_dst.data_ptr(), kd.data(), v_dst.data_ptr(), vd.data(), k_mean.data_ptr(),
                                 ms.data(), dst_off, pool_off, &g, stream_of(k_src)));
}

void untile(const at::Tensor& src, at::Tensor& dst, c10::IntArrayRef geom) {
  gpu(src, "src");
  rank(src, 5, "src");
  rank(dst, 4, "dst");
  c10::DeviceGuard guard(src.device());
  const li_tile_geom g = geom_of(geom);
  const auto ss = strides<5>(src);
  const auto ds = strides<4>(dst);
  check("li_untile", li_untile(dtype_code(src), (int32_t)dst.size(0), (int32_t)dst.size(1), (int32_t)dst.size(3),
                               src.data_ptr(), ss.data(), dst.data_ptr(), ds.data(), &g, stream_of(src)));
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> block_mask(const at::Tensor& q_pool, const at::Tensor& k_pool,
                                                          int64_t metric, int64_t budget_mode, double ratio,
                                                          int64_t min_budget, int64_t n_recent, bool force_diag,
                                                          bool force_sink, bool force_neighbors, int64_t nh,
                                                          int64_t nw, int64_t num_txt_blk, int64_t kmax,
                                                          const c10::optional<at::Tensor>& row_budget,
                                                          bool return_scores, bool k_normalized) {
  gpu(q_pool, "q_pool");
  rank(q_pool, 4, "q_pool");
  rank(k_pool, 4, "k_pool");
  c10::DeviceGuard guard(q_pool.device());
  const int64_t B = q_pool.size(0), NH = q_pool.size(1), nq = q_pool.size(2), D = q_pool.size(3);
  const int64_t nk = k_pool.size(2);
  auto iopt = q_pool.options().dtype(at::kInt);
  at::Tensor indices = at::empty({B, NH, nq, kmax}, iopt);
  at::Tensor counts = at::empty({B, NH, nq}, iopt);
  at::Tensor scores = at::empty(return_scores ? c10::IntArrayRef({B, NH, nq, nk}) : c10::IntArrayRef({0}),
                                q_pool.options());
  li_mask_params p{};
  p.metric = (int32_t)metric;
  p.budget_mode = (int32_t)budget_mode;
  p.topk_ratio = ratio;
  p.min_budget = (int32_t)min_budget;
  p.n_recent = (int32_t)n_recent;
  p.force_diag = force_diag;
  p.force_sink = force_sink;
  p.force_neighbors = force_neighbors;
  p.nq = (int32_t)nq;
  p.nk = (int32_t)nk;
  p.nh = (int32_t)nh;
  p.nw = (int32_t)nw;
  p.num_txt_blk = (int32_t)num_txt_blk;
  p.kmax = (int32_t)kmax;
  if (row_budget.has_value() && row_budget->defined()) {
    TORCH_CHECK(row_budget->scalar_type() == at::kInt && row_budget->is_contiguous() && row_budget->numel() == nq,
                "row_budget must be a contiguous int32 tensor of ", nq, " entries");
    p.row_budget = row_budget->data_ptr<int32_t>();
  }
  p.scale = (float)(1.0 / std::sqrt((double)D));
  p.k_normalized = k_normalized;
  const auto qs = strides<4>(q_pool);
  const auto ks = strides<4>(k_pool);
  check("li_block_mask", li_block_mask(dtype_code(q_pool), (int32_t)B, (int32_t)NH, (int32_t)D, q_pool.data_ptr(),
                                       qs.data(), k_pool.data_ptr(), ks.data(), &p, indices.data_ptr<int32_t>(),
                                       counts.data_ptr<int32_t>(), return_scores ? scores.data_ptr() : nullptr,
                                       stream_of(q_pool)));
  return {indices, counts, scores};
}

void index_checks(const at::Tensor& indices, const at::Tensor& counts) {
  TORCH_CHECK(indices.scalar_type() == at::kInt && counts.scalar_type() == at::kInt,
              "block indices and counts must be int32");
  rank(indices, 4, "block_indices");
  rank(counts, 3, "block_counts");
}

at::Tensor bsa_fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v, const at::Tensor& indices,
                   const at::Tensor& counts, double sm_scale, int64_t block_size, at::Tensor& out, bool return_lse,
                   bool split, bool balance) {
  gpu(q, "q");
  rank(q, 4, "q");
  rank(k, 4, "k");
  rank(v, 4, "v");
  index_checks(indices, counts);
  c10::DeviceGuard guard(q.device());
  const int64_t B = q.size(0), NH = q.size(1), Lq = q.size(2), D = q.size(3), Lk = k.size(2);
  TORCH_CHECK(out.is_contiguous() && out.sizes() == q.sizes() && out.scalar_type() == q.scalar_type(),
              "out must be a contiguous tensor of q's shape and dtype");
  at::Tensor lse = lse_or_empty(q, return_lse, B, NH, Lq);
  at::Tensor ws = workspace(q, B, NH, Lq, D, block_size, split || balance);
  const auto is = strides<4>(indices);
  const auto cs = strides<3>(counts);
  const int st = li_bsa_fwd(dtype_code(q), (int32_t)B, (int32_t)NH, (int32_t)Lq, (int32_t)Lk, (int32_t)D,
                            q.data_ptr(), k.data_ptr(), v.data_ptr(), indices.data_ptr<int32_t>(), is.data(),
                            (int32_t)indices.size(3), counts.data_ptr<int32_t>(), cs.data(), (float)sm_scale,
                            (int32_t)block_size, out.data_ptr(), return_lse ? lse.data_ptr<float>() : nullptr,
                            ptr(ws), ws.defined() ? ws.numel() * 4 : 0, balance ? LI_BSA_BALANCE : 0, stream_of(q));
  check("li_bsa_fwd", st);
  return lse;
}

at::Tensor bsa_fwd_gather(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                          const c10::optional<at::Tensor>& k_txt, const c10::optional<at::Tensor>& v_txt,
                          int64_t num_txt_blk, c10::IntArrayRef q_geom, c10::IntArrayRef k_geom,
                          const at::Tensor& indices, const at::Tensor& counts, double sm_scale, at::Tensor& out,
                          bool return_lse, bool split, bool balance, bool sorted) {
  gpu(q, "q");
  rank(q, 4, "q");
  rank(k, 4, "k");
  rank(v, 4, "v");
  index_checks(indices, counts);
  c10::DeviceGuard guard(q.device());
  const li_tile_geom gq = geom_of(q_geom), gk = geom_of(k_geom);
  const int64_t B = q.size(0), NH = q.size(1), D = q.size(3);
  const int64_t nq = (int64_t)((gq.T + gq.tt - 1) / gq.tt) * gq.nh * gq.nw;
  const int64_t bs = (int64_t)gq.tt * gq.th * gq.tw;
  rank(out, 4, "out");
  at::Tensor lse = lse_or_empty(q, return_lse, B, NH, nq * bs);
  at::Tensor ws = workspace(q, B, NH, nq * bs, D, bs, split || balance);
  const at::Tensor kt = num_txt_blk > 0 && k_txt.has_value() ? *k_txt : at::Tensor();
  const at::Tensor vt = num_txt_blk > 0 && v_txt.has_value() ? *v_txt : at::Tensor();
  const auto qs = strides<4>(q);
  const auto ks = strides<4>(k);
  const auto vs = strides<4>(v);
  const auto os = strides<4>(out);
  const auto is = strides<4>(indices);
  const auto cs = strides<3>(counts);
  const int st = li_bsa_fwd_gather(
      dtype_code(q), (int32_t)B, (int32_t)NH, (int32_t)D, q.data_ptr(), qs.data(), k.data_ptr(), ks.data(),
      v.data_ptr(), vs.data(), ptr(kt), ptr(vt), (int32_t)num_txt_blk, &gq, &gk, indices.data_ptr<int32_t>(),
      is.data(), (int32_t)indices.size(3), counts.data_ptr<int32_t>(), cs.data(), (float)sm_scale, out.data_ptr(),
      os.data(), return_lse ? lse.data_ptr<float>() : nullptr, ptr(ws), ws.defined() ? ws.numel() * 4 : 0,
      (balance ? LI_BSA_BALANCE : 0) | (sorted ? LI_BSA_SORTED : 0), stream_of(q));
  check("li_bsa_fwd_gather", st);
  return lse;
}

at::Tensor attn_dense(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                      const c10::optional<at::Tensor>& k_txt, const c10::optional<at::Tensor>& v_txt,
                      int64_t txt_len, double sm_scale, at::Tensor& out, bool return_lse, bool split) {
  gpu(q, "q");
  rank(q, 4, "q");
  rank(k, 4, "k");
  rank(v, 4, "v");
  c10::DeviceGuard guard(q.device());
  const int64_t B = q.size(0), NH = q.size(1), Lq = q.size(2), D = q.size(3), Lk = k.size(2);
  const int64_t nq = (Lq + 127) / 128;
  rank(out, 4, "out");
  at::Tensor lse = lse_or_empty(q, return_lse, B, NH, nq * 128);
  at::Tensor ws = workspace(q, B, NH, nq * 128, D, 128, split);
  const at::Tensor kt = txt_len > 0 && k_txt.has_value() ? *k_txt : at::Tensor();
  const at::Tensor vt = txt_len > 0 && v_txt.has_value() ? *v_txt : at::Tensor();
  const auto qs = strides<4>(q);
  const auto ks = strides<4>(k);
  const auto vs = strides<4>(v);
  const auto os = strides<4>(out);
  const int st = li_attn_fwd_dense(dtype_code(q), (int32_t)B, (int32_t)NH, (int32_t)D, (int32_t)Lq, (int32_t)Lk,
                                   q.data_ptr(), qs.data(), k.data_ptr(), ks.data(), v.data_ptr(), vs.data(),
                                   ptr(kt), ptr(vt), (int32_t)txt_len, (float)sm_scale, out.data_ptr(), os.data(),
                                   return_lse ? lse.data_ptr<float>() : nullptr, ptr(ws),
                                   ws.defined() ? ws.numel() * 4 : 0, stream_of(q));
  check("li_attn_fwd_dense", st);
  return lse;
}

void tile_prep_fp8(const at::Tensor& src, at::Tensor& dst, at::Tensor& scales, const c10::optional<at::Tensor>& mean,
                   int64_t dst_off, int64_t pool_off, c10::IntArrayRef geom) {
  gpu(src, "src");
  rank(src, 4, "src");
  rank(dst, 5, "dst");
  rank(scales, 3, "scales");
  c10::DeviceGuard guard(src.device());
  const li_tile_geom g = geom_of(geom);
  const at::Tensor m = mean.has_value() ? *mean : at::Tensor();
  const auto ss = strides<4>(src);
  const auto ds = strides<5>(dst);
  const auto cs = strides<3>(scales);
  std::array<int64_t, 4> ms{};
  if (m.defined()) ms = strides<4>(m);
  check("li_tile_prep_fp8",
        li_tile_prep_fp8(dtype_code(src), (int32_t)src.size(0), (int32_t)src.size(1), (int32_t)src.size(3),
                         src.data_ptr(), ss.data(), dst.data_ptr(), ds.data(), scales.data_ptr<float>(), cs.data(),
                         ptr(m), m.defined() ? ms.data() : nullptr, dst_off, pool_off, &g, stream_of(src)));
}

void kv_prep_fp8(const at::Tensor& k_src, const at::Tensor& v_src, at::Tensor& k_dst, at::Tensor& k_scales,
                 at::Tensor& v_dst, at::Tensor& k_mean, int64_t dst_off, int64_t pool_off, c10::IntArrayRef geom) {
  gpu(k_src, "k_src");
  rank(k_src, 4, "k_src");
  rank(v_src, 4, "v_src");
  rank(k_dst, 5, "k_dst");
  rank(k_scales, 3, "k_scales");
  rank(v_dst, 5, "v_dst");
  rank(k_mean, 4, "k_mean");
  c10::DeviceGuard guard(k_src.device());
  const li_tile_geom g = geom_of(geom);
  const auto ks = strides<4>(k_src);
  const auto vs = strides<4>(v_src);
  const auto kd = strides<5>(k_dst);
  const auto sc = strides<3>(k_scales);
  const auto vd = strides<5>(v_dst);
  const auto ms = strides<4>(k_mean);
  check("li_kv_prep_fp8",
        li_kv_prep_fp8(dtype_code(k_src), (int32_t)k_src.size(0), (int32_t)k_src.size(1), (int32_t)k_src.size(3),
                       k_src.data_ptr(), ks.data(), v_src.data_ptr(), vs.data(), k_dst.data_ptr(), kd.data(),
                       k_scales.data_ptr<float>(), sc.data(), v_dst.data_ptr(), vd.data(), k_mean.data_ptr(),
                       ms.data(), dst_off, pool_off, &g, stream_of(k_src)));
}

at::Tensor bsa_fwd_fp8(const at::Tensor& q8, const at::Tensor& q_scale, const at::Tensor& k8,
                       const at::Tensor& k_scale, const at::Tensor& v, const at::Tensor& indices,
                       const at::Tensor& counts, double sm_scale, int64_t block_size, at::Tensor& out,
                       bool return_lse, bool split, bool balance) {
  gpu(q8, "q8");
  rank(q8, 4, "q8");
  rank(k8, 4, "k8");
  rank(v, 4, "v");
  index_checks(indices, counts);
  TORCH_CHECK(v.scalar_type() == at::kBFloat16, "v must be bfloat16");
  c10::DeviceGuard guard(q8.device());
  const int64_t B = q8.size(0), NH = q8.size(1), Lq = q8.size(2), D = q8.size(3), Lk = k8.size(2);
  TORCH_CHECK(out.is_contiguous() && out.dim() == 4 && out.size(0) == B && out.size(1) == NH && out.size(2) == Lq &&
                  out.size(3) == D && out.scalar_type() == at::kBFloat16,
              "out must be a contiguous bfloat16 tensor of q8's shape");
  at::Tensor lse = lse_or_empty(v, return_lse, B, NH, Lq);
  at::Tensor ws = workspace(v, B, NH, Lq, D, block_size, split || balance);
  const auto is = strides<4>(indices);
  const auto cs = strides<3>(counts);
  const int st = li_bsa_fwd_fp8((int32_t)B, (int32_t)NH, (int32_t)Lq, (int32_t)Lk, (int32_t)D, q8.data_ptr(),
                                q_scale.data_ptr<float>(), k8.data_ptr(), k_scale.data_ptr<float>(), v.data_ptr(),
                                indices.data_ptr<int32_t>(), is.data(), (int32_t)indices.size(3),
                                counts.data_ptr<int32_t>(), cs.data(), (float)sm_scale, (int32_t)block_size,
                                out.data_ptr(), return_lse ? lse.data_ptr<float>() : nullptr, ptr(ws),
                                ws.defined() ? ws.numel() * 4 : 0, balance ? LI_BSA_BALANCE : 0, stream_of(v));
  check("li_bsa_fwd_fp8", st);
  return lse;
}

at::Tensor bsa_fwd_fp8_gather(const at::Tensor& q8, const at::Tensor& q_scale, const at::Tensor& k8,
                              const at::Tensor& k_scale, const at::Tensor& v, const c10::optional<at::Tensor>& v_txt,
                              int64_t num_txt_blk, c10::IntArrayRef q_geom, c10::IntArrayRef k_geom,
                              const at::Tensor& indices, const at::Tensor& counts, double sm_scale, at::Tensor& out,
                              bool return_lse, bool balance, bool sorted) {
  gpu(q8, "q8");
  rank(v, 4, "v");
  rank(out, 4, "out");
  index_checks(indices, counts);
  c10::DeviceGuard guard(q8.device());
  const li_tile_geom gq = geom_of(q_geom), gk = geom_of(k_geom);
  const int64_t B = v.size(0), NH = v.size(1), D = v.size(3);
  const int64_t nq = (int64_t)((gq.T + gq.tt - 1) / gq.tt) * gq.nh * gq.nw;
  at::Tensor lse = lse_or_empty(v, return_lse, B, NH, nq * 128);
  at::Tensor ws = workspace(v, B, NH, nq * 128, D, 128, true);
  const at::Tensor vt = num_txt_blk > 0 && v_txt.has_value() ? *v_txt : at::Tensor();
  const auto vs = strides<4>(v);
  const auto os = strides<4>(out);
  const auto is = strides<4>(indices);
  const auto cs = strides<3>(counts);
  const int st = li_bsa_fwd_fp8_gather(
      (int32_t)B, (int32_t)NH, (int32_t)D, q8.data_ptr(), q_scale.data_ptr<float>(), k8.data_ptr(),
      k_scale.data_ptr<float>(), v.data_ptr(), vs.data(), ptr(vt), (int32_t)num_txt_blk, &gq, &gk,
      indices.data_ptr<int32_t>(), is.data(), (int32_t)indices.size(3), counts.data_ptr<int32_t>(), cs.data(),
      (float)sm_scale, out.data_ptr(), os.data(), return_lse ? lse.data_ptr<float>() : nullptr, ptr(ws),
      ws.defined() ? ws.numel() * 4 : 0, (balance ? LI_BSA_BALANCE : 0) | (sorted ? LI_BSA_SORTED : 0),
      stream_of(v));
  check("li_bsa_fwd_fp8_gather", st);
  return lse;
}

}  // namespace

TORCH_LIBRARY(li, m) {
  m.def("pool(Tensor src, Tensor(a!) mean, int pool_off, int[] geom) -> ()");
  m.def("pool_pair(Tensor src0, Tensor(a!) mean0, int pool_off0, int[] geom0, Tensor src1, Tensor(b!) mean1, "
        "int pool_off1, int[] geom1, Tensor(c!)? mean1_normalized=None) -> ()");
  m.def("q_prep(Tensor src, Tensor(a!) dst, Tensor(b!) mean, int[] geom) -> ()");
  m.def("kv_prep(Tensor k_src, Tensor v_src, Tensor(a!) k_dst, Tensor(b!) v_dst, Tensor(c!) k_mean, int dst_off, "
        "int pool_off, int[] geom) -> ()");
  m.def("untile(Tensor src, Tensor(a!) dst, int[] geom) -> ()");
  m.def("block_mask(Tensor q_pool, Tensor k_pool, int metric, int budget_mode, float ratio, int min_budget, "
        "int n_recent, bool force_diag, bool force_sink, bool force_neighbors, int nh, int nw, int num_txt_blk, "
        "int kmax, Tensor? row_budget, bool return_scores, bool k_normalized=False) -> (Tensor, Tensor, Tensor)");
  m.def("bsa_fwd(Tensor q, Tensor k, Tensor v, Tensor indices, Tensor counts, float sm_scale, int block_size, "
        "Tensor(a!) out, bool return_lse, bool split, bool balance) -> Tensor");
  m.def("bsa_fwd_gather(Tensor q, Tensor k, Tensor v, Tensor? k_txt, Tensor? v_txt, int num_txt_blk, int[] q_geom, "
        "int[] k_geom, Tensor indices, Tensor counts, float sm_scale, Tensor(a!) out, bool return_lse, bool split, "
        "bool balance, bool sorted=False) -> Tensor");
  m.def("attn_dense(Tensor q, Tensor k, Tensor v, Tensor? k_txt, Tensor? v_txt, int txt_len, float sm_scale, "
        "Tensor(a!) out, bool return_lse, bool split) -> Tensor");
  m.def("tile_prep_fp8(Tensor src, Tensor(a!) dst, Tensor(b!) scales, Tensor(c!)? mean, int dst_off, int pool_off, "
        "int[] geom) -> ()");
  m.def("kv_prep_fp8(Tensor k_src, Tensor v_src, Tensor(a!) k_dst, Tensor(b!) k_scales, Tensor(c!) v_dst, "
        "Tensor(d!) k_mean, int dst_off, int pool_off, int[] geom) -> ()");
  m.def("bsa_fwd_fp8(Tensor q8, Tensor q_scale, Tensor k8, Tensor k_scale, Tensor v, Tensor indices, Tensor counts, "
        "float sm_scale, int block_size, Tensor(a!) out, bool return_lse, bool split, bool balance) -> Tensor");
  m.def("bsa_fwd_fp8_gather(Tensor q8, Tensor q_scale, Tensor k8, Tensor k_scale, Tensor v, Tensor? v_txt, "
        "int num_txt_blk, int[] q_geom, int[] k_geom, Tensor indices, Tensor counts, float sm_scale, "
        "Tensor(a!) out, bool return_lse, bool balance, bool sorted=False) -> Tensor");
}

TORCH_LIBRARY_IMPL(li, CUDA, m) {
  m.impl("pool", &pool);
  m.impl("pool_pair", &pool_pair);
  m.impl("q_prep", &q_prep);
  m.impl("kv_prep", &kv_prep);
  m.impl("untile", &untile);
  m.impl("block_mask", &block_mask);
  m.impl("bsa_fwd", &bsa_fwd);
  m.impl("bsa_fwd_gather", &bsa_fwd_gather);
  m.impl("attn_dense", &attn_dense);
  m.impl("tile_prep_fp8", &tile_prep_fp8);
  m.impl("kv_prep_fp8", &kv_prep_fp8);
  m.impl("bsa_fwd_fp8", &bsa_fwd_fp8);
  m.impl("bsa_fwd_fp8_gather", &bsa_fwd_fp8_gather);
}
