// PyTorch custom operators torch.ops.li.* over the C ABI of libli_sparse_attn.so.
//
// Each operator checks dtypes, ranks, devices and every tensor's extent
// against the geometry and lists it is indexed by (so that a direct call
// cannot make a kernel read or write past a tensor), allocates what it
// returns (and the attention workspace) through the caching allocator, writes
// the tensors its schema marks as mutated (Tensor(a!): tiles, pools, attention
// outputs), and enqueues the C-ABI call on torch's current HIP stream of the
// tensors' device.  The reference's error messages stay in the Python
// wrappers that call these operators (li_sparse/_core.py); the fake (meta)
// implementations, which give output shapes for tracing, are registered in
// li_sparse/_ops.py.
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
  TORCH_CHECK(g[0] >= 0 && g[1] > 0 && g[2] > 0 && g[3] > 0 && g[4] > 0 && g[5] > 0 && g[6] > 0 && g[7] > 0,
              "geometry (T, H, W, tt, th, tw, nh, nw) must have T >= 0 and the other fields positive, got ", g);
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

// Extent checks.  The C ABI takes pointers and strides only, so these are
// what keeps a direct call of an operator (outside the Python wrappers) from
// reading or writing past a tensor: every tensor must reach at least as far
// as the kernels index it, on the device of the first one.

int64_t blocks_of(const li_tile_geom& g) { return (int64_t)((g.T + g.tt - 1) / g.tt) * g.nh * g.nw; }
int64_t tokens_of(const li_tile_geom& g) { return (int64_t)g.T * g.H * g.W; }
int64_t block_size_of(const li_tile_geom& g) { return (int64_t)g.tt * g.th * g.tw; }

void on_device(const at::Tensor& ref, const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.device() == ref.device(), name, " must be on ", ref.device(), ", got ", t.device());
}

// (B, NH, >= rows, D), with the element type of `like` when given.  With
// `exact`, exactly `rows` rows: for contiguous tensors that a kernel indexes at
// a per-head pitch implied by the geometry rather than by a stride, where a
// longer tensor would make every head after the first read another head's
// rows.
void rows4(const at::Tensor& t, int64_t B, int64_t NH, int64_t rows, int64_t D, const char* name,
           const at::Tensor* like = nullptr, bool exact = false) {
  TORCH_CHECK(t.dim() == 4 && t.size(0) == B && t.size(1) == NH && (exact ? t.size(2) == rows : t.size(2) >= rows) &&
                  t.size(3) == D,
              name, " must be (", B, ", ", NH, ", ", exact ? "" : ">= ", rows, ", ", D, "), got ", t.sizes());
  if (like) {
    on_device(*like, t, name);
    TORCH_CHECK(t.scalar_type() == like->scalar_type(), name, " must be ", like->scalar_type(), ", got ",
                t.scalar_type());
  }
}

// (B, NH, >= blocks, BS, D) tiles.
void tiles5(const at::Tensor& t, int64_t B, int64_t NH, int64_t blocks, int64_t BS, int64_t D, const char* name,
            const at::Tensor& ref) {
  TORCH_CHECK(t.dim() == 5 && t.size(0) == B && t.size(1) == NH && t.size(2) >= blocks && t.size(3) == BS &&
                  t.size(4) == D,
              name, " must be (", B, ", ", NH, ", >= ", blocks, ", ", BS, ", ", D, "), got ", t.sizes());
  on_device(ref, t, name);
}

// (B, NH, >= blocks) fp32 scales; exactly `blocks` with `exact` (as for rows4).
void scales3(const at::Tensor& t, int64_t B, int64_t NH, int64_t blocks, const char* name, const at::Tensor& ref,
             bool exact = false) {
  TORCH_CHECK(t.dim() == 3 && t.size(0) == B && t.size(1) == NH &&
                  (exact ? t.size(2) == blocks : t.size(2) >= blocks) && t.scalar_type() == at::kFloat,
              name, " must be float32 (", B, ", ", NH, ", ", exact ? "" : ">= ", blocks, "), got ", t.scalar_type(),
              " ", t.sizes());
  on_device(ref, t, name);
}

void codes(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.element_size() == 1, name, " must hold 1-byte e4m3 codes, got ", t.scalar_type());
}

// Lists over nq query tiles: indices (B, NH, nq, n_cols), counts (B, NH, nq), int32.
void lists(const at::Tensor& indices, const at::Tensor& counts, int64_t B, int64_t NH, int64_t nq,
           const at::Tensor& ref) {
  TORCH_CHECK(indices.size(0) == B && indices.size(1) == NH && indices.size(2) >= nq, "block_indices must be (",
              B, ", ", NH, ", >= ", nq, ", n), got ", indices.sizes());
  TORCH_CHECK(counts.size(0) == B && counts.size(1) == NH && counts.size(2) >= nq, "block_counts must be (", B,
              ", ", NH, ", >= ", nq, "), got ", counts.sizes());
  on_device(ref, indices, "block_indices");
  on_device(ref, counts, "block_counts");
}

// Contiguous zero-padded text rows, exactly (B, NH, rows, D), when there are
// any: the kernels index them at a per-head pitch of `rows` rows.
void text(const c10::optional<at::Tensor>& t, int64_t rows, int64_t B, int64_t NH, int64_t D, const char* name,
          const at::Tensor& like) {
  if (rows <= 0) return;
  TORCH_CHECK(t.has_value() && t->defined(), name, " is required with text blocks");
  TORCH_CHECK(t->is_contiguous(), name, " must be contiguous");
  rows4(*t, B, NH, rows, D, name, &like, true);
}

// ---------------------------------------------------------------------------

void pool(const at::Tensor& src, at::Tensor& mean, int64_t pool_off, c10::IntArrayRef geom) {
  gpu(src, "src");
  rank(src, 4, "src");
  rank(mean, 4, "mean");
  c10::DeviceGuard guard(src.device());
  const li_tile_geom g = geom_of(geom);
  const int64_t B = src.size(0), NH = src.size(1), D = src.size(3);
  rows4(src, B, NH, tokens_of(g), D, "src");
  rows4(mean, B, NH, blocks_of(g) + pool_off, D, "mean", &src);
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
  {
    const int64_t B = src0.size(0), NH = src0.size(1), D = src0.size(3);
    rows4(src0, B, NH, tokens_of(g0), D, "src0");
    rows4(mean0, B, NH, blocks_of(g0) + off0, D, "mean0", &src0);
    rows4(src1, B, NH, tokens_of(g1), D, "src1", &src0);
    rows4(mean1, B, NH, blocks_of(g1) + off1, D, "mean1", &src0);
  }
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
  const int64_t B = src.size(0), NH = src.size(1), D = src.size(3);
  rows4(src, B, NH, tokens_of(g), D, "src");
  tiles5(dst, B, NH, blocks_of(g), block_size_of(g), D, "dst", src);
  TORCH_CHECK(dst.scalar_type() == src.scalar_type(), "dst must be ", src.scalar_type());
  rows4(mean, B, NH, blocks_of(g), D, "mean", &src);
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
  {
    const int64_t B = k_src.size(0), NH = k_src.size(1), D = k_src.size(3), nb = blocks_of(g);
    rows4(k_src, B, NH, tokens_of(g), D, "k_src");
    rows4(v_src, B, NH, tokens_of(g), D, "v_src", &k_src);
    tiles5(k_dst, B, NH, nb + dst_off, block_size_of(g), D, "k_dst", k_src);
    tiles5(v_dst, B, NH, nb + dst_off, block_size_of(g), D, "v_dst", k_src);
    TORCH_CHECK(k_dst.scalar_type() == k_src.scalar_type() && v_dst.scalar_type() == k_src.scalar_type(),
                "k_dst and v_dst must be ", k_src.scalar_type());
    rows4(k_mean, B, NH, nb + pool_off, D, "k_mean", &k_src);
  }
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
  {
    const int64_t B = dst.size(0), NH = dst.size(1), D = dst.size(3);
    tiles5(src, B, NH, blocks_of(g), block_size_of(g), D, "src", src);
    rows4(dst, B, NH, tokens_of(g), D, "dst", &src);
  }
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
  rows4(k_pool, B, NH, 0, D, "k_pool", &q_pool);
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
    on_device(q_pool, *row_budget, "row_budget");
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
  TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(), "q, k, v must be contiguous");
  TORCH_CHECK(block_size > 0, "block_size must be positive");
  rows4(k, B, NH, Lk, D, "k", &q);
  TORCH_CHECK(v.sizes() == k.sizes(), "v must have k's shape ", k.sizes(), ", got ", v.sizes());
  rows4(v, B, NH, Lk, D, "v", &q);
  on_device(q, out, "out");
  lists(indices, counts, B, NH, (Lq + block_size - 1) / block_size, q);
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
  const int64_t nq = blocks_of(gq);
  const int64_t bs = block_size_of(gq);
  rank(out, 4, "out");
  rows4(q, B, NH, tokens_of(gq), D, "q");
  rows4(k, B, NH, tokens_of(gk), D, "k", &q);
  rows4(v, B, NH, tokens_of(gk), D, "v", &q);
  rows4(out, B, NH, tokens_of(gq), D, "out", &q);
  text(k_txt, num_txt_blk * bs, B, NH, D, "k_txt", q);
  text(v_txt, num_txt_blk * bs, B, NH, D, "v_txt", q);
  lists(indices, counts, B, NH, nq, q);
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
  rows4(k, B, NH, Lk, D, "k", &q);
  rows4(v, B, NH, Lk, D, "v", &q);
  rows4(out, B, NH, Lq, D, "out", &q);
  TORCH_CHECK(txt_len >= 0, "txt_len must be >= 0");
  text(k_txt, (txt_len + 127) / 128 * 128, B, NH, D, "k_txt", q);
  text(v_txt, (txt_len + 127) / 128 * 128, B, NH, D, "v_txt", q);
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
  {
    const int64_t B = src.size(0), NH = src.size(1), D = src.size(3), nb = blocks_of(g);
    rows4(src, B, NH, tokens_of(g), D, "src");
    tiles5(dst, B, NH, nb + dst_off, block_size_of(g), D, "dst", src);
    codes(dst, "dst");
    scales3(scales, B, NH, nb + dst_off, "scales", src);
    if (m.defined()) rows4(m, B, NH, nb + pool_off, D, "mean", &src);
  }
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
  {
    const int64_t B = k_src.size(0), NH = k_src.size(1), D = k_src.size(3), nb = blocks_of(g);
    rows4(k_src, B, NH, tokens_of(g), D, "k_src");
    rows4(v_src, B, NH, tokens_of(g), D, "v_src", &k_src);
    tiles5(k_dst, B, NH, nb + dst_off, block_size_of(g), D, "k_dst", k_src);
    codes(k_dst, "k_dst");
    scales3(k_scales, B, NH, nb + dst_off, "k_scales", k_src);
    tiles5(v_dst, B, NH, nb + dst_off, block_size_of(g), D, "v_dst", k_src);
    TORCH_CHECK(v_dst.scalar_type() == k_src.scalar_type(), "v_dst must be ", k_src.scalar_type());
    rows4(k_mean, B, NH, nb + pool_off, D, "k_mean", &k_src);
  }
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
  TORCH_CHECK(q8.is_contiguous() && k8.is_contiguous() && v.is_contiguous() && q_scale.is_contiguous() &&
                  k_scale.is_contiguous(),
              "q8, k8, v and the scales must be contiguous");
  codes(q8, "q8");
  codes(k8, "k8");
  rows4(k8, B, NH, Lk, D, "k8");
  rows4(v, B, NH, Lk, D, "v");
  TORCH_CHECK(v.size(2) == Lk, "v must have k8's length ", Lk);
  TORCH_CHECK(block_size > 0, "block_size must be positive");
  // One scale per block of block_size rows (the library takes 128 only),
  // indexed at per-head pitches of the tile and block counts.
  scales3(q_scale, B, NH, (Lq + block_size - 1) / block_size, "q_scale", q8, true);
  scales3(k_scale, B, NH, Lk / block_size, "k_scale", q8, true);
  on_device(q8, k8, "k8");
  on_device(q8, v, "v");
  on_device(q8, out, "out");
  lists(indices, counts, B, NH, (Lq + block_size - 1) / block_size, q8);
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
  const int64_t nq = blocks_of(gq);
  TORCH_CHECK(block_size_of(gq) == 128, "the e4m3 gather path is built for 128-token tiles");
  TORCH_CHECK(q8.is_contiguous() && k8.is_contiguous() && q_scale.is_contiguous() && k_scale.is_contiguous(),
              "q8, k8 and the scales must be contiguous");
  codes(q8, "q8");
  codes(k8, "k8");
  TORCH_CHECK(v.scalar_type() == at::kBFloat16, "v must be bfloat16");
  // Tiles and scales are indexed at per-head pitches of the geometry's block
  // counts: exact extents.
  rows4(q8, B, NH, nq * 128, D, "q8", nullptr, true);
  rows4(k8, B, NH, (num_txt_blk + blocks_of(gk)) * 128, D, "k8", nullptr, true);
  scales3(q_scale, B, NH, nq, "q_scale", v, true);
  scales3(k_scale, B, NH, num_txt_blk + blocks_of(gk), "k_scale", v, true);
  rows4(v, B, NH, tokens_of(gk), D, "v");
  rows4(out, B, NH, tokens_of(gq), D, "out", &v);
  on_device(v, q8, "q8");
  on_device(v, k8, "k8");
  text(v_txt, num_txt_blk * 128, B, NH, D, "v_txt", v);
  lists(indices, counts, B, NH, nq, v);
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
