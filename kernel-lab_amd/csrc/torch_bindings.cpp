// PyTorch-ROCm registration of the kernel_lab operators: torch.ops.kernel_lab.*.
//
// Schemas are those of csrc/torch_bindings.cpp:107-113 in the reference, so
// callers and torch.compile graphs see the same operators:
//   rms_norm(Tensor! out, Tensor x, Tensor weight, float eps) -> ()
//   fused_add_rms_norm(Tensor! out, Tensor x, Tensor! residual, Tensor weight, float eps) -> ()
//   paged_decode_attention(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache,
//                          Tensor block_table, Tensor seq_lens, float scale) -> ()
// plus `fused_add_rmsnorm` (same schema as fused_add_rms_norm), the overload
// `paged_decode_attention.splits(..., int num_splits, int max_seq_len)` for
// the split-KV controls of the reference's Triton wrapper
// (kernel_lab/triton_kernels/paged_attention.py:176-211; 0 means "planner
// decides" and "block-table width" respectively, num_splits -1 the balanced
// schedule), and
//   paged_decode_attention_fp8(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache,
//                              Tensor block_table, Tensor seq_lens, float scale,
//                              Tensor k_scale, Tensor v_scale, int num_splits, int max_seq_len) -> ()
// for a float8_e4m3fn cache with fp32 per-KV-head scales (the FP8 KV cache the
// reference lists as planned work, README.md:98), and
//   cascade_decode_attention(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache,
//                            Tensor prefix_block_table, Tensor prefix_len,
//                            Tensor block_table, Tensor seq_lens, float scale) -> ()
// for a prefix shared by every sequence (docs/design.md:96-100 of the reference
// names cascade/shared-prefix attention).
//
// Outputs are caller-allocated ("Tensor!" = mutated in place). The only
// allocation here is the split-KV workspace, taken from PyTorch's caching
// allocator on the current stream. This file is the only one that includes
// PyTorch; it calls the kernels through the C-ABI in kernel_lab.h.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include "kernel_lab.h"

namespace {

kl_dtype to_kl_dtype(at::ScalarType t) {
  switch (t) {
    case at::kFloat:
      return KL_DTYPE_F32;
    case at::kHalf:
      return KL_DTYPE_F16;
    case at::kBFloat16:
      return KL_DTYPE_BF16;
    default:
      TORCH_CHECK(false, "kernel_lab: unsupported dtype ", t);
  }
}

void check_status(int status, const char* what) {
  TORCH_CHECK(status == KL_OK, "kernel_lab: ", what, " failed: ", kl_status_string(status), ": ",
              kl_last_error());
}

kl_stream_t current_stream(const at::Device& device) {
  return reinterpret_cast<kl_stream_t>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(device.index()).stream());
}

// The argument contract of the reference's RMSNorm operators
// (csrc/torch_bindings.cpp:31-49 there): GPU tensors on one device and of one
// dtype; x's last dimension contiguous; out and weight contiguous, out shaped
// like x, one weight per hidden element; a residual contiguous and shaped like x.
void check_norm_args(const at::Tensor& out, const at::Tensor& x, const at::Tensor* residual,
                     const at::Tensor& weight) {
  for (const at::Tensor* t : {&x, &weight, &out, residual}) {
    if (t == nullptr) continue;
    TORCH_CHECK(t->is_cuda(), "tensors must be on the GPU");
    TORCH_CHECK(t->device() == x.device(), "tensors must share a device");
    TORCH_CHECK(t->scalar_type() == x.scalar_type(), "x, weight, out and residual must share a dtype");
  }
  TORCH_CHECK(x.dim() >= 1 && x.stride(-1) == 1, "x must have a contiguous last dimension");
  TORCH_CHECK(weight.is_contiguous() && weight.numel() == x.size(-1), "weight needs one contiguous value per hidden "
              "element (", weight.numel(), " values, hidden ", x.size(-1), ")");
  TORCH_CHECK(out.is_contiguous() && out.sizes() == x.sizes(), "out must be contiguous and shaped like x");
  if (residual != nullptr) {
    TORCH_CHECK(residual->is_contiguous() && residual->sizes() == x.sizes(),
                "residual must be contiguous and shaped like x");
  }
}

// x as `count` rows of its last dimension, row i at data + i * stride
// elements. The kernels take one row stride, which the strides of x's
// leading dimensions give when they nest (each steps over the next one's
// span; size-1 dimensions are free). Otherwise, or when rows would overlap,
// the rows are read from a contiguous copy: x is only read, so the result is
// the same.
struct NormRows {
  at::Tensor data;  // x, or its contiguous copy
  int64_t count;
  int64_t stride;
};

NormRows norm_rows(const at::Tensor& x) {
  const int64_t hidden = x.size(-1);
  const int64_t count = hidden > 0 ? x.numel() / hidden : 0;
  int64_t stride = hidden;  // a single row
  bool nested = true;
  int64_t inner_size = 0, inner_stride = 0;  // the next non-trivial dimension inward
  for (int64_t d = x.dim() - 2; d >= 0; --d) {
    if (x.size(d) == 1) continue;
    if (inner_size == 0) {
      stride = x.stride(d);  // the innermost leading dimension steps from row to row
    } else if (x.stride(d) != inner_stride * inner_size) {
      nested = false;
    }
    inner_size = x.size(d);
    inner_stride = x.stride(d);
  }
  if (!nested || (count > 1 && stride < hidden)) return {x.contiguous(), count, hidden};
  return {x, count, stride};
}

void rms_norm_impl(at::Tensor& out, const at::Tensor& x, at::Tensor* residual, const at::Tensor& weight,
                   double eps) {
  check_norm_args(out, x, residual, weight);
  const NormRows rows = norm_rows(x);
  if (rows.count == 0) return;
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  check_status(kl_rms_norm(to_kl_dtype(x.scalar_type()), out.data_ptr(), rows.data.data_ptr(),
                           residual != nullptr ? residual->data_ptr() : nullptr, weight.data_ptr(), rows.count,
                           x.size(-1), rows.stride, static_cast<float>(eps), current_stream(x.device())),
               "rms_norm");
}

void rms_norm(at::Tensor& out, const at::Tensor& x, const at::Tensor& weight, double eps) {
  rms_norm_impl(out, x, nullptr, weight, eps);
}

void fused_add_rms_norm(at::Tensor& out, const at::Tensor& x, at::Tensor& residual, const at::Tensor& weight,
                        double eps) {
  rms_norm_impl(out, x, &residual, weight, eps);
}

// Same checks as paged_decode_attention in the reference
// (csrc/torch_bindings.cpp:71-93), plus device agreement and max_seq_len.
// k_scale / v_scale non-null: the caches hold float8_e4m3fn codes.
void paged_decode_impl(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                       const at::Tensor& block_table, const at::Tensor& seq_lens, double scale, int64_t num_splits,
                       int64_t max_seq_len, const at::Tensor* k_scale = nullptr, const at::Tensor* v_scale = nullptr) {
  const bool kv8 = k_scale != nullptr;
  TORCH_CHECK(q.is_cuda() && k_cache.is_cuda() && v_cache.is_cuda() && out.is_cuda() && block_table.is_cuda() &&
                  seq_lens.is_cuda(),
              "tensors must be on the GPU");
  const auto dev = q.device();
  TORCH_CHECK(k_cache.device() == dev && v_cache.device() == dev && out.device() == dev &&
                  block_table.device() == dev && seq_lens.device() == dev,
              "tensors must share a device");
  TORCH_CHECK(q.dim() == 3 && k_cache.dim() == 4, "q is [batch, heads, dim]; caches are 4-D");
  TORCH_CHECK(q.is_contiguous() && out.is_contiguous() && k_cache.is_contiguous() && v_cache.is_contiguous(),
              "q, out and both caches must be contiguous");
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes(), "k_cache and v_cache shapes differ");
  TORCH_CHECK(out.sizes() == q.sizes(), "out must match q");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seq_lens.scalar_type() == at::kInt,
              "block_table and seq_lens must be int32");
  TORCH_CHECK(block_table.dim() == 2 && seq_lens.dim() == 1, "block_table is 2-D and seq_lens 1-D");
  TORCH_CHECK(block_table.stride(-1) == 1 && seq_lens.is_contiguous(),
              "block_table rows and seq_lens must be contiguous");
  if (kv8) {
    TORCH_CHECK(k_cache.scalar_type() == at::kFloat8_e4m3fn && v_cache.scalar_type() == at::kFloat8_e4m3fn,
                "an FP8 cache must be float8_e4m3fn");
    TORCH_CHECK((q.scalar_type() == at::kHalf || q.scalar_type() == at::kBFloat16) &&
                    q.scalar_type() == out.scalar_type(),
                "with an FP8 cache, q and out must be float16 or bfloat16 and match");
    TORCH_CHECK(k_scale->is_cuda() && v_scale->is_cuda() && k_scale->device() == dev && v_scale->device() == dev,
                "k_scale and v_scale must be on the tensors' device");
    TORCH_CHECK(k_scale->scalar_type() == at::kFloat && v_scale->scalar_type() == at::kFloat &&
                    k_scale->is_contiguous() && v_scale->is_contiguous(),
                "k_scale and v_scale must be contiguous float32");
    TORCH_CHECK(k_scale->numel() == k_cache.size(2) && v_scale->numel() == k_cache.size(2),
                "k_scale and v_scale need one value per KV head");
  } else {
    TORCH_CHECK(q.scalar_type() == k_cache.scalar_type() && q.scalar_type() == v_cache.scalar_type() &&
                    q.scalar_type() == out.scalar_type(),
                "q, caches and out must share a dtype");
  }

  const int batch = static_cast<int>(q.size(0));
  const int num_q_heads = static_cast<int>(q.size(1));
  const int head_dim = static_cast<int>(q.size(2));
  const int page_size = static_cast<int>(k_cache.size(1));
  const int num_kv_heads = static_cast<int>(k_cache.size(2));
  TORCH_CHECK(k_cache.size(3) == head_dim, "cache head_dim differs from q");
  TORCH_CHECK(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
              "num_q_heads must be a multiple of num_kv_heads");
  TORCH_CHECK(block_table.size(0) == batch && seq_lens.size(0) == batch,
              "block_table and seq_lens need one row per sequence");
  TORCH_CHECK(num_splits >= KL_SPLITS_BALANCED && max_seq_len >= 0,
              "num_splits must be >= 0 or -1 (balanced), max_seq_len >= 0");
  if (batch == 0) return;

  int64_t max_pages = block_table.size(1);
  if (max_seq_len > 0) max_pages = std::min<int64_t>(max_pages, (max_seq_len + page_size - 1) / page_size);
  TORCH_CHECK(max_pages >= 1, "block_table needs at least one column");
  const int64_t bt_stride = batch > 1 ? block_table.stride(0) : block_table.size(1);

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  const kl_dtype dtype = to_kl_dtype(q.scalar_type());
  int splits = 0;
  size_t ws_bytes = 0;
  check_status(kl_paged_decode_plan(dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size,
                                    static_cast<int>(max_pages), static_cast<int>(num_splits), 0, &splits,
                                    &ws_bytes),
               "paged_decode_attention planning");
  at::Tensor workspace;
  if (ws_bytes > 0) {
    workspace = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  }
  void* ws = ws_bytes > 0 ? workspace.data_ptr() : nullptr;
  if (kv8) {
    check_status(kl_paged_decode_attention_fp8(
                     dtype, out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                     k_scale->data_ptr<float>(), v_scale->data_ptr<float>(), block_table.data_ptr<int32_t>(),
                     seq_lens.data_ptr<int32_t>(), batch, num_q_heads, num_kv_heads, head_dim, page_size, bt_stride,
                     static_cast<int>(max_pages), static_cast<float>(scale), static_cast<int>(num_splits), ws,
                     ws_bytes, current_stream(dev)),
                 "paged_decode_attention_fp8");
    return;
  }
  check_status(kl_paged_decode_attention(dtype, out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                         block_table.data_ptr<int32_t>(), seq_lens.data_ptr<int32_t>(), batch,
                                         num_q_heads, num_kv_heads, head_dim, page_size, bt_stride,
                                         static_cast<int>(max_pages), static_cast<float>(scale),
                                         static_cast<int>(num_splits), ws, ws_bytes, current_stream(dev)),
               "paged_decode_attention");
}

void paged_decode_attention(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
                            const at::Tensor& v_cache, const at::Tensor& block_table, const at::Tensor& seq_lens,
                            double scale) {
  paged_decode_impl(out, q, k_cache, v_cache, block_table, seq_lens, scale, 0, 0);
}

void paged_decode_attention_splits(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
                                   const at::Tensor& v_cache, const at::Tensor& block_table,
                                   const at::Tensor& seq_lens, double scale, int64_t num_splits,
                                   int64_t max_seq_len) {
  paged_decode_impl(out, q, k_cache, v_cache, block_table, seq_lens, scale, num_splits, max_seq_len);
}

void paged_decode_attention_fp8(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
                                const at::Tensor& v_cache, const at::Tensor& block_table, const at::Tensor& seq_lens,
                                double scale, const at::Tensor& k_scale, const at::Tensor& v_scale,
                                int64_t num_splits, int64_t max_seq_len) {
  paged_decode_impl(out, q, k_cache, v_cache, block_table, seq_lens, scale, num_splits, max_seq_len, &k_scale,
                    &v_scale);
}

// Shared-prefix decode: attention over prefix tokens, then each sequence's own.
void cascade_decode_attention(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
                              const at::Tensor& v_cache, const at::Tensor& prefix_block_table,
                              const at::Tensor& prefix_len, const at::Tensor& block_table,
                              const at::Tensor& seq_lens, double scale) {
  const auto dev = q.device();
  const std::initializer_list<const at::Tensor*> all = {&k_cache, &v_cache,    &out,    &prefix_block_table,
                                                        &prefix_len, &block_table, &seq_lens};
  for (const at::Tensor* t : all) {
    TORCH_CHECK(t->is_cuda() && t->device() == dev, "tensors must share q's GPU");
  }
  TORCH_CHECK(q.dim() == 3 && k_cache.dim() == 4, "q is [batch, heads, dim]; caches are 4-D");
  TORCH_CHECK(q.is_contiguous() && out.is_contiguous() && k_cache.is_contiguous() && v_cache.is_contiguous(),
              "q, out and both caches must be contiguous");
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes() && out.sizes() == q.sizes(), "cache or output shapes differ");
  TORCH_CHECK(q.scalar_type() == k_cache.scalar_type() && q.scalar_type() == v_cache.scalar_type() &&
                  q.scalar_type() == out.scalar_type(),
              "q, caches and out must share a dtype");
  TORCH_CHECK(prefix_block_table.scalar_type() == at::kInt && prefix_block_table.dim() == 1 &&
                  prefix_block_table.is_contiguous(),
              "prefix_block_table is a contiguous 1-D int32 tensor");
  TORCH_CHECK(prefix_len.scalar_type() == at::kInt && prefix_len.numel() == 1, "prefix_len is one int32");
  TORCH_CHECK(block_table.scalar_type() == at::kInt && seq_lens.scalar_type() == at::kInt &&
                  block_table.dim() == 2 && seq_lens.dim() == 1 && block_table.stride(-1) == 1 &&
                  seq_lens.is_contiguous(),
              "block_table is 2-D int32 with contiguous rows; seq_lens contiguous 1-D int32");
  const int batch = static_cast<int>(q.size(0));
  const int num_q_heads = static_cast<int>(q.size(1));
  const int head_dim = static_cast<int>(q.size(2));
  const int page_size = static_cast<int>(k_cache.size(1));
  const int num_kv_heads = static_cast<int>(k_cache.size(2));
  TORCH_CHECK(k_cache.size(3) == head_dim, "cache head_dim differs from q");
  TORCH_CHECK(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  TORCH_CHECK(block_table.size(0) == batch && seq_lens.size(0) == batch,
              "block_table and seq_lens need one row per sequence");
  if (batch == 0) return;
  const int64_t max_pages = block_table.size(1);
  TORCH_CHECK(max_pages >= 1, "block_table needs at least one column");
  const int64_t bt_stride = batch > 1 ? block_table.stride(0) : block_table.size(1);
  const int prefix_pages = static_cast<int>(prefix_block_table.numel());

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  const kl_dtype dtype = to_kl_dtype(q.scalar_type());
  size_t ws_bytes = 0;
  check_status(kl_cascade_decode_plan(dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, prefix_pages,
                                      static_cast<int>(max_pages), 0, &ws_bytes),
               "cascade_decode_attention planning");
  at::Tensor workspace = at::empty({static_cast<int64_t>(ws_bytes)}, q.options().dtype(at::kByte));
  check_status(kl_cascade_decode_attention(
                   dtype, out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                   prefix_pages > 0 ? prefix_block_table.data_ptr<int32_t>() : nullptr,
                   prefix_len.data_ptr<int32_t>(), prefix_pages, block_table.data_ptr<int32_t>(),
                   seq_lens.data_ptr<int32_t>(), batch, num_q_heads, num_kv_heads, head_dim, page_size, bt_stride,
                   static_cast<int>(max_pages), static_cast<float>(scale), workspace.data_ptr(), ws_bytes,
                   current_stream(dev)),
               "cascade_decode_attention");
}

}  // namespace

TORCH_LIBRARY(kernel_lab, m) {
  m.def("rms_norm(Tensor! out, Tensor x, Tensor weight, float eps) -> ()");
  m.def("fused_add_rms_norm(Tensor! out, Tensor x, Tensor! residual, Tensor weight, float eps) -> ()");
  m.def("fused_add_rmsnorm(Tensor! out, Tensor x, Tensor! residual, Tensor weight, float eps) -> ()");
  m.def(
      "paged_decode_attention(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, "
      "Tensor block_table, Tensor seq_lens, float scale) -> ()");
  m.def(
      "paged_decode_attention.splits(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, "
      "Tensor block_table, Tensor seq_lens, float scale, int num_splits, int max_seq_len) -> ()");
  m.def(
      "paged_decode_attention_fp8(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, "
      "Tensor block_table, Tensor seq_lens, float scale, Tensor k_scale, Tensor v_scale, "
      "int num_splits=0, int max_seq_len=0) -> ()");
  m.def(
      "cascade_decode_attention(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, "
      "Tensor prefix_block_table, Tensor prefix_len, Tensor block_table, Tensor seq_lens, float scale) -> ()");
}

// ROCm tensors carry PyTorch's CUDA dispatch key.
TORCH_LIBRARY_IMPL(kernel_lab, CUDA, m) {
  m.impl("rms_norm", &rms_norm);
  m.impl("fused_add_rms_norm", &fused_add_rms_norm);
  m.impl("fused_add_rmsnorm", &fused_add_rms_norm);
  m.impl("paged_decode_attention", &paged_decode_attention);
  m.impl("paged_decode_attention.splits", &paged_decode_attention_splits);
  m.impl("paged_decode_attention_fp8", &paged_decode_attention_fp8);
  m.impl("cascade_decode_attention", &cascade_decode_attention);
}
