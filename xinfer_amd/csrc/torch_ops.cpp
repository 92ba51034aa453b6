// torch.library registration and AOTInductor C shims of the xinfer operators.
//
// A thin layer over the C ABI (include/xinfer_attention.h): it validates the
// torch-specific parts of the reference contract with the reference's
// messages, makes layout copies where the reference does, allocates the output
// and workspace through the caching allocator, and launches on the current
// stream of the inputs' device.
//   schemas          compiler/common/kernels/attention.cpp:128-135 and the
//                    triton_op schema of compiler/common/kernels/kv_cache.py:45-52
//   CUDA-key impls   attention.cpp:137-140 (ROCm torch keeps the CUDA key)
//   C shims          compiler/common/kernels/attention_shim.cpp:5-32
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/inductor/aoti_torch/utils.h>
#include <torch/library.h>

#include <cmath>
#include <vector>

#include "xinfer_attention.h"
#include "xinfer_attention_aoti.h"

namespace xinfer {
namespace {

xinfer_view4 view_of(const at::Tensor &t) {
  xinfer_view4 v{};
  v.data = t.data_ptr();
  for (int i = 0; i < 4; ++i) {
    v.size[i] = t.size(i);
    v.stride[i] = t.stride(i);
  }
  return v;
}

// The kernels read 16-byte feature chunks: unit feature stride, strides of the
// other dimensions divisible by 8 elements and a 16-byte aligned base.
bool kernel_layout(const at::Tensor &t) {
  if ((reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) != 0) return false;
  if (t.size(3) > 1 && t.stride(3) != 1) return false;
  for (int i = 0; i < 3; ++i)
    if (t.size(i) > 1 && t.stride(i) % 8 != 0) return false;
  // One (row, head) slice is addressed with 32-bit byte offsets.
  if ((t.size(2) + 1) * t.stride(2) * 2 >= (int64_t(1) << 31)) return false;
  return true;
}

// Q additionally fits one batch row ([Hq, T, D]) in 32-bit byte offsets.
bool query_layout(const at::Tensor &q) {
  return kernel_layout(q) && (q.size(1) * q.stride(1) + q.size(2) * q.stride(2)) * 2 < (int64_t(1) << 31);
}

void *current_stream(const at::Tensor &t) {
  return static_cast<void *>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_status(int status) { TORCH_CHECK(status == XINFER_OK, xinfer_status_string(status)); }

}  // namespace

// Replaces compiler/common/kernels/attention.cpp:14-79.  With `bthd` the
// output is a contiguous [B,T,Hq,D] tensor instead (the optional variant).
at::Tensor batched_attention(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                             const at::Tensor &offsets, const at::Tensor &cuda_offsets, const at::Tensor &blocks,
                             double scale, bool bthd) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.sizes() == k.sizes() && k.size(0) == q.size(0) &&
                  k.size(3) == q.size(3),
              "Invalid Q/K/V shapes");
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device() &&
                  q.scalar_type() == at::kBFloat16 && k.scalar_type() == q.scalar_type() &&
                  v.scalar_type() == q.scalar_type(),
              "Expected colocated CUDA BF16 Q/K/V");
  const auto batch = q.size(0);
  TORCH_CHECK(offsets.device().is_cpu() && offsets.scalar_type() == at::kInt &&
                  offsets.is_contiguous() && offsets.sizes() == at::IntArrayRef({2, batch + 1}),
              "Expected CPU int32 cumulative query/KV lengths [2,B+1]");
  TORCH_CHECK(cuda_offsets.device() == q.device() && cuda_offsets.scalar_type() == at::kInt &&
                  cuda_offsets.sizes() == offsets.sizes() && cuda_offsets.is_contiguous() &&
                  blocks.device() == q.device() && blocks.scalar_type() == at::kInt &&
                  blocks.sizes() == at::IntArrayRef({batch, 1}),
              "Invalid CUDA attention metadata");
  const int32_t *cuq = static_cast<const int32_t *>(offsets.data_ptr());
  const int32_t *cuk = cuq + batch + 1;
  TORCH_CHECK(cuq[0] == 0 && cuk[0] == 0, "Cumulative lengths must start at zero");
  int64_t max_length = 0;
  for (int64_t row = 0; row < batch; ++row) {
    const int64_t count = cuq[row + 1] - cuq[row], length = cuk[row + 1] - cuk[row];
    TORCH_CHECK(count >= 0 && count <= q.size(2) && length >= count && length >= 1 &&
                    length <= k.size(2),
                "Invalid query/KV lengths");
    max_length = std::max(max_length, length);
  }
  c10::DeviceGuard guard(q.device());
  auto output = bthd ? at::empty({q.size(0), q.size(2), q.size(1), q.size(3)}, q.options())
                     : at::empty(q.sizes(), q.options());
  if (batch == 0 || q.size(2) == 0) return output;
  // Row r's KV lives in k[page]/v[page], page = blocks[r] when the capacity
  // is a multiple of 256 (the reference's paged call, :39-40, :56-58, :68-70),
  // else k[r]/v[r].  The kernels read the table on the device.  Copy only
  // what the kernels cannot read in place, as the reference does (:58-61,
  // :108-114); a copy of the longest populated prefix covers every key any
  // row reads, in every row of the batch dimension.
  auto query = query_layout(q) ? q : q.contiguous();
  auto key = kernel_layout(k) ? k : k.narrow(2, 0, max_length).contiguous();
  auto value = kernel_layout(v) ? v : v.narrow(2, 0, max_length).contiguous();
  if (key.size(2) != value.size(2)) {
    key = k.narrow(2, 0, max_length).contiguous();
    value = v.narrow(2, 0, max_length).contiguous();
  }
  auto qv = view_of(query), kv = view_of(key), vv = view_of(value);
  const int32_t *pages = k.size(2) % 256 == 0 ? static_cast<const int32_t *>(blocks.data_ptr()) : nullptr;
  const size_t bytes = xinfer_batched_flash_attention_workspace_size(&qv, &kv, cuq);
  auto workspace = at::empty({static_cast<int64_t>(bytes)}, q.options().dtype(at::kByte));
  if (bthd) {
    auto ov = view_of(output.transpose(1, 2));
    check_status(xinfer_batched_flash_attention_out(&qv, &kv, &vv, cuq, pages, blocks.stride(0), scale, &ov,
                                                    workspace.data_ptr(), bytes, current_stream(q)));
  } else {
    check_status(xinfer_batched_flash_attention(&qv, &kv, &vv, cuq, pages, blocks.stride(0), scale,
                                                output.data_ptr(), workspace.data_ptr(), bytes, current_stream(q)));
  }
  return output;
}

at::Tensor batched_flash_attention(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                                   const at::Tensor &offsets, const at::Tensor &cuda_offsets,
                                   const at::Tensor &blocks, double scale) {
  return batched_attention(q, k, v, offsets, cuda_offsets, blocks, scale, false);
}

// The optional variant of compiler/qwen3/adapters/attention.py:58-61: the same
// operation with the output already in the [B,T,Hq,D] order the adapter
// reshapes to [B,T,Hq*D], so that reshape is a view instead of a copy.
at::Tensor batched_flash_attention_bthd(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                                        const at::Tensor &offsets, const at::Tensor &cuda_offsets,
                                        const at::Tensor &blocks, double scale) {
  return batched_attention(q, k, v, offsets, cuda_offsets, blocks, scale, true);
}

// Graph-capture variant of batched_flash_attention: the same schema, but the
// row lengths come from cuda_offsets when the kernels run (prefill shapes are
// planned on the device from them);
// the CPU offsets are checked for shape only, so a graph captured once stays
// valid while the caller rewrites cuda_offsets (and the caches) in place
// between replays.  Output and workspace shapes depend on the tensor shapes
// only.
at::Tensor batched_flash_attention_graph(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                                         const at::Tensor &offsets, const at::Tensor &cuda_offsets,
                                         const at::Tensor &blocks, double scale) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.sizes() == k.sizes() && k.size(0) == q.size(0) &&
                  k.size(3) == q.size(3),
              "Invalid Q/K/V shapes");
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device() &&
                  q.scalar_type() == at::kBFloat16 && k.scalar_type() == q.scalar_type() &&
                  v.scalar_type() == q.scalar_type(),
              "Expected colocated CUDA BF16 Q/K/V");
  const auto batch = q.size(0);
  TORCH_CHECK(offsets.device().is_cpu() && offsets.scalar_type() == at::kInt &&
                  offsets.sizes() == at::IntArrayRef({2, batch + 1}),
              "Expected CPU int32 cumulative query/KV lengths [2,B+1]");
  TORCH_CHECK(cuda_offsets.device() == q.device() && cuda_offsets.scalar_type() == at::kInt &&
                  cuda_offsets.sizes() == offsets.sizes() && cuda_offsets.is_contiguous() &&
                  blocks.device() == q.device() && blocks.scalar_type() == at::kInt &&
                  blocks.sizes() == at::IntArrayRef({batch, 1}),
              "Invalid CUDA attention metadata");
  c10::DeviceGuard guard(q.device());
  auto output = at::empty(q.sizes(), q.options());
  if (batch == 0 || q.size(2) == 0) return output;
  // Any row may read up to the capacity, so a layout copy covers all of it.
  auto query = query_layout(q) ? q : q.contiguous();
  auto key = kernel_layout(k) ? k : k.contiguous();
  auto value = kernel_layout(v) ? v : v.contiguous();
  auto qv = view_of(query), kv = view_of(key), vv = view_of(value);
  const size_t bytes = xinfer_batched_flash_attention_graph_workspace_size(&qv, &kv);
  auto workspace = at::empty({static_cast<int64_t>(bytes)}, q.options().dtype(at::kByte));
  const int32_t *pages = k.size(2) % 256 == 0 ? static_cast<const int32_t *>(blocks.data_ptr()) : nullptr;
  check_status(xinfer_batched_flash_attention_graph(&qv, &kv, &vv, static_cast<const int32_t *>(cuda_offsets.data_ptr()),
                                                    pages, blocks.stride(0), scale, output.data_ptr(),
                                                    workspace.data_ptr(), bytes, current_stream(q)));
  return output;
}

// Replaces compiler/common/kernels/attention.cpp:82-124.
at::Tensor flash_attention(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v,
                           const at::Tensor &extent, double scale) {
  TORCH_CHECK(q.is_cuda() && k.device() == q.device() && v.device() == q.device(),
              "xinfer attention requires Q/K/V on the same CUDA device");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16 &&
                  v.scalar_type() == at::kBFloat16,
              "xinfer attention requires BF16");
  TORCH_CHECK(q.dim() == 4 && q.size(0) > 0 && q.size(2) >= 1 && q.size(2) <= 512,
              "Unsupported Q shape");
  TORCH_CHECK(k.dim() == 4 && v.dim() == 4 && k.size(0) == q.size(0) && k.size(2) > 0 &&
                  k.size(3) == q.size(3) && v.sizes() == k.sizes(),
              "Expected matching full-capacity K/V inputs [batch,kv_heads,capacity,head_dim]");
  TORCH_CHECK(q.size(1) > 0 && k.size(1) > 0 && q.size(1) % k.size(1) == 0,
              "Query heads must be a positive multiple of KV heads");
  TORCH_CHECK(q.size(3) >= 8 && q.size(3) <= 256 && q.size(3) % 8 == 0,
              "Flash head dimension must be a multiple of 8 in 8..256");
  TORCH_CHECK(extent.device().is_cpu() && extent.scalar_type() == at::kByte && extent.dim() == 1,
              "Expected a CPU uint8 extent vector");
  const int64_t length = extent.size(0) - 1;  // metadata only; the data is never read
  TORCH_CHECK(length >= q.size(2) && length <= k.size(2), "Invalid valid-prefix length");
  TORCH_CHECK(std::isfinite(scale) && scale > 0, "Attention scale must be finite and positive");
  TORCH_CHECK(!q.requires_grad() && !k.requires_grad() && !v.requires_grad(),
              "xinfer attention supports inference only");
  c10::DeviceGuard guard(q.device());
  auto query = query_layout(q) ? q : q.contiguous();
  auto key = kernel_layout(k) ? k : k.slice(2, 0, length).contiguous();
  auto value = kernel_layout(v) ? v : v.slice(2, 0, length).contiguous();
  if (key.size(2) != value.size(2)) {
    key = k.slice(2, 0, length).contiguous();
    value = v.slice(2, 0, length).contiguous();
  }
  auto output = at::empty(q.sizes(), q.options());
  auto qv = view_of(query), kv = view_of(key), vv = view_of(value);
  const size_t bytes = xinfer_flash_attention_workspace_size(&qv, &kv, length);
  auto workspace = at::empty({static_cast<int64_t>(bytes)}, q.options().dtype(at::kByte));
  check_status(xinfer_flash_attention(&qv, &kv, &vv, length, scale, output.data_ptr(),
                                      workspace.data_ptr(), bytes, current_stream(q)));
  return output;
}

// Replaces the Triton op compiler/common/kernels/kv_cache.py:45-72.
void append_kv_batched(const at::Tensor &key, const at::Tensor &value, const at::Tensor &positions,
                       const at::Tensor &cu_query, const at::Tensor &cache_key,
                       const at::Tensor &cache_value) {
  TORCH_CHECK(cache_key.is_contiguous() && cache_value.is_contiguous(),
              "Expected contiguous KV caches");
  TORCH_CHECK(key.dim() == 4 && value.sizes() == key.sizes() && cache_key.dim() == 4 &&
                  cache_value.sizes() == cache_key.sizes(),
              "Expected key/value [B,H,T,D] and caches [B,H,C,D]");
  TORCH_CHECK(key.scalar_type() == at::kBFloat16 && value.scalar_type() == at::kBFloat16 &&
                  cache_key.scalar_type() == at::kBFloat16 &&
                  cache_value.scalar_type() == at::kBFloat16,
              "xinfer KV append requires BF16");
  TORCH_CHECK(key.is_cuda() && value.device() == key.device() && cache_key.device() == key.device() &&
                  cache_value.device() == key.device() && positions.device() == key.device() &&
                  cu_query.device() == key.device(),
              "xinfer KV append requires colocated CUDA tensors");
  TORCH_CHECK(positions.scalar_type() == at::kLong && positions.dim() == 2 &&
                  positions.size(0) == key.size(0) && positions.size(1) == key.size(2),
              "Expected int64 positions [B,T]");
  TORCH_CHECK(cu_query.scalar_type() == at::kInt && cu_query.dim() == 1 &&
                  cu_query.size(0) == key.size(0) + 1,
              "Expected int32 cumulative query lengths [B+1]");
  c10::DeviceGuard guard(key.device());
  // A strided cu_query row (e.g. cuda_offsets[0]) is contiguous; other strides are copied.
  auto cu = cu_query.is_contiguous() ? cu_query : cu_query.contiguous();
  auto kv = view_of(key), vv = view_of(value), ck = view_of(cache_key), cv = view_of(cache_value);
  check_status(xinfer_append_kv_batched(&kv, &vv, static_cast<const int64_t *>(positions.data_ptr()),
                                        positions.stride(0), positions.stride(1),
                                        static_cast<const int32_t *>(cu.data_ptr()), &ck, &cv, current_stream(key)));
}

// Replaces the eager step before the attention operator,
// compiler/qwen3/adapters/attention.py:44-51: q/k RMSNorm (transformers
// Qwen3RMSNorm), apply_rotary_pos_emb and KVCache.update (the append).
// q [B,T,Hq,D], key/value [B,T,Hkv,D] are the projections viewed per head
// (`proj(x).view(B, T, -1, D)`), cos/sin [B,T,D]; returns the rotated query
// as a contiguous [B,Hq,T,D] tensor and appends the rotated key and the value
// to the caches in place.
at::Tensor qk_norm_rope_append(const at::Tensor &q, const at::Tensor &key, const at::Tensor &value,
                               const at::Tensor &q_weight, const at::Tensor &k_weight, double eps,
                               const at::Tensor &cos, const at::Tensor &sin, const at::Tensor &positions,
                               const at::Tensor &cu_query, const at::Tensor &cache_key,
                               const at::Tensor &cache_value) {
  TORCH_CHECK(q.dim() == 4 && key.dim() == 4 && value.sizes() == key.sizes() && key.size(0) == q.size(0) &&
                  key.size(1) == q.size(1) && key.size(3) == q.size(3) && cos.dim() == 3 &&
                  cos.sizes() == sin.sizes() && cos.size(0) == q.size(0) && cos.size(1) == q.size(1) &&
                  cos.size(2) == q.size(3) && q_weight.dim() == 1 && q_weight.size(0) == q.size(3) &&
                  k_weight.sizes() == q_weight.sizes(),
              "Expected q [B,T,Hq,D], key/value [B,T,Hkv,D], cos/sin [B,T,D] and [D] weights");
  for (const at::Tensor *t : {&q, &key, &value, &q_weight, &k_weight, &cos, &sin, &cache_key, &cache_value})
    TORCH_CHECK(t->scalar_type() == at::kBFloat16, "xinfer norm/rope append requires BF16");
  for (const at::Tensor *t : {&key, &value, &q_weight, &k_weight, &cos, &sin, &positions, &cu_query, &cache_key,
                              &cache_value})
    TORCH_CHECK(q.is_cuda() && t->device() == q.device(), "xinfer norm/rope append requires colocated CUDA tensors");
  TORCH_CHECK(cache_key.is_contiguous() && cache_value.is_contiguous(), "Expected contiguous KV caches");
  TORCH_CHECK(positions.scalar_type() == at::kLong && positions.dim() == 2 && positions.size(0) == q.size(0) &&
                  positions.size(1) == q.size(1),
              "Expected int64 positions [B,T]");
  TORCH_CHECK(cu_query.scalar_type() == at::kInt && cu_query.dim() == 1 && cu_query.size(0) == q.size(0) + 1,
              "Expected int32 cumulative query lengths [B+1]");
  c10::DeviceGuard guard(q.device());
  auto output = at::empty({q.size(0), q.size(2), q.size(1), q.size(3)}, q.options());
  // Per-head views [B,H,T,D]; rows the kernel cannot read in place are copied.
  auto rows = [](const at::Tensor &t) { return kernel_layout(t) ? t : t.contiguous(); };
  auto qh = rows(q.transpose(1, 2)), kh = rows(key.transpose(1, 2)), vh = rows(value.transpose(1, 2));
  auto cs = rows(cos.unsqueeze(1)), sn = rows(sin.unsqueeze(1));
  auto qw = q_weight.contiguous(), kw = k_weight.contiguous();
  auto cu = cu_query.is_contiguous() ? cu_query : cu_query.contiguous();
  auto qv = view_of(qh), kv = view_of(kh), vv = view_of(vh), cv = view_of(cs), sv = view_of(sn);
  auto ck = view_of(cache_key), cvv = view_of(cache_value);
  check_status(xinfer_qk_norm_rope_append(&qv, &kv, &vv, qw.data_ptr(), kw.data_ptr(), eps, &cv, &sv,
                                          static_cast<const int64_t *>(positions.data_ptr()), positions.stride(0),
                                          positions.stride(1), static_cast<const int32_t *>(cu.data_ptr()),
                                          output.data_ptr(), &ck, &cvv, current_stream(q)));
  return output;
}

// Replaces the Triton op compiler/common/kernels/projection_gemv.py:35-62,
// with its checks, their order and messages (ValueError in Python).
at::Tensor projection_gemv(const at::Tensor &x, const at::Tensor &weight) {
  TORCH_CHECK_VALUE(x.is_cuda() && weight.device() == x.device(), "Projection GEMV requires colocated CUDA tensors");
  TORCH_CHECK_VALUE((x.scalar_type() == at::kBFloat16 || x.scalar_type() == at::kFloat) &&
                        weight.scalar_type() == x.scalar_type(),
                    "Projection GEMV requires matching BF16 or FP32 tensors");
  bool singleton = x.dim() >= 2 && weight.dim() == 2;
  for (int64_t d = 0; singleton && d + 1 < x.dim(); ++d) singleton = x.size(d) == 1;
  TORCH_CHECK_VALUE(singleton, "Projection GEMV requires one input row and a 2D weight");
  TORCH_CHECK_VALUE(x.size(-1) == weight.size(1) && x.stride(-1) == 1 && weight.is_contiguous(),
                    "Projection GEMV requires matching contiguous reduction dimensions");
  const int64_t n = weight.size(0), k = weight.size(1);
  TORCH_CHECK_VALUE(n > 0 && k > 0, "Projection GEMV requires positive dimensions");
  c10::DeviceGuard guard(x.device());
  std::vector<int64_t> shape(x.sizes().begin(), x.sizes().end());
  shape.back() = n;
  auto output = at::empty(shape, x.options());
  check_status(xinfer_projection_gemv(x.data_ptr(), weight.data_ptr(), output.data_ptr(), n, k,
                                      x.scalar_type() == at::kFloat ? XINFER_FP32 : XINFER_BF16, current_stream(x)));
  return output;
}

}  // namespace xinfer

TORCH_LIBRARY(xinfer, m) {
  m.def("batched_flash_attention(Tensor q, Tensor k, Tensor v, Tensor offsets, "
        "Tensor cuda_offsets, Tensor blocks, float scale) -> Tensor",
        {at::Tag::flexible_layout});
  m.def("flash_attention(Tensor q, Tensor k, Tensor v, Tensor kv_extent, float scale) -> Tensor",
        {at::Tag::flexible_layout});
  m.def("batched_flash_attention_bthd(Tensor q, Tensor k, Tensor v, Tensor offsets, "
        "Tensor cuda_offsets, Tensor blocks, float scale) -> Tensor",
        {at::Tag::flexible_layout});
  m.def("batched_flash_attention_graph(Tensor q, Tensor k, Tensor v, Tensor offsets, "
        "Tensor cuda_offsets, Tensor blocks, float scale) -> Tensor",
        {at::Tag::flexible_layout});
  m.def("append_kv_batched(Tensor key, Tensor value, Tensor positions, Tensor cu_query, "
        "Tensor(a4!) cache_key, Tensor(a5!) cache_value) -> ()");
  m.def("projection_gemv(Tensor x, Tensor weight) -> Tensor");
  m.def("qk_norm_rope_append(Tensor q, Tensor key, Tensor value, Tensor q_weight, Tensor k_weight, "
        "float eps, Tensor cos, Tensor sin, Tensor positions, Tensor cu_query, Tensor(a10!) cache_key, "
        "Tensor(a11!) cache_value) -> Tensor");
}

TORCH_LIBRARY_IMPL(xinfer, CUDA, m) {
  m.impl("batched_flash_attention", TORCH_FN(xinfer::batched_flash_attention));
  m.impl("flash_attention", TORCH_FN(xinfer::flash_attention));
  m.impl("batched_flash_attention_bthd", TORCH_FN(xinfer::batched_flash_attention_bthd));
  m.impl("batched_flash_attention_graph", TORCH_FN(xinfer::batched_flash_attention_graph));
  m.impl("append_kv_batched", TORCH_FN(xinfer::append_kv_batched));
  m.impl("qk_norm_rope_append", TORCH_FN(xinfer::qk_norm_rope_append));
  m.impl("projection_gemv", TORCH_FN(xinfer::projection_gemv));
}

using torch::aot_inductor::new_tensor_handle;
using torch::aot_inductor::resolve_tensor_dispatch_flags;

extern "C" {

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_batched_flash_attention(
    AtenTensorHandle q, AtenTensorHandle k, AtenTensorHandle v, AtenTensorHandle offsets,
    AtenTensorHandle cuda_offsets, AtenTensorHandle blocks, double scale, AtenTensorHandle *output) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    *output = new_tensor_handle(xinfer::batched_flash_attention(
        resolve_tensor_dispatch_flags(q), resolve_tensor_dispatch_flags(k),
        resolve_tensor_dispatch_flags(v), resolve_tensor_dispatch_flags(offsets),
        resolve_tensor_dispatch_flags(cuda_offsets), resolve_tensor_dispatch_flags(blocks), scale));
  });
}

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_batched_flash_attention_bthd(
    AtenTensorHandle q, AtenTensorHandle k, AtenTensorHandle v, AtenTensorHandle offsets,
    AtenTensorHandle cuda_offsets, AtenTensorHandle blocks, double scale, AtenTensorHandle *output) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    *output = new_tensor_handle(xinfer::batched_flash_attention_bthd(
        resolve_tensor_dispatch_flags(q), resolve_tensor_dispatch_flags(k),
        resolve_tensor_dispatch_flags(v), resolve_tensor_dispatch_flags(offsets),
        resolve_tensor_dispatch_flags(cuda_offsets), resolve_tensor_dispatch_flags(blocks), scale));
  });
}

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_flash_attention(AtenTensorHandle q, AtenTensorHandle k,
                                                                 AtenTensorHandle v, AtenTensorHandle extent,
                                                                 double scale, AtenTensorHandle *output) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    *output = new_tensor_handle(xinfer::flash_attention(
        resolve_tensor_dispatch_flags(q), resolve_tensor_dispatch_flags(k),
        resolve_tensor_dispatch_flags(v), resolve_tensor_dispatch_flags(extent), scale));
  });
}

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_append_kv_batched(
    AtenTensorHandle key, AtenTensorHandle value, AtenTensorHandle positions, AtenTensorHandle cu_query,
    AtenTensorHandle cache_key, AtenTensorHandle cache_value, AtenTensorHandle * /*unused_output*/) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    xinfer::append_kv_batched(resolve_tensor_dispatch_flags(key), resolve_tensor_dispatch_flags(value),
                              resolve_tensor_dispatch_flags(positions),
                              resolve_tensor_dispatch_flags(cu_query),
                              resolve_tensor_dispatch_flags(cache_key),
                              resolve_tensor_dispatch_flags(cache_value));
  });
}

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_qk_norm_rope_append(
    AtenTensorHandle q, AtenTensorHandle key, AtenTensorHandle value, AtenTensorHandle q_weight,
    AtenTensorHandle k_weight, double eps, AtenTensorHandle cos, AtenTensorHandle sin, AtenTensorHandle positions,
    AtenTensorHandle cu_query, AtenTensorHandle cache_key, AtenTensorHandle cache_value, AtenTensorHandle *output) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    *output = new_tensor_handle(xinfer::qk_norm_rope_append(
        resolve_tensor_dispatch_flags(q), resolve_tensor_dispatch_flags(key), resolve_tensor_dispatch_flags(value),
        resolve_tensor_dispatch_flags(q_weight), resolve_tensor_dispatch_flags(k_weight), eps,
        resolve_tensor_dispatch_flags(cos), resolve_tensor_dispatch_flags(sin),
        resolve_tensor_dispatch_flags(positions), resolve_tensor_dispatch_flags(cu_query),
        resolve_tensor_dispatch_flags(cache_key), resolve_tensor_dispatch_flags(cache_value)));
  });
}

AOTI_TORCH_EXPORT AOTITorchError aoti_torch_cuda_projection_gemv(AtenTensorHandle x, AtenTensorHandle weight,
                                                                 AtenTensorHandle *output) {
  AOTI_TORCH_CONVERT_EXCEPTION_TO_ERROR_CODE({
    *output = new_tensor_handle(
        xinfer::projection_gemv(resolve_tensor_dispatch_flags(x), resolve_tensor_dispatch_flags(weight)));
  });
}

}  // extern "C"
