// PyTorch-ROCm binding of the `flash_attn_wmma` module: the drop-in
// replacement of the reference's csrc/flash_attn.cpp:4-29 (same module name,
// function names, argument names, defaults and return values).
//
// The torch-side half of the reference host entries lives here, with the
// reference's checks in the reference's order and with its messages:
//   forward_flash2: csrc/kernel_flash2.cu:741-767,
//   forward_naive:  csrc/kernel_naive.cu:252-276, 285.
// Then the call goes through the C ABI (include/flashlite_attn.h) on the
// current HIP stream of the tensors' device.  A non-zero status becomes a
// RuntimeError carrying the library's message (the reference's CUDA_CHECK,
// csrc/includes/flash_attn.h:15-22).  Plain C++: compiled by the host
// compiler, no hipify.

#include <torch/extension.h>

// ROCm PyTorch reports HIP devices as device type `cuda`; its HIP guard and
// stream accessors for that case are the "MasqueradingAsCUDA" variants.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <optional>

#include "flashlite_attn.h"

namespace flash_attn {

namespace {

void* current_stream(const torch::Tensor& t) {
  return static_cast<void*>(
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

fl_attn_params make_params(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                           torch::Tensor& o, double sm_scale, bool is_causal) {
  fl_attn_params p;
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.o = o.data_ptr();
  p.batch = q.size(0);
  p.heads = q.size(1);
  p.seq_q = q.size(2);
  p.seq_k = k.size(2);
  p.head_dim = q.size(3);
  p.sm_scale = sm_scale;
  p.causal = is_causal ? 1 : 0;
  return p;
}

void check_same_device(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v) {
  TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
              "All tensors must be on the same device");
}

}  // namespace

torch::Tensor flash_attn_forward_naive(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                       double sm_scale, bool is_causal) {
  TORCH_CHECK(q.is_cuda(), "Query tensor must be on CUDA");
  TORCH_CHECK(k.is_cuda(), "Key tensor must be on CUDA");
  TORCH_CHECK(v.is_cuda(), "Value tensor must be on CUDA");

  TORCH_CHECK(q.is_contiguous(), "Query tensor must be contiguous");
  TORCH_CHECK(k.is_contiguous(), "Key tensor must be contiguous");
  TORCH_CHECK(v.is_contiguous(), "Value tensor must be contiguous");

  TORCH_CHECK(q.dtype() == torch::kHalf, "Query tensor must be FP16 (Half)");
  TORCH_CHECK(k.dtype() == torch::kHalf, "Key tensor must be FP16 (Half)");
  TORCH_CHECK(v.dtype() == torch::kHalf, "Value tensor must be FP16 (Half)");

  TORCH_CHECK(q.dim() == 4, "Query tensor must have 4 dimensions [B, H, N, D]");
  TORCH_CHECK(k.dim() == 4, "Key tensor must have 4 dimensions [B, H, N, D]");
  TORCH_CHECK(v.dim() == 4, "Value tensor must have 4 dimensions [B, H, N, D]");

  TORCH_CHECK(k.size(0) == q.size(0) && k.size(1) == q.size(1) && k.size(3) == q.size(3),
              "Key dimensions must match Query dimensions [B, H, N_k, D]");
  TORCH_CHECK(v.size(0) == q.size(0) && v.size(1) == q.size(1) && v.size(2) == k.size(2) &&
                  v.size(3) == q.size(3),
              "Value dimensions must match Key dimensions [B, H, N_k, D]");
  check_same_device(q, k, v);

  auto out = torch::empty_like(q);

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  fl_attn_params p = make_params(q, k, v, out, sm_scale, is_causal);
  const int rc = fl_attn_naive_f16(&p, current_stream(q));
  TORCH_CHECK(rc == FL_OK, "FlashLite HIP error: ", fl_attn_last_error());
  return out;
}

torch::Tensor flash_attn_forward_flash2(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                        double sm_scale, bool is_causal,
                                        std::optional<torch::Tensor> out) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "All tensors must be on CUDA");
  TORCH_CHECK(q.is_contiguous() && k.is_contiguous() && v.is_contiguous(),
              "All tensors must be contiguous");
  TORCH_CHECK(q.dtype() == torch::kHalf && k.dtype() == torch::kHalf && v.dtype() == torch::kHalf,
              "All tensors must be FP16 (Half)");
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "Tensors must be 4D [B, H, N, D]");

  const int64_t batch_size = q.size(0);
  const int64_t num_heads = q.size(1);
  const int64_t head_dim = q.size(3);

  TORCH_CHECK(k.size(0) == batch_size && k.size(1) == num_heads && k.size(3) == head_dim,
              "Key dimensions must match Query dimensions [B, H, N_k, D]");
  TORCH_CHECK(v.size(0) == batch_size && v.size(1) == num_heads && v.size(2) == k.size(2) &&
                  v.size(3) == head_dim,
              "Value dimensions must match Key dimensions [B, H, N_k, D]");
  TORCH_CHECK(head_dim == 64, "FlashLite WMMA kernel currently requires head_dim == 64");
  check_same_device(q, k, v);

  torch::Tensor out_tensor;
  if (out.has_value() && out.value().defined()) {
    out_tensor = out.value();
    TORCH_CHECK(out_tensor.is_cuda() && out_tensor.is_contiguous(),
                "out tensor must be contiguous CUDA tensor");
    TORCH_CHECK(out_tensor.sizes() == q.sizes(), "out tensor shape must match q");
    TORCH_CHECK(out_tensor.dtype() == torch::kHalf, "out tensor dtype must be FP16");
    TORCH_CHECK(out_tensor.device() == q.device(), "out tensor must be on the same device as q");
  } else {
    out_tensor = torch::empty_like(q);
  }

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  fl_attn_params p = make_params(q, k, v, out_tensor, sm_scale, is_causal);
  const int rc = fl_attn_fwd_f16(&p, current_stream(q));
  TORCH_CHECK(rc == FL_OK, "FlashLite HIP error: ", fl_attn_last_error());
  return out_tensor;
}

// Beyond the reference surface: any [B, H, N, 64] strided views with a
// unit-stride head dimension (e.g. the transpose of a [B, N, H, 64] tensor),
// N_k != N_q (bottom-right causal), optionally the fp32 log-sum-exp
// [B, H, N_q], and split-KV for few query rows over many keys.  Returns
// `out`, or (out, lse) with return_lse.  An omitted `out` is allocated with
// q's layout (empty_like keeps dense strides); an omitted `lse` (with
// return_lse) as a contiguous fp32 [B, H, N_q] tensor.  Passing both keeps
// the call free of allocations (apart from a split-KV workspace, see below).
// num_splits: 0 = the library's choice, 1 = one pass, n > 1 = n key chunks.
// A split-KV call needs a workspace: `workspace` (any device tensor of
// enough bytes, reused across calls for an allocation-free loop) or else
// one from the caching allocator.
py::object flash_attn_forward_flash2_ex(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                        double sm_scale, bool is_causal,
                                        std::optional<torch::Tensor> out, bool return_lse,
                                        int64_t num_splits,
                                        std::optional<torch::Tensor> workspace,
                                        std::optional<torch::Tensor> lse_out) {
  TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda(), "All tensors must be on CUDA");
  const auto dt = q.scalar_type();
  TORCH_CHECK((dt == torch::kHalf || dt == torch::kBFloat16) && k.scalar_type() == dt &&
                  v.scalar_type() == dt,
              "All tensors must be FP16 (Half), or all BF16");
  const bool bf16 = dt == torch::kBFloat16;
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "Tensors must be 4D [B, H, N, D]");
  const int64_t batch_size = q.size(0);
  const int64_t num_heads = q.size(1);
  const int64_t head_dim = q.size(3);
  TORCH_CHECK(k.size(0) == batch_size && k.size(1) == num_heads && k.size(3) == head_dim,
              "Key dimensions must match Query dimensions [B, H, N_k, D]");
  TORCH_CHECK(v.size(0) == batch_size && v.size(1) == num_heads && v.size(2) == k.size(2) &&
                  v.size(3) == head_dim,
              "Value dimensions must match Key dimensions [B, H, N_k, D]");
  TORCH_CHECK(head_dim == 64 || head_dim == 128, "forward_flash2_ex requires head_dim 64 or 128");
  TORCH_CHECK(q.stride(3) == 1 && k.stride(3) == 1 && v.stride(3) == 1,
              "The head dimension must have unit stride");
  check_same_device(q, k, v);

  torch::Tensor out_tensor;
  if (out.has_value() && out.value().defined()) {
    out_tensor = out.value();
    TORCH_CHECK(out_tensor.is_cuda() && out_tensor.stride(3) == 1,
                "out tensor must be a CUDA tensor with a unit-stride head dimension");
    TORCH_CHECK(out_tensor.sizes() == q.sizes(), "out tensor shape must match q");
    TORCH_CHECK(out_tensor.scalar_type() == dt, "out tensor dtype must match q");
    TORCH_CHECK(out_tensor.device() == q.device(), "out tensor must be on the same device as q");
  } else {
    out_tensor = torch::empty_like(q);
  }
  torch::Tensor lse;
  const bool lse_given = lse_out.has_value() && lse_out.value().defined();
  TORCH_CHECK(!lse_given || return_lse, "lse= needs return_lse=True");
  if (lse_given) {
    lse = lse_out.value();
    TORCH_CHECK(lse.is_cuda() && lse.device() == q.device(),
                "lse tensor must be on the same device as q");
    TORCH_CHECK(lse.scalar_type() == torch::kFloat32, "lse tensor dtype must be float32");
    TORCH_CHECK(lse.dim() == 3 && lse.size(0) == batch_size && lse.size(1) == num_heads &&
                    lse.size(2) == q.size(2) && lse.is_contiguous(),
                "lse tensor must be a contiguous [B, H, N_q] tensor");
  } else if (return_lse)
    lse = torch::empty({batch_size, num_heads, q.size(2)},
                       q.options().dtype(torch::kFloat32).memory_format(torch::MemoryFormat::Contiguous));

  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  fl_attn_params_ex p;
  p.base = make_params(q, k, v, out_tensor, sm_scale, is_causal);
  const torch::Tensor* ts[4] = {&q, &k, &v, &out_tensor};
  int64_t* st[4] = {p.q_stride, p.k_stride, p.v_stride, p.o_stride};
  for (int i = 0; i < 4; ++i)
    for (int d = 0; d < 3; ++d) st[i][d] = ts[i]->stride(d);
  p.lse = return_lse ? lse.data_ptr<float>() : nullptr;
  TORCH_CHECK(num_splits >= 0 && num_splits <= INT32_MAX, "num_splits must be >= 0");
  // Split-KV is built for fp16 at head_dim 64; bf16 and head_dim 128 run one pass.
  const bool one_pass_only = bf16 || head_dim != 64;
  TORCH_CHECK(!one_pass_only || num_splits <= 1,
              "split-KV (num_splits > 1) needs fp16 tensors with head_dim 64");
  const int64_t ws_bytes = (num_splits == 1 || one_pass_only)
                               ? 0
                               : fl_attn_splitkv_workspace_bytes(&p, (int32_t)num_splits);
  TORCH_CHECK(ws_bytes >= 0, "FlashLite HIP error: ", fl_attn_last_error());
  int rc;
  if (ws_bytes == 0) {
    rc = bf16 ? fl_attn_fwd_bf16_ex(&p, -1, current_stream(q))
              : fl_attn_fwd_f16_ex(&p, -1, current_stream(q));
  } else {
    torch::Tensor ws;
    if (workspace.has_value() && workspace.value().defined() &&
        workspace.value().nbytes() >= (size_t)ws_bytes) {
      ws = workspace.value();
      TORCH_CHECK(ws.is_cuda() && ws.device() == q.device() && ws.is_contiguous(),
                  "workspace must be a contiguous tensor on q's device");
    } else {
      ws = torch::empty({(ws_bytes + 3) / 4}, q.options().dtype(torch::kFloat32));
    }
    rc = fl_attn_fwd_f16_splitkv(&p, (int32_t)num_splits, ws.data_ptr(), (int64_t)ws.nbytes(),
                                 current_stream(q));
  }
  TORCH_CHECK(rc == FL_OK, "FlashLite HIP error: ", fl_attn_last_error());
  if (return_lse) return py::make_tuple(out_tensor, lse);
  return py::cast(out_tensor);
}

}  // namespace flash_attn

PYBIND11_MODULE(flash_attn_wmma, m) {
  m.doc() = "FlashAttention-2 forward for AMD Instinct MI355X (gfx950): MFMA + LDS HIP kernels";

  m.def("forward_naive", &flash_attn::flash_attn_forward_naive,
        "Naive attention forward (HIP baseline, one work-group per query row)", py::arg("q"),
        py::arg("k"), py::arg("v"), py::arg("sm_scale") = 0.0, py::arg("is_causal") = false);

  m.def("forward_flash2", &flash_attn::flash_attn_forward_flash2,
        "FlashAttention-2 forward (gfx950 MFMA)", py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("sm_scale") = 0.0, py::arg("is_causal") = false, py::arg("out") = py::none());

  m.def("forward_flash2_ex", &flash_attn::flash_attn_forward_flash2_ex,
        "FlashAttention-2 forward on strided [B, H, N, D] views (fp16 or bf16, D 64 or 128), "
        "N_k != N_q (bottom-right causal), optional log-sum-exp",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("sm_scale") = 0.0,
        py::arg("is_causal") = false, py::arg("out") = py::none(), py::arg("return_lse") = false,
        py::arg("num_splits") = 0, py::arg("workspace") = py::none(), py::arg("lse") = py::none());

  m.def("splitkv_workspace_bytes",
        [](torch::Tensor q, torch::Tensor k, bool is_causal, int64_t num_splits) {
          fl_attn_params_ex p;
          p.base = fl_attn_params{nullptr, nullptr, nullptr, nullptr, q.size(0), q.size(1),
                                  q.size(2), k.size(2), q.size(3), 0.0, is_causal ? 1 : 0};
          const int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
          const int64_t ks[3] = {k.stride(0), k.stride(1), k.stride(2)};
          for (int d = 0; d < 3; ++d) {
            p.q_stride[d] = p.o_stride[d] = qs[d];
            p.k_stride[d] = p.v_stride[d] = ks[d];
          }
          p.lse = nullptr;
          if (num_splits == 1 || q.scalar_type() != torch::kHalf || q.size(3) != 64)
            return (int64_t)0;  // one pass: split-KV is built for fp16 at head_dim 64
          const int64_t b = fl_attn_splitkv_workspace_bytes(&p, (int32_t)num_splits);
          TORCH_CHECK(b >= 0, "FlashLite HIP error: ", fl_attn_last_error());
          return b;
        },
        "Workspace bytes forward_flash2_ex needs for these q / k shapes and num_splits "
        "(0 when it runs one pass)",
        py::arg("q"), py::arg("k"), py::arg("is_causal") = false, py::arg("num_splits") = 0);
}
