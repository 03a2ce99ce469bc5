// PyTorch-ROCm binding of the MoE expert path.
//
// Exposes the eight functions of the reference extension module under their
// reference names and argument orders (reference csrc/bindings.cpp:6-57,
// 59-92), plus the fused dispatch and the inverse-map combine/backward used
// by the HIP MoE layer. Every function validates its tensors (raising
// RuntimeError like the reference's TORCH_CHECKs), allocates outputs and
// workspace through torch's caching allocator, and calls the C ABI of
// libnanotitan_moe.so on the current HIP stream of the input's device. No
// function synchronises the host.
#include <torch/extension.h>

#include <c10/hip/HIPGuard.h>
#include <c10/hip/HIPStream.h>

#include <tuple>

#include "nanotitan_moe.h"

namespace {

using torch::Tensor;

int dtype_code(const Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return NT_F32;
    case at::kDouble: return NT_F64;
    case at::kHalf: return NT_F16;
    case at::kBFloat16: return NT_BF16;
    default:
      TORCH_CHECK(false, "unsupported dtype ", t.scalar_type(),
                  " (expected float32, float64, float16 or bfloat16)");
  }
  return -1;
}

at::ScalarType scalar_of(int code) {
  switch (code) {
    case NT_F32: return at::kFloat;
    case NT_F64: return at::kDouble;
    case NT_F16: return at::kHalf;
    default: return at::kBFloat16;
  }
}

void check_status(int st, const char* what) {
  TORCH_CHECK(st == NT_OK, what, ": ", nt_strerror(st));
}

void check_device(const Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
}

void check_i32(const Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kInt, name, " must be int32");
  check_device(t, name);
}

void check_f32(const Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be float32");
  check_device(t, name);
}

// Every tensor of one call lives on the device of the first.
void check_same_device(const Tensor& first, std::initializer_list<const Tensor*> rest) {
  for (const Tensor* t : rest)
    TORCH_CHECK(t->device() == first.device(), "all tensors must be on the same device (",
                first.device(), " vs ", t->device(), ")");
}

hipStream_t stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.get_device()).stream();
}

Tensor workspace(const Tensor& like, size_t bytes) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// ------------------------------------------------------ reference surface

// count_expert_kernel(topk_experts_per_token, mask, num_experts, num_topk_experts)
// reference csrc/kernels/count_experts.cu:32-57.
Tensor count_expert_kernel(Tensor topk, Tensor mask, int64_t num_experts, int64_t num_topk) {
  check_i32(topk, "topk_experts_per_token");
  check_i32(mask, "mask");
  TORCH_CHECK(topk.is_contiguous() && mask.is_contiguous(), "inputs must be contiguous");
  TORCH_CHECK(topk.dim() == 2 && topk.size(1) == num_topk,
              "topk_experts_per_token must be [num_tokens, num_topk_experts]");
  TORCH_CHECK(mask.numel() == topk.size(0), "mask must have one entry per token");
  const int64_t T = topk.size(0);
  c10::hip::HIPGuard guard(topk.get_device());
  Tensor counts = at::empty({num_experts}, topk.options().dtype(at::kInt));
  Tensor ws = workspace(topk, nt_dispatch_workspace_bytes(T, (int32_t)num_topk,
                                                          (int32_t)num_experts, 0, NT_F32));
  check_status(nt_count_experts(topk.data_ptr<int32_t>(), mask.data_ptr<int32_t>(), T,
                                (int32_t)num_topk, (int32_t)num_experts, counts.data_ptr<int32_t>(),
                                ws.data_ptr(), ws.numel(), stream_of(topk)),
               "count_expert_kernel");
  return counts;
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> pack_impl(Tensor X, Tensor w, Tensor topk,
                                                             Tensor cursor) {
  TORCH_CHECK(X.is_contiguous(), "X must be contiguous");
  TORCH_CHECK(w.is_contiguous(), "topk_weights must be contiguous");
  check_device(X, "X");
  check_f32(w, "topk_weights");
  check_i32(topk, "topk_experts");
  check_i32(cursor, "expert_offset_cpy");
  TORCH_CHECK(topk.is_contiguous() && cursor.is_contiguous(), "indices must be contiguous");
  TORCH_CHECK(X.dim() == 2 && w.dim() == 2 && topk.sizes() == w.sizes() && w.size(0) == X.size(0),
              "expected X [T,d], topk_weights [T,k], topk_experts [T,k]");
  TORCH_CHECK(cursor.numel() >= 2, "expert_offset_cpy must hold num_experts + 1 entries");
  const int64_t T = X.size(0), d = X.size(1), k = w.size(1), A = T * k;
  const int32_t E = (int32_t)(cursor.numel() - 1);
  const int dt = dtype_code(X);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor packed_X = at::empty({A, d}, X.options());
  Tensor token_id = at::empty({A}, X.options().dtype(at::kInt));
  Tensor expert = at::empty({A}, X.options().dtype(at::kInt));
  Tensor packed_w = at::empty({A}, X.options().dtype(at::kFloat));
  Tensor inv = at::empty({T, k}, X.options().dtype(at::kInt));
  Tensor ws = workspace(X, nt_dispatch_workspace_bytes(T, (int32_t)k, E, d, dt));
  check_status(nt_pack_tokens(dt, X.data_ptr(), w.data_ptr<float>(), topk.data_ptr<int32_t>(), T,
                              (int32_t)k, d, E, cursor.data_ptr<int32_t>(), packed_X.data_ptr(),
                              token_id.data_ptr<int32_t>(), expert.data_ptr<int32_t>(),
                              packed_w.data_ptr<float>(), inv.data_ptr<int32_t>(), ws.data_ptr(),
                              ws.numel(), stream_of(X)),
               "pack_tokens_kernel");
  return {packed_X, token_id, expert, packed_w, inv};
}

// pack_tokens_kernel(X, topk_weights, topk_experts, expert_offset_cpy)
// reference csrc/kernels/pack_tokens.cu:51-111; mutates the cursor like it.
std::tuple<Tensor, Tensor, Tensor, Tensor> pack_tokens_kernel(Tensor X, Tensor w, Tensor topk,
                                                              Tensor cursor) {
  auto r = pack_impl(X, w, topk, cursor);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r)};
}

// combine_tokens_kernel(expert_outputs, packed_tokenId, packed_topk_weights, num_tokens, d_model)
// reference csrc/kernels/combine_kernels.cu:36-78. Returns float32 [T, d].
Tensor combine_tokens_kernel(Tensor y, Tensor token_id, Tensor w, int64_t num_tokens,
                             int64_t d_model) {
  TORCH_CHECK(y.is_contiguous(), "Expert output tensor should be contiguous");
  TORCH_CHECK(token_id.is_contiguous(), "packed token ids tensor should be contiguous");
  TORCH_CHECK(w.is_contiguous(), "packed topk weights tensor should be contiguous");
  check_device(y, "expert_outputs");
  check_i32(token_id, "packed_tokenId");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && y.size(1) == d_model, "expert_outputs must be [A, d_model]");
  TORCH_CHECK(token_id.numel() == y.size(0) && w.numel() == y.size(0),
              "one token id and one weight per packed row");
  const int64_t A = y.size(0);
  c10::hip::HIPGuard guard(y.get_device());
  Tensor out = at::empty({num_tokens, d_model}, y.options().dtype(at::kFloat));
  Tensor ws = workspace(y, nt_combine_workspace_bytes(A, num_tokens));
  check_status(nt_combine_tokens(dtype_code(y), y.data_ptr(), token_id.data_ptr<int32_t>(),
                                 w.data_ptr<float>(), A, num_tokens, d_model,
                                 out.data_ptr<float>(), ws.data_ptr(), ws.numel(), stream_of(y)),
               "combine_tokens_kernel");
  return out;
}

// combine_kernel_backward(expert_outputs, packed_tokenIds, packed_topk_weights,
//                         residual_stream_grad, hidden_dim)
// reference csrc/kernels/backward_combine_kernel.cu:42-93.
std::tuple<Tensor, Tensor> combine_kernel_backward(Tensor y, Tensor token_id, Tensor w, Tensor dY,
                                                   int64_t hidden_dim) {
  TORCH_CHECK(y.is_contiguous() && token_id.is_contiguous() && w.is_contiguous() &&
                  dY.is_contiguous(),
              "Tensor should be laid out in contiguous memory location");
  TORCH_CHECK(dY.scalar_type() == at::kFloat, "residual_stream_grad must be float32");
  check_device(y, "expert_outputs");
  check_device(dY, "residual_stream_grad");
  check_i32(token_id, "packed_tokenIds");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && y.size(1) == hidden_dim && dY.dim() == 2 &&
                  dY.size(1) == hidden_dim,
              "expert_outputs and residual_stream_grad must have hidden_dim columns");
  TORCH_CHECK(token_id.numel() == y.size(0) && w.numel() == y.size(0),
              "one token id and one weight per packed row");
  const int64_t A = y.size(0), T = dY.size(0);
  c10::hip::HIPGuard guard(y.get_device());
  Tensor dy = at::empty_like(y);
  Tensor dw = at::empty(w.sizes(), w.options());
  check_status(nt_combine_backward(dtype_code(y), y.data_ptr(), token_id.data_ptr<int32_t>(),
                                   w.data_ptr<float>(), dY.data_ptr<float>(), A, T, hidden_dim,
                                   dy.data_ptr(), dw.data_ptr<float>(), stream_of(y)),
               "combine_kernel_backward");
  return {dy, dw};
}

// pack_kernel_backward(packed_X_grad, packed_topk_weights_grad, packed_tokenId,
//                      packed_expert, topk_experts)
// reference csrc/kernels/backward_pack_kernel.cu:46-101.
std::tuple<Tensor, Tensor> pack_kernel_backward(Tensor dpX, Tensor dpw, Tensor token_id,
                                                Tensor expert, Tensor topk) {
  TORCH_CHECK(dpX.is_contiguous(), "packed_X_grad must be contiguous");
  TORCH_CHECK(dpw.is_contiguous(), "packed_topk_weights_grad must be contiguous");
  TORCH_CHECK(token_id.is_contiguous(), "packed_tokenId must be contiguous");
  TORCH_CHECK(expert.is_contiguous(), "packed_expert must be contiguous");
  TORCH_CHECK(topk.is_contiguous(), "topk_experts must be contiguous");
  TORCH_CHECK(dpw.scalar_type() == at::kFloat, "packed_topk_weights_grad must be float32");
  check_device(dpX, "packed_X_grad");
  check_i32(token_id, "packed_tokenId");
  check_i32(expert, "packed_expert");
  check_i32(topk, "topk_experts");
  TORCH_CHECK(dpX.dim() == 2 && topk.dim() == 2, "expected packed_X_grad [A,d], topk [T,k]");
  const int64_t A = dpX.size(0), d = dpX.size(1), T = topk.size(0), k = topk.size(1);
  TORCH_CHECK(dpw.numel() == A && token_id.numel() == A && expert.numel() == A,
              "one gate grad, token id and expert id per packed row");
  c10::hip::HIPGuard guard(dpX.get_device());
  Tensor dX = at::empty({T, d}, dpX.options());
  Tensor dw = at::empty({T, k}, dpw.options());
  Tensor ws = workspace(dpX, nt_combine_workspace_bytes(A, T));
  check_status(nt_pack_backward(dtype_code(dpX), dpX.data_ptr(), dpw.data_ptr<float>(),
                                token_id.data_ptr<int32_t>(), expert.data_ptr<int32_t>(),
                                topk.data_ptr<int32_t>(), A, T, (int32_t)k, d, dX.data_ptr(),
                                dw.data_ptr<float>(), ws.data_ptr(), ws.numel(), stream_of(dpX)),
               "pack_kernel_backward");
  return {dX, dw};
}

void check_gemm_inputs(const Tensor& a, const Tensor& offsets, const Tensor& b) {
  TORCH_CHECK(a.is_contiguous(), "X must be contiguous");
  TORCH_CHECK(b.is_contiguous(), "weights must be contiguous");
  check_device(a, "X");
  check_device(b, "weights");
  check_i32(offsets, "expert_offset");
  TORCH_CHECK(offsets.is_contiguous() && offsets.dim() == 1 && offsets.numel() >= 2,
              "expert_offset must be a 1-D [num_experts + 1] tensor");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "operands must share one dtype");
}

// grouped_gemm_kernel(X, expert_offset, weights) -> [A, N]
// reference csrc/kernels/grouped_gemm.cu:43-91.
Tensor grouped_gemm_kernel(Tensor X, Tensor offsets, Tensor W) {
  check_gemm_inputs(X, offsets, W);
  TORCH_CHECK(X.dim() == 2 && W.dim() == 3 && W.size(1) == X.size(1),
              "expected X [A,K] and weights [E,K,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = X.size(0), K = X.size(1), N = W.size(2);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor out = at::empty({A, N}, X.options());
  const int dt = dtype_code(X);
  // The forward and dX GEMMs need no workspace (only the dW split does).
  check_status(nt_grouped_gemm(dt, X.data_ptr(), offsets.data_ptr<int32_t>(), W.data_ptr(), E, A,
                               K, N, out.data_ptr(), nullptr, 0, stream_of(X)),
               "grouped_gemm_kernel");
  return out;
}

// bwd_grouped_gemm_dW_kernel(X, expert_offset, dOut) -> [E, K, N]
// reference csrc/kernels/bwd_grouped_gemm_dW.cu:43-86.
Tensor bwd_grouped_gemm_dW_kernel(Tensor X, Tensor offsets, Tensor dOut) {
  check_gemm_inputs(X, offsets, dOut);
  TORCH_CHECK(X.dim() == 2 && dOut.dim() == 2 && dOut.size(0) == X.size(0),
              "expected X [A,K] and dOut [A,N]");
  const int64_t A = X.size(0), K = X.size(1), N = dOut.size(1);
  const int32_t E = (int32_t)(offsets.numel() - 1);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor dW = at::empty({E, K, N}, X.options());
  const int dt = dtype_code(X);
  Tensor ws = workspace(X, nt_grouped_gemm_workspace_bytes(dt, E, A, K, N));
  check_status(nt_grouped_gemm_dw(dt, X.data_ptr(), offsets.data_ptr<int32_t>(), dOut.data_ptr(),
                                  E, A, K, N, dW.data_ptr(), ws.data_ptr(), ws.numel(),
                                  stream_of(X)),
               "bwd_grouped_gemm_dW_kernel");
  return dW;
}

// bwd_grouped_gemm_dX_kernel(W_gate, expert_offset, dOut) -> [A, K]
// reference csrc/kernels/bwd_grouped_gemm_dX.cu:46-96.
Tensor bwd_grouped_gemm_dX_kernel(Tensor W, Tensor offsets, Tensor dOut) {
  check_gemm_inputs(dOut, offsets, W);
  TORCH_CHECK(W.dim() == 3 && dOut.dim() == 2 && dOut.size(1) == W.size(2),
              "expected W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = dOut.size(0), K = W.size(1), N = W.size(2);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(W.get_device());
  Tensor dX = at::empty({A, K}, W.options());
  const int dt = dtype_code(W);
  check_status(nt_grouped_gemm_dx(dt, W.data_ptr(), offsets.data_ptr<int32_t>(), dOut.data_ptr(),
                                  E, A, K, N, dX.data_ptr(), nullptr, 0, stream_of(W)),
               "bwd_grouped_gemm_dX_kernel");
  return dX;
}

// grouped_gemm_gelu(X, expert_offset, W_up) -> (gelu(h), gelu'(h)), both
// [A, N], h = X @ W_up per expert: the up-projection with the activation
// fused into its epilogue.
std::tuple<Tensor, Tensor> grouped_gemm_gelu(Tensor X, Tensor offsets, Tensor W) {
  check_gemm_inputs(X, offsets, W);
  TORCH_CHECK(X.dim() == 2 && W.dim() == 3 && W.size(1) == X.size(1),
              "expected X [A,K] and weights [E,K,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = X.size(0), K = X.size(1), N = W.size(2);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor act = at::empty({A, N}, X.options());
  Tensor act_grad = at::empty({A, N}, X.options());
  const int dt = dtype_code(X);
  check_status(nt_grouped_gemm_gelu(dt, X.data_ptr(), offsets.data_ptr<int32_t>(), W.data_ptr(), E,
                                    A, K, N, act.data_ptr(), act_grad.data_ptr(), nullptr, 0,
                                    stream_of(X)),
               "grouped_gemm_gelu");
  return {act, act_grad};
}

// bwd_grouped_gemm_dX_gelu(W_down, expert_offset, dOut, act_grad) -> dH [A, K]:
// (dOut @ W^T) * gelu'(h) in one kernel.
Tensor bwd_grouped_gemm_dX_gelu(Tensor W, Tensor offsets, Tensor dOut, Tensor act_grad) {
  check_gemm_inputs(dOut, offsets, W);
  TORCH_CHECK(W.dim() == 3 && dOut.dim() == 2 && dOut.size(1) == W.size(2),
              "expected W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  TORCH_CHECK(act_grad.is_contiguous() && act_grad.dim() == 2 &&
                  act_grad.size(0) == dOut.size(0) && act_grad.size(1) == W.size(1) &&
                  act_grad.scalar_type() == W.scalar_type(),
              "expected act_grad [A,K] contiguous, in the weights' dtype");
  check_device(act_grad, "act_grad");
  const int64_t A = dOut.size(0), K = W.size(1), N = W.size(2);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(W.get_device());
  Tensor dH = at::empty({A, K}, W.options());
  const int dt = dtype_code(W);
  check_status(nt_grouped_gemm_dx_gelu(dt, W.data_ptr(), offsets.data_ptr<int32_t>(),
                                       dOut.data_ptr(), act_grad.data_ptr(), E, A, K, N,
                                       dH.data_ptr(), nullptr, 0, stream_of(W)),
               "bwd_grouped_gemm_dX_gelu");
  return dH;
}

// bwd_grouped_gemm_dW_dX(X, W, expert_offset, dOut) -> (dW [E,K,N], dX [A,K]):
// the dW and dX of one projection in one call (a dW with few tiles runs
// beside the dX in the same kernel launch).
std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX(Tensor X, Tensor W, Tensor offsets, Tensor dOut) {
  check_gemm_inputs(X, offsets, dOut);
  check_gemm_inputs(dOut, offsets, W);
  TORCH_CHECK(X.dim() == 2 && W.dim() == 3 && dOut.dim() == 2 && dOut.size(0) == X.size(0) &&
                  W.size(1) == X.size(1) && W.size(2) == dOut.size(1),
              "expected X [A,K], W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = X.size(0), K = X.size(1), N = dOut.size(1);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor dW = at::empty({E, K, N}, X.options());
  Tensor dX = at::empty({A, K}, X.options());
  const int dt = dtype_code(X);
  Tensor ws = workspace(X, nt_grouped_gemm_workspace_bytes(dt, E, A, K, N));
  check_status(nt_grouped_gemm_dw_dx(dt, X.data_ptr(), W.data_ptr(), offsets.data_ptr<int32_t>(),
                                     dOut.data_ptr(), E, A, K, N, dW.data_ptr(), dX.data_ptr(),
                                     ws.data_ptr(), ws.numel(), stream_of(X)),
               "bwd_grouped_gemm_dW_dX");
  return {dW, dX};
}

// bwd_grouped_gemm_dW_dX_gelu(act, W, expert_offset, dOut, act_grad) -> (dW, dH):
// bwd_grouped_gemm_dW_kernel(act, ., dOut) and bwd_grouped_gemm_dX_gelu(W, ., dOut,
// act_grad) in one call, paired like bwd_grouped_gemm_dW_dX.
std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX_gelu(Tensor act, Tensor W, Tensor offsets,
                                                       Tensor dOut, Tensor act_grad) {
  check_gemm_inputs(act, offsets, dOut);
  check_gemm_inputs(dOut, offsets, W);
  TORCH_CHECK(act.dim() == 2 && W.dim() == 3 && dOut.dim() == 2 && dOut.size(0) == act.size(0) &&
                  W.size(1) == act.size(1) && W.size(2) == dOut.size(1),
              "expected act [A,K], W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  TORCH_CHECK(act_grad.is_contiguous() && act_grad.sizes() == act.sizes() &&
                  act_grad.scalar_type() == W.scalar_type(),
              "expected act_grad [A,K] contiguous, in the weights' dtype");
  check_device(act_grad, "act_grad");
  const int64_t A = act.size(0), K = act.size(1), N = dOut.size(1);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(act.get_device());
  Tensor dW = at::empty({E, K, N}, act.options());
  Tensor dH = at::empty({A, K}, act.options());
  const int dt = dtype_code(act);
  Tensor ws = workspace(act, nt_grouped_gemm_workspace_bytes(dt, E, A, K, N));
  check_status(nt_grouped_gemm_dw_dx_gelu(dt, act.data_ptr(), W.data_ptr(),
                                          offsets.data_ptr<int32_t>(), dOut.data_ptr(),
                                          act_grad.data_ptr(), E, A, K, N, dW.data_ptr(),
                                          dH.data_ptr(), ws.data_ptr(), ws.numel(), stream_of(act)),
               "bwd_grouped_gemm_dW_dX_gelu");
  return {dW, dH};
}

// bwd_grouped_gemm_dW_dX_swiglu(hidden, W_out, expert_offset, dOut, gate, value)
// -> (dW_out, dgate, dvalue): bwd_grouped_gemm_dW_kernel(hidden, ., dOut) and
// bwd_grouped_gemm_dX_swiglu(W_out, ., dOut, gate, value) in one call.
std::tuple<Tensor, Tensor, Tensor> bwd_grouped_gemm_dW_dX_swiglu(Tensor hidden, Tensor W,
                                                                 Tensor offsets, Tensor dOut,
                                                                 Tensor gate, Tensor value) {
  check_gemm_inputs(hidden, offsets, dOut);
  check_gemm_inputs(dOut, offsets, W);
  TORCH_CHECK(hidden.dim() == 2 && W.dim() == 3 && dOut.dim() == 2 &&
                  dOut.size(0) == hidden.size(0) && W.size(1) == hidden.size(1) &&
                  W.size(2) == dOut.size(1),
              "expected hidden [A,K], W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  for (const Tensor* t : {&gate, &value}) {
    TORCH_CHECK(t->is_contiguous() && t->sizes() == hidden.sizes() &&
                    t->scalar_type() == W.scalar_type(),
                "expected gate and value [A,K] contiguous, in the weights' dtype");
    check_device(*t, "gate/value");
  }
  const int64_t A = hidden.size(0), K = hidden.size(1), N = dOut.size(1);
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(hidden.get_device());
  Tensor dW = at::empty({E, K, N}, hidden.options());
  Tensor dgate = at::empty({A, K}, hidden.options());
  Tensor dvalue = at::empty({A, K}, hidden.options());
  const int dt = dtype_code(hidden);
  Tensor ws = workspace(hidden, nt_grouped_gemm_workspace_bytes(dt, E, A, K, N));
  check_status(nt_grouped_gemm_dw_dx_swiglu(dt, hidden.data_ptr(), W.data_ptr(),
                                            offsets.data_ptr<int32_t>(), dOut.data_ptr(),
                                            gate.data_ptr(), value.data_ptr(), E, A, K, N,
                                            dW.data_ptr(), dgate.data_ptr(), dvalue.data_ptr(),
                                            ws.data_ptr(), ws.numel(), stream_of(hidden)),
               "bwd_grouped_gemm_dW_dX_swiglu");
  return {dW, dgate, dvalue};
}

// bwd_grouped_gemm_dW_dX2(X, W1, W2, expert_offset, dOut1, dOut2) -> (dW1, dX):
// bwd_grouped_gemm_dW_kernel(X, ., dOut1) and bwd_grouped_gemm_dX2 in one call.
std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX2(Tensor X, Tensor W1, Tensor W2,
                                                   Tensor offsets, Tensor dOut1, Tensor dOut2) {
  check_gemm_inputs(X, offsets, dOut1);
  check_gemm_inputs(dOut1, offsets, W1);
  check_gemm_inputs(dOut2, offsets, W2);
  TORCH_CHECK(X.dim() == 2 && W1.dim() == 3 && W2.sizes() == W1.sizes() && dOut1.dim() == 2 &&
                  dOut2.sizes() == dOut1.sizes() && dOut1.size(0) == X.size(0) &&
                  W1.size(1) == X.size(1) && W1.size(2) == dOut1.size(1),
              "expected X [A,K], W1, W2 [E,K,N] and dOut1, dOut2 [A,N]");
  TORCH_CHECK(offsets.numel() == W1.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = X.size(0), K = X.size(1), N = dOut1.size(1);
  const int32_t E = (int32_t)W1.size(0);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor dW1 = at::empty({E, K, N}, X.options());
  Tensor dX = at::empty({A, K}, X.options());
  const int dt = dtype_code(X);
  Tensor ws = workspace(X, nt_grouped_gemm_workspace_bytes(dt, E, A, K, N));
  check_status(nt_grouped_gemm_dw_dx2(dt, X.data_ptr(), W1.data_ptr(), W2.data_ptr(),
                                      offsets.data_ptr<int32_t>(), dOut1.data_ptr(),
                                      dOut2.data_ptr(), E, A, K, N, dW1.data_ptr(), dX.data_ptr(),
                                      ws.data_ptr(), ws.numel(), stream_of(X)),
               "bwd_grouped_gemm_dW_dX2");
  return {dW1, dX};
}

// Checks a [rows, cols] activation that travels with W's dtype and device.
void check_act(const Tensor& t, int64_t rows, int64_t cols, const Tensor& like, const char* name) {
  TORCH_CHECK(t.is_contiguous() && t.dim() == 2 && t.size(0) == rows && t.size(1) == cols &&
                  t.scalar_type() == like.scalar_type(),
              name, ": expected a contiguous [", rows, ",", cols, "] tensor in the weights' dtype");
  check_device(t, name);
}

// grouped_gemm_swiglu(X, expert_offset, W_gate, W_val) -> (hidden, gate, value),
// each [A, N]: gate and value GEMMs in one kernel, hidden = silu(gate) * value
// in its epilogue.
std::tuple<Tensor, Tensor, Tensor> grouped_gemm_swiglu(Tensor X, Tensor offsets, Tensor Wg,
                                                       Tensor Wv) {
  check_gemm_inputs(X, offsets, Wg);
  check_gemm_inputs(X, offsets, Wv);
  TORCH_CHECK(X.dim() == 2 && Wg.dim() == 3 && Wg.size(1) == X.size(1) && Wv.sizes() == Wg.sizes(),
              "expected X [A,K] and gate / value weights [E,K,N]");
  TORCH_CHECK(offsets.numel() == Wg.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = X.size(0), K = X.size(1), N = Wg.size(2);
  const int32_t E = (int32_t)Wg.size(0);
  c10::hip::HIPGuard guard(X.get_device());
  Tensor hidden = at::empty({A, N}, X.options());
  Tensor gate = at::empty({A, N}, X.options());
  Tensor value = at::empty({A, N}, X.options());
  check_status(nt_grouped_gemm_swiglu(dtype_code(X), X.data_ptr(), offsets.data_ptr<int32_t>(),
                                      Wg.data_ptr(), Wv.data_ptr(), E, A, K, N, hidden.data_ptr(),
                                      gate.data_ptr(), value.data_ptr(), nullptr, 0, stream_of(X)),
               "grouped_gemm_swiglu");
  return {hidden, gate, value};
}

// bwd_grouped_gemm_dX_swiglu(W_out, expert_offset, dOut, gate, value) ->
// (dgate, dvalue), each [A, K]: dhidden = dOut @ W_out^T and the SwiGLU
// backward in one kernel.
std::tuple<Tensor, Tensor> bwd_grouped_gemm_dX_swiglu(Tensor W, Tensor offsets, Tensor dOut,
                                                      Tensor gate, Tensor value) {
  check_gemm_inputs(dOut, offsets, W);
  TORCH_CHECK(W.dim() == 3 && dOut.dim() == 2 && dOut.size(1) == W.size(2),
              "expected W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = dOut.size(0), K = W.size(1), N = W.size(2);
  check_act(gate, A, K, W, "gate");
  check_act(value, A, K, W, "value");
  const int32_t E = (int32_t)W.size(0);
  c10::hip::HIPGuard guard(W.get_device());
  Tensor dgate = at::empty({A, K}, W.options());
  Tensor dvalue = at::empty({A, K}, W.options());
  check_status(nt_grouped_gemm_dx_swiglu(dtype_code(W), W.data_ptr(), offsets.data_ptr<int32_t>(),
                                         dOut.data_ptr(), gate.data_ptr(), value.data_ptr(), E, A,
                                         K, N, dgate.data_ptr(), dvalue.data_ptr(), nullptr, 0,
                                         stream_of(W)),
               "bwd_grouped_gemm_dX_swiglu");
  return {dgate, dvalue};
}

// bwd_grouped_gemm_dX2(W1, W2, expert_offset, dOut1, dOut2) -> dX [A, K] =
// dOut1 @ W1^T + dOut2 @ W2^T per expert, one reduction, one rounding.
Tensor bwd_grouped_gemm_dX2(Tensor W1, Tensor W2, Tensor offsets, Tensor dOut1, Tensor dOut2) {
  check_gemm_inputs(dOut1, offsets, W1);
  check_gemm_inputs(dOut2, offsets, W2);
  TORCH_CHECK(W1.dim() == 3 && W2.sizes() == W1.sizes() && dOut1.dim() == 2 &&
                  dOut1.size(1) == W1.size(2) && dOut2.sizes() == dOut1.sizes(),
              "expected W1, W2 [E,K,N] and dOut1, dOut2 [A,N]");
  TORCH_CHECK(offsets.numel() == W1.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  const int64_t A = dOut1.size(0), K = W1.size(1), N = W1.size(2);
  const int32_t E = (int32_t)W1.size(0);
  c10::hip::HIPGuard guard(W1.get_device());
  Tensor dX = at::empty({A, K}, W1.options());
  check_status(nt_grouped_gemm_dx2(dtype_code(W1), W1.data_ptr(), W2.data_ptr(),
                                   offsets.data_ptr<int32_t>(), dOut1.data_ptr(), dOut2.data_ptr(),
                                   E, A, K, N, dX.data_ptr(), nullptr, 0, stream_of(W1)),
               "bwd_grouped_gemm_dX2");
  return dX;
}

// ------------------------------------------------------- layer extensions

// Fused router gate: (gates [T,k] f32, topk [T,k] i32).
std::tuple<Tensor, Tensor> route_topk(Tensor logits, int64_t k) {
  TORCH_CHECK(logits.is_contiguous() && logits.dim() == 2, "logits must be a contiguous [T,E]");
  check_f32(logits, "logits");
  const int64_t T = logits.size(0), E = logits.size(1);
  TORCH_CHECK(k >= 1 && k <= E && k <= 32, "top_k must be in [1, min(E, 32)]");
  c10::hip::HIPGuard guard(logits.get_device());
  Tensor gates = at::empty({T, k}, logits.options());
  Tensor topk = at::empty({T, k}, logits.options().dtype(at::kInt));
  check_status(nt_route_topk(logits.data_ptr<float>(), T, (int32_t)E, (int32_t)k,
                             gates.data_ptr<float>(), topk.data_ptr<int32_t>(), nullptr,
                             stream_of(logits)),
               "route_topk");
  return {gates, topk};
}

// Router gate fused with the expert count: (gates, topk, dispatch workspace)
// where the workspace already holds the per-block expert counts that
// dispatch_tokens_counted(X, ...) starts from. X only fixes the dispatch's
// block size (its row bytes) and device.
std::tuple<Tensor, Tensor, Tensor> route_topk_count(Tensor logits, int64_t k, Tensor X) {
  TORCH_CHECK(logits.is_contiguous() && logits.dim() == 2, "logits must be a contiguous [T,E]");
  check_f32(logits, "logits");
  check_device(X, "X");
  const int64_t T = logits.size(0), E = logits.size(1);
  TORCH_CHECK(X.dim() == 2 && X.size(0) == T, "X must be [T,d] with the logits' T");
  TORCH_CHECK(k >= 1 && k <= E && k <= 32, "top_k must be in [1, min(E, 32)]");
  const int dt = dtype_code(X);
  c10::hip::HIPGuard guard(logits.get_device());
  Tensor gates = at::empty({T, k}, logits.options());
  Tensor topk = at::empty({T, k}, logits.options().dtype(at::kInt));
  Tensor ws = workspace(X, nt_dispatch_workspace_bytes(T, (int32_t)k, (int32_t)E, X.size(1), dt));
  const int32_t TB = nt_dispatch_block_tokens(T, (int32_t)k, X.size(1), dt);
  check_status(nt_route_topk_count(logits.data_ptr<float>(), T, (int32_t)E, (int32_t)k,
                                   gates.data_ptr<float>(), topk.data_ptr<int32_t>(), nullptr, TB,
                                   static_cast<int32_t*>(ws.data_ptr()), stream_of(logits)),
               "route_topk_count");
  return {gates, topk, ws};
}

Tensor route_topk_backward(Tensor gates, Tensor topk, Tensor dgates, int64_t num_experts) {
  TORCH_CHECK(gates.is_contiguous() && topk.is_contiguous() && dgates.is_contiguous(),
              "inputs must be contiguous");
  check_f32(gates, "gates");
  check_f32(dgates, "dgates");
  check_i32(topk, "topk");
  TORCH_CHECK(gates.sizes() == topk.sizes() && gates.sizes() == dgates.sizes() &&
                  gates.dim() == 2,
              "gates, topk and dgates must all be [T,k]");
  const int64_t T = gates.size(0), k = gates.size(1);
  c10::hip::HIPGuard guard(gates.get_device());
  Tensor dlogits = at::empty({T, num_experts}, gates.options());
  check_status(nt_route_topk_backward(gates.data_ptr<float>(), topk.data_ptr<int32_t>(),
                                      dgates.data_ptr<float>(), T, (int32_t)num_experts,
                                      (int32_t)k, dlogits.data_ptr<float>(), stream_of(gates)),
               "route_topk_backward");
  return dlogits;
}

// Fused count + scan + pack: (counts [E], offsets [E+1], packed_X, token_id,
// expert, packed_w, inv [T,k]).
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_impl(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts, c10::optional<Tensor> counted_ws) {
  TORCH_CHECK(X.is_contiguous() && w.is_contiguous() && topk.is_contiguous(),
              "inputs must be contiguous");
  check_device(X, "X");
  check_f32(w, "topk_weights");
  check_i32(topk, "topk_experts");
  TORCH_CHECK(X.dim() == 2 && w.dim() == 2 && topk.sizes() == w.sizes() && w.size(0) == X.size(0),
              "expected X [T,d], topk_weights [T,k], topk_experts [T,k]");
  const int64_t T = X.size(0), d = X.size(1), k = w.size(1), A = T * k;
  const int32_t E = (int32_t)num_experts;
  const int dt = dtype_code(X);
  c10::hip::HIPGuard guard(X.get_device());
  auto i32 = X.options().dtype(at::kInt);
  Tensor counts = at::empty({E}, i32);
  Tensor offsets = at::empty({E + 1}, i32);
  Tensor packed_X = at::empty({A, d}, X.options());
  Tensor token_id = at::empty({A}, i32);
  Tensor expert = at::empty({A}, i32);
  Tensor packed_w = at::empty({A}, X.options().dtype(at::kFloat));
  Tensor inv = at::empty({T, k}, i32);
  const size_t ws_need = nt_dispatch_workspace_bytes(T, (int32_t)k, E, d, dt);
  Tensor ws;
  if (counted_ws.has_value()) {
    ws = *counted_ws;
    check_device(ws, "dispatch workspace");
    TORCH_CHECK(ws.is_contiguous() && (size_t)ws.numel() * ws.element_size() >= ws_need,
                "dispatch workspace from route_topk_count is too small for these sizes");
  } else {
    ws = workspace(X, ws_need);
  }
  auto fn = counted_ws.has_value() ? nt_dispatch_counted : nt_dispatch;
  check_status(fn(dt, X.data_ptr(), w.data_ptr<float>(), topk.data_ptr<int32_t>(), T, (int32_t)k,
                  d, E, counts.data_ptr<int32_t>(), offsets.data_ptr<int32_t>(),
                  packed_X.data_ptr(), token_id.data_ptr<int32_t>(), expert.data_ptr<int32_t>(),
                  packed_w.data_ptr<float>(), inv.data_ptr<int32_t>(), ws.data_ptr(),
                  (size_t)ws.numel() * ws.element_size(), stream_of(X)),
               "dispatch_tokens");
  return {counts, offsets, packed_X, token_id, expert, packed_w, inv};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_tokens(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts) {
  return dispatch_impl(X, w, topk, num_experts, c10::nullopt);
}

// dispatch_tokens starting from the per-block counts route_topk_count left
// in `ws` (no counting pass). The counts stay as they are (a second call on
// the same ws gives the same outputs); the rest of ws is overwritten scratch.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_tokens_counted(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts, Tensor ws) {
  return dispatch_impl(X, w, topk, num_experts, ws);
}

// pack_tokens_kernel plus the inverse map.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> pack_tokens_inv(Tensor X, Tensor w, Tensor topk,
                                                                   Tensor cursor) {
  return pack_impl(X, w, topk, cursor);
}

Tensor combine_inv(Tensor y, Tensor inv, Tensor w, c10::ScalarType out_dtype) {
  TORCH_CHECK(y.is_contiguous() && inv.is_contiguous() && w.is_contiguous(),
              "inputs must be contiguous");
  check_device(y, "expert_outputs");
  check_i32(inv, "inv");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && inv.dim() == 2, "expected y [A,d], inv [T,k]");
  // The kernels read rows p < T*k of y and w (and skip larger entries of inv).
  TORCH_CHECK(y.size(0) == inv.numel() && w.numel() == inv.numel(),
              "expert_outputs and packed_topk_weights must have T*k = inv.numel() rows");
  check_same_device(y, {&inv, &w});
  const int64_t T = inv.size(0), k = inv.size(1), d = y.size(1);
  c10::hip::HIPGuard guard(y.get_device());
  Tensor out = at::empty({T, d}, y.options().dtype(out_dtype));
  Tensor probe = at::empty({0}, y.options().dtype(out_dtype));
  check_status(nt_combine_inv(dtype_code(y), y.data_ptr(), inv.data_ptr<int32_t>(),
                              w.data_ptr<float>(), T, (int32_t)k, d, dtype_code(probe),
                              out.data_ptr(), stream_of(y)),
               "combine_inv");
  return out;
}

std::tuple<Tensor, Tensor> combine_backward_inv(Tensor y, Tensor inv, Tensor w, Tensor dY) {
  TORCH_CHECK(y.is_contiguous() && inv.is_contiguous() && w.is_contiguous() && dY.is_contiguous(),
              "inputs must be contiguous");
  check_device(y, "expert_outputs");
  check_device(dY, "grad");
  check_i32(inv, "inv");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && inv.dim() == 2 && dY.dim() == 2 && dY.size(0) == inv.size(0) &&
                  dY.size(1) == y.size(1),
              "expected y [A,d], inv [T,k], grad [T,d]");
  TORCH_CHECK(dY.scalar_type() == at::kFloat || dY.scalar_type() == y.scalar_type(),
              "grad must be float32 or the activation dtype");
  // The kernel reads and writes rows p < T*k of y, dy, w and dw.
  TORCH_CHECK(y.size(0) == inv.numel() && w.numel() == inv.numel(),
              "expert_outputs and packed_topk_weights must have T*k = inv.numel() rows");
  check_same_device(y, {&inv, &w, &dY});
  const int64_t T = inv.size(0), k = inv.size(1), d = y.size(1);
  c10::hip::HIPGuard guard(y.get_device());
  Tensor dy = at::empty_like(y);
  Tensor dw = at::empty(w.sizes(), w.options());
  check_status(nt_combine_backward_inv(dtype_code(y), y.data_ptr(), inv.data_ptr<int32_t>(),
                                       w.data_ptr<float>(), dtype_code(dY), dY.data_ptr(), T,
                                       (int32_t)k, d, dy.data_ptr(), dw.data_ptr<float>(),
                                       stream_of(y)),
               "combine_backward_inv");
  return {dy, dw};
}

std::tuple<Tensor, Tensor> pack_backward_inv(Tensor dpX, Tensor dpw, Tensor inv) {
  TORCH_CHECK(dpX.is_contiguous() && dpw.is_contiguous() && inv.is_contiguous(),
              "inputs must be contiguous");
  check_device(dpX, "packed_X_grad");
  check_f32(dpw, "packed_topk_weights_grad");
  check_i32(inv, "inv");
  TORCH_CHECK(dpX.dim() == 2 && inv.dim() == 2, "expected packed_X_grad [A,d], inv [T,k]");
  // The kernel reads rows p < T*k of dpX and dpw.
  TORCH_CHECK(dpX.size(0) == inv.numel() && dpw.numel() == inv.numel(),
              "packed_X_grad and packed_topk_weights_grad must have T*k = inv.numel() rows");
  check_same_device(dpX, {&dpw, &inv});
  const int64_t T = inv.size(0), k = inv.size(1), d = dpX.size(1);
  c10::hip::HIPGuard guard(dpX.get_device());
  Tensor dX = at::empty({T, d}, dpX.options());
  Tensor dw = at::empty({T, k}, dpw.options());
  check_status(nt_pack_backward_inv(dtype_code(dpX), dpX.data_ptr(), dpw.data_ptr<float>(),
                                    inv.data_ptr<int32_t>(), T, (int32_t)k, d, dX.data_ptr(),
                                    dw.data_ptr<float>(), stream_of(dpX)),
               "pack_backward_inv");
  return {dX, dw};
}

// pack_backward_inv whose dw feeds route_topk_backward, fused: (dX [T,d],
// dlogits [T,E]).
std::tuple<Tensor, Tensor> pack_backward_inv_route(Tensor dpX, Tensor dpw, Tensor inv, Tensor gates,
                                                   Tensor topk, int64_t num_experts) {
  TORCH_CHECK(dpX.is_contiguous() && dpw.is_contiguous() && inv.is_contiguous() &&
                  gates.is_contiguous() && topk.is_contiguous(),
              "inputs must be contiguous");
  check_device(dpX, "packed_X_grad");
  check_f32(dpw, "packed_topk_weights_grad");
  check_i32(inv, "inv");
  check_f32(gates, "gates");
  check_i32(topk, "topk");
  TORCH_CHECK(dpX.dim() == 2 && inv.dim() == 2, "expected packed_X_grad [A,d], inv [T,k]");
  TORCH_CHECK(dpX.size(0) == inv.numel() && dpw.numel() == inv.numel(),
              "packed_X_grad and packed_topk_weights_grad must have T*k = inv.numel() rows");
  TORCH_CHECK(gates.sizes() == inv.sizes() && topk.sizes() == inv.sizes(),
              "gates and topk must be [T,k] like inv");
  TORCH_CHECK(num_experts >= 1 && num_experts <= NT_MAX_EXPERTS, "num_experts out of range");
  check_same_device(dpX, {&dpw, &inv, &gates, &topk});
  const int64_t T = inv.size(0), k = inv.size(1), d = dpX.size(1);
  c10::hip::HIPGuard guard(dpX.get_device());
  Tensor dX = at::empty({T, d}, dpX.options());
  Tensor dlogits = at::empty({T, num_experts}, gates.options());
  // The fused kernel takes k <= 8; above, the two launches need dw.
  Tensor dw = k > 8 ? at::empty({T, k}, dpw.options()) : Tensor();
  check_status(nt_pack_backward_inv_route(
                   dtype_code(dpX), dpX.data_ptr(), dpw.data_ptr<float>(),
                   inv.data_ptr<int32_t>(), gates.data_ptr<float>(), topk.data_ptr<int32_t>(), T,
                   (int32_t)k, d, (int32_t)num_experts, dX.data_ptr(), dlogits.data_ptr<float>(),
                   k > 8 ? dw.data_ptr<float>() : nullptr, stream_of(dpX)),
               "pack_backward_inv_route");
  return {dX, dlogits};
}

// stream_copy(dst, src, blocks=0): the library's 16-byte streaming copy of
// src's bytes into dst (the achievable-bandwidth reference of the benchmark).
void stream_copy(Tensor dst, Tensor src, int64_t blocks) {
  check_device(dst, "dst");
  check_device(src, "src");
  TORCH_CHECK(dst.is_contiguous() && src.is_contiguous(), "tensors must be contiguous");
  const size_t bytes = (size_t)src.numel() * src.element_size();
  TORCH_CHECK((size_t)dst.numel() * dst.element_size() >= bytes, "dst is smaller than src");
  check_same_device(dst, {&src});
  c10::hip::HIPGuard guard(src.get_device());
  check_status(nt_stream_copy(dst.data_ptr(), src.data_ptr(), bytes, (int32_t)blocks,
                              stream_of(src)),
               "stream_copy");
}

// stream_fill(dst, value) / stream_read(src, sink): the write-only and
// read-only bandwidth references (sink: one int32 on src's device).
void stream_fill(Tensor dst, int64_t value) {
  check_device(dst, "dst");
  TORCH_CHECK(dst.is_contiguous(), "dst must be contiguous");
  c10::hip::HIPGuard guard(dst.get_device());
  check_status(nt_stream_fill(dst.data_ptr(), (size_t)dst.numel() * dst.element_size(),
                              (uint32_t)value, stream_of(dst)),
               "stream_fill");
}
void stream_read(Tensor src, Tensor sink) {
  check_device(src, "src");
  check_device(sink, "sink");
  TORCH_CHECK(src.is_contiguous() && sink.numel() >= 1 && sink.element_size() == 4,
              "src must be contiguous and sink one 32-bit word");
  check_same_device(src, {&sink});
  c10::hip::HIPGuard guard(src.get_device());
  check_status(nt_stream_read(src.data_ptr(), (size_t)src.numel() * src.element_size(),
                              static_cast<uint32_t*>(sink.data_ptr()), stream_of(src)),
               "stream_read");
}

// ------------------------------------------------------------ Meta kernels
//
// Output shapes and dtypes only (fake / meta tensors, torch.compile tracing):
// every output's shape follows from the input shapes, none from their values.
namespace meta {

Tensor count_expert_kernel(Tensor topk, Tensor mask, int64_t num_experts, int64_t num_topk) {
  return at::empty({num_experts}, topk.options().dtype(at::kInt));
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> pack_tokens_inv(Tensor X, Tensor w, Tensor topk,
                                                                   Tensor cursor) {
  const int64_t T = X.size(0), d = X.size(1), k = w.size(1), A = T * k;
  auto i32 = X.options().dtype(at::kInt);
  return {at::empty({A, d}, X.options()), at::empty({A}, i32), at::empty({A}, i32),
          at::empty({A}, X.options().dtype(at::kFloat)), at::empty({T, k}, i32)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> pack_tokens_kernel(Tensor X, Tensor w, Tensor topk,
                                                              Tensor cursor) {
  auto r = pack_tokens_inv(X, w, topk, cursor);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r)};
}

Tensor combine_tokens_kernel(Tensor y, Tensor token_id, Tensor w, int64_t num_tokens,
                             int64_t d_model) {
  return at::empty({num_tokens, d_model}, y.options().dtype(at::kFloat));
}

std::tuple<Tensor, Tensor> combine_kernel_backward(Tensor y, Tensor token_id, Tensor w, Tensor dY,
                                                   int64_t hidden_dim) {
  return {at::empty_like(y), at::empty(w.sizes(), w.options())};
}

std::tuple<Tensor, Tensor> pack_kernel_backward(Tensor dpX, Tensor dpw, Tensor token_id,
                                                Tensor expert, Tensor topk) {
  return {at::empty({topk.size(0), dpX.size(1)}, dpX.options()),
          at::empty({topk.size(0), topk.size(1)}, dpw.options())};
}

Tensor grouped_gemm_kernel(Tensor X, Tensor offsets, Tensor W) {
  return at::empty({X.size(0), W.size(2)}, X.options());
}

Tensor bwd_grouped_gemm_dW_kernel(Tensor X, Tensor offsets, Tensor dOut) {
  return at::empty({offsets.size(0) - 1, X.size(1), dOut.size(1)}, X.options());
}

Tensor bwd_grouped_gemm_dX_kernel(Tensor W, Tensor offsets, Tensor dOut) {
  return at::empty({dOut.size(0), W.size(1)}, W.options());
}

std::tuple<Tensor, Tensor> grouped_gemm_gelu(Tensor X, Tensor offsets, Tensor W) {
  return {grouped_gemm_kernel(X, offsets, W), grouped_gemm_kernel(X, offsets, W)};
}

Tensor bwd_grouped_gemm_dX_gelu(Tensor W, Tensor offsets, Tensor dOut, Tensor act_grad) {
  return bwd_grouped_gemm_dX_kernel(W, offsets, dOut);
}

std::tuple<Tensor, Tensor, Tensor> grouped_gemm_swiglu(Tensor X, Tensor offsets, Tensor Wg,
                                                       Tensor Wv) {
  return {grouped_gemm_kernel(X, offsets, Wg), grouped_gemm_kernel(X, offsets, Wg),
          grouped_gemm_kernel(X, offsets, Wg)};
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dX_swiglu(Tensor W, Tensor offsets, Tensor dOut,
                                                      Tensor gate, Tensor value) {
  return {bwd_grouped_gemm_dX_kernel(W, offsets, dOut), bwd_grouped_gemm_dX_kernel(W, offsets, dOut)};
}

Tensor bwd_grouped_gemm_dX2(Tensor W1, Tensor W2, Tensor offsets, Tensor dOut1, Tensor dOut2) {
  return bwd_grouped_gemm_dX_kernel(W1, offsets, dOut1);
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX(Tensor X, Tensor W, Tensor offsets, Tensor dOut) {
  return {at::empty_like(W), at::empty_like(X)};
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX_gelu(Tensor act, Tensor W, Tensor offsets,
                                                       Tensor dOut, Tensor act_grad) {
  return {at::empty_like(W), at::empty_like(act)};
}

std::tuple<Tensor, Tensor, Tensor> bwd_grouped_gemm_dW_dX_swiglu(Tensor hidden, Tensor W,
                                                                 Tensor offsets, Tensor dOut,
                                                                 Tensor gate, Tensor value) {
  return {at::empty_like(W), at::empty_like(hidden), at::empty_like(hidden)};
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX2(Tensor X, Tensor W1, Tensor W2, Tensor offsets,
                                                   Tensor dOut1, Tensor dOut2) {
  return {at::empty_like(W1), at::empty_like(X)};
}

std::tuple<Tensor, Tensor> route_topk(Tensor logits, int64_t k) {
  return {at::empty({logits.size(0), k}, logits.options()),
          at::empty({logits.size(0), k}, logits.options().dtype(at::kInt))};
}

std::tuple<Tensor, Tensor, Tensor> route_topk_count(Tensor logits, int64_t k, Tensor X) {
  const int64_t T = logits.size(0), E = logits.size(1);
  const size_t bytes =
      nt_dispatch_workspace_bytes(T, (int32_t)k, (int32_t)E, X.size(1), dtype_code(X));
  return {at::empty({T, k}, logits.options()), at::empty({T, k}, logits.options().dtype(at::kInt)),
          at::empty({(int64_t)std::max<size_t>(bytes, 1)}, X.options().dtype(at::kByte))};
}

Tensor route_topk_backward(Tensor gates, Tensor topk, Tensor dgates, int64_t num_experts) {
  return at::empty({gates.size(0), num_experts}, gates.options());
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_tokens(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts) {
  const int64_t T = X.size(0), d = X.size(1), k = w.size(1), A = T * k;
  auto i32 = X.options().dtype(at::kInt);
  return {at::empty({num_experts}, i32),       at::empty({num_experts + 1}, i32),
          at::empty({A, d}, X.options()),      at::empty({A}, i32),
          at::empty({A}, i32),                 at::empty({A}, X.options().dtype(at::kFloat)),
          at::empty({T, k}, i32)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_tokens_counted(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts, Tensor ws) {
  return dispatch_tokens(X, w, topk, num_experts);
}

Tensor combine_inv(Tensor y, Tensor inv, Tensor w, c10::ScalarType out_dtype) {
  return at::empty({inv.size(0), y.size(1)}, y.options().dtype(out_dtype));
}

std::tuple<Tensor, Tensor> combine_backward_inv(Tensor y, Tensor inv, Tensor w, Tensor dY) {
  return {at::empty_like(y), at::empty(w.sizes(), w.options())};
}

std::tuple<Tensor, Tensor> pack_backward_inv(Tensor dpX, Tensor dpw, Tensor inv) {
  return {at::empty({inv.size(0), dpX.size(1)}, dpX.options()),
          at::empty({inv.size(0), inv.size(1)}, dpw.options())};
}

std::tuple<Tensor, Tensor> pack_backward_inv_route(Tensor dpX, Tensor dpw, Tensor inv, Tensor gates,
                                                   Tensor topk, int64_t num_experts) {
  return {at::empty({inv.size(0), dpX.size(1)}, dpX.options()),
          at::empty({inv.size(0), num_experts}, gates.options())};
}

}  // namespace meta

}  // namespace

// The op library: torch.ops.nanotitan.<op>. The eight reference ops keep the
// names and argument orders of csrc/bindings.cpp:59-92 (pack_tokens_kernel
// mutates its cursor argument, like the reference's atomic cursor); the
// others are the layer's fused ops. Implementations: the HIP kernels for GPU
// tensors (CUDA dispatch key, which ROCm builds of torch use for HIP
// devices), plain C++ for CPU tensors (cpu_ops.cpp), shapes only for Meta.
TORCH_LIBRARY(nanotitan, m) {
  m.def("count_expert_kernel(Tensor topk_experts_per_token, Tensor mask, int num_experts, "
        "int num_topk_experts) -> Tensor");
  m.def("pack_tokens_kernel(Tensor X, Tensor topk_weights, Tensor topk_experts, "
        "Tensor(a!) expert_offset_cpy) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("combine_tokens_kernel(Tensor expert_outputs, Tensor packed_tokenId, "
        "Tensor packed_topk_weights, int num_tokens, int d_model) -> Tensor");
  m.def("combine_kernel_backward(Tensor expert_outputs, Tensor packed_tokenIds, "
        "Tensor packed_topk_weights, Tensor residual_stream_grad, int hidden_dim) "
        "-> (Tensor, Tensor)");
  m.def("pack_kernel_backward(Tensor packed_X_grad, Tensor packed_topk_weights_grad, "
        "Tensor packed_tokenId, Tensor packed_expert, Tensor topk_experts) -> (Tensor, Tensor)");
  m.def("grouped_gemm_kernel(Tensor X, Tensor expert_offset, Tensor weights) -> Tensor");
  m.def("bwd_grouped_gemm_dW_kernel(Tensor X, Tensor expert_offset, Tensor dOut) -> Tensor");
  m.def("bwd_grouped_gemm_dX_kernel(Tensor W_gate, Tensor expert_offset, Tensor dOut) -> Tensor");
  m.def("grouped_gemm_gelu(Tensor X, Tensor expert_offset, Tensor W) -> (Tensor, Tensor)");
  m.def("bwd_grouped_gemm_dX_gelu(Tensor W, Tensor expert_offset, Tensor dOut, Tensor act_grad) "
        "-> Tensor");
  m.def("grouped_gemm_swiglu(Tensor X, Tensor expert_offset, Tensor W_gate, Tensor W_val) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("bwd_grouped_gemm_dX_swiglu(Tensor W, Tensor expert_offset, Tensor dOut, Tensor gate, "
        "Tensor value) -> (Tensor, Tensor)");
  m.def("bwd_grouped_gemm_dX2(Tensor W1, Tensor W2, Tensor expert_offset, Tensor dOut1, "
        "Tensor dOut2) -> Tensor");
  m.def("bwd_grouped_gemm_dW_dX(Tensor X, Tensor W, Tensor expert_offset, Tensor dOut) "
        "-> (Tensor, Tensor)");
  m.def("bwd_grouped_gemm_dW_dX_gelu(Tensor act, Tensor W, Tensor expert_offset, Tensor dOut, "
        "Tensor act_grad) -> (Tensor, Tensor)");
  m.def("bwd_grouped_gemm_dW_dX_swiglu(Tensor hidden, Tensor W, Tensor expert_offset, "
        "Tensor dOut, Tensor gate, Tensor value) -> (Tensor, Tensor, Tensor)");
  m.def("bwd_grouped_gemm_dW_dX2(Tensor X, Tensor W1, Tensor W2, Tensor expert_offset, "
        "Tensor dOut1, Tensor dOut2) -> (Tensor, Tensor)");
  m.def("route_topk(Tensor logits, int top_k) -> (Tensor, Tensor)");
  m.def("route_topk_count(Tensor logits, int top_k, Tensor X) -> (Tensor, Tensor, Tensor)");
  m.def("route_topk_backward(Tensor gates, Tensor topk, Tensor dgates, int num_experts) -> Tensor");
  m.def("dispatch_tokens(Tensor X, Tensor topk_weights, Tensor topk_experts, int num_experts) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  // ws: the per-block counts at its start are only read; the rest is scratch
  // the HIP kernel overwrites (so the schema marks it mutable).
  m.def("dispatch_tokens_counted(Tensor X, Tensor topk_weights, Tensor topk_experts, "
        "int num_experts, Tensor(a!) ws) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
        "Tensor)");
  m.def("pack_tokens_inv(Tensor X, Tensor topk_weights, Tensor topk_experts, "
        "Tensor(a!) expert_offset_cpy) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("combine_inv(Tensor expert_outputs, Tensor inv, Tensor packed_topk_weights, "
        "ScalarType out_dtype) -> Tensor");
  m.def("combine_backward_inv(Tensor expert_outputs, Tensor inv, Tensor packed_topk_weights, "
        "Tensor grad) -> (Tensor, Tensor)");
  m.def("pack_backward_inv(Tensor packed_X_grad, Tensor packed_topk_weights_grad, Tensor inv) "
        "-> (Tensor, Tensor)");
  m.def("pack_backward_inv_route(Tensor packed_X_grad, Tensor packed_topk_weights_grad, "
        "Tensor inv, Tensor gates, Tensor topk, int num_experts) -> (Tensor, Tensor)");
}

#define NT_IMPL_ALL(m, NS)                                                  \
  m.impl("count_expert_kernel", &NS count_expert_kernel);                   \
  m.impl("pack_tokens_kernel", &NS pack_tokens_kernel);                     \
  m.impl("combine_tokens_kernel", &NS combine_tokens_kernel);               \
  m.impl("combine_kernel_backward", &NS combine_kernel_backward);           \
  m.impl("pack_kernel_backward", &NS pack_kernel_backward);                 \
  m.impl("grouped_gemm_kernel", &NS grouped_gemm_kernel);                   \
  m.impl("bwd_grouped_gemm_dW_kernel", &NS bwd_grouped_gemm_dW_kernel);     \
  m.impl("bwd_grouped_gemm_dX_kernel", &NS bwd_grouped_gemm_dX_kernel);     \
  m.impl("grouped_gemm_gelu", &NS grouped_gemm_gelu);                       \
  m.impl("bwd_grouped_gemm_dX_gelu", &NS bwd_grouped_gemm_dX_gelu);         \
  m.impl("grouped_gemm_swiglu", &NS grouped_gemm_swiglu);                   \
  m.impl("bwd_grouped_gemm_dX_swiglu", &NS bwd_grouped_gemm_dX_swiglu);     \
  m.impl("bwd_grouped_gemm_dX2", &NS bwd_grouped_gemm_dX2);                 \
  m.impl("bwd_grouped_gemm_dW_dX", &NS bwd_grouped_gemm_dW_dX);             \
  m.impl("bwd_grouped_gemm_dW_dX_gelu", &NS bwd_grouped_gemm_dW_dX_gelu);   \
  m.impl("bwd_grouped_gemm_dW_dX_swiglu", &NS bwd_grouped_gemm_dW_dX_swiglu); \
  m.impl("bwd_grouped_gemm_dW_dX2", &NS bwd_grouped_gemm_dW_dX2);           \
  m.impl("route_topk", &NS route_topk);                                     \
  m.impl("route_topk_count", &NS route_topk_count);                         \
  m.impl("route_topk_backward", &NS route_topk_backward);                   \
  m.impl("dispatch_tokens", &NS dispatch_tokens);                           \
  m.impl("dispatch_tokens_counted", &NS dispatch_tokens_counted);           \
  m.impl("pack_tokens_inv", &NS pack_tokens_inv);                           \
  m.impl("combine_inv", &NS combine_inv);                                   \
  m.impl("combine_backward_inv", &NS combine_backward_inv);                 \
  m.impl("pack_backward_inv", &NS pack_backward_inv);                       \
  m.impl("pack_backward_inv_route", &NS pack_backward_inv_route)

TORCH_LIBRARY_IMPL(nanotitan, CUDA, m) { NT_IMPL_ALL(m, ); }

TORCH_LIBRARY_IMPL(nanotitan, Meta, m) { NT_IMPL_ALL(m, meta::); }

#undef NT_IMPL_ALL

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "nanoTitan MoE expert path on MI355X (gfx950): HIP kernels behind the reference op surface";
  m.def("count_expert_kernel", &count_expert_kernel,
        "Histogram of expert ids over unmasked tokens -> int32 [E]");
  m.def("pack_tokens_kernel", &pack_tokens_kernel,
        "[num_tokens, d] -> [num_tokens * k, d] expert-major packing (canonical stable order)");
  m.def("combine_tokens_kernel", &combine_tokens_kernel,
        "Gate-weighted sum of packed rows per token -> float32 [T, d]");
  m.def("combine_kernel_backward", &combine_kernel_backward,
        "Backward of combine -> (expert_output_grad, packed_topk_weights_grad)");
  m.def("pack_kernel_backward", &pack_kernel_backward,
        "Backward of pack -> (X_grad, topk_weights_grad)");
  m.def("grouped_gemm_kernel", &grouped_gemm_kernel, "Expert-grouped GEMM forward");
  m.def("bwd_grouped_gemm_dW_kernel", &bwd_grouped_gemm_dW_kernel,
        "Expert-grouped GEMM weight gradient");
  m.def("bwd_grouped_gemm_dX_kernel", &bwd_grouped_gemm_dX_kernel,
        "Expert-grouped GEMM input gradient");
  m.def("grouped_gemm_gelu", &grouped_gemm_gelu,
        "Up-projection grouped GEMM with fused GELU -> (gelu(h), gelu'(h))");
  m.def("grouped_gemm_swiglu", &grouped_gemm_swiglu,
        "Gate and value grouped GEMMs with fused SwiGLU -> (hidden, gate, value)");
  m.def("bwd_grouped_gemm_dX_swiglu", &bwd_grouped_gemm_dX_swiglu,
        "dX grouped GEMM of the down projection with the SwiGLU backward -> (dgate, dvalue)");
  m.def("bwd_grouped_gemm_dX2", &bwd_grouped_gemm_dX2,
        "Sum of two dX grouped GEMMs over one concatenated reduction");
  m.def("bwd_grouped_gemm_dX_gelu", &bwd_grouped_gemm_dX_gelu,
        "dX grouped GEMM with fused GELU backward -> (dOut @ W^T) * act_grad");
  m.def("dispatch_tokens", &dispatch_tokens,
        "Fused count + offsets + pack -> (counts, offsets, packed_X, token_id, expert, packed_w, inv)");
  m.def("pack_tokens_inv", &pack_tokens_inv, "pack_tokens_kernel that also returns the inverse map");
  m.def("combine_inv", &combine_inv, "Combine driven by the inverse map");
  m.def("combine_backward_inv", &combine_backward_inv, "Combine backward driven by the inverse map");
  m.def("pack_backward_inv", &pack_backward_inv, "Pack backward driven by the inverse map");
  m.def("pack_backward_inv_route", &pack_backward_inv_route,
        "pack_backward_inv with the router's backward on its dw -> (X_grad, dlogits)");
  m.def("route_topk", &route_topk, "Fused softmax / top-k / renorm router gate -> (gates, topk)");
  m.def("bwd_grouped_gemm_dW_dX", &bwd_grouped_gemm_dW_dX,
        "dW and dX of one projection in one call (a dW with few tiles runs beside the dX)");
  m.def("bwd_grouped_gemm_dW_dX_gelu", &bwd_grouped_gemm_dW_dX_gelu,
        "dW of the down projection and the GELU-backward dX in one call");
  m.def("bwd_grouped_gemm_dW_dX_swiglu", &bwd_grouped_gemm_dW_dX_swiglu,
        "dW of the SwiGLU output projection and the SwiGLU-backward dX in one call");
  m.def("bwd_grouped_gemm_dW_dX2", &bwd_grouped_gemm_dW_dX2,
        "dW of the gate projection and the two-part dX in one call");
  m.def("route_topk_count", &route_topk_count,
        "Router gate fused with the per-block expert count -> (gates, topk, dispatch workspace)");
  m.def("dispatch_tokens_counted", &dispatch_tokens_counted,
        "dispatch_tokens from the counts route_topk_count computed");
  m.def("route_topk_backward", &route_topk_backward, "Gradient of route_topk's gates -> dlogits");
  m.def("stream_fill", &stream_fill, "16-byte streaming device fill (write bandwidth reference)",
        pybind11::arg("dst"), pybind11::arg("value") = 0);
  m.def("stream_read", &stream_read, "16-byte streaming device read (read bandwidth reference)",
        pybind11::arg("src"), pybind11::arg("sink"));
  m.def("stream_copy", &stream_copy, "16-byte streaming device copy (bandwidth reference)",
        pybind11::arg("dst"), pybind11::arg("src"), pybind11::arg("blocks") = 0);
  m.def("version", []() { return nt_version(); });
}
