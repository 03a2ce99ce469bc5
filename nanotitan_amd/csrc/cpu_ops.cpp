// CPU kernels of the nanotitan op library (torch.ops.nanotitan.*, CPU dispatch key).
//
// The same ops as the HIP kernels, for tensors that live in host memory, so
// the op surface can run (and be tested) on a machine without a GPU. A GPU
// tensor never reaches this file: the dispatcher sends it to the HIP
// implementation, and a call with tensors on both sides is rejected.
//
// Results follow the GPU kernels' definitions:
//  * counts, offsets, packed order (stable counting sort of the flat
//    assignment index by expert), inverse map, packed rows and gates, and
//    the cursor post-state are bit-identical;
//  * the ordered fp32 sums (combine forward: products rounded, then added in
//    ascending packed order; pack backward's dX and gate gradients) are
//    bit-identical; this file is compiled with -ffp-contract=off;
//  * dot products (combine backward's gate gradient), GEMMs, softmax and the
//    GELU / SwiGLU activations are computed in fp32 (fp64 for float64) or
//    better and rounded at the same points as the GPU, so they agree within
//    the tolerances the GPU tests use.
// Reference interfaces: csrc/bindings.cpp:9-57 (op names and argument
// orders), src/model/cuda_backend.py:30-67 (router and dispatch glue).
#include <torch/extension.h>

#include <ATen/Parallel.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <tuple>
#include <vector>

#include "nanotitan_moe.h"

namespace nt_cpu {
namespace {

using torch::Tensor;

void check_cpu(const Tensor& t, const char* name) {
  TORCH_CHECK(t.device().is_cpu(), name, " must be a CPU tensor (all arguments on one device)");
}
void check_i32(const Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kInt, name, " must be int32");
  check_cpu(t, name);
}
void check_f32(const Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kFloat, name, " must be float32");
  check_cpu(t, name);
}
void check_float_type(const Tensor& t, const char* name) {
  const auto s = t.scalar_type();
  TORCH_CHECK(s == at::kFloat || s == at::kDouble || s == at::kHalf || s == at::kBFloat16,
              "unsupported dtype ", s, " for ", name,
              " (expected float32, float64, float16 or bfloat16)");
  check_cpu(t, name);
}

// Element <-> float conversions with the GPU's rounding (nearest even).
template <typename S>
inline float to_f(S v) {
  return static_cast<float>(v);
}
template <typename S>
inline S from_f(float v) {
  return static_cast<S>(v);
}

// Row range of expert e clamped to [0, A] and non-decreasing (the GPU
// scheduler's rule for a malformed offsets array).
inline void expert_rows(const int32_t* off, int e, int64_t A, int64_t& a, int64_t& b) {
  a = std::min<int64_t>(std::max<int64_t>(off[e], 0), A);
  b = std::min<int64_t>(std::max<int64_t>(off[e + 1], a), A);
}

// ----------------------------------------------------------- dispatch

Tensor count_expert_kernel(Tensor topk, Tensor mask, int64_t num_experts, int64_t num_topk) {
  check_i32(topk, "topk_experts_per_token");
  check_i32(mask, "mask");
  TORCH_CHECK(topk.is_contiguous() && mask.is_contiguous(), "inputs must be contiguous");
  TORCH_CHECK(topk.dim() == 2 && topk.size(1) == num_topk,
              "topk_experts_per_token must be [num_tokens, num_topk_experts]");
  TORCH_CHECK(mask.numel() == topk.size(0), "mask must have one entry per token");
  TORCH_CHECK(num_experts >= 1 && num_experts <= NT_MAX_EXPERTS,
              "num_experts must be in [1, ", NT_MAX_EXPERTS, "]");
  const int64_t T = topk.size(0), k = num_topk;
  Tensor counts = at::zeros({num_experts}, topk.options());
  int32_t* c = counts.data_ptr<int32_t>();
  const int32_t* tk = topk.data_ptr<int32_t>();
  const int32_t* m = mask.data_ptr<int32_t>();
  for (int64_t t = 0; t < T; ++t) {
    if (m[t] == 0) continue;
    for (int64_t j = 0; j < k; ++j) {
      const int32_t e = tk[t * k + j];
      if (e >= 0 && e < num_experts) ++c[e];
    }
  }
  return counts;
}

// Canonical pack from a per-expert base (cursor): slot(f) = base[e] + rank
// of f among the earlier assignments of expert e. Slots outside [0, A) are
// dropped (inv = -1). Returns the per-expert counts of valid ids.
std::vector<int64_t> pack_rows(const Tensor& X, const Tensor& w, const Tensor& topk,
                               const std::vector<int64_t>& base, Tensor& packed_X,
                               Tensor& token_id, Tensor& expert, Tensor& packed_w, Tensor& inv) {
  const int64_t T = X.size(0), d = X.size(1), k = topk.size(1), A = T * k;
  const int64_t E = (int64_t)base.size();
  const int64_t rb = d * X.element_size();
  const int32_t* tk = topk.data_ptr<int32_t>();
  const float* wp = w.data_ptr<float>();
  int32_t* iv = inv.data_ptr<int32_t>();
  std::vector<int64_t> slot(A, -1), run(E, 0);
  for (int64_t f = 0; f < A; ++f) {
    const int32_t e = tk[f];
    if (e < 0 || e >= E) continue;
    const int64_t p = base[e] + run[e]++;
    if (p >= 0 && p < A) slot[f] = p;
  }
  int32_t* tid = token_id.data_ptr<int32_t>();
  int32_t* ex = expert.data_ptr<int32_t>();
  float* pw = packed_w.data_ptr<float>();
  const char* src = static_cast<const char*>(X.data_ptr());
  char* dst = static_cast<char*>(packed_X.data_ptr());
  at::parallel_for(0, T, 256, [&](int64_t t0, int64_t t1) {
    for (int64_t t = t0; t < t1; ++t)
      for (int64_t j = 0; j < k; ++j) {
        const int64_t f = t * k + j, p = slot[f];
        iv[f] = (int32_t)p;
        if (p < 0) continue;
        tid[p] = (int32_t)t;
        ex[p] = tk[f];
        pw[p] = wp[f];
        if (rb > 0) std::memcpy(dst + p * rb, src + t * rb, (size_t)rb);
      }
  });
  return run;
}

void check_pack_inputs(const Tensor& X, const Tensor& w, const Tensor& topk) {
  TORCH_CHECK(X.is_contiguous() && w.is_contiguous() && topk.is_contiguous(),
              "inputs must be contiguous");
  check_float_type(X, "X");
  check_f32(w, "topk_weights");
  check_i32(topk, "topk_experts");
  TORCH_CHECK(X.dim() == 2 && w.dim() == 2 && topk.sizes() == w.sizes() && w.size(0) == X.size(0),
              "expected X [T,d], topk_weights [T,k], topk_experts [T,k]");
  TORCH_CHECK(w.size(1) >= 1, "top-k must be at least 1");
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> pack_impl(Tensor X, Tensor w, Tensor topk,
                                                             Tensor cursor) {
  check_pack_inputs(X, w, topk);
  check_i32(cursor, "expert_offset_cpy");
  TORCH_CHECK(cursor.is_contiguous() && cursor.numel() >= 2,
              "expert_offset_cpy must hold num_experts + 1 entries");
  const int64_t T = X.size(0), d = X.size(1), k = w.size(1), A = T * k;
  const int64_t E = cursor.numel() - 1;
  TORCH_CHECK(E <= NT_MAX_EXPERTS, "number of experts exceeds ", NT_MAX_EXPERTS);
  auto i32 = X.options().dtype(at::kInt);
  Tensor packed_X = at::empty({A, d}, X.options());
  Tensor token_id = at::empty({A}, i32);
  Tensor expert = at::empty({A}, i32);
  Tensor packed_w = at::empty({A}, X.options().dtype(at::kFloat));
  Tensor inv = at::empty({T, k}, i32);
  int32_t* cur = cursor.data_ptr<int32_t>();
  std::vector<int64_t> base(cur, cur + E);
  const std::vector<int64_t> counts =
      pack_rows(X, w, topk, base, packed_X, token_id, expert, packed_w, inv);
  for (int64_t e = 0; e < E; ++e) cur[e] = (int32_t)(cur[e] + counts[e]);
  return {packed_X, token_id, expert, packed_w, inv};
}

std::tuple<Tensor, Tensor, Tensor, Tensor> pack_tokens_kernel(Tensor X, Tensor w, Tensor topk,
                                                              Tensor cursor) {
  auto r = pack_impl(X, w, topk, cursor);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r)};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> pack_tokens_inv(Tensor X, Tensor w, Tensor topk,
                                                                   Tensor cursor) {
  return pack_impl(X, w, topk, cursor);
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_tokens(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts) {
  check_pack_inputs(X, w, topk);
  TORCH_CHECK(num_experts >= 1 && num_experts <= NT_MAX_EXPERTS,
              "num_experts must be in [1, ", NT_MAX_EXPERTS, "]");
  const int64_t T = X.size(0), d = X.size(1), k = w.size(1), A = T * k, E = num_experts;
  auto i32 = X.options().dtype(at::kInt);
  // Counts of valid ids and their exclusive scan: the pack's base.
  std::vector<int64_t> base(E, 0), cnt(E, 0);
  const int32_t* tk = topk.data_ptr<int32_t>();
  for (int64_t f = 0; f < A; ++f)
    if (tk[f] >= 0 && tk[f] < E) ++cnt[tk[f]];
  for (int64_t e = 1; e < E; ++e) base[e] = base[e - 1] + cnt[e - 1];
  Tensor counts = at::empty({E}, i32);
  Tensor offsets = at::empty({E + 1}, i32);
  for (int64_t e = 0; e < E; ++e) {
    counts.data_ptr<int32_t>()[e] = (int32_t)cnt[e];
    offsets.data_ptr<int32_t>()[e] = (int32_t)base[e];
  }
  offsets.data_ptr<int32_t>()[E] = (int32_t)(E > 0 ? base[E - 1] + cnt[E - 1] : 0);
  Tensor packed_X = at::empty({A, d}, X.options());
  Tensor token_id = at::empty({A}, i32);
  Tensor expert = at::empty({A}, i32);
  Tensor packed_w = at::empty({A}, X.options().dtype(at::kFloat));
  Tensor inv = at::empty({T, k}, i32);
  pack_rows(X, w, topk, base, packed_X, token_id, expert, packed_w, inv);
  return {counts, offsets, packed_X, token_id, expert, packed_w, inv};
}

// The dispatch workspace route_topk_count hands over: hist[e*nb + b], the
// tokens of block b (TB = nt_dispatch_block_tokens) routed to expert e.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> dispatch_tokens_counted(
    Tensor X, Tensor w, Tensor topk, int64_t num_experts, Tensor ws) {
  check_cpu(ws, "dispatch workspace");
  const size_t need = nt_dispatch_workspace_bytes(X.size(0), (int32_t)w.size(1),
                                                  (int32_t)num_experts, X.size(1),
                                                  X.scalar_type() == at::kFloat    ? NT_F32
                                                  : X.scalar_type() == at::kDouble ? NT_F64
                                                  : X.scalar_type() == at::kHalf   ? NT_F16
                                                                                   : NT_BF16);
  TORCH_CHECK(ws.is_contiguous() && (size_t)ws.numel() * ws.element_size() >= need,
              "dispatch workspace from route_topk_count is too small for these sizes");
  // The per-block counts in ws describe these ids; the host pack recounts
  // them. ws is left as it is: the counts must survive the call on every
  // device, and the scratch after them holds nothing the caller reads.
  return dispatch_tokens(X, w, topk, num_experts);
}

// ------------------------------------------------------------ combine

// Rows of each token in ascending packed order (a stable counting sort of
// the packed rows by token id); ids outside [0, T) are dropped.
void token_csr(const int32_t* tid, int64_t A, int64_t T, std::vector<int64_t>& start,
               std::vector<int64_t>& rows) {
  start.assign(T + 1, 0);
  for (int64_t p = 0; p < A; ++p)
    if (tid[p] >= 0 && tid[p] < T) ++start[tid[p] + 1];
  for (int64_t t = 0; t < T; ++t) start[t + 1] += start[t];
  rows.assign(start[T], 0);
  std::vector<int64_t> fill(start.begin(), start.end() - 1);
  for (int64_t p = 0; p < A; ++p)
    if (tid[p] >= 0 && tid[p] < T) rows[fill[tid[p]]++] = p;
}

// out[t,:] = sum over rows p (in the given order) of fl32(w[p] * y[p,:]).
template <typename S, typename SO>
void combine_rows(const S* y, const float* w, int64_t d, const int64_t* rows, int64_t n,
                  SO* out, float* acc) {
  std::fill(acc, acc + d, 0.f);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t p = rows[i];
    const float wp = w[p];
    const S* yr = y + p * d;
    for (int64_t h = 0; h < d; ++h) {
      const float prod = wp * to_f(yr[h]);  // rounded to fp32, then added (no FMA)
      acc[h] = acc[h] + prod;
    }
  }
  for (int64_t h = 0; h < d; ++h) out[h] = from_f<SO>(acc[h]);
}

Tensor combine_tokens_kernel(Tensor y, Tensor token_id, Tensor w, int64_t num_tokens,
                             int64_t d_model) {
  TORCH_CHECK(y.is_contiguous(), "Expert output tensor should be contiguous");
  TORCH_CHECK(token_id.is_contiguous(), "packed token ids tensor should be contiguous");
  TORCH_CHECK(w.is_contiguous(), "packed topk weights tensor should be contiguous");
  check_float_type(y, "expert_outputs");
  check_i32(token_id, "packed_tokenId");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && y.size(1) == d_model, "expert_outputs must be [A, d_model]");
  TORCH_CHECK(token_id.numel() == y.size(0) && w.numel() == y.size(0),
              "one token id and one weight per packed row");
  const int64_t A = y.size(0), T = num_tokens, d = d_model;
  Tensor out = at::empty({T, d}, y.options().dtype(at::kFloat));
  std::vector<int64_t> start, rows;
  token_csr(token_id.data_ptr<int32_t>(), A, T, start, rows);
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, y.scalar_type(), "combine_cpu", [&] {
    const scalar_t* yp = y.data_ptr<scalar_t>();
    float* op = out.data_ptr<float>();
    at::parallel_for(0, T, 64, [&](int64_t t0, int64_t t1) {
      std::vector<float> acc(d);
      for (int64_t t = t0; t < t1; ++t)
        combine_rows<scalar_t, float>(yp, w.data_ptr<float>(), d, rows.data() + start[t],
                                      start[t + 1] - start[t], op + t * d, acc.data());
    });
  });
  return out;
}

// dy[p] = cast(dY[t] * w[p]); dw[p] = sum_h dY[t,h] * y[p,h] (double sum).
template <typename S, typename SG>
void combine_bwd_row(const S* y, const SG* g, float wp, int64_t d, S* dy, float* dw) {
  double s = 0.0;
  for (int64_t h = 0; h < d; ++h) {
    const float gv = to_f(g[h]);
    dy[h] = from_f<S>(gv * wp);
    s += (double)gv * (double)to_f(y[h]);
  }
  *dw = (float)s;
}

std::tuple<Tensor, Tensor> combine_kernel_backward(Tensor y, Tensor token_id, Tensor w, Tensor dY,
                                                   int64_t hidden_dim) {
  TORCH_CHECK(y.is_contiguous() && token_id.is_contiguous() && w.is_contiguous() &&
                  dY.is_contiguous(),
              "Tensor should be laid out in contiguous memory location");
  TORCH_CHECK(dY.scalar_type() == at::kFloat, "residual_stream_grad must be float32");
  check_float_type(y, "expert_outputs");
  check_cpu(dY, "residual_stream_grad");
  check_i32(token_id, "packed_tokenIds");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && y.size(1) == hidden_dim && dY.dim() == 2 &&
                  dY.size(1) == hidden_dim,
              "expert_outputs and residual_stream_grad must have hidden_dim columns");
  TORCH_CHECK(token_id.numel() == y.size(0) && w.numel() == y.size(0),
              "one token id and one weight per packed row");
  const int64_t A = y.size(0), T = dY.size(0), d = hidden_dim;
  Tensor dy = at::zeros_like(y);
  Tensor dw = at::zeros(w.sizes(), w.options());
  const int32_t* tid = token_id.data_ptr<int32_t>();
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, y.scalar_type(), "combine_bwd_cpu",
                                  [&] {
    const scalar_t* yp = y.data_ptr<scalar_t>();
    scalar_t* dyp = dy.data_ptr<scalar_t>();
    const float* g = dY.data_ptr<float>();
    at::parallel_for(0, A, 64, [&](int64_t p0, int64_t p1) {
      for (int64_t p = p0; p < p1; ++p) {
        const int32_t t = tid[p];
        const float wp = w.data_ptr<float>()[p];
        if (t < 0 || t >= T) {
          // The GPU kernel multiplies a zero grad row: dy = 0 * w (signed), dw = +0.
          for (int64_t h = 0; h < d; ++h) dyp[p * d + h] = from_f<scalar_t>(0.f * wp);
          continue;
        }
        combine_bwd_row<scalar_t, float>(yp + p * d, g + t * d, wp, d, dyp + p * d,
                                         dw.data_ptr<float>() + p);
      }
    });
  });
  return {dy, dw};
}

std::tuple<Tensor, Tensor> pack_kernel_backward(Tensor dpX, Tensor dpw, Tensor token_id,
                                                Tensor expert, Tensor topk) {
  TORCH_CHECK(dpX.is_contiguous(), "packed_X_grad must be contiguous");
  TORCH_CHECK(dpw.is_contiguous(), "packed_topk_weights_grad must be contiguous");
  TORCH_CHECK(token_id.is_contiguous(), "packed_tokenId must be contiguous");
  TORCH_CHECK(expert.is_contiguous(), "packed_expert must be contiguous");
  TORCH_CHECK(topk.is_contiguous(), "topk_experts must be contiguous");
  TORCH_CHECK(dpw.scalar_type() == at::kFloat, "packed_topk_weights_grad must be float32");
  check_float_type(dpX, "packed_X_grad");
  check_cpu(dpw, "packed_topk_weights_grad");
  check_i32(token_id, "packed_tokenId");
  check_i32(expert, "packed_expert");
  check_i32(topk, "topk_experts");
  TORCH_CHECK(dpX.dim() == 2 && topk.dim() == 2, "expected packed_X_grad [A,d], topk [T,k]");
  const int64_t A = dpX.size(0), d = dpX.size(1), T = topk.size(0), k = topk.size(1);
  TORCH_CHECK(dpw.numel() == A && token_id.numel() == A && expert.numel() == A,
              "one gate grad, token id and expert id per packed row");
  Tensor dX = at::empty({T, d}, dpX.options());
  Tensor dw = at::empty({T, k}, dpw.options());
  std::vector<int64_t> start, rows;
  token_csr(token_id.data_ptr<int32_t>(), A, T, start, rows);
  const int32_t* ex = expert.data_ptr<int32_t>();
  const int32_t* tk = topk.data_ptr<int32_t>();
  const float* gw = dpw.data_ptr<float>();
  float* dwp = dw.data_ptr<float>();
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, dpX.scalar_type(), "pack_bwd_cpu",
                                  [&] {
    const scalar_t* xp = dpX.data_ptr<scalar_t>();
    scalar_t* op = dX.data_ptr<scalar_t>();
    at::parallel_for(0, T, 64, [&](int64_t t0, int64_t t1) {
      std::vector<float> acc(d);
      for (int64_t t = t0; t < t1; ++t) {
        const int64_t* r = rows.data() + start[t];
        const int64_t n = start[t + 1] - start[t];
        std::fill(acc.begin(), acc.end(), 0.f);
        for (int64_t i = 0; i < n; ++i)
          for (int64_t h = 0; h < d; ++h) acc[h] = acc[h] + to_f(xp[r[i] * d + h]);
        for (int64_t h = 0; h < d; ++h) op[t * d + h] = from_f<scalar_t>(acc[h]);
        // Reference rule (csrc/kernels/backward_pack_kernel.cu:35-42): the
        // first slot whose expert matches receives the row's gate gradient,
        // summed in ascending packed order.
        for (int64_t j = 0; j < k; ++j) dwp[t * k + j] = 0.f;
        for (int64_t i = 0; i < n; ++i) {
          for (int64_t j = 0; j < k; ++j)
            if (tk[t * k + j] == ex[r[i]]) {
              dwp[t * k + j] = dwp[t * k + j] + gw[r[i]];
              break;
            }
        }
      }
    });
  });
  return {dX, dw};
}

// Packed rows of token t from the inverse map: valid entries in ascending
// order (slot order above 256 of them, as the GPU kernels walk them).
void inv_rows(const int32_t* inv, int64_t t, int64_t k, int64_t A, std::vector<int64_t>& rows) {
  rows.clear();
  for (int64_t j = 0; j < k; ++j) {
    const int32_t p = inv[t * k + j];
    if (p >= 0 && p < A) rows.push_back(p);
  }
  if (k <= 256) std::sort(rows.begin(), rows.end());
}

Tensor combine_inv(Tensor y, Tensor inv, Tensor w, c10::ScalarType out_dtype) {
  TORCH_CHECK(y.is_contiguous() && inv.is_contiguous() && w.is_contiguous(),
              "inputs must be contiguous");
  check_float_type(y, "expert_outputs");
  check_i32(inv, "inv");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && inv.dim() == 2, "expected y [A,d], inv [T,k]");
  TORCH_CHECK(y.size(0) == inv.numel() && w.numel() == inv.numel(),
              "expert_outputs and packed_topk_weights must have T*k = inv.numel() rows");
  const int64_t T = inv.size(0), k = inv.size(1), d = y.size(1), A = T * k;
  Tensor out = at::empty({T, d}, y.options().dtype(out_dtype));
  check_float_type(out, "out_dtype");
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, y.scalar_type(), "combine_inv_cpu",
                                  [&] {
    using S = scalar_t;
    AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, out_dtype, "combine_inv_out", [&] {
      const S* yp = y.data_ptr<S>();
      scalar_t* op = out.data_ptr<scalar_t>();
      at::parallel_for(0, T, 64, [&](int64_t t0, int64_t t1) {
        std::vector<float> acc(d);
        std::vector<int64_t> rows;
        for (int64_t t = t0; t < t1; ++t) {
          inv_rows(inv.data_ptr<int32_t>(), t, k, A, rows);
          combine_rows<S, scalar_t>(yp, w.data_ptr<float>(), d, rows.data(),
                                    (int64_t)rows.size(), op + t * d, acc.data());
        }
      });
    });
  });
  return out;
}

std::tuple<Tensor, Tensor> combine_backward_inv(Tensor y, Tensor inv, Tensor w, Tensor dY) {
  TORCH_CHECK(y.is_contiguous() && inv.is_contiguous() && w.is_contiguous() && dY.is_contiguous(),
              "inputs must be contiguous");
  check_float_type(y, "expert_outputs");
  check_cpu(dY, "grad");
  check_i32(inv, "inv");
  check_f32(w, "packed_topk_weights");
  TORCH_CHECK(y.dim() == 2 && inv.dim() == 2 && dY.dim() == 2 && dY.size(0) == inv.size(0) &&
                  dY.size(1) == y.size(1),
              "expected y [A,d], inv [T,k], grad [T,d]");
  TORCH_CHECK(dY.scalar_type() == at::kFloat || dY.scalar_type() == y.scalar_type(),
              "grad must be float32 or the activation dtype");
  TORCH_CHECK(y.size(0) == inv.numel() && w.numel() == inv.numel(),
              "expert_outputs and packed_topk_weights must have T*k = inv.numel() rows");
  const int64_t T = inv.size(0), k = inv.size(1), d = y.size(1), A = T * k;
  Tensor dy = at::zeros_like(y);
  Tensor dw = at::zeros(w.sizes(), w.options());
  const int32_t* iv = inv.data_ptr<int32_t>();
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, y.scalar_type(), "combine_bwd_inv",
                                  [&] {
    using S = scalar_t;
    auto run = [&](auto* g) {
      at::parallel_for(0, T, 64, [&](int64_t t0, int64_t t1) {
        for (int64_t t = t0; t < t1; ++t)
          for (int64_t j = 0; j < k; ++j) {
            const int32_t p = iv[t * k + j];
            if (p < 0 || p >= A) continue;
            combine_bwd_row(y.data_ptr<S>() + p * d, g + t * d, w.data_ptr<float>()[p], d,
                            dy.data_ptr<S>() + p * d, dw.data_ptr<float>() + p);
          }
      });
    };
    if (dY.scalar_type() == at::kFloat) run(dY.data_ptr<float>());
    else run(dY.data_ptr<S>());
  });
  return {dy, dw};
}

std::tuple<Tensor, Tensor> pack_backward_inv(Tensor dpX, Tensor dpw, Tensor inv) {
  TORCH_CHECK(dpX.is_contiguous() && dpw.is_contiguous() && inv.is_contiguous(),
              "inputs must be contiguous");
  check_float_type(dpX, "packed_X_grad");
  check_f32(dpw, "packed_topk_weights_grad");
  check_i32(inv, "inv");
  TORCH_CHECK(dpX.dim() == 2 && inv.dim() == 2, "expected packed_X_grad [A,d], inv [T,k]");
  TORCH_CHECK(dpX.size(0) == inv.numel() && dpw.numel() == inv.numel(),
              "packed_X_grad and packed_topk_weights_grad must have T*k = inv.numel() rows");
  const int64_t T = inv.size(0), k = inv.size(1), d = dpX.size(1), A = T * k;
  Tensor dX = at::empty({T, d}, dpX.options());
  Tensor dw = at::empty({T, k}, dpw.options());
  const int32_t* iv = inv.data_ptr<int32_t>();
  const float* gw = dpw.data_ptr<float>();
  float* dwp = dw.data_ptr<float>();
  AT_DISPATCH_FLOATING_TYPES_AND2(at::kHalf, at::kBFloat16, dpX.scalar_type(), "pack_bwd_inv",
                                  [&] {
    const scalar_t* xp = dpX.data_ptr<scalar_t>();
    scalar_t* op = dX.data_ptr<scalar_t>();
    at::parallel_for(0, T, 64, [&](int64_t t0, int64_t t1) {
      std::vector<float> acc(d);
      std::vector<int64_t> rows;
      for (int64_t t = t0; t < t1; ++t) {
        inv_rows(iv, t, k, A, rows);
        std::fill(acc.begin(), acc.end(), 0.f);
        for (int64_t p : rows)
          for (int64_t h = 0; h < d; ++h) acc[h] = acc[h] + to_f(xp[p * d + h]);
        for (int64_t h = 0; h < d; ++h) op[t * d + h] = from_f<scalar_t>(acc[h]);
        for (int64_t j = 0; j < k; ++j) {
          const int32_t p = iv[t * k + j];
          dwp[t * k + j] = (p >= 0 && p < A) ? gw[p] : 0.f;
        }
      }
    });
  });
  return {dX, dw};
}

// -------------------------------------------------------------- router

// Order of selection: larger logit first, ties to the lower expert id;
// -0 equals +0 and NaN ranks below every number (the GPU's order keys).
inline bool before(float a, int ia, float b, int ib) {
  const bool na = std::isnan(a), nb = std::isnan(b);
  if (na || nb) return na != nb ? nb : ia < ib;
  if (a != b) return a > b;
  return ia < ib;
}

void route_rows(const float* logits, int64_t T, int64_t E, int64_t k, float* gates, int32_t* topk,
                int32_t* hist, int64_t TB, int64_t nb) {
  at::parallel_for(0, T, 256, [&](int64_t t0, int64_t t1) {
    std::vector<int> order(E);
    for (int64_t t = t0; t < t1; ++t) {
      const float* z = logits + t * E;
      std::iota(order.begin(), order.end(), 0);
      std::partial_sort(order.begin(), order.begin() + k, order.end(),
                        [&](int a, int b) { return before(z[a], a, z[b], b); });
      const float m = z[order[0]];
      float den = 0.f;
      for (int64_t j = 0; j < k; ++j) den += std::exp(z[order[j]] - m);
      const float r = 1.f / den;
      for (int64_t j = 0; j < k; ++j) {
        gates[t * k + j] = std::exp(z[order[j]] - m) * r;
        topk[t * k + j] = order[j];
      }
    }
  });
  if (hist != nullptr) {
    std::fill(hist, hist + E * nb, 0);
    for (int64_t t = 0; t < T; ++t)
      for (int64_t j = 0; j < k; ++j) ++hist[(int64_t)topk[t * k + j] * nb + t / TB];
  }
}

void check_logits(const Tensor& logits, int64_t k) {
  TORCH_CHECK(logits.is_contiguous() && logits.dim() == 2, "logits must be a contiguous [T,E]");
  check_f32(logits, "logits");
  const int64_t E = logits.size(1);
  TORCH_CHECK(E <= NT_MAX_EXPERTS, "number of experts exceeds ", NT_MAX_EXPERTS);
  TORCH_CHECK(k >= 1 && k <= E && k <= 32, "top_k must be in [1, min(E, 32)]");
}

std::tuple<Tensor, Tensor> route_topk(Tensor logits, int64_t k) {
  check_logits(logits, k);
  const int64_t T = logits.size(0), E = logits.size(1);
  Tensor gates = at::empty({T, k}, logits.options());
  Tensor topk = at::empty({T, k}, logits.options().dtype(at::kInt));
  route_rows(logits.data_ptr<float>(), T, E, k, gates.data_ptr<float>(), topk.data_ptr<int32_t>(),
             nullptr, 1, 0);
  return {gates, topk};
}

int dtype_code(const Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return NT_F32;
    case at::kDouble: return NT_F64;
    case at::kHalf: return NT_F16;
    default: return NT_BF16;
  }
}

std::tuple<Tensor, Tensor, Tensor> route_topk_count(Tensor logits, int64_t k, Tensor X) {
  check_logits(logits, k);
  check_float_type(X, "X");
  const int64_t T = logits.size(0), E = logits.size(1);
  TORCH_CHECK(X.dim() == 2 && X.size(0) == T, "X must be [T,d] with the logits' T");
  Tensor gates = at::empty({T, k}, logits.options());
  Tensor topk = at::empty({T, k}, logits.options().dtype(at::kInt));
  const int dt = dtype_code(X);
  const size_t bytes = nt_dispatch_workspace_bytes(T, (int32_t)k, (int32_t)E, X.size(1), dt);
  Tensor ws = at::zeros({(int64_t)std::max<size_t>(bytes, 4)}, X.options().dtype(at::kByte));
  const int64_t TB = nt_dispatch_block_tokens(T, (int32_t)k, X.size(1), dt);
  const int64_t nb = TB > 0 ? (T + TB - 1) / TB : 0;
  route_rows(logits.data_ptr<float>(), T, E, k, gates.data_ptr<float>(), topk.data_ptr<int32_t>(),
             T > 0 ? static_cast<int32_t*>(ws.data_ptr()) : nullptr, std::max<int64_t>(TB, 1), nb);
  return {gates, topk, ws};
}

Tensor route_topk_backward(Tensor gates, Tensor topk, Tensor dgates, int64_t num_experts) {
  TORCH_CHECK(gates.is_contiguous() && topk.is_contiguous() && dgates.is_contiguous(),
              "inputs must be contiguous");
  check_f32(gates, "gates");
  check_f32(dgates, "dgates");
  check_i32(topk, "topk");
  TORCH_CHECK(gates.sizes() == topk.sizes() && gates.sizes() == dgates.sizes() && gates.dim() == 2,
              "gates, topk and dgates must all be [T,k]");
  const int64_t T = gates.size(0), k = gates.size(1), E = num_experts;
  Tensor dl = at::zeros({T, E}, gates.options());
  const float* g = gates.data_ptr<float>();
  const float* dg = dgates.data_ptr<float>();
  const int32_t* tk = topk.data_ptr<int32_t>();
  float* o = dl.data_ptr<float>();
  at::parallel_for(0, T, 256, [&](int64_t t0, int64_t t1) {
    for (int64_t t = t0; t < t1; ++t) {
      float part = 0.f;
      for (int64_t j = 0; j < k; ++j) part += dg[t * k + j] * g[t * k + j];
      for (int64_t j = 0; j < k; ++j) {
        const int32_t e = tk[t * k + j];
        if (e >= 0 && e < E) o[t * E + e] += g[t * k + j] * (dg[t * k + j] - part);
      }
    }
  });
  return dl;
}

// The pack backward whose dw is the router's gate gradient, then the router
// backward on it (the two ops above, in sequence).
std::tuple<Tensor, Tensor> pack_backward_inv_route(Tensor dpX, Tensor dpw, Tensor inv, Tensor gates,
                                                   Tensor topk, int64_t num_experts) {
  TORCH_CHECK(gates.sizes() == inv.sizes() && topk.sizes() == inv.sizes(),
              "gates and topk must be [T,k] like inv");
  auto [dX, dw] = pack_backward_inv(dpX, dpw, inv);
  return {dX, route_topk_backward(gates, topk, dw, num_experts)};
}

// --------------------------------------------------------- grouped GEMM
//
// Per expert segment: fp32 (fp64 for float64) products of the rows, one
// rounding to the dtype. Rows past offsets[E] are zero.

at::ScalarType acc_type(const Tensor& t) {
  return t.scalar_type() == at::kDouble ? at::kDouble : at::kFloat;
}

void check_gemm(const Tensor& a, const Tensor& offsets, const Tensor& b) {
  TORCH_CHECK(a.is_contiguous(), "X must be contiguous");
  TORCH_CHECK(b.is_contiguous(), "weights must be contiguous");
  check_float_type(a, "X");
  check_float_type(b, "weights");
  check_i32(offsets, "expert_offset");
  TORCH_CHECK(offsets.is_contiguous() && offsets.dim() == 1 && offsets.numel() >= 2,
              "expert_offset must be a 1-D [num_experts + 1] tensor");
  TORCH_CHECK(offsets.numel() - 1 <= NT_MAX_EXPERTS, "number of experts exceeds ",
              NT_MAX_EXPERTS);
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "operands must share one dtype");
}

// fp32/fp64 products h[a] = X[a] @ W[e] (op 0), dOut[a] @ W[e]^T (op 1).
Tensor rows_product(const Tensor& a, const Tensor& offsets, const Tensor& W, int op) {
  const int64_t A = a.size(0);
  const int64_t cols = op == 0 ? W.size(2) : W.size(1);
  const auto at_ = acc_type(a);
  Tensor h = at::zeros({A, cols}, a.options().dtype(at_));
  const int32_t* off = offsets.data_ptr<int32_t>();
  for (int64_t e = 0; e + 1 < offsets.numel(); ++e) {
    int64_t r0, r1;
    expert_rows(off, (int)e, A, r0, r1);
    if (r1 <= r0) continue;
    Tensor we = W[e].to(at_);
    h.slice(0, r0, r1).copy_(at::mm(a.slice(0, r0, r1).to(at_), op == 0 ? we : we.t()));
  }
  return h;
}

Tensor grouped_gemm_kernel(Tensor X, Tensor offsets, Tensor W) {
  check_gemm(X, offsets, W);
  TORCH_CHECK(X.dim() == 2 && W.dim() == 3 && W.size(1) == X.size(1),
              "expected X [A,K] and weights [E,K,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  return rows_product(X, offsets, W, 0).to(X.scalar_type());
}

Tensor bwd_grouped_gemm_dX_kernel(Tensor W, Tensor offsets, Tensor dOut) {
  check_gemm(dOut, offsets, W);
  TORCH_CHECK(W.dim() == 3 && dOut.dim() == 2 && dOut.size(1) == W.size(2),
              "expected W [E,K,N] and dOut [A,N]");
  TORCH_CHECK(offsets.numel() == W.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  return rows_product(dOut, offsets, W, 1).to(W.scalar_type());
}

Tensor bwd_grouped_gemm_dW_kernel(Tensor X, Tensor offsets, Tensor dOut) {
  check_gemm(X, offsets, dOut);
  TORCH_CHECK(X.dim() == 2 && dOut.dim() == 2 && dOut.size(0) == X.size(0),
              "expected X [A,K] and dOut [A,N]");
  const int64_t A = X.size(0), K = X.size(1), N = dOut.size(1), E = offsets.numel() - 1;
  const auto at_ = acc_type(X);
  Tensor dW = at::zeros({E, K, N}, X.options());
  const int32_t* off = offsets.data_ptr<int32_t>();
  for (int64_t e = 0; e < E; ++e) {
    int64_t r0, r1;
    expert_rows(off, (int)e, A, r0, r1);
    if (r1 <= r0) continue;
    dW[e].copy_(at::mm(X.slice(0, r0, r1).to(at_).t(), dOut.slice(0, r0, r1).to(at_)));
  }
  return dW;
}

// Elementwise activations in the accumulation type, from the rounded inputs.
template <typename AT>
inline void gelu_pair(AT x, AT& act, AT& grad) {
  const AT cdf = AT(0.5) * (AT(1) + std::erf(x * AT(0.70710678118654752440)));
  const AT pdf = std::exp(AT(-0.5) * x * x) * AT(0.39894228040143267794);
  act = x * cdf;
  grad = cdf + x * pdf;
}

// h rounded to the dtype; gelu(h) and gelu'(h) evaluated in double and
// rounded once (fp64: in double).
std::tuple<Tensor, Tensor> grouped_gemm_gelu(Tensor X, Tensor offsets, Tensor W) {
  Tensor h = grouped_gemm_kernel(X, offsets, W);
  Tensor hd = h.to(at::kDouble);
  Tensor act = at::empty_like(hd), g = at::empty_like(hd);
  const double* hp = hd.data_ptr<double>();
  double* ap = act.data_ptr<double>();
  double* gp = g.data_ptr<double>();
  at::parallel_for(0, hd.numel(), 4096, [&](int64_t i0, int64_t i1) {
    for (int64_t i = i0; i < i1; ++i) gelu_pair<double>(hp[i], ap[i], gp[i]);
  });
  return {act.to(X.scalar_type()), g.to(X.scalar_type())};
}

Tensor bwd_grouped_gemm_dX_gelu(Tensor W, Tensor offsets, Tensor dOut, Tensor act_grad) {
  check_cpu(act_grad, "act_grad");
  TORCH_CHECK(act_grad.is_contiguous() && act_grad.dim() == 2 &&
                  act_grad.size(0) == dOut.size(0) && act_grad.size(1) == W.size(1) &&
                  act_grad.scalar_type() == W.scalar_type(),
              "expected act_grad [A,K] contiguous, in the weights' dtype");
  Tensor dA = bwd_grouped_gemm_dX_kernel(W, offsets, dOut);
  const auto at_ = acc_type(W);
  return (dA.to(at_) * act_grad.to(at_)).to(W.scalar_type());
}

// SwiGLU in the accumulation type with the unfused graph's roundings: gate,
// value, silu(gate), hidden (and in the backward dhidden, dhidden * value,
// dvalue, dgate) each rounded to the dtype.
std::tuple<Tensor, Tensor, Tensor> grouped_gemm_swiglu(Tensor X, Tensor offsets, Tensor Wg,
                                                       Tensor Wv) {
  TORCH_CHECK(Wv.sizes() == Wg.sizes(), "expected X [A,K] and gate / value weights [E,K,N]");
  Tensor gate = grouped_gemm_kernel(X, offsets, Wg);
  Tensor value = grouped_gemm_kernel(X, offsets, Wv);
  const auto dt = X.scalar_type();
  const auto at_ = acc_type(X);
  Tensor g = gate.to(at_), v = value.to(at_);
  Tensor silu = (g * at::sigmoid(g)).to(dt).to(at_);
  Tensor hidden = (silu * v).to(dt);
  return {hidden, gate, value};
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dX_swiglu(Tensor W, Tensor offsets, Tensor dOut,
                                                      Tensor gate, Tensor value) {
  for (const Tensor* t : {&gate, &value}) {
    check_cpu(*t, "gate/value");
    TORCH_CHECK(t->is_contiguous() && t->dim() == 2 && t->size(0) == dOut.size(0) &&
                    t->size(1) == W.size(1) && t->scalar_type() == W.scalar_type(),
                "expected gate and value [A,K] contiguous, in the weights' dtype");
  }
  const auto dt = W.scalar_type();
  const auto at_ = acc_type(W);
  Tensor dh = bwd_grouped_gemm_dX_kernel(W, offsets, dOut).to(at_);
  Tensor g = gate.to(at_), v = value.to(at_);
  Tensor sg = at::sigmoid(g);
  Tensor dvalue = (dh * (g * sg).to(dt).to(at_)).to(dt);
  Tensor ds = (dh * v).to(dt).to(at_);
  Tensor dgate = ((ds * sg) * (1 + g * (1 - sg))).to(dt);
  return {dgate, dvalue};
}

Tensor bwd_grouped_gemm_dX2(Tensor W1, Tensor W2, Tensor offsets, Tensor dOut1, Tensor dOut2) {
  check_gemm(dOut1, offsets, W1);
  check_gemm(dOut2, offsets, W2);
  TORCH_CHECK(W1.dim() == 3 && W2.sizes() == W1.sizes() && dOut1.dim() == 2 &&
                  dOut1.size(1) == W1.size(2) && dOut2.sizes() == dOut1.sizes(),
              "expected W1, W2 [E,K,N] and dOut1, dOut2 [A,N]");
  TORCH_CHECK(offsets.numel() == W1.size(0) + 1, "expert_offset must hold num_experts + 1 entries");
  // One accumulation over both products, one rounding.
  return (rows_product(dOut1, offsets, W1, 1) + rows_product(dOut2, offsets, W2, 1))
      .to(W1.scalar_type());
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX(Tensor X, Tensor W, Tensor offsets, Tensor dOut) {
  return {bwd_grouped_gemm_dW_kernel(X, offsets, dOut),
          bwd_grouped_gemm_dX_kernel(W, offsets, dOut)};
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX_gelu(Tensor act, Tensor W, Tensor offsets,
                                                       Tensor dOut, Tensor act_grad) {
  return {bwd_grouped_gemm_dW_kernel(act, offsets, dOut),
          bwd_grouped_gemm_dX_gelu(W, offsets, dOut, act_grad)};
}

std::tuple<Tensor, Tensor, Tensor> bwd_grouped_gemm_dW_dX_swiglu(Tensor hidden, Tensor W,
                                                                 Tensor offsets, Tensor dOut,
                                                                 Tensor gate, Tensor value) {
  Tensor dW = bwd_grouped_gemm_dW_kernel(hidden, offsets, dOut);
  auto r = bwd_grouped_gemm_dX_swiglu(W, offsets, dOut, gate, value);
  return {dW, std::get<0>(r), std::get<1>(r)};
}

std::tuple<Tensor, Tensor> bwd_grouped_gemm_dW_dX2(Tensor X, Tensor W1, Tensor W2, Tensor offsets,
                                                   Tensor dOut1, Tensor dOut2) {
  return {bwd_grouped_gemm_dW_kernel(X, offsets, dOut1),
          bwd_grouped_gemm_dX2(W1, W2, offsets, dOut1, dOut2)};
}

}  // namespace
}  // namespace nt_cpu

TORCH_LIBRARY_IMPL(nanotitan, CPU, m) {
  using namespace nt_cpu;
  m.impl("count_expert_kernel", &count_expert_kernel);
  m.impl("pack_tokens_kernel", &pack_tokens_kernel);
  m.impl("combine_tokens_kernel", &combine_tokens_kernel);
  m.impl("combine_kernel_backward", &combine_kernel_backward);
  m.impl("pack_kernel_backward", &pack_kernel_backward);
  m.impl("grouped_gemm_kernel", &grouped_gemm_kernel);
  m.impl("bwd_grouped_gemm_dW_kernel", &bwd_grouped_gemm_dW_kernel);
  m.impl("bwd_grouped_gemm_dX_kernel", &bwd_grouped_gemm_dX_kernel);
  m.impl("grouped_gemm_gelu", &grouped_gemm_gelu);
  m.impl("bwd_grouped_gemm_dX_gelu", &bwd_grouped_gemm_dX_gelu);
  m.impl("grouped_gemm_swiglu", &grouped_gemm_swiglu);
  m.impl("bwd_grouped_gemm_dX_swiglu", &bwd_grouped_gemm_dX_swiglu);
  m.impl("bwd_grouped_gemm_dX2", &bwd_grouped_gemm_dX2);
  m.impl("bwd_grouped_gemm_dW_dX", &bwd_grouped_gemm_dW_dX);
  m.impl("bwd_grouped_gemm_dW_dX_gelu", &bwd_grouped_gemm_dW_dX_gelu);
  m.impl("bwd_grouped_gemm_dW_dX_swiglu", &bwd_grouped_gemm_dW_dX_swiglu);
  m.impl("bwd_grouped_gemm_dW_dX2", &bwd_grouped_gemm_dW_dX2);
  m.impl("route_topk", &route_topk);
  m.impl("route_topk_count", &route_topk_count);
  m.impl("route_topk_backward", &route_topk_backward);
  m.impl("dispatch_tokens", &dispatch_tokens);
  m.impl("dispatch_tokens_counted", &dispatch_tokens_counted);
  m.impl("pack_tokens_inv", &pack_tokens_inv);
  m.impl("combine_inv", &combine_inv);
  m.impl("combine_backward_inv", &combine_backward_inv);
  m.impl("pack_backward_inv", &pack_backward_inv);
  m.impl("pack_backward_inv_route", &pack_backward_inv_route);
}
