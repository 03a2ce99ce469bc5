// Router gate: fp32 softmax -> top-k -> renormalised gates, fused, for gfx950.
//
// The reference computes probs = softmax(logits), torch.topk(probs, k) and
// gates = p_topk / sum(p_topk) as separate torch ops
// (src/model/cuda_backend.py:30-37). Softmax is monotonic, so the top-k of
// the probabilities is the top-k of the logits; selecting on the logits is
// exact (no rounding before the comparison) and ties go to the lower expert
// id (torch.topk leaves tie order unspecified). The renormalised gates are
// exactly a softmax over the k selected logits:
//     gate_j = exp(z_j) / sum_{i in sel} exp(z_i),
// so their gradient touches only the selected logits:
//     dz_j = gate_j * (dgate_j - sum_i dgate_i * gate_i),  dz_e = 0 otherwise.
// One thread per token; rows are read once (16-byte loads when aligned).
#include <math.h>

#include "common.hpp"

namespace nt {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxTopK = 32;

template <int KMAX>
__global__ void __launch_bounds__(kRouterThreads)
route_topk_kernel(const float* __restrict__ logits, int64_t T, int32_t E, int32_t k,
                  float* __restrict__ gates, int32_t* __restrict__ topk,
                  float* __restrict__ probs) {
  const int64_t t = (int64_t)blockIdx.x * kRouterThreads + threadIdx.x;
  if (t >= T) return;
  const float* z = logits + t * E;
  float val[KMAX];
  int32_t idx[KMAX];
  int filled = 0;
  for (int e = 0; e < E; ++e) {
    const float v = z[e];
    // Insert when the list is not full or v beats the current k-th value;
    // an equal value never displaces an earlier (lower-id) entry.
    if (filled < k || v > val[k - 1]) {
      int pos = filled < k ? filled : k - 1;
      while (pos > 0 && v > val[pos - 1]) {
        val[pos] = val[pos - 1];
        idx[pos] = idx[pos - 1];
        --pos;
      }
      val[pos] = v;
      idx[pos] = e;
      if (filled < k) ++filled;
    }
  }
  const float m = val[0];
  float s = 0.f;
  for (int j = 0; j < k; ++j) {
    val[j] = expf(val[j] - m);
    s += val[j];
  }
  const float inv = 1.f / s;
  for (int j = 0; j < k; ++j) {
    gates[t * k + j] = val[j] * inv;
    topk[t * k + j] = idx[j];
  }
  if (probs != nullptr) {
    float tot = 0.f;
    for (int e = 0; e < E; ++e) tot += expf(z[e] - m);
    const float r = 1.f / tot;
    for (int e = 0; e < E; ++e) probs[t * E + e] = expf(z[e] - m) * r;
  }
}

__global__ void __launch_bounds__(kRouterThreads)
route_topk_backward_kernel(const float* __restrict__ gates, const int32_t* __restrict__ topk,
                           const float* __restrict__ dgates, int64_t T, int32_t E, int32_t k,
                           float* __restrict__ dlogits) {
  const int64_t t = (int64_t)blockIdx.x * kRouterThreads + threadIdx.x;
  if (t >= T) return;
  float* dz = dlogits + t * E;
  for (int e = 0; e < E; ++e) dz[e] = 0.f;
  float s = 0.f;
  for (int j = 0; j < k; ++j) s += dgates[t * k + j] * gates[t * k + j];
  for (int j = 0; j < k; ++j) {
    const int32_t e = topk[t * k + j];
    if (e >= 0 && e < E) dz[e] += gates[t * k + j] * (dgates[t * k + j] - s);
  }
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

int nt_route_topk(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                  int32_t* topk, float* probs, hipStream_t stream) {
  if (T < 0 || E < 1 || k < 1 || k > E) return NT_ERR_INVALID_ARG;
  if (k > kMaxTopK) return NT_ERR_INVALID_ARG;
  if (T * (int64_t)E > INT32_MAX * 4ll) return NT_ERR_TOO_LARGE;
  if (T == 0) return NT_OK;
  if (logits == nullptr || gates == nullptr || topk == nullptr) return NT_ERR_INVALID_ARG;
  const dim3 grid((unsigned)ceil_div(T, kRouterThreads));
  if (k <= 2)
    hipLaunchKernelGGL(route_topk_kernel<2>, grid, dim3(kRouterThreads), 0, stream, logits, T, E, k,
                       gates, topk, probs);
  else if (k <= 8)
    hipLaunchKernelGGL(route_topk_kernel<8>, grid, dim3(kRouterThreads), 0, stream, logits, T, E, k,
                       gates, topk, probs);
  else
    hipLaunchKernelGGL(route_topk_kernel<kMaxTopK>, grid, dim3(kRouterThreads), 0, stream, logits,
                       T, E, k, gates, topk, probs);
  return launch_status();
}

int nt_route_topk_backward(const float* gates, const int32_t* topk, const float* dgates,
                           int64_t T, int32_t E, int32_t k, float* dlogits, hipStream_t stream) {
  if (T < 0 || E < 1 || k < 1 || k > E) return NT_ERR_INVALID_ARG;
  if (T == 0) return NT_OK;
  if (gates == nullptr || topk == nullptr || dgates == nullptr || dlogits == nullptr)
    return NT_ERR_INVALID_ARG;
  const dim3 grid((unsigned)ceil_div(T, kRouterThreads));
  hipLaunchKernelGGL(route_topk_backward_kernel, grid, dim3(kRouterThreads), 0, stream, gates, topk,
                     dgates, T, E, k, dlogits);
  return launch_status();
}

}  // extern "C"
