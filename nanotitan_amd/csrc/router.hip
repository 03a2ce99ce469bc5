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
// A segment of lanes per token (one lane per expert up to 64 experts); the
// k selections are segment-wide argmax reductions over wave shuffles.
#include <math.h>

#include <type_traits>

#include "common.hpp"

namespace nt {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxTopK = 32;

// Lane layout: each token is served by a segment of S lanes (S = the power
// of two >= E, at most 64); lane s of the segment holds experts s, s+S,
// s+2S, ... (V = ceil(E/S) of them, at most VMAX). A wave serves 64/S
// tokens. Loads and stores of a row are coalesced across the segment.
struct RouterLayout {
  int S;      // lanes per token
  int V;      // experts per lane
  int tpw;    // tokens per wave
};

__host__ __device__ inline RouterLayout router_layout(int32_t E) {
  RouterLayout L;
  int s = 1;
  while (s < E && s < kWave) s <<= 1;
  L.S = s;
  L.V = (E + s - 1) / s;
  L.tpw = kWave / s;
  return L;
}

// (value, expert) order used for selection: a larger value wins; equal
// values go to the lower expert id; NaN ranks below -inf.
__device__ __forceinline__ bool beats(float v, int i, float w, int j) {
  const bool vn = v != v, wn = w != w;
  if (vn || wn) return !vn && wn ? true : (vn && wn ? i < j : false);
  return v > w || (v == w && i < j);
}

// Top-k of each token's logits (ties to the lower id), gates = softmax of
// the selected logits, optional full softmax. Each of the k rounds takes the
// best untaken (value, expert) of every lane and reduces it across the
// segment with xor shuffles.
template <int KMAX, int VMAX>
__global__ void __launch_bounds__(kRouterThreads)
route_topk_kernel(const float* __restrict__ logits, int64_t T, int32_t E, int32_t k,
                  float* __restrict__ gates, int32_t* __restrict__ topk,
                  float* __restrict__ probs) {
  const RouterLayout L = router_layout(E);
  const int lane = lane_id();
  const int s = lane % L.S;
  const int64_t wave_g = ((int64_t)blockIdx.x * kRouterThreads + threadIdx.x) / kWave;
  const int64_t t = wave_g * L.tpw + lane / L.S;
  const bool live = t < T;
  const float* z = logits + t * E;
  float x[VMAX];
#pragma unroll
  for (int v = 0; v < VMAX; ++v) {
    const int e = v * L.S + s;
    x[v] = (live && v < L.V && e < E) ? z[e] : -INFINITY;
  }
  uint32_t taken = 0;
  for (int v = 0; v < VMAX; ++v)
    if (v >= L.V || v * L.S + s >= E) taken |= 1u << v;  // padding never wins
  float sel_v[KMAX];
  int sel_i[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= k) break;
    // Best untaken candidate of this lane.
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
      const int e = v * L.S + s;
      if (!((taken >> v) & 1u) && (bi == 0x7fffffff || beats(x[v], e, bv, bi))) {
        bv = x[v];
        bi = e;
      }
    }
    // Segment-wide best.
    for (int o = 1; o < L.S; o <<= 1) {
      const float ov = __shfl_xor(bv, o, kWave);
      const int oi = __shfl_xor(bi, o, kWave);
      if (oi != 0x7fffffff && (bi == 0x7fffffff || beats(ov, oi, bv, bi))) {
        bv = ov;
        bi = oi;
      }
    }
    sel_v[j] = bv;
    sel_i[j] = bi;
    if (bi != 0x7fffffff && bi % L.S == s) taken |= 1u << (bi / L.S);
  }
  const float m = sel_v[0];
  float den = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j)
    if (j < k) den += expf(sel_v[j] - m);
  const float inv = 1.f / den;
  if (live) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k && j % L.S == s) {
        gates[t * k + j] = expf(sel_v[j] - m) * inv;
        topk[t * k + j] = sel_i[j];
      }
    }
  }
  if (probs != nullptr) {
    float part = 0.f;
#pragma unroll
    for (int v = 0; v < VMAX; ++v)
      if (v < L.V && v * L.S + s < E) part += expf(x[v] - m);
    for (int o = 1; o < L.S; o <<= 1) part += __shfl_xor(part, o, kWave);
    const float r = 1.f / part;
    if (live) {
#pragma unroll
      for (int v = 0; v < VMAX; ++v) {
        const int e = v * L.S + s;
        if (v < L.V && e < E) probs[t * E + e] = expf(x[v] - m) * r;
      }
    }
  }
}

// dlogits[t, :] = 0 except dz[topk[t,j]] = g_j * (dg_j - sum_i dg_i * g_i),
// same lane layout as the forward; every element of the row is written once.
template <int KMAX, int VMAX>
__global__ void __launch_bounds__(kRouterThreads)
route_topk_backward_kernel(const float* __restrict__ gates, const int32_t* __restrict__ topk,
                           const float* __restrict__ dgates, int64_t T, int32_t E, int32_t k,
                           float* __restrict__ dlogits) {
  const RouterLayout L = router_layout(E);
  const int lane = lane_id();
  const int s = lane % L.S;
  const int64_t wave_g = ((int64_t)blockIdx.x * kRouterThreads + threadIdx.x) / kWave;
  const int64_t t = wave_g * L.tpw + lane / L.S;
  const bool live = t < T;
  // Segment lanes j < k load slot j; the sum and the slots are shared by shuffles.
  float g = 0.f, dg = 0.f;
  int id = -1;
  for (int j = s; j < k; j += L.S) {  // k <= S here (k <= E, S >= min(E, 64), k <= 32)
    if (live) {
      g = gates[t * k + j];
      dg = dgates[t * k + j];
      id = topk[t * k + j];
    }
  }
  float part = s < k ? dg * g : 0.f;
  for (int o = 1; o < L.S; o <<= 1) part += __shfl_xor(part, o, kWave);
  const float dz_mine = g * (dg - part);
  float out[VMAX];
#pragma unroll
  for (int v = 0; v < VMAX; ++v) out[v] = 0.f;
  const int base_lane = (lane / L.S) * L.S;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= k) break;
    const int ej = __shfl(id, base_lane + j, kWave);
    const float dj = __shfl(dz_mine, base_lane + j, kWave);
    if (ej >= 0 && ej < E && ej % L.S == s) {
#pragma unroll
      for (int v = 0; v < VMAX; ++v)
        if (v == ej / L.S) out[v] += dj;
    }
  }
  if (live) {
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
      const int e = v * L.S + s;
      if (v < L.V && e < E) dlogits[t * E + e] = out[v];
    }
  }
}

template <int KMAX, int VMAX>
void launch_route(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                  int32_t* topk, float* probs, hipStream_t stream) {
  const RouterLayout L = router_layout(E);
  const int64_t waves = ceil_div(T, L.tpw);
  const dim3 grid((unsigned)ceil_div(waves, kRouterThreads / kWave));
  hipLaunchKernelGGL((route_topk_kernel<KMAX, VMAX>), grid, dim3(kRouterThreads), 0, stream,
                     logits, T, E, k, gates, topk, probs);
}

template <int KMAX, int VMAX>
void launch_route_bwd(const float* gates, const int32_t* topk, const float* dgates, int64_t T,
                      int32_t E, int32_t k, float* dlogits, hipStream_t stream) {
  const RouterLayout L = router_layout(E);
  const int64_t waves = ceil_div(T, L.tpw);
  const dim3 grid((unsigned)ceil_div(waves, kRouterThreads / kWave));
  hipLaunchKernelGGL((route_topk_backward_kernel<KMAX, VMAX>), grid, dim3(kRouterThreads), 0,
                     stream, gates, topk, dgates, T, E, k, dlogits);
}

// Dispatch on (top-k bound, experts-per-lane bound).
template <typename F>
bool router_dispatch(int32_t E, int32_t k, F&& f) {
  const int V = router_layout(E).V;
  auto by_v = [&](auto kmax) -> bool {
    constexpr int KM = decltype(kmax)::value;
    if (V <= 1) return f(std::integral_constant<int, KM>(), std::integral_constant<int, 1>());
    if (V <= 2) return f(std::integral_constant<int, KM>(), std::integral_constant<int, 2>());
    if (V <= 4) return f(std::integral_constant<int, KM>(), std::integral_constant<int, 4>());
    return f(std::integral_constant<int, KM>(), std::integral_constant<int, 16>());
  };
  if (k <= 2) return by_v(std::integral_constant<int, 2>());
  if (k <= 8) return by_v(std::integral_constant<int, 8>());
  return by_v(std::integral_constant<int, kMaxTopK>());
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
  router_dispatch(E, k, [&](auto km, auto vm) {
    launch_route<decltype(km)::value, decltype(vm)::value>(logits, T, E, k, gates, topk, probs,
                                                           stream);
    return true;
  });
  return launch_status();
}

int nt_route_topk_backward(const float* gates, const int32_t* topk, const float* dgates,
                           int64_t T, int32_t E, int32_t k, float* dlogits, hipStream_t stream) {
  if (T < 0 || E < 1 || k < 1 || k > E) return NT_ERR_INVALID_ARG;
  if (T == 0) return NT_OK;
  if (gates == nullptr || topk == nullptr || dgates == nullptr || dlogits == nullptr)
    return NT_ERR_INVALID_ARG;
  router_dispatch(E, k, [&](auto km, auto vm) {
    launch_route_bwd<decltype(km)::value, decltype(vm)::value>(gates, topk, dgates, T, E, k,
                                                               dlogits, stream);
    return true;
  });
  return launch_status();
}

}  // extern "C"
