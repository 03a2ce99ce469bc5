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
// A segment of S lanes serves a token, each lane holding about eight
// experts; every one of the k selections is a per-lane max over 64-bit order
// keys followed by log2(S) shuffle steps.
#include <math.h>

#include <type_traits>

#include "common.hpp"

namespace nt {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kRouterWaves = kRouterThreads / kWave;
constexpr int kLanePerExperts = 8;  // target experts per lane
constexpr int kRouterHistMax = 2048;  // LDS ints of the fused count (see route_topk_hist_kernel)

// Lane layout: a token is served by a segment of S lanes, S the power of two
// >= ceil(E/8) (at most 64); lane s of the segment holds experts s, s+S,
// s+2S, ... (V = ceil(E/S) <= 16 of them for E <= 1024). A wave serves 64/S
// tokens, 4 waves 256/S. The segment reads a row with coalesced loads; the
// selection runs over registers with few shuffles (one token per lane for
// E <= 8).
struct RouterLayout {
  int S;      // lanes per token
  int lgS;    // log2(S)
  int V;      // experts per lane
  int tpw;    // tokens per wave
};

__host__ __device__ inline RouterLayout router_layout(int32_t E) {
  RouterLayout L;
  const int want = (E + kLanePerExperts - 1) / kLanePerExperts;
  int s = 1, lg = 0;
  while (s < want && s < kWave) {
    s <<= 1;
    ++lg;
  }
  L.S = s;
  L.lgS = lg;
  L.V = (E + s - 1) / s;
  L.tpw = kWave / s;
  return L;
}

// Selection order as one unsigned 64-bit key, larger = chosen first: the
// high word maps the float's bits to an unsigned integer of the same order
// (sign flipped; -0 taken as +0 so the two tie; every NaN maps to 0, below
// -inf),
// the low word is ~expert so equal values go to the lower expert id. Key 0
// marks an empty slot (padding or already taken): it ranks below every
// expert, NaNs included, since ~e >= 2^31 for e < 2^31.
__device__ __forceinline__ uint64_t order_key(float x, int e) {
  // Integer-only, so denormals keep their order whatever the float mode.
  uint32_t u = __float_as_uint(x);
  if (u == 0x80000000u) u = 0u;  // -0 -> +0
  const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
  const uint32_t hi = nan ? 0u : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
  return ((uint64_t)hi << 32) | (uint32_t)~(uint32_t)e;
}

__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t hi = (uint32_t)(key >> 32);
  if (hi == 0u) return __uint_as_float(0x7fffffffu);  // NaN
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
}

__device__ __forceinline__ int key_expert(uint64_t key) { return (int)~(uint32_t)key; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int o) {
  const uint32_t lo = __shfl_xor((uint32_t)v, o, kWave);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, kWave);
  return ((uint64_t)hi << 32) | lo;
}

// Top-k of token t's logits (ties to the lower id), gates = softmax of the
// selected logits, optional full softmax into probs. With s_hist, each
// selected expert also bumps s_hist[expert] (an LDS count).
template <int KMAX, int VMAX>
__device__ __forceinline__ void route_token(const float* __restrict__ logits, int64_t t, bool live,
                                            int32_t E, int32_t k, const RouterLayout& L,
                                            float* __restrict__ gates,
                                            int32_t* __restrict__ topk,
                                            float* __restrict__ probs, int32_t* s_hist) {
  const int s = lane_id() & (L.S - 1);
  const float* z = logits + t * E;
  float x[VMAX];
  uint64_t key[VMAX];
#pragma unroll
  for (int v = 0; v < VMAX; ++v) {
    const int e = v * L.S + s;
    const bool in = live && v < L.V && e < E;
    x[v] = in ? z[e] : -INFINITY;
    key[v] = in ? order_key(x[v], e) : 0ull;
  }
  float sel_v[KMAX];
  int sel_i[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= k) break;
    uint64_t best = key[0];
#pragma unroll
    for (int v = 1; v < VMAX; ++v) best = key[v] > best ? key[v] : best;
    for (int o = 1; o < L.S; o <<= 1) {
      const uint64_t other = shfl_xor_u64(best, o);
      best = other > best ? other : best;
    }
#pragma unroll
    for (int v = 0; v < VMAX; ++v) key[v] = key[v] == best ? 0ull : key[v];
    sel_v[j] = key_value(best);
    sel_i[j] = key_expert(best);
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
      if (j < k && (j & (L.S - 1)) == s) {
        gates[t * k + j] = expf(sel_v[j] - m) * inv;
        topk[t * k + j] = sel_i[j];
        if (s_hist != nullptr) atomicAdd(&s_hist[sel_i[j]], 1);  // LDS, integer
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

template <int KMAX, int VMAX>
__global__ void __launch_bounds__(kRouterThreads)
route_topk_kernel(const float* __restrict__ logits, int64_t T, int32_t E, int32_t k,
                  float* __restrict__ gates, int32_t* __restrict__ topk,
                  float* __restrict__ probs) {
  const RouterLayout L = router_layout(E);
  const int64_t wave_g = (int64_t)blockIdx.x * kRouterWaves + threadIdx.x / kWave;
  const int64_t t = wave_g * L.tpw + (lane_id() >> L.lgS);
  route_token<KMAX, VMAX>(logits, t, t < T, E, k, L, gates, topk, probs, nullptr);
}

// The count fused into the gate: the dispatch counts tokens in blocks of TB
// (a power of two) and wants hist[e*nb + c] = #{(t, j) : t in block c,
// topk[t,j] = e} for every c < nb = ceil(T/TB). Workgroup b routes the BT =
// max(TB, 256/S) tokens [b*BT, (b+1)*BT) in BT/(256/S) passes, keeps the
// BT/TB block histograms in LDS (at most 2048 counts: 256/S <= 2048/E), and
// writes each of its columns once (no zero-fill, no global atomics).
template <int KMAX, int VMAX>
__global__ void __launch_bounds__(kRouterThreads)
route_topk_hist_kernel(const float* __restrict__ logits, int64_t T, int32_t E, int32_t k,
                       float* __restrict__ gates, int32_t* __restrict__ topk,
                       float* __restrict__ probs, int32_t TB, int32_t BT, int32_t nb,
                       int32_t* __restrict__ hist) {
  __shared__ int32_t s_hist[kRouterHistMax];
  const RouterLayout L = router_layout(E);
  const int sub = BT / TB;
  for (int i = threadIdx.x; i < sub * E; i += kRouterThreads) s_hist[i] = 0;
  __syncthreads();
  const int64_t t0 = (int64_t)blockIdx.x * BT;
  const int64_t t1 = t0 + BT < T ? t0 + BT : T;
  const int per_pass = kRouterWaves * L.tpw;
  const int mine = (threadIdx.x / kWave) * L.tpw + (lane_id() >> L.lgS);
  for (int p = 0; p < BT; p += per_pass) {
    const int64_t t = t0 + p + mine;
    const int c = (p + mine) / TB;  // block within this workgroup
    route_token<KMAX, VMAX>(logits, t, t < t1, E, k, L, gates, topk, probs,
                            s_hist + (c < sub ? c : 0) * E);
  }
  __syncthreads();
  const int64_t c0 = (int64_t)blockIdx.x * sub;
  for (int i = threadIdx.x; i < sub * E; i += kRouterThreads) {
    const int e = i / sub, c = i - e * sub;
    if (c0 + c < nb) hist[(int64_t)e * nb + c0 + c] = s_hist[c * E + e];
  }
}

// dlogits[t, :] = 0 except dz[topk[t,j]] = g_j * (dg_j - sum_i dg_i * g_i).
// Same lane layout as the forward; every lane of a segment reads the token's
// k slots itself (one cache line for the segment) and every element of the
// row is written once.
template <int KMAX, int VMAX>
__global__ void __launch_bounds__(kRouterThreads)
route_topk_backward_kernel(const float* __restrict__ gates, const int32_t* __restrict__ topk,
                           const float* __restrict__ dgates, int64_t T, int32_t E, int32_t k,
                           float* __restrict__ dlogits) {
  const RouterLayout L = router_layout(E);
  const int s = lane_id() & (L.S - 1);
  const int64_t wave_g = (int64_t)blockIdx.x * kRouterWaves + threadIdx.x / kWave;
  const int64_t t = wave_g * L.tpw + (lane_id() >> L.lgS);
  if (t >= T) return;  // no shuffles below: lanes are independent
  float g[KMAX], dg[KMAX];
  float part = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= k) break;
    g[j] = gates[t * k + j];
    dg[j] = dgates[t * k + j];
    part += dg[j] * g[j];
  }
  float out[VMAX];
#pragma unroll
  for (int v = 0; v < VMAX; ++v) out[v] = 0.f;
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    if (j >= k) break;
    const int ej = topk[t * k + j];
    const float dz = g[j] * (dg[j] - part);
    if (ej >= 0 && ej < E && (ej & (L.S - 1)) == s) {
      const int vj = ej >> L.lgS;
#pragma unroll
      for (int v = 0; v < VMAX; ++v)
        if (v == vj) out[v] += dz;
    }
  }
#pragma unroll
  for (int v = 0; v < VMAX; ++v) {
    const int e = v * L.S + s;
    if (v < L.V && e < E) dlogits[t * E + e] = out[v];
  }
}

template <int KMAX, int VMAX>
void launch_route(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                  int32_t* topk, float* probs, hipStream_t stream) {
  const RouterLayout L = router_layout(E);
  const dim3 grid((unsigned)ceil_div(T, (int64_t)kRouterWaves * L.tpw));
  hipLaunchKernelGGL((route_topk_kernel<KMAX, VMAX>), grid, dim3(kRouterThreads), 0, stream,
                     logits, T, E, k, gates, topk, probs);
}

template <int KMAX, int VMAX>
void launch_route_hist(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                       int32_t* topk, float* probs, int32_t TB, int32_t nb, int32_t* hist,
                       hipStream_t stream) {
  const RouterLayout L = router_layout(E);
  const int32_t per_pass = kRouterWaves * L.tpw;
  const int32_t BT = TB > per_pass ? TB : per_pass;
  const dim3 grid((unsigned)ceil_div(T, (int64_t)BT));
  hipLaunchKernelGGL((route_topk_hist_kernel<KMAX, VMAX>), grid, dim3(kRouterThreads), 0, stream,
                     logits, T, E, k, gates, topk, probs, TB, BT, nb, hist);
}

template <int KMAX, int VMAX>
void launch_route_bwd(const float* gates, const int32_t* topk, const float* dgates, int64_t T,
                      int32_t E, int32_t k, float* dlogits, hipStream_t stream) {
  const RouterLayout L = router_layout(E);
  const dim3 grid((unsigned)ceil_div(T, (int64_t)kRouterWaves * L.tpw));
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
    if (V <= 8) return f(std::integral_constant<int, KM>(), std::integral_constant<int, 8>());
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
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
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

int nt_route_topk_count(const float* logits, int64_t T, int32_t E, int32_t k, float* gates,
                        int32_t* topk, float* probs, int32_t TB, int32_t* hist,
                        hipStream_t stream) {
  if (T < 0 || E < 1 || k < 1 || k > E || TB < 1 || (TB & (TB - 1)) != 0)
    return NT_ERR_INVALID_ARG;
  if (k > kMaxTopK) return NT_ERR_INVALID_ARG;
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
  if (T * (int64_t)E > INT32_MAX * 4ll) return NT_ERR_TOO_LARGE;
  if (T == 0) return NT_OK;
  if (logits == nullptr || gates == nullptr || topk == nullptr || hist == nullptr)
    return NT_ERR_INVALID_ARG;
  const int64_t nb = ceil_div(T, (int64_t)TB);
  if (nb > INT32_MAX) return NT_ERR_TOO_LARGE;
  // LDS holds the max(TB, 256/S) / TB block histograms of a workgroup.
  const RouterLayout L = router_layout(E);
  const int32_t per_pass = kRouterWaves * L.tpw;
  if (TB < per_pass && (int64_t)(per_pass / TB) * E > kRouterHistMax) return NT_ERR_INVALID_ARG;
  router_dispatch(E, k, [&](auto km, auto vm) {
    launch_route_hist<decltype(km)::value, decltype(vm)::value>(logits, T, E, k, gates, topk,
                                                                probs, TB, (int32_t)nb, hist,
                                                                stream);
    return true;
  });
  return launch_status();
}

int nt_route_topk_backward(const float* gates, const int32_t* topk, const float* dgates,
                           int64_t T, int32_t E, int32_t k, float* dlogits, hipStream_t stream) {
  if (T < 0 || E < 1 || k < 1 || k > E || k > kMaxTopK) return NT_ERR_INVALID_ARG;
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
  if (T * (int64_t)E > INT32_MAX * 4ll) return NT_ERR_TOO_LARGE;
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
