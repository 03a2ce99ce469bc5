// Shared device helpers for the gfx950 MoE kernels: element conversions,
// wave64 primitives, launch/argument checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nanotitan_moe.h"

namespace nt {

constexpr int kWave = 64;
constexpr int kMaxTopK = 32;  // the router's largest top-k (lane registers per token)

// ---------------------------------------------------------------- elements
// bf16 and fp16 are carried as raw 16-bit patterns; all arithmetic is fp32.

struct bf16 {
  uint16_t bits;
};
struct f16 {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even, NaN kept quiet: the rounding torch's .to(bfloat16)
// performs (c10::BFloat16 round_to_nearest_even).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// v_cvt_f16_f32 rounds to nearest even (the default MODE rounding).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <typename T>
struct elem;

template <>
struct elem<float> {
  using storage = float;
  __device__ static float load(float v) { return v; }
  __device__ static float store(float v) { return v; }
};
template <>
struct elem<double> {
  using storage = double;
  __device__ static float load(double v) { return static_cast<float>(v); }
  __device__ static double store(float v) { return static_cast<double>(v); }
};
template <>
struct elem<bf16> {
  using storage = uint16_t;
  __device__ static float load(uint16_t v) { return bf16_to_f32(v); }
  __device__ static uint16_t store(float v) { return f32_to_bf16(v); }
};
template <>
struct elem<f16> {
  using storage = uint16_t;
  __device__ static float load(uint16_t v) { return f16_to_f32(v); }
  __device__ static uint16_t store(float v) { return f32_to_f16(v); }
};

inline int dtype_bytes(int dtype) {
  switch (dtype) {
    case NT_F32: return 4;
    case NT_F64: return 8;
    case NT_F16: return 2;
    case NT_BF16: return 2;
    default: return 0;
  }
}

// Integer or integer-vector type of B bytes, for __builtin_nontemporal_load
// of B-byte chunks (the builtin takes scalar and vector types only).
template <int B>
struct nt_word;
// 32 and 64 bytes: instantiated by vector-width switches for wide element
// types, never selected at run time (16-byte accesses at most).
template <>
struct nt_word<64> {
  typedef uint32_t type __attribute__((ext_vector_type(16)));
};
template <>
struct nt_word<32> {
  typedef uint32_t type __attribute__((ext_vector_type(8)));
};
template <>
struct nt_word<16> {
  typedef uint32_t type __attribute__((ext_vector_type(4)));
};
template <>
struct nt_word<8> {
  typedef uint32_t type __attribute__((ext_vector_type(2)));
};
template <>
struct nt_word<4> {
  typedef uint32_t type;
};
template <>
struct nt_word<2> {
  typedef uint16_t type;
};
template <>
struct nt_word<1> {
  typedef uint8_t type;
};

// Non-temporal load of one V (any trivially copyable 1/2/4/8/16-byte type).
template <typename V>
__device__ __forceinline__ V load_nt(const V* p) {
  using W = typename nt_word<sizeof(V)>::type;
  return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const W*>(p)));
}

// ------------------------------------------------------------ wave64 helpers

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

__device__ __forceinline__ int popc64(uint64_t m) { return __popcll(m); }

// Butterfly sum over the 64 lanes; every lane receives the total. The
// association order is fixed, so the result is run-to-run deterministic.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Inclusive prefix sum across the wave (Hillis-Steele).
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    int u = __shfl_up(v, o, kWave);
    if (l >= o) v += u;
  }
  return v;
}

// Orders a wave's LDS writes before its later LDS reads by other lanes of the
// same wave (waits for outstanding LDS operations; no workgroup barrier, so
// it is safe after lanes or waves have diverged).
__device__ __forceinline__ void lds_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// Scheduling fence, then s_waitcnt vmcnt(0) (expcnt and lgkmcnt left at
// their gfx9 maxima): every vector memory operation the wave has issued has
// completed. The gathers and copies issue a batch of loads, call this once,
// and then store with no further wait: the compiler, unsure whether the
// stores under uniform branches were issued, would otherwise wait for a
// count that includes them before each next group of stores. A real wait
// instruction, so the compiler's own wait insertion accounts for it.
__device__ __forceinline__ void wait_batch_loads() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xF70);
}

// One round of a workgroup-wide stable counting rank. Every thread of the
// workgroup passes one item (key in [0, nkeys) when valid); the result is the
// number of valid items with the same key that precede it in thread order in
// this round plus in all earlier rounds (s_run[nkeys] carries those counts and
// is updated; s_wc[waves][nkeys] is scratch, zero on entry and on exit).
// Peers with equal keys inside a wave are found with one ballot per key bit.
// Contains workgroup barriers: all threads must call it. Returns -1 for an
// invalid item.
__device__ __forceinline__ int block_rank_round(int key, bool valid, int nbits, int nkeys,
                                                int32_t* s_run, int32_t* s_wc) {
  const int wave = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  uint64_t peers = ballot(valid);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool set = valid && ((key >> bit) & 1);
    const uint64_t bb = ballot(set);
    peers &= set ? bb : ~bb;
  }
  const int rank_w = popc64(peers & lanemask_lt());
  if (valid && rank_w == 0) s_wc[wave * nkeys + key] = popc64(peers);
  __syncthreads();
  int q = -1;
  if (valid) {
    q = s_run[key] + rank_w;
    for (int w2 = 0; w2 < wave; ++w2) q += s_wc[w2 * nkeys + key];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nkeys; e += blockDim.x) {
    int add = 0;
    for (int w2 = 0; w2 < nwaves; ++w2) {
      add += s_wc[w2 * nkeys + e];
      s_wc[w2 * nkeys + e] = 0;
    }
    s_run[e] += add;
  }
  __syncthreads();
  return q;
}

// Round a non-negative size up to a multiple of a.
__host__ __device__ constexpr int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }
__host__ __device__ constexpr int64_t ceil_div(int64_t x, int64_t a) { return (x + a - 1) / a; }

inline int launch_status() { return hipGetLastError() == hipSuccess ? NT_OK : NT_ERR_LAUNCH; }

}  // namespace nt
