// Expert counting and top-k token packing (dispatch) for gfx950.
//
// Three stream-ordered launches, no host synchronisation, no atomics on the
// packed order:
//   1. hist_kernel   one workgroup per block of TB tokens builds an LDS
//                    histogram of its assignments over the E experts and
//                    stores it expert-major: hist[e*nb + b].
//   2. scan_kernel   one workgroup per expert turns hist[e, :] into an
//                    exclusive scan over blocks and writes counts[e] (and the
//                    reference's cursor post-state).
//   3. pack_rows_kernel  one workgroup per token block ranks its assignments
//                    within the block (wave64 ballots over the bits of the
//                    expert id give each lane its same-expert peers; a small
//                    LDS table carries counts across waves and rounds), adds
//                    the block's base, then copies every token row once from
//                    X into its k packed slots with 16-byte accesses.
// Packed order is the stable counting sort of the flat assignment index by
// expert: exactly the order of the reference torch backend
// (src/model/torch_backend.py:58-66), deterministic run to run.
#include <mutex>

#include "common.hpp"

namespace nt {
namespace {

constexpr int kDispatchThreads = 256;
constexpr int kDispatchWaves = kDispatchThreads / kWave;

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// hist[e*nb + b] = #{ assignments of tokens [b*TB, b*TB+TB) with expert e,
//                     token unmasked }.
__global__ void __launch_bounds__(kDispatchThreads)
hist_kernel(const int32_t* __restrict__ topk, const int32_t* __restrict__ mask, int64_t T,
            int32_t k, int32_t E, int32_t TB, int32_t nb, int32_t* __restrict__ hist) {
  extern __shared__ int32_t s_hist[];
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e < E; e += blockDim.x) s_hist[e] = 0;
  __syncthreads();
  const int64_t tok0 = (int64_t)b * TB;
  const int64_t ntok = min((int64_t)TB, T - tok0);
  const int64_t na = ntok * k;
  const int64_t f0 = tok0 * k;
  for (int64_t i = threadIdx.x; i < na; i += blockDim.x) {
    const int32_t e = topk[f0 + i];
    bool ok = e >= 0 && e < E;
    if (mask != nullptr) ok = ok && mask[tok0 + i / k] != 0;
    if (ok) atomicAdd(&s_hist[e], 1);  // integer: order-independent
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) hist[(int64_t)e * nb + b] = s_hist[e];
}

// Workgroup e: scan[e, 0..nb) = exclusive scan of hist[e, 0..nb),
// counts[e] = total. `scan` may be `hist` itself (in place); the counted
// dispatch scans into a region of its own, so the per-block counts the
// router left in the workspace survive the call. With a cursor: base[e] =
// cursor[e]; cursor[e] += total (the state the reference's atomic cursor is
// left in, csrc/kernels/pack_tokens.cu:37).
__global__ void __launch_bounds__(kDispatchThreads)
scan_kernel(const int32_t* hist, int32_t* scan, int32_t nb, int32_t* __restrict__ counts,
            int32_t* __restrict__ cursor, int32_t* __restrict__ base) {
  __shared__ int32_t s_wsum[kDispatchWaves];
  __shared__ int32_t s_carry;
  const int e = blockIdx.x;
  const int32_t* h = hist + (int64_t)e * nb;
  int32_t* o = scan + (int64_t)e * nb;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (int start = 0; start < nb; start += kDispatchThreads) {
    const int i = start + threadIdx.x;
    const int v = i < nb ? h[i] : 0;
    const int incl = wave_incl_scan(v);
    if (lane == kWave - 1) s_wsum[wave] = incl;
    __syncthreads();
    int before = s_carry;
    for (int w = 0; w < wave; ++w) before += s_wsum[w];
    if (i < nb) o[i] = before + incl - v;
    __syncthreads();
    if (threadIdx.x == 0) {
      int tot = 0;
      for (int w = 0; w < kDispatchWaves; ++w) tot += s_wsum[w];
      s_carry += tot;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const int total = s_carry;
    if (counts != nullptr) counts[e] = total;
    if (cursor != nullptr) {
      const int c = cursor[e];
      base[e] = c;
      cursor[e] = c + total;
    }
  }
}

// Long rows: each lane loads up to kLongRowBatch 16-byte vectors of a row
// before it stores any (measured cold: C4 8 KiB rows 89 -> 78 us, C5 4 KiB
// rows 555 -> 497 us against one vector at a time; with the long-row
// instantiation at 8 waves per SIMD, C4 78 -> 76 us, and 4 or 16 vectors
// the same).
constexpr int kLongRowBatch = 8;

template <typename V>
__device__ __forceinline__ void copy_row_to_slots(const V* __restrict__ src, V* __restrict__ dst,
                                                  int64_t nv, const int32_t* slots, int k) {
  const int lane = lane_id();
  for (int64_t c0 = lane; c0 < nv; c0 += (int64_t)kWave * kLongRowBatch) {
    V v[kLongRowBatch];
#pragma unroll
    for (int u = 0; u < kLongRowBatch; ++u) {
      const int64_t c = c0 + (int64_t)u * kWave;
      if (c < nv) v[u] = load_nt(src + c);  // each token row is read once
    }
#pragma unroll
    for (int u = 0; u < kLongRowBatch; ++u) {
      const int64_t c = c0 + (int64_t)u * kWave;
      if (c >= nv) break;
      for (int j = 0; j < k; ++j) {
        const int32_t p = slots[j];
        if (p >= 0) dst[(int64_t)p * nv + c] = v[u];
      }
    }
  }
}

// The same copy for 16-byte vectors and k <= kSlotRegs: the token's slots
// are read once into scalar registers, every load of a batch of LB vectors
// per lane is issued before the first store (a vector beyond the row loads
// the batch's first again and is not stored), and one wait covers the batch
// (wait_batch_loads). Before, the stores of each vector waited for those of
// the one before (the wait count also covers stores).
constexpr int kSlotRegs = 8;

template <typename V, int LB>
__device__ __forceinline__ void copy_row_to_slot_regs(const V* __restrict__ src,
                                                      V* __restrict__ dst, int64_t nv,
                                                      const int32_t* slots, int k) {
  int32_t ps[kSlotRegs];
#pragma unroll
  for (int j = 0; j < kSlotRegs; ++j) ps[j] = j < k ? __builtin_amdgcn_readfirstlane(slots[j]) : -1;
  const int lane = lane_id();
  for (int64_t c0 = lane; c0 < nv; c0 += (int64_t)kWave * LB) {
    V v[LB];
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int64_t c = c0 + (int64_t)u * kWave;
      v[u] = load_nt(src + (c < nv ? c : c0));  // each token row is read once
    }
    wait_batch_loads();
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int64_t c = c0 + (int64_t)u * kWave;
      if (c >= nv) break;
#pragma unroll
      for (int j = 0; j < kSlotRegs; ++j)
        if (ps[j] >= 0) dst[(int64_t)ps[j] * nv + c] = v[u];
    }
  }
}

constexpr int kRowBatch = 16;  // rows in flight per wave in the short-row copy

// Rank, place and copy. base_mode 0: base[e] comes from `base` (cursor copy);
// base_mode 1: base[e] = exclusive scan of counts (offsets), written to
// `offsets` by workgroup 0; `hist` holds the per-expert exclusive scans over
// blocks (scan_kernel). base_mode 2 (no scan launch): `hist` holds the raw
// per-block counts; every workgroup sums expert e's row of it (wave e mod 4)
// into its total and the part before this block, and workgroup 0 writes
// counts and offsets.
// SHORT: the instantiation for rows of one 16-byte vector per lane or less
// (its 16-row batches hold 128 registers, which would cap the long-row copy
// at two waves per SIMD).
template <typename V, bool SHORT>
__global__ void __launch_bounds__(kDispatchThreads)
pack_rows_kernel(const V* __restrict__ X, const float* __restrict__ w,
                 const int32_t* __restrict__ topk, int64_t T, int32_t k, int32_t E,
                 int32_t nbits, int32_t TB, int32_t nb, int64_t nv, int64_t A_cap,
                 const int32_t* __restrict__ hist, int base_mode,
                 const int32_t* __restrict__ base, int32_t* __restrict__ counts,
                 int32_t* __restrict__ offsets, V* __restrict__ packed_X,
                 int32_t* __restrict__ token_id, int32_t* __restrict__ expert,
                 float* __restrict__ packed_w, int32_t* __restrict__ inv) {
  extern __shared__ int32_t smem[];
  int32_t* s_base = smem;                 // [E]
  int32_t* s_run = s_base + E;            // [E]
  int32_t* s_wc = s_run + E;              // [waves][E]
  int32_t* s_pos = s_wc + kDispatchWaves * E;  // [TB*k]

  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;

  const int64_t tok0 = (int64_t)b * TB;
  const int ntok = (int)min((int64_t)TB, T - tok0);
  const int na = ntok * k;
  const int64_t f0 = tok0 * k;

  // Short rows (one 16-byte vector per lane): the wave's first kRowBatch
  // token rows are loaded before the bases and the ranking, so their latency
  // hides behind them; only the store addresses depend on the ranks.
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  constexpr bool kVec16 = sizeof(V) == 16 && SHORT;
  const bool short_rows = kVec16 && nv > 0 && nv <= kWave;
  const bool on = lane < nv;
  u32x4 pre[kRowBatch];
  if (short_rows) {
    const u32x4* src = reinterpret_cast<const u32x4*>(X);
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int tt = wave + u * kDispatchWaves;
      if (on && tt < ntok) pre[u] = load_nt(src + (tok0 + tt) * nv + lane);
    }
  }

  // Per-expert base of this block.
  if (base_mode == 0) {
    for (int e = tid; e < E; e += kDispatchThreads) s_base[e] = base[e];
  } else if (base_mode == 2) {
    for (int e = wave; e < E; e += kDispatchWaves) {
      const int32_t* h = hist + (int64_t)e * nb;
      int tot = 0, before = 0;
      // Eight loads in flight per lane (the entries are L2-resident).
      for (int i0 = 0; i0 < nb; i0 += 8 * kWave) {
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = i0 + u * kWave + lane;
          v[u] = i < nb ? h[i] : 0;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int i = i0 + u * kWave + lane;
          tot += v[u];
          before += i < b ? v[u] : 0;
        }
      }
      tot = wave_sum_int(tot);
      before = wave_sum_int(before);
      if (lane == 0) {
        s_run[e] = tot;
        s_base[e] = before;
      }
    }
    __syncthreads();
    if (wave == 0) {
      int carry = 0;
      for (int s0 = 0; s0 < E; s0 += kWave) {
        const int e = s0 + lane;
        const int v = e < E ? s_run[e] : 0;
        const int incl = wave_incl_scan(v);
        if (e < E) {
          s_base[e] += carry + incl - v;
          if (b == 0) {
            counts[e] = v;
            offsets[e] = carry + incl - v;
          }
        }
        carry += __shfl(incl, kWave - 1, kWave);
      }
      if (b == 0 && lane == 0) offsets[E] = carry;
    }
    __syncthreads();
  } else {
    // Exclusive scan of counts over experts (E <= NT_MAX_EXPERTS) in s_base.
    for (int e = tid; e < E; e += kDispatchThreads) s_base[e] = counts[e];
    __syncthreads();
    if (wave == 0) {
      int carry = 0;
      for (int s = 0; s < E; s += kWave) {
        const int e = s + lane;
        const int v = e < E ? s_base[e] : 0;
        const int incl = wave_incl_scan(v);
        if (e < E) s_base[e] = carry + incl - v;
        carry += __shfl(incl, kWave - 1, kWave);
      }
      if (b == 0 && offsets != nullptr) {
        for (int e = lane; e < E; e += kWave) offsets[e] = s_base[e];
        if (lane == 0) offsets[E] = carry;
      }
    }
    __syncthreads();
  }
  for (int e = tid; e < E; e += kDispatchThreads) {
    if (base_mode != 2) s_base[e] += hist[(int64_t)e * nb + b];
    s_run[e] = 0;
  }
  for (int i = tid; i < kDispatchWaves * E; i += kDispatchThreads) s_wc[i] = 0;
  __syncthreads();


  // Stable rank of each assignment among same-expert assignments of the block.
  for (int r = 0; r < na; r += kDispatchThreads) {
    const int i = r + tid;
    const int32_t e = i < na ? topk[f0 + i] : -1;
    const bool valid = e >= 0 && e < E;
    const int q = block_rank_round(e, valid, nbits, E, s_run, s_wc);
    if (i < na) {
      int32_t p = -1;
      if (valid) {
        p = s_base[e] + q;
        if (p < 0 || (int64_t)p >= A_cap) p = -1;
      }
      s_pos[i] = p;
    }
  }
  __syncthreads();  // s_pos complete before other threads read it

  // Metadata: one thread per assignment.
  for (int i = tid; i < na; i += kDispatchThreads) {
    const int32_t p = s_pos[i];
    const int64_t f = f0 + i;
    if (inv != nullptr) inv[f] = p;
    if (p >= 0) {
      token_id[p] = (int32_t)(tok0 + i / k);
      expert[p] = topk[f];
      packed_w[p] = w[f];
    }
  }

  // Rows: each wave copies whole token rows, read once, written k times.
  if (nv <= 0) return;
  if constexpr (kVec16) {
    if (short_rows) {
      // One vector per lane per row: kRowBatch rows are loaded before any is
      // stored, so a wave waits for memory once per batch rather than once
      // per row. The first batch was loaded before the ranking.
      const u32x4* src = reinterpret_cast<const u32x4*>(X);
      u32x4* dst = reinterpret_cast<u32x4*>(packed_X);
      for (int t = wave; t < ntok; t += kRowBatch * kDispatchWaves) {
        u32x4 v[kRowBatch];
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) {
          const int tt = t + u * kDispatchWaves;
          if (t == wave) v[u] = pre[u];
          else if (on && tt < ntok) v[u] = load_nt(src + (tok0 + tt) * nv + lane);
        }
#pragma unroll
        for (int u = 0; u < kRowBatch; ++u) {
          const int tt = t + u * kDispatchWaves;
          if (on && tt < ntok) {
            for (int j = 0; j < k; ++j) {
              const int32_t p = s_pos[tt * k + j];
              if (p >= 0) dst[(int64_t)p * nv + lane] = v[u];
            }
          }
        }
      }
      return;
    }
  }
  if (sizeof(V) == 16 && k <= kSlotRegs) {
    // 8 vectors per lane per batch from rows of 4 KiB up, 4 for rows up to
    // 4 KiB, 2 for rows up to 2 KiB (one batch covers the row; fewer
    // vectors would issue loads that only repeat the first)
    for (int t = wave; t < ntok; t += kDispatchWaves) {
      const V* src = X + (tok0 + t) * nv;
      if (nv > (int64_t)kWave * kLongRowBatch / 2)
        copy_row_to_slot_regs<V, kLongRowBatch>(src, packed_X, nv, s_pos + t * k, k);
      else if (nv > (int64_t)kWave * kLongRowBatch / 4)
        copy_row_to_slot_regs<V, kLongRowBatch / 2>(src, packed_X, nv, s_pos + t * k, k);
      else
        copy_row_to_slot_regs<V, kLongRowBatch / 4>(src, packed_X, nv, s_pos + t * k, k);
    }
    return;
  }
  for (int t = wave; t < ntok; t += kDispatchWaves) {
    copy_row_to_slots<V>(X + (tok0 + t) * nv, packed_X, nv, s_pos + t * k, k);
  }
}

struct PackPlan {
  int32_t TB;
  int32_t nb;
  int64_t row_bytes;
};

constexpr int64_t kMinLongRowBlocks = 512;

PackPlan plan_pack(int64_t T, int32_t k, int64_t row_bytes) {
  // Rows of 2 KiB and more: 32 tokens per block (measured cold against 16
  // and 8: C4 75.6 -> 74.5 us, C5 499 -> 493 us; 64 the same as 32).
  int32_t tb = row_bytes >= 2048 ? 32 : 64;
  while (tb > 1 && (int64_t)tb * k > 2048) tb >>= 1;
  // Long rows (beyond one 16-byte vector per lane) with few tokens: at least
  // two blocks per CU (measured cold, C1 at 2 KiB rows: 22.6 -> 17.2 us).
  // Short rows keep their blocks: each wave batches 16 of them, and smaller
  // blocks were slower (C2 26 -> 34 us).
  if (row_bytes > 1024)
    while (tb > 4 && ceil_div(T, (int64_t)tb) < kMinLongRowBlocks) tb >>= 1;
  PackPlan p;
  p.TB = tb;
  p.nb = (int32_t)ceil_div(T, tb);
  p.row_bytes = row_bytes;
  return p;
}

size_t hist_bytes(const PackPlan& p, int32_t E) {
  return (size_t)round_up((int64_t)E * p.nb * 4, 256);
}

// [hist | base | scan]: the per-block histogram, the per-expert bases of
// nt_pack_tokens, and the counted dispatch's scan of the histogram (kept
// apart from it, so that the histogram is only read).
size_t dispatch_ws_bytes(const PackPlan& p, int32_t E) {
  return 2 * hist_bytes(p, E) + (size_t)round_up((int64_t)E * 4, 256);
}
int32_t* scan_region(void* ws, const PackPlan& p, int32_t E) {
  return reinterpret_cast<int32_t*>(static_cast<char*>(ws) + hist_bytes(p, E) +
                                    (size_t)round_up((int64_t)E * 4, 256));
}

int nbits_for(int32_t E) {
  int n = 0;
  while ((1 << n) < E) ++n;
  return n;
}

int check_common(int64_t T, int32_t k, int32_t E) {
  if (T < 0 || k < 1 || E < 1) return NT_ERR_INVALID_ARG;
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
  if (T * (int64_t)k > INT32_MAX) return NT_ERR_TOO_LARGE;
  return NT_OK;
}

size_t pack_lds_bytes(const PackPlan& p, int32_t E, int32_t k) {
  return (size_t)(2 * E + kDispatchWaves * E + (int64_t)p.TB * k) * 4;
}

template <typename V>
int launch_pack_rows(const PackPlan& plan, const void* X, const float* w, const int32_t* topk,
                     int64_t T, int32_t k, int32_t E, const int32_t* hist, int base_mode,
                     const int32_t* base, int32_t* counts, int32_t* offsets,
                     void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                     int32_t* inv, hipStream_t stream) {
  const int64_t nv = plan.row_bytes / (int64_t)sizeof(V);
  const size_t lds = pack_lds_bytes(plan, E, k);
  auto kern = sizeof(V) == 16 && nv > 0 && nv <= kWave ? pack_rows_kernel<V, true>
                                                      : pack_rows_kernel<V, false>;
  hipLaunchKernelGGL(kern, dim3(plan.nb), dim3(kDispatchThreads), lds, stream,
                     static_cast<const V*>(X), w, topk, T, k, E, nbits_for(E), plan.TB, plan.nb,
                     nv, T * k, hist, base_mode, base, counts, offsets, static_cast<V*>(packed_X),
                     token_id, expert, packed_w, inv);
  return launch_status();
}

int pack_rows_dispatch(const PackPlan& plan, const void* X, void* packed_X, const float* w,
                       const int32_t* topk, int64_t T, int32_t k, int32_t E, const int32_t* hist,
                       int base_mode, const int32_t* base, int32_t* counts,
                       int32_t* offsets, int32_t* token_id, int32_t* expert, float* packed_w,
                       int32_t* inv, hipStream_t stream) {
  const uintptr_t align = reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(packed_X) |
                          static_cast<uintptr_t>(plan.row_bytes);
  if (align % 16 == 0)
    return launch_pack_rows<uint4>(plan, X, w, topk, T, k, E, hist, base_mode, base, counts,
                                   offsets, packed_X, token_id, expert, packed_w, inv, stream);
  if (align % 8 == 0)
    return launch_pack_rows<uint2>(plan, X, w, topk, T, k, E, hist, base_mode, base, counts,
                                   offsets, packed_X, token_id, expert, packed_w, inv, stream);
  if (align % 4 == 0)
    return launch_pack_rows<uint32_t>(plan, X, w, topk, T, k, E, hist, base_mode, base, counts,
                                      offsets, packed_X, token_id, expert, packed_w, inv, stream);
  if (align % 2 == 0)
    return launch_pack_rows<uint16_t>(plan, X, w, topk, T, k, E, hist, base_mode, base, counts,
                                      offsets, packed_X, token_id, expert, packed_w, inv, stream);
  return launch_pack_rows<uint8_t>(plan, X, w, topk, T, k, E, hist, base_mode, base, counts,
                                   offsets, packed_X, token_id, expert, packed_w, inv, stream);
}

int launch_hist_scan(const PackPlan& plan, const int32_t* topk, const int32_t* mask, int64_t T,
                     int32_t k, int32_t E, int32_t* hist, int32_t* counts, int32_t* cursor,
                     int32_t* base, hipStream_t stream) {
  if (plan.nb > 0) {
    hipLaunchKernelGGL(hist_kernel, dim3(plan.nb), dim3(kDispatchThreads), (size_t)E * 4, stream,
                       topk, mask, T, k, E, plan.TB, plan.nb, hist);
    int st = launch_status();
    if (st != NT_OK) return st;
  }
  hipLaunchKernelGGL(scan_kernel, dim3(E), dim3(kDispatchThreads), 0, stream, hist, hist,
                     plan.nb, counts, cursor, base);
  return launch_status();
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

size_t nt_dispatch_workspace_bytes(int64_t T, int32_t k, int32_t E, int64_t d, int dtype) {
  if (T < 0 || k < 1 || E < 1 || d < 0) return 0;
  const PackPlan p = plan_pack(T, k, d * dtype_bytes(dtype));
  return dispatch_ws_bytes(p, E);
}

int nt_count_experts(const int32_t* topk, const int32_t* mask, int64_t T, int32_t k, int32_t E,
                     int32_t* counts, void* ws, size_t ws_bytes, hipStream_t stream) {
  int st = check_common(T, k, E);
  if (st != NT_OK) return st;
  if (counts == nullptr || (T > 0 && topk == nullptr)) return NT_ERR_INVALID_ARG;
  const PackPlan plan = plan_pack(T, k, 0);
  if (ws == nullptr || ws_bytes < dispatch_ws_bytes(plan, E)) return NT_ERR_WORKSPACE;
  return launch_hist_scan(plan, topk, mask, T, k, E, static_cast<int32_t*>(ws), counts, nullptr,
                          nullptr, stream);
}

int nt_pack_tokens(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                   int32_t k, int64_t d, int32_t E, int32_t* cursor, void* packed_X,
                   int32_t* token_id, int32_t* expert, float* packed_w, int32_t* inv, void* ws,
                   size_t ws_bytes, hipStream_t stream) {
  int st = check_common(T, k, E);
  if (st != NT_OK) return st;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return NT_ERR_DTYPE;
  if (d < 0 || cursor == nullptr) return NT_ERR_INVALID_ARG;
  if (T > 0 && (X == nullptr && d > 0)) return NT_ERR_INVALID_ARG;
  if (T > 0 && (w == nullptr || topk == nullptr || token_id == nullptr || expert == nullptr ||
                packed_w == nullptr || (packed_X == nullptr && d > 0)))
    return NT_ERR_INVALID_ARG;
  const PackPlan plan = plan_pack(T, k, d * eb);
  if (ws == nullptr || ws_bytes < dispatch_ws_bytes(plan, E)) return NT_ERR_WORKSPACE;
  int32_t* hist = static_cast<int32_t*>(ws);
  int32_t* base = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + hist_bytes(plan, E));
  st = launch_hist_scan(plan, topk, nullptr, T, k, E, hist, nullptr, cursor, base, stream);
  if (st != NT_OK || plan.nb == 0) return st;
  return pack_rows_dispatch(plan, X, packed_X, w, topk, T, k, E, hist, 0, base, nullptr, nullptr,
                            token_id, expert, packed_w, inv, stream);
}

int32_t nt_dispatch_block_tokens(int64_t T, int32_t k, int64_t d, int dtype) {
  if (T < 0 || k < 1 || d < 0 || dtype_bytes(dtype) == 0) return 0;
  return plan_pack(T, k, d * dtype_bytes(dtype)).TB;
}

}  // extern "C"

namespace nt {
namespace {

// nt_dispatch / nt_dispatch_counted: counted = the per-block histogram is
// already in ws (written by nt_route_topk_count); otherwise hist_kernel
// builds it. Up to kFoldMaxEntries histogram entries (E * blocks: C1, C2 and
// C4 of the configs) the pack workgroups sum it themselves, each reading it
// whole from L2, instead of a scan launch.
constexpr int64_t kFoldMaxEntries = 8192;
int dispatch_impl(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                  int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                  void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                  int32_t* inv, void* ws, size_t ws_bytes, bool counted, hipStream_t stream) {
  int st = check_common(T, k, E);
  if (st != NT_OK) return st;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return NT_ERR_DTYPE;
  if (d < 0 || counts == nullptr || offsets == nullptr) return NT_ERR_INVALID_ARG;
  if (T > 0 && (w == nullptr || topk == nullptr || token_id == nullptr || expert == nullptr ||
                packed_w == nullptr || ((X == nullptr || packed_X == nullptr) && d > 0)))
    return NT_ERR_INVALID_ARG;
  const PackPlan plan = plan_pack(T, k, d * eb);
  if (ws == nullptr || ws_bytes < dispatch_ws_bytes(plan, E)) return NT_ERR_WORKSPACE;
  int32_t* hist = static_cast<int32_t*>(ws);
  // Small histograms are summed inside the pack (base_mode 2): no scan launch.
  const bool fold = plan.nb > 0 && (int64_t)E * plan.nb <= kFoldMaxEntries;
  if (fold) {
    st = NT_OK;
    if (!counted) {
      hipLaunchKernelGGL(hist_kernel, dim3(plan.nb), dim3(kDispatchThreads), (size_t)E * 4,
                         stream, topk, nullptr, T, k, E, plan.TB, plan.nb, hist);
      st = launch_status();
    }
  } else if (counted) {
    // The router's counts stay as they are: a second call on the same
    // workspace sees the same histogram.
    int32_t* scan = scan_region(ws, plan, E);
    hipLaunchKernelGGL(scan_kernel, dim3(E), dim3(kDispatchThreads), 0, stream, hist, scan,
                       plan.nb, counts, nullptr, nullptr);
    st = launch_status();
    hist = scan;
  } else {
    st = launch_hist_scan(plan, topk, nullptr, T, k, E, hist, counts, nullptr, nullptr, stream);
  }
  if (st != NT_OK) return st;
  if (plan.nb == 0) {
    // No tokens: offsets are all zero.
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(kDispatchThreads), 0, stream, offsets,
                       (int64_t)E + 1, 0);
    return launch_status();
  }
  return pack_rows_dispatch(plan, X, packed_X, w, topk, T, k, E, hist, fold ? 2 : 1, nullptr,
                            counts, offsets, token_id, expert, packed_w, inv, stream);
}

}  // namespace
}  // namespace nt

extern "C" {

int nt_dispatch(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w, int32_t* inv,
                void* ws, size_t ws_bytes, hipStream_t stream) {
  return dispatch_impl(dtype, X, w, topk, T, k, d, E, counts, offsets, packed_X, token_id,
                       expert, packed_w, inv, ws, ws_bytes, false, stream);
}

int nt_dispatch_counted(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                        int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                        void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                        int32_t* inv, void* ws, size_t ws_bytes, hipStream_t stream) {
  return dispatch_impl(dtype, X, w, topk, T, k, d, E, counts, offsets, packed_X, token_id,
                       expert, packed_w, inv, ws, ws_bytes, true, stream);
}

}  // extern "C"

// ------------------------------------------------ no-allocation dispatch
//
// nt_dispatch with its workspace (the per-block expert histogram and the
// per-expert bases, dispatch_ws_bytes) in a device array the library owns,
// for callers that cannot allocate: code under graph capture, tight serving
// loops. Each GPU the library runs on holds its own copy of the array until
// the process ends. Every call on a GPU shares that GPU's copy and leaves its
// contents behind; nothing in it needs to start at zero (the histogram kernel
// writes every entry the scan and the pack read), but two calls that overlap
// on one GPU (different streams, no ordering between them) race on it.
static __device__ __align__(256) unsigned char scratch[NT_NOALLOC_SCRATCH_BYTES];

namespace nt {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the device `stream` belongs to. The
// array's host-side name is only a handle: the address comes from
// hipGetSymbolAddress, called once per device with that device current.
int scratch_on(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return NT_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return NT_ERR_LAUNCH;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return NT_ERR_LAUNCH;
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (err != hipSuccess || ptr == nullptr) return NT_ERR_LAUNCH;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return NT_OK;
}

}  // namespace
}  // namespace nt

extern "C" {

int nt_dispatch_noalloc(int dtype, const void* X, const float* w, const int32_t* topk, int64_t T,
                        int32_t k, int64_t d, int32_t E, int32_t* counts, int32_t* offsets,
                        void* packed_X, int32_t* token_id, int32_t* expert, float* packed_w,
                        int32_t* inv, hipStream_t stream) {
  int st = check_common(T, k, E);
  if (st != NT_OK) return st;
  const int eb = dtype_bytes(dtype);
  if (eb == 0) return NT_ERR_DTYPE;
  if (d < 0) return NT_ERR_INVALID_ARG;
  // The same workspace nt_dispatch would take; beyond the array it is an error.
  const size_t need = dispatch_ws_bytes(plan_pack(T, k, d * eb), E);
  if (need > (size_t)NT_NOALLOC_SCRATCH_BYTES) return NT_ERR_SCRATCH;
  void* ws = nullptr;
  st = scratch_on(stream, &ws);
  if (st != NT_OK) return st;
  return dispatch_impl(dtype, X, w, topk, T, k, d, E, counts, offsets, packed_X, token_id, expert,
                       packed_w, inv, ws, (size_t)NT_NOALLOC_SCRATCH_BYTES, false, stream);
}

}  // extern "C"
