// Weighted combine (forward and backward) and pack backward for gfx950.
//
// All three are per-token gathers: one wave owns one token, takes the packed
// rows that belong to it in ascending packed index, and accumulates in fp32
// in that fixed order. No floating-point atomics, so results are identical
// run to run, and the combine equals a sequential index_add_ in packed
// order bit for bit (products are rounded before the add: no FMA).
//
// The rows of a token come either from the inverse map written by the pack
// (inv[t*k + j] = packed slot of token t's j-th choice; the k slots are put
// in ascending order in LDS) or, on the reference's token-id surface, from a
// token CSR built here: rows per token (integer atomics) and their exclusive
// scan give each token's segment, and a stable LSD radix sort of the packed
// rows by token id (8-bit digits, workgroup-stable ranks from wave ballots)
// lays every segment out in ascending packed order, for any fan-in.
#include <algorithm>

#include "common.hpp"

namespace nt {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxSorted = 256;
// Tokens per wave of the small-fan-in inverse-map kernels (measured at
// d = 512, k = 2: one for the combine, two for the pack backward; one at
// k <= 8).
constexpr int kCombineU = 1;
constexpr int kPackBwdU = 2;
// Rows beyond one 16-byte vector per lane: one token per wave (measured
// cold, C4 8 KiB rows: 80 -> 75 us against two).
constexpr int kPackBwdULong = 1;
constexpr int64_t kLongRowBytes = 1024;
constexpr int fan_u(int kmax, int u) { return kmax <= 2 ? u : 1; }

template <typename S, int N>
struct alignas(sizeof(S) * N) vpack {
  S v[N];
};

// VE consecutive elements of type T, as floats. Every row these kernels read
// (packed rows, gradient rows) is read once: the load is non-temporal, so it
// does not displace lines other waves still need.
template <typename T, int VE>
__device__ __forceinline__ void load_vec(const typename elem<T>::storage* p, float (&out)[VE]) {
  using S = typename elem<T>::storage;
  using W = typename nt_word<sizeof(S) * VE>::type;
  const vpack<S, VE> v =
      __builtin_bit_cast(vpack<S, VE>, __builtin_nontemporal_load(reinterpret_cast<const W*>(p)));
#pragma unroll
  for (int i = 0; i < VE; ++i) out[i] = elem<T>::load(v.v[i]);
}

// The same load kept as the raw word (VE 16-bit elements take half the
// registers of VE floats), converted by unpack_vec where it is summed: the
// gathers that hold k rows in flight then keep their occupancy.
template <typename T, int VE>
using raw_vec = typename nt_word<sizeof(typename elem<T>::storage) * VE>::type;
template <typename T, int VE>
__device__ __forceinline__ raw_vec<T, VE> load_raw(const typename elem<T>::storage* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const raw_vec<T, VE>*>(p));
}
template <typename T, int VE>
__device__ __forceinline__ void unpack_vec(raw_vec<T, VE> w, float (&out)[VE]) {
  using S = typename elem<T>::storage;
  const vpack<S, VE> v = __builtin_bit_cast(vpack<S, VE>, w);
#pragma unroll
  for (int i = 0; i < VE; ++i) out[i] = elem<T>::load(v.v[i]);
}

// The small-fan-in gathers issue every row load of a pass before the first
// is used, then wait once for all of them (wait_batch_loads, a scheduling
// fence and a full wait): without the fence the compiler converts each row
// as it arrives and waits for it before issuing the next load, so a wave
// kept one row chunk in flight.
// A pass covers H consecutive 16-byte-per-lane chunks of each row: rows of
// several chunks (k <= 2) take kLongChunks per pass; a chunk beyond the row
// loads the pass's first chunk again and is discarded.
constexpr int kLongChunks = 4;

template <typename T, int VE>
__device__ __forceinline__ void store_vec(typename elem<T>::storage* p, const float (&in)[VE]) {
  using S = typename elem<T>::storage;
  vpack<S, VE> v;
#pragma unroll
  for (int i = 0; i < VE; ++i) v.v[i] = elem<T>::store(in[i]);
  *reinterpret_cast<vpack<S, VE>*>(p) = v;
}

// ----------------------------------------------------------- token lists

// List source: either CSR (start[t], start[t+1]) into `list`, or the inverse
// map (t*k .. t*k+k) of `inv`.
struct ListSrc {
  const int32_t* start;  // [T+1] or nullptr
  const int32_t* list;   // CSR entries or inv
  int32_t k;             // used when start == nullptr
  int64_t rows;          // packed rows; entries outside [0, rows) are skipped
};

// Packed rows of token t in ascending order. A CSR list is already sorted
// and is walked in place: returns -(length). An inverse-map row is compacted
// (dropping empty slots) and sorted into s_out (wave-private LDS of
// kMaxSorted ints): returns its count; a row longer than kMaxSorted (top-k
// above 256) is walked in place, in slot order.
__device__ int gather_sorted(const ListSrc& src, int64_t t, int32_t* s_in, int32_t* s_out,
                             int64_t* first) {
  const int lane = lane_id();
  int64_t b, n;
  if (src.start != nullptr) {
    b = src.start[t];
    n = src.start[t + 1] - b;
    *first = b;
    return -(int)n;
  }
  b = t * src.k;
  n = src.k;
  *first = b;
  if (n > kMaxSorted) return -(int)n;
  // Compact valid (>= 0) entries into s_in.
  int cnt = 0;
  for (int64_t base = 0; base < n; base += kWave) {
    const int64_t i = base + lane;
    const int32_t p = i < n ? src.list[b + i] : -1;
    const bool ok = p >= 0 && p < src.rows;
    const uint64_t m = ballot(ok);
    if (ok) s_in[cnt + popc64(m & lanemask_lt())] = p;
    cnt += popc64(m);
  }
  lds_wave_sync();
  // Rank each entry (ties broken by position, so the ranks form a permutation).
  for (int i = lane; i < cnt; i += kWave) {
    const int32_t pi = s_in[i];
    int r = 0;
    for (int m = 0; m < cnt; ++m) {
      const int32_t pm = s_in[m];
      r += (pm < pi) || (pm == pi && m < i);
    }
    s_out[r] = pi;
  }
  lds_wave_sync();
  return cnt;
}

__device__ __forceinline__ int32_t list_entry(const ListSrc& src, const int32_t* s_sorted, int n,
                                              int64_t first, int i) {
  if (n >= 0) return s_sorted[i];
  const int32_t p = src.list[first + i];
  return p < src.rows ? p : -1;
}

// --------------------------------------------------------- CSR building

__global__ void zero_i32(int32_t* __restrict__ p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

__global__ void token_count_kernel(const int32_t* __restrict__ token_id, int64_t A, int64_t T,
                                   int32_t* __restrict__ cnt) {
  for (int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; p < A;
       p += (int64_t)gridDim.x * blockDim.x) {
    const int32_t t = token_id[p];
    if (t >= 0 && t < T) atomicAdd(&cnt[t], 1);
  }
}

// One workgroup of 1024 threads: start[0..T] = exclusive scan of cnt; cnt is
// reset to zero for reuse as the fill cursor.
__global__ void __launch_bounds__(1024)
token_scan_kernel(int32_t* __restrict__ cnt, int64_t T, int32_t* __restrict__ start) {
  __shared__ int32_t s_wsum[16];
  __shared__ int32_t s_carry;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (int64_t s = 0; s < T; s += 1024) {
    const int64_t i = s + threadIdx.x;
    const int v = i < T ? cnt[i] : 0;
    const int incl = wave_incl_scan(v);
    if (lane == kWave - 1) s_wsum[wave] = incl;
    __syncthreads();
    int before = s_carry;
    for (int w = 0; w < wave; ++w) before += s_wsum[w];
    if (i < T) {
      start[i] = before + incl - v;
      cnt[i] = 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int tot = 0;
      for (int w = 0; w < 16; ++w) tot += s_wsum[w];
      s_carry += tot;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) start[T] = s_carry;
}

// Stable LSD radix sort of the packed rows by token id, 8 bits per pass.
// Keys outside [0, T) are mapped to T and sort last (outside every segment).
constexpr int kRadixBits = 8;
constexpr int kRadixBins = 1 << kRadixBits;
constexpr int kRadixChunk = 1024;  // rows per workgroup

__device__ __forceinline__ int radix_key(int32_t v, int64_t T) {
  return (v >= 0 && v < T) ? v : (int)T;
}

__global__ void __launch_bounds__(256)
radix_hist_kernel(const int32_t* __restrict__ keys, int64_t n, int64_t T, int shift, int32_t nb,
                  int32_t* __restrict__ hist) {
  __shared__ int32_t s_h[kRadixBins];
  s_h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t i0 = (int64_t)blockIdx.x * kRadixChunk;
  for (int r = threadIdx.x; r < kRadixChunk; r += 256) {
    const int64_t i = i0 + r;
    if (i < n) atomicAdd(&s_h[(radix_key(keys[i], T) >> shift) & (kRadixBins - 1)], 1);
  }
  __syncthreads();
  hist[(int64_t)threadIdx.x * nb + blockIdx.x] = s_h[threadIdx.x];
}

// One workgroup: exclusive scan in place of hist[0..count) (digit-major).
__global__ void __launch_bounds__(1024)
radix_scan_kernel(int32_t* __restrict__ hist, int64_t count) {
  __shared__ int32_t s_wsum[16];
  __shared__ int32_t s_carry;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  if (threadIdx.x == 0) s_carry = 0;
  __syncthreads();
  for (int64_t s0 = 0; s0 < count; s0 += 1024) {
    const int64_t i = s0 + threadIdx.x;
    const int v = i < count ? hist[i] : 0;
    const int incl = wave_incl_scan(v);
    if (lane == kWave - 1) s_wsum[wave] = incl;
    __syncthreads();
    int before = s_carry;
    for (int w = 0; w < wave; ++w) before += s_wsum[w];
    if (i < count) hist[i] = before + incl - v;
    __syncthreads();
    if (threadIdx.x == 0) {
      int tot = 0;
      for (int w = 0; w < 16; ++w) tot += s_wsum[w];
      s_carry += tot;
    }
    __syncthreads();
  }
}

// vals_in == nullptr: the values are the row indices themselves.
__global__ void __launch_bounds__(256)
radix_scatter_kernel(const int32_t* __restrict__ keys_in, const int32_t* __restrict__ vals_in,
                     int64_t n, int64_t T, int shift, int32_t nb,
                     const int32_t* __restrict__ hist, int32_t* __restrict__ keys_out,
                     int32_t* __restrict__ vals_out) {
  __shared__ int32_t s_base[kRadixBins];
  __shared__ int32_t s_run[kRadixBins];
  __shared__ int32_t s_wc[4 * kRadixBins];
  s_base[threadIdx.x] = hist[(int64_t)threadIdx.x * nb + blockIdx.x];
  s_run[threadIdx.x] = 0;
  for (int i = threadIdx.x; i < 4 * kRadixBins; i += 256) s_wc[i] = 0;
  __syncthreads();
  const int64_t i0 = (int64_t)blockIdx.x * kRadixChunk;
  for (int r = 0; r < kRadixChunk; r += 256) {
    const int64_t i = i0 + r + threadIdx.x;
    const bool valid = i < n;
    const int key = valid ? radix_key(keys_in[i], T) : 0;
    const int digit = (key >> shift) & (kRadixBins - 1);
    const int q = block_rank_round(digit, valid, kRadixBits, kRadixBins, s_run, s_wc);
    if (valid) {
      const int64_t pos = s_base[digit] + q;
      keys_out[pos] = key;
      vals_out[pos] = vals_in != nullptr ? vals_in[i] : (int32_t)i;
    }
  }
}

struct CsrWs {
  int32_t* cnt;    // [T]
  int32_t* start;  // [T+1]
  int32_t* keys[2];  // [A] each
  int32_t* vals[2];  // [A] each
  int32_t* hist;   // [256 * nb]
};

int radix_passes(int64_t T) {
  int bits = 1;
  while (bits < 62 && ((int64_t)1 << bits) <= T) ++bits;  // T itself must fit (sentinel)
  return (bits + kRadixBits - 1) / kRadixBits;
}

size_t csr_bytes(int64_t A, int64_t T) {
  const int64_t nb = ceil_div(std::max<int64_t>(A, 1), kRadixChunk);
  return (size_t)(round_up(T * 4, 256) + round_up((T + 1) * 4, 256) + 4 * round_up(A * 4, 256) +
                  round_up(kRadixBins * nb * 4, 256));
}

CsrWs carve_csr(void* ws, int64_t A, int64_t T) {
  char* c = static_cast<char*>(ws);
  CsrWs r;
  r.cnt = reinterpret_cast<int32_t*>(c);
  c += round_up(T * 4, 256);
  r.start = reinterpret_cast<int32_t*>(c);
  c += round_up((T + 1) * 4, 256);
  for (int i = 0; i < 2; ++i) {
    r.keys[i] = reinterpret_cast<int32_t*>(c);
    c += round_up(A * 4, 256);
    r.vals[i] = reinterpret_cast<int32_t*>(c);
    c += round_up(A * 4, 256);
  }
  r.hist = reinterpret_cast<int32_t*>(c);
  return r;
}

// Builds start[0..T] and returns the sorted list (rows of each token in
// ascending packed order) through *list.
int build_csr(const int32_t* token_id, int64_t A, int64_t T, const CsrWs& c, const int32_t** list,
              hipStream_t s) {
  const int grid_t = (int)std::min<int64_t>(ceil_div(std::max<int64_t>(T, 1), 256), 4096);
  const int grid_a = (int)std::min<int64_t>(ceil_div(std::max<int64_t>(A, 1), 256), 4096);
  hipLaunchKernelGGL(zero_i32, dim3(grid_t), dim3(256), 0, s, c.cnt, T);
  hipLaunchKernelGGL(token_count_kernel, dim3(grid_a), dim3(256), 0, s, token_id, A, T, c.cnt);
  hipLaunchKernelGGL(token_scan_kernel, dim3(1), dim3(1024), 0, s, c.cnt, T, c.start);
  int st = launch_status();
  if (st != NT_OK) return st;
  *list = nullptr;
  if (A == 0) return NT_OK;
  const int32_t nb = (int32_t)ceil_div(A, kRadixChunk);
  const int passes = radix_passes(T);
  const int32_t* kin = token_id;
  const int32_t* vin = nullptr;
  for (int pass = 0; pass < passes; ++pass) {
    const int shift = pass * kRadixBits;
    int32_t* kout = c.keys[pass & 1];
    int32_t* vout = c.vals[pass & 1];
    hipLaunchKernelGGL(radix_hist_kernel, dim3(nb), dim3(256), 0, s, kin, A, T, shift, nb, c.hist);
    hipLaunchKernelGGL(radix_scan_kernel, dim3(1), dim3(1024), 0, s, c.hist,
                       (int64_t)kRadixBins * nb);
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(nb), dim3(256), 0, s, kin, vin, A, T, shift, nb,
                       c.hist, kout, vout);
    st = launch_status();
    if (st != NT_OK) return st;
    kin = kout;
    vin = vout;
  }
  *list = vin;
  return NT_OK;
}

// ------------------------------------------------------------- combine fwd

// out[t, :] = sum_{p in rows(t), ascending} fl(w[p] * float(y[p, :])).
template <typename T, typename TO, int VE>
__global__ void __launch_bounds__(kThreads)
combine_kernel(const typename elem<T>::storage* __restrict__ y, ListSrc src,
               const float* __restrict__ w, int64_t T_, int64_t d,
               typename elem<TO>::storage* __restrict__ out) {
  __shared__ int32_t s_lists[kWaves][2][kMaxSorted];
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kWaves + wave;
  if (t >= T_) return;
  int64_t first;
  const int n = gather_sorted(src, t, s_lists[wave][0], s_lists[wave][1], &first);
  const int nn = n >= 0 ? n : -n;
  const int32_t* sorted = s_lists[wave][1];
  for (int64_t h = (int64_t)lane * VE; h < d; h += (int64_t)kWave * VE) {
    float acc[VE];
#pragma unroll
    for (int v = 0; v < VE; ++v) acc[v] = 0.f;
    for (int i = 0; i < nn; ++i) {
      const int32_t p = list_entry(src, sorted, n, first, i);
      if (p < 0) continue;
      const float wp = w[p];
      float x[VE];
      load_vec<T, VE>(y + (int64_t)p * d + h, x);
      // The product is rounded to fp32 before the add (no fused multiply-add),
      // exactly as a sequential index_add_ of a pre-multiplied tensor.
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int v = 0; v < VE; ++v) acc[v] = acc[v] + wp * x[v];
      }
    }
    store_vec<TO, VE>(out + t * d + h, acc);
  }
}

// Inverse-map form for small fan-in (k <= KMAX): a wave serves U tokens
// at once. Each token's k slots are loaded by one segment of 64/U lanes,
// broadcast and sorted ascending in registers; then every row load of the U
// tokens is issued before the ordered accumulation, so a wave keeps U * k
// row loads in flight. Same arithmetic and order as combine_kernel.
template <int KMAX, int U>
__device__ __forceinline__ void sorted_slots(const int32_t* __restrict__ inv, int64_t t0,
                                             int64_t T_, int32_t k, int32_t& mine,
                                             int32_t (&p)[U][KMAX], int (&n)[U]) {
  constexpr int kSeg = kWave / U;
  static_assert(KMAX <= kSeg, "a token's slots fit its lane segment");
  const int lane = lane_id();
  const int64_t rows = T_ * k;
  const int64_t tl = t0 + lane / kSeg;
  const int jl = lane % kSeg;
  mine = (jl < k && tl < T_) ? inv[tl * k + jl] : -1;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    n[u] = 0;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      const int32_t v = __shfl(mine, u * kSeg + j, kWave);
      const bool ok = j < k && v >= 0 && v < rows;
      p[u][j] = ok ? v : INT32_MAX;
      n[u] += ok;
    }
#pragma unroll
    for (int i = 0; i < KMAX - 1; ++i)
#pragma unroll
      for (int j = 0; j < KMAX - 1 - i; ++j) {
        const int32_t a = p[u][j], b = p[u][j + 1];
        p[u][j] = a < b ? a : b;
        p[u][j + 1] = a < b ? b : a;
      }
    // Every lane computed the same slots from the same broadcasts: moving
    // them to scalar registers makes the row loads' conditions uniform, so
    // the loads are issued back to back instead of one per branch.
    n[u] = __builtin_amdgcn_readfirstlane(n[u]);
#pragma unroll
    for (int j = 0; j < KMAX; ++j) p[u][j] = __builtin_amdgcn_readfirstlane(p[u][j]);
  }
}

// A row every lane may load for a slot that has none: the first valid slot
// of the wave's tokens (-1 when none has one). Loading it for the empty
// slots lets every row load of a pass be issued unconditionally, back to
// back; the empty slots' data is never used.
template <int KMAX, int U>
__device__ __forceinline__ int32_t fill_row(const int32_t (&p)[U][KMAX], const int (&n)[U]) {
  int32_t r = -1;
#pragma unroll
  for (int u = U - 1; u >= 0; --u)
    if (n[u] > 0) r = p[u][0];
  return r;
}

template <typename T, typename TO, int VE, int KMAX, int U, int H>
__global__ void __launch_bounds__(kThreads)
combine_inv_kernel(const typename elem<T>::storage* __restrict__ y,
                   const int32_t* __restrict__ inv, int32_t k, const float* __restrict__ w,
                   int64_t T_, int64_t d, typename elem<TO>::storage* __restrict__ out) {
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t t0 = ((int64_t)blockIdx.x * kWaves + wave) * U;
  if (t0 >= T_) return;
  int32_t mine, p[U][KMAX];
  int n[U];
  sorted_slots<KMAX, U>(inv, t0, T_, k, mine, p, n);
  float wp[U][KMAX];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int j = 0; j < KMAX; ++j) wp[u][j] = j < n[u] ? w[p[u][j]] : 0.f;
  const int32_t fill = fill_row<KMAX, U>(p, n);
  constexpr int64_t kStep = (int64_t)kWave * VE;
  for (int64_t h0 = (int64_t)lane * VE; h0 < d; h0 += H * kStep) {
    raw_vec<T, VE> x[H][U][KMAX];
    if (fill >= 0) {
#pragma unroll
      for (int c = 0; c < H; ++c) {
        const int64_t hl = h0 + c * kStep < d ? h0 + c * kStep : h0;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < KMAX; ++j)
            x[c][u][j] = load_raw<T, VE>(y + (int64_t)(j < n[u] ? p[u][j] : fill) * d + hl);
      }
    }
    wait_batch_loads();
#pragma unroll
    for (int c = 0; c < H; ++c) {
      const int64_t h = h0 + c * kStep;
      if (h >= d) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u >= T_) break;
        float acc[VE];
#pragma unroll
        for (int v = 0; v < VE; ++v) acc[v] = 0.f;
        {
#pragma clang fp contract(off)
#pragma unroll
          for (int j = 0; j < KMAX; ++j)
            if (j < n[u]) {
              float xf[VE];
              unpack_vec<T, VE>(x[c][u][j], xf);
#pragma unroll
              for (int v = 0; v < VE; ++v) acc[v] = acc[v] + wp[u][j] * xf[v];
            }
        }
        store_vec<TO, VE>(out + (t0 + u) * d + h, acc);
      }
    }
  }
}

// ------------------------------------------------------------- combine bwd

// Generic form, one wave per packed row p:
// dy[p,:] = cast(dY[t,:] * w[p]); dw[p] = sum_h dY[t,h] * y[p,h].
template <typename T, typename TG, int VE>
__global__ void __launch_bounds__(kThreads)
combine_bwd_kernel(const typename elem<T>::storage* __restrict__ y,
                   const int32_t* __restrict__ token_id, const float* __restrict__ w,
                   const typename elem<TG>::storage* __restrict__ dY, int64_t A, int64_t T_,
                   int64_t d, typename elem<T>::storage* __restrict__ dy, float* __restrict__ dw) {
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t p = (int64_t)blockIdx.x * kWaves + wave;
  if (p >= A) return;
  const int32_t t = token_id[p];
  const bool ok = t >= 0 && t < T_;
  const float wp = w[p];
  float part = 0.f;
  for (int64_t h = (int64_t)lane * VE; h < d; h += (int64_t)kWave * VE) {
    float g[VE], x[VE], o[VE];
    if (ok) {
      load_vec<TG, VE>(dY + (int64_t)t * d + h, g);
      load_vec<T, VE>(y + p * d + h, x);
    } else {
#pragma unroll
      for (int v = 0; v < VE; ++v) g[v] = x[v] = 0.f;
    }
#pragma unroll
    for (int v = 0; v < VE; ++v) {
      o[v] = __fmul_rn(g[v], wp);
      part = fmaf(g[v], x[v], part);
    }
    store_vec<T, VE>(dy + p * d + h, o);
  }
  part = wave_sum(part);
  if (lane == 0) dw[p] = part;
}

// Inverse-map form, one wave per token: the dY row is read once and serves
// all k packed rows of the token. Same per-row arithmetic and reduction
// order as combine_bwd_kernel, so dw and dy are bit-identical to it. The
// block's slots are read by one load and held in scalar registers, and every
// row load of a pass is issued before the first is used (an empty slot
// loads the block's first valid row and discards it).
template <typename T, typename TG, int VE, int KB, int H>
__global__ void __launch_bounds__(kThreads)
combine_bwd_inv_kernel(const typename elem<T>::storage* __restrict__ y,
                       const int32_t* __restrict__ inv, const float* __restrict__ w,
                       const typename elem<TG>::storage* __restrict__ dY, int64_t T_, int32_t k,
                       int64_t d, typename elem<T>::storage* __restrict__ dy,
                       float* __restrict__ dw) {
  static_assert(KB <= kWave, "a block's slots fit one wave");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kWaves + wave;
  if (t >= T_) return;
  const int64_t rows = T_ * k;
  for (int j0 = 0; j0 < k; j0 += KB) {
    const int nj = min(KB, k - j0);
    int32_t mine = lane < nj ? inv[t * k + j0 + lane] : -1;
    if (mine >= rows) mine = -1;
    const float wmine = mine >= 0 ? w[mine] : 0.f;
    int32_t pj[KB];
    float wj[KB], part[KB];
    int32_t fill = -1;
#pragma unroll
    for (int j = KB - 1; j >= 0; --j) {
      pj[j] = __builtin_amdgcn_readlane(mine, j);
      wj[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wmine), j));
      part[j] = 0.f;
      if (pj[j] >= 0) fill = pj[j];
    }
    if (fill < 0) continue;  // no valid slot in this block
    constexpr int64_t kStep = (int64_t)kWave * VE;
    for (int64_t h0 = (int64_t)lane * VE; h0 < d; h0 += H * kStep) {
      raw_vec<TG, VE> gw[H];
      raw_vec<T, VE> xw[H][KB];
#pragma unroll
      for (int c = 0; c < H; ++c) {
        const int64_t hl = h0 + c * kStep < d ? h0 + c * kStep : h0;
        gw[c] = load_raw<TG, VE>(dY + t * d + hl);
#pragma unroll
        for (int j = 0; j < KB; ++j)
          xw[c][j] = load_raw<T, VE>(y + (int64_t)(pj[j] >= 0 ? pj[j] : fill) * d + hl);
      }
      wait_batch_loads();
#pragma unroll
      for (int c = 0; c < H; ++c) {
        const int64_t h = h0 + c * kStep;
        if (h >= d) break;
        float g[VE];
        unpack_vec<TG, VE>(gw[c], g);
        // Every slot sums (an empty one its discarded fill row), so no row
        // load is moved behind a slot's condition; only the stores test it.
#pragma unroll
        for (int j = 0; j < KB; ++j) {
          float x[VE], o[VE];
          unpack_vec<T, VE>(xw[c][j], x);
#pragma unroll
          for (int v = 0; v < VE; ++v) {
            o[v] = __fmul_rn(g[v], wj[j]);
            part[j] = fmaf(g[v], x[v], part[j]);
          }
          if (pj[j] >= 0) store_vec<T, VE>(dy + (int64_t)pj[j] * d + h, o);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const float sum = wave_sum(part[j]);
      if (lane == 0 && pj[j] >= 0) dw[pj[j]] = sum;
    }
  }
}

// --------------------------------------------------------------- pack bwd

// dX[t,:] = cast(sum over rows(t) ascending of dpX[p,:]).
// dw: generic form (expert != nullptr): dw[t,j] = sum of dpw[p] for rows p
// whose expert first matches topk[t,j]; inverse form: dw[t,j] = dpw[inv[t*k+j]].
template <typename T, int VE>
__global__ void __launch_bounds__(kThreads)
pack_bwd_kernel(const typename elem<T>::storage* __restrict__ dpX, const float* __restrict__ dpw,
                ListSrc src, const int32_t* __restrict__ expert, const int32_t* __restrict__ topk,
                int64_t T_, int32_t k, int64_t d, typename elem<T>::storage* __restrict__ dX,
                float* __restrict__ dw) {
  __shared__ int32_t s_lists[kWaves][2][kMaxSorted];
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t t = (int64_t)blockIdx.x * kWaves + wave;
  if (t >= T_) return;
  int64_t first;
  const int n = gather_sorted(src, t, s_lists[wave][0], s_lists[wave][1], &first);
  const int nn = n >= 0 ? n : -n;
  const int32_t* sorted = s_lists[wave][1];
  for (int64_t h = (int64_t)lane * VE; h < d; h += (int64_t)kWave * VE) {
    float acc[VE];
#pragma unroll
    for (int v = 0; v < VE; ++v) acc[v] = 0.f;
    for (int i = 0; i < nn; ++i) {
      const int32_t p = list_entry(src, sorted, n, first, i);
      if (p < 0) continue;
      float x[VE];
      load_vec<T, VE>(dpX + (int64_t)p * d + h, x);
#pragma unroll
      for (int v = 0; v < VE; ++v) acc[v] = __fadd_rn(acc[v], x[v]);
    }
    store_vec<T, VE>(dX + t * d + h, acc);
  }
  if (expert == nullptr) {
    // Inverse map: slot j of token t sits at inv[t*k + j].
    for (int j = lane; j < k; j += kWave) {
      const int32_t p = src.list[t * k + j];
      dw[t * k + j] = (p >= 0 && p < src.rows) ? dpw[p] : 0.f;
    }
  } else {
    // Reference rule (csrc/kernels/backward_pack_kernel.cu:35-42): the first
    // slot whose expert matches receives the row's gate gradient. Lane j
    // owns slot j and sums its rows in ascending packed order.
    for (int j = lane; j < k; j += kWave) {
      const int32_t ej = topk[t * k + j];
      float acc = 0.f;
      for (int i = 0; i < nn; ++i) {
        const int32_t p = list_entry(src, sorted, n, first, i);
        if (p < 0) continue;
        const int32_t e = expert[p];
        if (e != ej) continue;
        int jf = 0;
        while (topk[t * k + jf] != e) ++jf;  // terminates: slot j matches
        if (jf == j) acc = __fadd_rn(acc, dpw[p]);
      }
      dw[t * k + j] = acc;
    }
  }
}

// The router's backward fused into the inverse-map pack backward (a null
// dlogits: none). For token t with gates g_j = gates[t,k+j], experts
// topk[t,j] and gate gradients dg_j = dpw[inv[t,j]] (0 when inv < 0),
// dlogits[t,:] is zero except at the selected experts, where it is
// g_j (dg_j - sum_i dg_i g_i): the arithmetic and order of
// route_topk_backward_kernel, so the result is the two-launch one bit for bit.
struct RouteGrad {
  const float* gates;
  const int32_t* topk;
  int32_t E;
  float* dlogits;
};
// Wave-wide (every lane calls it): lane `sl` of the `seg` lanes serving
// token t (sl < k) holds slot sl's gate gradient `dg`; the slots' gates and
// experts are read once per lane and broadcast by shuffles, so each token
// costs one round of loads. Lane sl writes experts sl, sl+seg, ... (live:
// t is a token).
__device__ __forceinline__ void route_grad_row(const RouteGrad& rg, int64_t t, bool live, int32_t k,
                                               int sl, int seg, float dg) {
  float g = 0.f;
  int32_t ej = -1;
  if (live && sl < k) {
    g = rg.gates[t * k + sl];
    ej = rg.topk[t * k + sl];
  }
  const int sb = lane_id() - sl;  // the segment's first lane
  float part = 0.f;
  for (int j = 0; j < k; ++j) part += __shfl(dg, sb + j, kWave) * __shfl(g, sb + j, kWave);
  for (int e0 = 0; e0 < rg.E; e0 += seg) {
    const int e = e0 + sl;
    float out = 0.f;
    for (int j = 0; j < k; ++j) {
      const int32_t ejj = __shfl(ej, sb + j, kWave);
      const float gj = __shfl(g, sb + j, kWave), dgj = __shfl(dg, sb + j, kWave);
      if (ejj == e) out += gj * (dgj - part);
    }
    if (live && e < rg.E) rg.dlogits[t * rg.E + e] = out;
  }
}

// Inverse-map pack backward for small fan-in: same sums as pack_bwd_kernel
// (ascending packed order, fp32), U tokens per wave with every row load
// issued up front. dw may be null (not written); rg.dlogits non-null adds
// the router's backward (route_grad_row).
template <typename T, int VE, int KMAX, int U, int H>
__global__ void __launch_bounds__(kThreads)
pack_bwd_inv_kernel(const typename elem<T>::storage* __restrict__ dpX,
                    const float* __restrict__ dpw, const int32_t* __restrict__ inv,
                    int64_t T_, int32_t k, int64_t d, typename elem<T>::storage* __restrict__ dX,
                    float* __restrict__ dw, RouteGrad rg) {
  constexpr int kSeg = kWave / U;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int64_t t0 = ((int64_t)blockIdx.x * kWaves + wave) * U;
  if (t0 >= T_) return;
  const int64_t rows = T_ * k;
  int32_t mine, p[U][KMAX];
  int n[U];
  sorted_slots<KMAX, U>(inv, t0, T_, k, mine, p, n);
  {
    const int64_t tl = t0 + lane / kSeg;
    const int jl = lane % kSeg;
    const float dg = (jl < k && tl < T_ && mine >= 0 && mine < rows) ? dpw[mine] : 0.f;
    if (dw != nullptr && jl < k && tl < T_) dw[tl * k + jl] = dg;
    if (rg.dlogits != nullptr) route_grad_row(rg, tl, tl < T_, k, jl, kSeg, dg);
  }
  const int32_t fill = fill_row<KMAX, U>(p, n);
  constexpr int64_t kStep = (int64_t)kWave * VE;
  for (int64_t h0 = (int64_t)lane * VE; h0 < d; h0 += H * kStep) {
    raw_vec<T, VE> x[H][U][KMAX];
    if (fill >= 0) {
#pragma unroll
      for (int c = 0; c < H; ++c) {
        const int64_t hl = h0 + c * kStep < d ? h0 + c * kStep : h0;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < KMAX; ++j)
            x[c][u][j] = load_raw<T, VE>(dpX + (int64_t)(j < n[u] ? p[u][j] : fill) * d + hl);
      }
    }
    wait_batch_loads();
#pragma unroll
    for (int c = 0; c < H; ++c) {
      const int64_t h = h0 + c * kStep;
      if (h >= d) break;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (t0 + u >= T_) break;
        float acc[VE];
#pragma unroll
        for (int v = 0; v < VE; ++v) acc[v] = 0.f;
#pragma unroll
        for (int j = 0; j < KMAX; ++j)
          if (j < n[u]) {
            float xf[VE];
            unpack_vec<T, VE>(x[c][u][j], xf);
#pragma unroll
            for (int v = 0; v < VE; ++v) acc[v] = __fadd_rn(acc[v], xf[v]);
          }
        store_vec<T, VE>(dX + (t0 + u) * d + h, acc);
      }
    }
  }
}

// ------------------------------------------------------------- dispatchers

template <typename T>
int vec_width(int64_t d, const void* a, const void* b, const void* c) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(c);
  const int eb = (int)sizeof(typename elem<T>::storage);
  const int max_ve = 16 / eb;
  for (int ve = max_ve; ve > 1; ve >>= 1) {
    if (d % ve == 0 && al % (uintptr_t)(ve * eb) == 0) return ve;
  }
  return 1;
}

template <typename T, typename TO>
int run_combine(const void* y, ListSrc src, const float* w, int64_t T_, int64_t d, void* out,
                hipStream_t s) {
  if (T_ == 0) return NT_OK;
  using S = typename elem<T>::storage;
  using SO = typename elem<TO>::storage;
  const dim3 grid((unsigned)ceil_div(T_, kWaves));
  const int ve = std::min(vec_width<T>(d, y, y, y), vec_width<TO>(d, out, out, out));
  const S* yp = static_cast<const S*>(y);
  SO* op = static_cast<SO*>(out);
  if (src.start == nullptr && src.k <= 8) {
    const bool long_rows = d * (int64_t)sizeof(S) > kLongRowBytes;
#define NT_CI(VE, KM) \
  do {                                                                                   \
    if (KM <= 2 && long_rows)                                                            \
      hipLaunchKernelGGL((combine_inv_kernel<T, TO, VE, KM, fan_u(KM, kCombineU), kLongChunks>), dim3((unsigned)ceil_div(T_, kWaves * fan_u(KM, kCombineU))), dim3(kThreads), 0, s, yp, src.list, src.k, w, T_, d, op); \
    else                                                                                 \
      hipLaunchKernelGGL((combine_inv_kernel<T, TO, VE, KM, fan_u(KM, kCombineU), 1>), dim3((unsigned)ceil_div(T_, kWaves * fan_u(KM, kCombineU))), dim3(kThreads), 0, s, yp, src.list, src.k, w, T_, d, op); \
  } while (0)
#define NT_CI_VE(KM)            \
  switch (ve) {                 \
    case 8: NT_CI(8, KM); break; \
    case 4: NT_CI(4, KM); break; \
    case 2: NT_CI(2, KM); break; \
    default: NT_CI(1, KM); break; \
  }
    if (src.k <= 2) {
      NT_CI_VE(2)
    } else {
      NT_CI_VE(8)
    }
#undef NT_CI_VE
#undef NT_CI
    return launch_status();
  }
  switch (ve) {
    case 8: hipLaunchKernelGGL((combine_kernel<T, TO, 8>), grid, dim3(kThreads), 0, s, yp, src, w, T_, d, op); break;
    case 4: hipLaunchKernelGGL((combine_kernel<T, TO, 4>), grid, dim3(kThreads), 0, s, yp, src, w, T_, d, op); break;
    case 2: hipLaunchKernelGGL((combine_kernel<T, TO, 2>), grid, dim3(kThreads), 0, s, yp, src, w, T_, d, op); break;
    default: hipLaunchKernelGGL((combine_kernel<T, TO, 1>), grid, dim3(kThreads), 0, s, yp, src, w, T_, d, op); break;
  }
  return launch_status();
}

template <typename T>
int combine_out_dispatch(int out_dtype, const void* y, ListSrc src, const float* w, int64_t T_,
                         int64_t d, void* out, hipStream_t s) {
  switch (out_dtype) {
    case NT_F32: return run_combine<T, float>(y, src, w, T_, d, out, s);
    case NT_F64: return run_combine<T, double>(y, src, w, T_, d, out, s);
    case NT_F16: return run_combine<T, f16>(y, src, w, T_, d, out, s);
    case NT_BF16: return run_combine<T, bf16>(y, src, w, T_, d, out, s);
    default: return NT_ERR_DTYPE;
  }
}

int combine_dispatch(int dtype, int out_dtype, const void* y, ListSrc src, const float* w,
                     int64_t T_, int64_t d, void* out, hipStream_t s) {
  switch (dtype) {
    case NT_F32: return combine_out_dispatch<float>(out_dtype, y, src, w, T_, d, out, s);
    case NT_F64: return combine_out_dispatch<double>(out_dtype, y, src, w, T_, d, out, s);
    case NT_F16: return combine_out_dispatch<f16>(out_dtype, y, src, w, T_, d, out, s);
    case NT_BF16: return combine_out_dispatch<bf16>(out_dtype, y, src, w, T_, d, out, s);
    default: return NT_ERR_DTYPE;
  }
}

template <typename T, typename TG>
int run_combine_bwd(const void* y, const int32_t* token_id, const float* w, const void* dY,
                    int64_t A, int64_t T_, int64_t d, void* dy, float* dw, hipStream_t s) {
  if (A == 0) return NT_OK;
  using S = typename elem<T>::storage;
  using SG = typename elem<TG>::storage;
  const dim3 grid((unsigned)ceil_div(A, kWaves));
  const int ve = std::min(vec_width<T>(d, y, dy, dy), vec_width<TG>(d, dY, dY, dY));
  const S* yp = static_cast<const S*>(y);
  const SG* gp = static_cast<const SG*>(dY);
  S* dyp = static_cast<S*>(dy);
  switch (ve) {
    case 8: hipLaunchKernelGGL((combine_bwd_kernel<T, TG, 8>), grid, dim3(kThreads), 0, s, yp, token_id, w, gp, A, T_, d, dyp, dw); break;
    case 4: hipLaunchKernelGGL((combine_bwd_kernel<T, TG, 4>), grid, dim3(kThreads), 0, s, yp, token_id, w, gp, A, T_, d, dyp, dw); break;
    case 2: hipLaunchKernelGGL((combine_bwd_kernel<T, TG, 2>), grid, dim3(kThreads), 0, s, yp, token_id, w, gp, A, T_, d, dyp, dw); break;
    default: hipLaunchKernelGGL((combine_bwd_kernel<T, TG, 1>), grid, dim3(kThreads), 0, s, yp, token_id, w, gp, A, T_, d, dyp, dw); break;
  }
  return launch_status();
}

template <typename T, typename TG>
int run_combine_bwd_inv(const void* y, const int32_t* inv, const float* w, const void* dY,
                        int64_t T_, int32_t k, int64_t d, void* dy, float* dw, hipStream_t s) {
  if (T_ == 0) return NT_OK;
  using S = typename elem<T>::storage;
  using SG = typename elem<TG>::storage;
  const dim3 grid((unsigned)ceil_div(T_, kWaves));
  const int ve = std::min(vec_width<T>(d, y, dy, dy), vec_width<TG>(d, dY, dY, dY));
  const S* yp = static_cast<const S*>(y);
  const SG* gp = static_cast<const SG*>(dY);
  S* dyp = static_cast<S*>(dy);
#define NT_CBI(VE, KB, H) \
  hipLaunchKernelGGL((combine_bwd_inv_kernel<T, TG, VE, KB, H>), grid, dim3(kThreads), 0, s, yp, inv, w, gp, T_, k, d, dyp, dw)
  const bool long_rows = d * (int64_t)sizeof(S) > kLongRowBytes;
  if (k <= 2 && long_rows) {
    switch (ve) {
      case 8: NT_CBI(8, 2, kLongChunks); break;
      case 4: NT_CBI(4, 2, kLongChunks); break;
      case 2: NT_CBI(2, 2, kLongChunks); break;
      default: NT_CBI(1, 2, kLongChunks); break;
    }
  } else if (k <= 2) {
    switch (ve) {
      case 8: NT_CBI(8, 2, 1); break;
      case 4: NT_CBI(4, 2, 1); break;
      case 2: NT_CBI(2, 2, 1); break;
      default: NT_CBI(1, 2, 1); break;
    }
  } else if (long_rows) {
    switch (ve) {
      case 8: NT_CBI(8, 8, 1); break;
      case 4: NT_CBI(4, 8, 1); break;
      case 2: NT_CBI(2, 8, 1); break;
      default: NT_CBI(1, 8, 1); break;
    }
  } else {
    // Short rows, k > 2: four rows per pass over dY (a second pass re-reads
    // the token's dY row from L2) keeps the kernel at 60 registers against
    // 75 with all eight (measured cold, C3: 126 -> 108 us before the row
    // loads were batched; long rows were 5% slower so).
    switch (ve) {
      case 8: NT_CBI(8, 4, 1); break;
      case 4: NT_CBI(4, 4, 1); break;
      case 2: NT_CBI(2, 4, 1); break;
      default: NT_CBI(1, 4, 1); break;
    }
  }
#undef NT_CBI
  return launch_status();
}

template <typename T>
int run_pack_bwd(const void* dpX, const float* dpw, ListSrc src, const int32_t* expert,
                 const int32_t* topk, int64_t T_, int32_t k, int64_t d, void* dX, float* dw,
                 hipStream_t s, RouteGrad rg) {
  if (T_ == 0) return NT_OK;
  using S = typename elem<T>::storage;
  const dim3 grid((unsigned)ceil_div(T_, kWaves));
  const int ve = vec_width<T>(d, dpX, dX, dX);
  const S* ip = static_cast<const S*>(dpX);
  S* op = static_cast<S*>(dX);
  if (src.start == nullptr && expert == nullptr && k <= 8) {
    const bool long_rows = d * (int64_t)sizeof(S) > kLongRowBytes;
#define NT_PBI_U(VE, KM, U, H) \
  hipLaunchKernelGGL((pack_bwd_inv_kernel<T, VE, KM, fan_u(KM, U), H>), dim3((unsigned)ceil_div(T_, kWaves * fan_u(KM, U))), dim3(kThreads), 0, s, ip, dpw, src.list, T_, k, d, op, dw, rg)
#define NT_PBI(VE, KM)                                                      \
  do {                                                                      \
    if (long_rows && KM <= 2) NT_PBI_U(VE, KM, kPackBwdULong, kLongChunks); \
    else if (long_rows) NT_PBI_U(VE, KM, kPackBwdULong, 1);                 \
    else NT_PBI_U(VE, KM, kPackBwdU, 1);                                    \
  } while (0)
#define NT_PBI_VE(KM)            \
  switch (ve) {                  \
    case 8: NT_PBI(8, KM); break; \
    case 4: NT_PBI(4, KM); break; \
    case 2: NT_PBI(2, KM); break; \
    default: NT_PBI(1, KM); break; \
  }
    if (k <= 2) {
      NT_PBI_VE(2)
    } else {
      NT_PBI_VE(8)
    }
#undef NT_PBI_VE
#undef NT_PBI
#undef NT_PBI_U
    return launch_status();
  }
  switch (ve) {
    case 8: hipLaunchKernelGGL((pack_bwd_kernel<T, 8>), grid, dim3(kThreads), 0, s, ip, dpw, src, expert, topk, T_, k, d, op, dw); break;
    case 4: hipLaunchKernelGGL((pack_bwd_kernel<T, 4>), grid, dim3(kThreads), 0, s, ip, dpw, src, expert, topk, T_, k, d, op, dw); break;
    case 2: hipLaunchKernelGGL((pack_bwd_kernel<T, 2>), grid, dim3(kThreads), 0, s, ip, dpw, src, expert, topk, T_, k, d, op, dw); break;
    default: hipLaunchKernelGGL((pack_bwd_kernel<T, 1>), grid, dim3(kThreads), 0, s, ip, dpw, src, expert, topk, T_, k, d, op, dw); break;
  }
  return launch_status();
}

// rg.dlogits non-null: the inverse-map kernel (src.start null, no expert
// array, k <= 8) also writes the router's gradient; the caller ensures that.
int pack_bwd_dispatch(int dtype, const void* dpX, const float* dpw, ListSrc src,
                      const int32_t* expert, const int32_t* topk, int64_t T_, int32_t k,
                      int64_t d, void* dX, float* dw, hipStream_t s, RouteGrad rg = RouteGrad{}) {
  switch (dtype) {
    case NT_F32: return run_pack_bwd<float>(dpX, dpw, src, expert, topk, T_, k, d, dX, dw, s, rg);
    case NT_F64: return run_pack_bwd<double>(dpX, dpw, src, expert, topk, T_, k, d, dX, dw, s, rg);
    case NT_F16: return run_pack_bwd<f16>(dpX, dpw, src, expert, topk, T_, k, d, dX, dw, s, rg);
    case NT_BF16: return run_pack_bwd<bf16>(dpX, dpw, src, expert, topk, T_, k, d, dX, dw, s, rg);
    default: return NT_ERR_DTYPE;
  }
}

bool sizes_ok(int64_t a, int64_t b, int64_t d) { return a >= 0 && b >= 0 && d >= 0; }

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

size_t nt_combine_workspace_bytes(int64_t A, int64_t T) {
  if (A < 0 || T < 0) return 0;
  return csr_bytes(A, T);
}

int nt_combine_tokens(int dtype, const void* y, const int32_t* token_id, const float* w,
                      int64_t A, int64_t T, int64_t d, float* out, void* ws, size_t ws_bytes,
                      hipStream_t stream) {
  if (dtype_bytes(dtype) == 0) return NT_ERR_DTYPE;
  if (!sizes_ok(A, T, d)) return NT_ERR_INVALID_ARG;
  if (A > INT32_MAX || T > INT32_MAX - 1) return NT_ERR_TOO_LARGE;
  if (T > 0 && d > 0 && out == nullptr) return NT_ERR_INVALID_ARG;
  if (A > 0 && (y == nullptr || token_id == nullptr || w == nullptr)) return NT_ERR_INVALID_ARG;
  if (ws == nullptr || ws_bytes < csr_bytes(A, T)) return NT_ERR_WORKSPACE;
  if (T == 0) return NT_OK;
  const CsrWs c = carve_csr(ws, A, T);
  const int32_t* list = nullptr;
  int st = build_csr(token_id, A, T, c, &list, stream);
  if (st != NT_OK) return st;
  ListSrc src{c.start, list, 0, A};
  return combine_dispatch(dtype, NT_F32, y, src, w, T, d, out, stream);
}

int nt_combine_inv(int dtype, const void* y, const int32_t* inv, const float* w, int64_t T,
                   int32_t k, int64_t d, int out_dtype, void* out, hipStream_t stream) {
  if (dtype_bytes(dtype) == 0 || dtype_bytes(out_dtype) == 0) return NT_ERR_DTYPE;
  if (!sizes_ok(T, k, d) || k < 1) return NT_ERR_INVALID_ARG;
  if (T * (int64_t)k > INT32_MAX) return NT_ERR_TOO_LARGE;
  if (T > 0 && (inv == nullptr || w == nullptr || (d > 0 && (y == nullptr || out == nullptr))))
    return NT_ERR_INVALID_ARG;
  ListSrc src{nullptr, inv, k, T * k};
  return combine_dispatch(dtype, out_dtype, y, src, w, T, d, out, stream);
}

int nt_combine_backward(int dtype, const void* y, const int32_t* token_id, const float* w,
                        const float* dY, int64_t A, int64_t T, int64_t d, void* dy, float* dw,
                        hipStream_t stream) {
  if (!sizes_ok(A, T, d)) return NT_ERR_INVALID_ARG;
  if (A > 0 && (token_id == nullptr || w == nullptr || dw == nullptr ||
                (d > 0 && (y == nullptr || dy == nullptr || dY == nullptr))))
    return NT_ERR_INVALID_ARG;
  switch (dtype) {
    case NT_F32: return run_combine_bwd<float, float>(y, token_id, w, dY, A, T, d, dy, dw, stream);
    case NT_F64: return run_combine_bwd<double, float>(y, token_id, w, dY, A, T, d, dy, dw, stream);
    case NT_F16: return run_combine_bwd<f16, float>(y, token_id, w, dY, A, T, d, dy, dw, stream);
    case NT_BF16: return run_combine_bwd<bf16, float>(y, token_id, w, dY, A, T, d, dy, dw, stream);
    default: return NT_ERR_DTYPE;
  }
}

int nt_combine_backward_inv(int dtype, const void* y, const int32_t* inv, const float* w,
                            int dY_dtype, const void* dY, int64_t T, int32_t k, int64_t d,
                            void* dy, float* dw, hipStream_t stream) {
  if (!sizes_ok(T, k, d) || k < 1) return NT_ERR_INVALID_ARG;
  if (T * (int64_t)k > INT32_MAX) return NT_ERR_TOO_LARGE;
  if (T > 0 && (inv == nullptr || w == nullptr || dw == nullptr ||
                (d > 0 && (y == nullptr || dy == nullptr || dY == nullptr))))
    return NT_ERR_INVALID_ARG;
  if (dY_dtype != NT_F32 && dY_dtype != dtype) return NT_ERR_DTYPE;
  const bool g32 = dY_dtype == NT_F32;
  switch (dtype) {
    case NT_F32: return run_combine_bwd_inv<float, float>(y, inv, w, dY, T, k, d, dy, dw, stream);
    case NT_F64:
      return g32 ? run_combine_bwd_inv<double, float>(y, inv, w, dY, T, k, d, dy, dw, stream)
                 : run_combine_bwd_inv<double, double>(y, inv, w, dY, T, k, d, dy, dw, stream);
    case NT_F16:
      return g32 ? run_combine_bwd_inv<f16, float>(y, inv, w, dY, T, k, d, dy, dw, stream)
                 : run_combine_bwd_inv<f16, f16>(y, inv, w, dY, T, k, d, dy, dw, stream);
    case NT_BF16:
      return g32 ? run_combine_bwd_inv<bf16, float>(y, inv, w, dY, T, k, d, dy, dw, stream)
                 : run_combine_bwd_inv<bf16, bf16>(y, inv, w, dY, T, k, d, dy, dw, stream);
    default: return NT_ERR_DTYPE;
  }
}

int nt_pack_backward(int dtype, const void* dpX, const float* dpw, const int32_t* token_id,
                     const int32_t* expert, const int32_t* topk, int64_t A, int64_t T, int32_t k,
                     int64_t d, void* dX, float* dw, void* ws, size_t ws_bytes,
                     hipStream_t stream) {
  if (dtype_bytes(dtype) == 0) return NT_ERR_DTYPE;
  if (!sizes_ok(A, T, d) || k < 1) return NT_ERR_INVALID_ARG;
  if (A > INT32_MAX || T * (int64_t)k > INT32_MAX) return NT_ERR_TOO_LARGE;
  if (T > 0 && (dw == nullptr || topk == nullptr || (d > 0 && dX == nullptr)))
    return NT_ERR_INVALID_ARG;
  if (A > 0 && (token_id == nullptr || expert == nullptr || dpw == nullptr ||
                (d > 0 && dpX == nullptr)))
    return NT_ERR_INVALID_ARG;
  if (ws == nullptr || ws_bytes < csr_bytes(A, T)) return NT_ERR_WORKSPACE;
  if (T == 0) return NT_OK;
  const CsrWs c = carve_csr(ws, A, T);
  const int32_t* list = nullptr;
  int st = build_csr(token_id, A, T, c, &list, stream);
  if (st != NT_OK) return st;
  ListSrc src{c.start, list, 0, A};
  return pack_bwd_dispatch(dtype, dpX, dpw, src, expert, topk, T, k, d, dX, dw, stream);
}

int nt_pack_backward_inv(int dtype, const void* dpX, const float* dpw, const int32_t* inv,
                         int64_t T, int32_t k, int64_t d, void* dX, float* dw,
                         hipStream_t stream) {
  if (dtype_bytes(dtype) == 0) return NT_ERR_DTYPE;
  if (!sizes_ok(T, k, d) || k < 1) return NT_ERR_INVALID_ARG;
  if (T * (int64_t)k > INT32_MAX) return NT_ERR_TOO_LARGE;
  if (T > 0 && (inv == nullptr || dpw == nullptr || dw == nullptr ||
                (d > 0 && (dpX == nullptr || dX == nullptr))))
    return NT_ERR_INVALID_ARG;
  ListSrc src{nullptr, inv, k, T * k};
  return pack_bwd_dispatch(dtype, dpX, dpw, src, nullptr, nullptr, T, k, d, dX, dw, stream);
}

int nt_pack_backward_inv_route(int dtype, const void* dpX, const float* dpw, const int32_t* inv,
                               const float* gates, const int32_t* topk, int64_t T, int32_t k,
                               int64_t d, int32_t E, void* dX, float* dlogits, float* dw,
                               hipStream_t stream) {
  if (dtype_bytes(dtype) == 0) return NT_ERR_DTYPE;
  // the router's limits (nt_route_topk_backward), checked before any launch
  if (!sizes_ok(T, k, d) || k < 1 || E < 1 || k > E || k > kMaxTopK) return NT_ERR_INVALID_ARG;
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
  if (T * (int64_t)k > INT32_MAX || T * (int64_t)E > INT32_MAX) return NT_ERR_TOO_LARGE;
  if (T > 0 && (inv == nullptr || dpw == nullptr || gates == nullptr || topk == nullptr ||
                dlogits == nullptr || (d > 0 && (dpX == nullptr || dX == nullptr))))
    return NT_ERR_INVALID_ARG;
  ListSrc src{nullptr, inv, k, T * k};
  if (k <= 8) {
    const RouteGrad rg{gates, topk, E, dlogits};
    return pack_bwd_dispatch(dtype, dpX, dpw, src, nullptr, nullptr, T, k, d, dX, dw, stream, rg);
  }
  // More slots than the inverse-map kernel takes: the two launches it fuses.
  if (T > 0 && dw == nullptr) return NT_ERR_INVALID_ARG;
  const int st = pack_bwd_dispatch(dtype, dpX, dpw, src, nullptr, nullptr, T, k, d, dX, dw, stream);
  if (st != NT_OK) return st;
  return nt_route_topk_backward(gates, topk, dw, T, E, k, dlogits, stream);
}

}  // extern "C"
