// Expert-grouped GEMM forward and its dX / dW gradients for gfx950.
//
//   fwd : out[a,:] = X[a,:] @ W[e]          rows a of expert e
//   dX  : dX[a,:]  = dOut[a,:] @ W[e]^T
//   dW  : dW[e]    = X_e^T @ dOut_e         reduction over the expert's rows
//
// bf16/fp16 with 16-byte-aligned shapes run on the MFMA kernel: 256 threads
// (4 waves, 2x2), a 128x128 output tile, K staged 64 at a time through LDS in
// a K-contiguous layout so every MFMA operand is one 16-byte LDS read.
// Operands that are K-contiguous in HBM (X rows, dOut rows, W rows for dX)
// are copied straight in; operands that are M/N-contiguous (W for the
// forward, both operands of dW) are transposed in registers on the way in
// (4x8 blocks, packed with byte permutes). fp32 accumulation, one
// round-to-nearest-even cast in the epilogue.
//
// A device-side tile scheduler maps the linear workgroup id to (expert,
// m-tile, n-tile) from the offsets array, so empty experts cost nothing, the
// host never reads offsets (no .item() syncs) and one launch covers every
// expert. fp32 / fp64 and shapes that are not multiples of 8 run on a simple
// LDS-tiled FMA kernel with the same scheduler.
#include <algorithm>
#include <atomic>
#include <chrono>
#include <type_traits>

#include "common.hpp"

namespace nt {
namespace {

#include "gelu_table_bf16.inc"

enum GemmMode { kFwd = 0, kDx = 1, kDw = 2 };


// ------------------------------------------------------------ scheduling

// Row range of expert e, clamped to [0, A] and made non-decreasing, so a
// malformed offsets array can never move an access outside the buffers.
__device__ __forceinline__ void expert_rows(const int32_t* __restrict__ offsets, int e, int64_t A,
                                            int64_t& r0, int64_t& r1) {
  int64_t a = offsets[e], b = offsets[e + 1];
  a = a < 0 ? 0 : (a > A ? A : a);
  b = b < a ? a : (b > A ? A : b);
  r0 = a;
  r1 = b;
}

// s_pref[e] = number of BM-row tiles of experts < e (s_pref[E] = total),
// built by the first wave; ends with a workgroup barrier.
__device__ void build_m_prefix(const int32_t* __restrict__ offsets, int E, int64_t A, int BM,
                               int32_t* s_pref) {
  if (threadIdx.x < kWave) {
    const int lane = lane_id();
    int carry = 0;
    for (int s = 0; s < E; s += kWave) {
      const int e = s + lane;
      int v = 0;
      if (e < E) {
        int64_t a, b;
        expert_rows(offsets, e, A, a, b);
        v = (int)ceil_div(b - a, BM);
      }
      const int incl = wave_incl_scan(v);
      if (e < E) s_pref[e + 1] = carry + incl;
      carry += __shfl(incl, kWave - 1, kWave);
    }
    if (lane == 0) s_pref[0] = 0;
  }
  __syncthreads();
}

// dW reduction chunks. An expert with more than `thr` rows is cut into
// nch(e) = ceil(M_e / R) chunks of R rows (R <= thr); every other expert is
// one chunk (an empty expert keeps one empty chunk, so its dW is still
// written, as zeros). s_pref[e] = chunks of experts < e; s_split[e] = chunks
// of experts < e that have at least two (those write fp32 partials, one slab
// per chunk, and a reduce pass sums them in chunk order). R = 0 means one
// chunk per expert.
//
// The workspace holds `cap` slabs, enough whenever the experts' row ranges
// are disjoint (non-decreasing offsets). expert_rows clamps each expert on
// its own, so a non-monotone offsets array can give ranges that overlap and
// more split chunks than that; then every expert is one chunk (no partial
// slab is written, and split_total() tells the reduce pass to do nothing).
// Ends with a workgroup barrier.
__device__ __forceinline__ int dw_chunks(int64_t rows, int32_t R, int32_t thr) {
  if (R <= 0 || rows <= thr) return 1;
  return (int)ceil_div(rows, R);
}
// Wave-wide: chunks of the split experts (those with two or more) over all
// E experts, the same on every lane.
__device__ int split_total(const int32_t* __restrict__ offsets, int E, int64_t A, int32_t R,
                           int32_t thr) {
  int tot = 0;
  for (int s = 0; s < E; s += kWave) {
    const int e = s + lane_id();
    int v = 0;
    if (e < E) {
      int64_t a, b;
      expert_rows(offsets, e, A, a, b);
      v = dw_chunks(b - a, R, thr);
      v = v >= 2 ? v : 0;
    }
    tot += wave_sum_int(v);
  }
  return tot;
}
__device__ void build_chunk_prefix(const int32_t* __restrict__ offsets, int E, int64_t A,
                                   int32_t R, int32_t thr, int32_t cap, int32_t* s_pref,
                                   int32_t* s_split) {
  if (threadIdx.x < kWave) {
    const int lane = lane_id();
    if (R > 0 && split_total(offsets, E, A, R, thr) > cap) R = 0;
    int carry = 0, carry_s = 0;
    for (int s = 0; s < E; s += kWave) {
      const int e = s + lane;
      int v = 0, vs = 0;
      if (e < E) {
        int64_t a, b;
        expert_rows(offsets, e, A, a, b);
        v = dw_chunks(b - a, R, thr);
        vs = v >= 2 ? v : 0;
      }
      const int incl = wave_incl_scan(v);
      const int incl_s = wave_incl_scan(vs);
      if (e < E) {
        s_pref[e + 1] = carry + incl;
        s_split[e + 1] = carry_s + incl_s;
      }
      carry += __shfl(incl, kWave - 1, kWave);
      carry_s += __shfl(incl_s, kWave - 1, kWave);
    }
    if (lane == 0) {
      s_pref[0] = 0;
      s_split[0] = 0;
    }
  }
  __syncthreads();
}

// Expert owning m-tile `mt_global` (expert-major order) and the tile's row
// range; false when mt_global is past the last tile.
__device__ bool find_m_tile(const int32_t* __restrict__ offsets, int E, int64_t A,
                            const int32_t* s_pref, int64_t mt_global, int& e_out, int64_t& r0,
                            int64_t& r1, int64_t& mt_local) {
  if (mt_global >= s_pref[E]) return false;
  int lo = 0, hi = E - 1;  // largest e with s_pref[e] <= mt_global
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= mt_global) lo = mid;
    else hi = mid - 1;
  }
  e_out = lo;
  expert_rows(offsets, lo, A, r0, r1);
  mt_local = mt_global - s_pref[lo];
  return true;
}

__device__ bool map_m_tile(const int32_t* __restrict__ offsets, int E, int64_t A, int BM,
                           int64_t mt_global, int32_t* s_pref, int& e_out, int64_t& r0,
                           int64_t& r1, int64_t& mt_local) {
  build_m_prefix(offsets, E, A, BM, s_pref);
  return find_m_tile(offsets, E, A, s_pref, mt_global, e_out, r0, r1, mt_local);
}

// ------------------------------------------------------- MFMA operand tiles

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));

// The 16-bit GEMMs run on v_mfma_f32_16x16x32: the same operand registers
// (8 elements per lane) and flops per register as 32x32x16, at lower power
// per flop. The GPU holds its power limit by lowering the clock, so this
// raises the sustained rate (measured on MI355X, MFMA chains from registers:
// 1,916-1,922 TF/s at 1.92 GHz against 1,660-1,681 at 1.64-1.67 GHz; this
// kernel's k-step with operands from LDS: 1,422-1,441 against 1,342-1,360;
// the GEMMs, outputs bit-identical: C4 forward 1,171 -> 1,245 TF/s, dX
// 1,120 -> 1,198, dW 1,090 -> 1,140, C2 layer step 1.028 -> 0.964 ms).
template <typename T>
struct mfma_op;
template <>
struct mfma_op<bf16> {
  typedef bf16x8_t vec;
  __device__ static f32x4_t run(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct mfma_op<f16> {
  typedef f16x8_t vec;
  __device__ static f32x4_t run(vec a, vec b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// Accumulators of one wave: acc[i][j][g] holds 16x16 block g of the 32x32
// sub-tile (i, j) of the wave's output block, with the B fragment issued as
// the MFMA's first operand, so that lane l, element q holds
//   C[32 i + acc_row(g, l)][32 j + acc_col(g, l) + q]:
// 4 consecutive output columns of one row per block.
template <int TM, int TN>
using AccTile = f32x4_t[TM][TN][4];
__device__ __forceinline__ int acc_row(int g, int lane) { return 16 * (g >> 1) + (lane & 15); }
__device__ __forceinline__ int acc_col(int g, int lane) { return 16 * (g & 1) + 4 * (lane >> 4); }

// Two fp32 values rounded to nearest-even and packed into 32 bits (first
// value in the low half). bf16 uses the hardware pair conversion
// (v_cvt_pk_bf16_f32, RNE); fp16 converts each value (v_cvt_f16_f32, RNE).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);
template <>
__device__ __forceinline__ uint32_t pack2<bf16>(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
template <>
__device__ __forceinline__ uint32_t pack2<f16>(float a, float b) {
  return (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaThreads = 512;  // 8 waves, two per SIMD
constexpr int kMfmaWaves = kMfmaThreads / kWave;

// Operand tiles are fetched with raw buffer loads that write straight into
// LDS (buffer_load_dwordx4 ... lds): lane i of one instruction lands at
// 16*i bytes past the instruction's LDS base (M0), so one instruction fills
// 1 KiB of LDS and the lane -> global-address map chooses the LDS layout.
// The descriptor's range check turns any offset past the range into a zero
// fill; lanes whose chunk lies past the reduction end get kOob.
//
// The loads are issued from inline assembly: the compiler then does not
// treat them as LDS writes that every later LDS read must wait for (it
// would wait for the next stage's loads before reading the current stage).
// Completion is explicit instead: s_waitcnt vmcnt(0) and a workgroup
// barrier before a stage is read.
constexpr uint32_t kBufConfig = 0x00020000u;  // gfx9 buffer descriptor word 3
constexpr uint32_t kOob = 0x80000000u;
constexpr int kCpolNT = 2;  // buffer instruction cache policy: non-temporal

__device__ __forceinline__ i32x4_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = (int32_t)(bytes <= 0 ? 0 : (bytes > 0x7ffffff0 ? 0x7ffffff0 : bytes));
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane(n);
  r[3] = (int)kBufConfig;
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)p);
}

__device__ __forceinline__ void load16_to_lds(i32x4_t rsrc, uint32_t voff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, 0 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(lds)
      : "memory", "m0");
}

// a + b (b wave-uniform) as an instruction the compiler cannot move or fold.
__device__ __forceinline__ uint32_t add_opaque(uint32_t a, uint32_t b) {
  uint32_t r;
  asm volatile("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(b), "v"(a));
  return r;
}

// Wait until at most N of this wave's vector-memory operations are in
// flight. The counter retires loads and stores in issue order, so every
// older operation is complete.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Buffer descriptor for the epilogue's stores to one output tile. Lanes
// outside the tile store at offset kOob, which the range check drops, so
// every wave issues the same number of store instructions per tile (the
// next tile's first wait counts them).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a) |
                     ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32))
                      << 32);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(u), 0, 0x7ffffff0,
                                           (int)kBufConfig);
}

__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t d = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(d[0], d[1], d[2], d[3]);
}

__device__ __forceinline__ void store16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t d = {v.x, v.y, v.z, v.w};
  // Non-temporal (cache policy NT): output tiles are written once and read
  // by a later kernel, so they should not displace the operand panels the
  // XCD's L2 shares between concurrent tiles (measured: -5 to -19 us per
  // C2-sized GEMM).
  __builtin_amdgcn_raw_buffer_store_b128(d, r, (int)off, 0, kCpolNT);
}

// One operand tile in LDS, ROWS (m or n) x BK (reduction, 64 or 32) 16-bit
// elements.
//
// K-major (the reduction index is contiguous in HBM): row r of the tile is
// BK elements = CPR chunks of 16 B; RPW = 16 / CPR rows share one 256-byte
// sweep of the 64 banks. Chunk c of row r is stored at c ^ ((r / RPW) % CPR).
// An MFMA fragment read (ds_read_b128, 16 lanes per LDS cycle: rows
// r..r+15, one chunk) then touches all 64 banks once.
//
// MN-major (m / n contiguous in HBM): row k of the tile holds ROWS elements
// (ROWS/8 chunks), chunk c stored at c ^ mn_swizzle(k). Fragments come from
// ds_read_b64_tr_b16, which transposes 4x4 blocks of 16-bit elements across
// each 16-lane group: source lane 4j+q reads the 4 elements at (k0 + j,
// mn0 + 4q .. 4q+3); destination lane 4q+e receives (k0 + 0..3, mn0 + 4q + e).
// Two such reads (k0 and k0 + 4) give a lane the 8 consecutive reduction
// elements of one m / n index that v_mfma_f32_16x16x32 takes; lane group g
// reads rows 8g .. 8g+7 of the substep. 32 lanes per LDS cycle (groups 0
// and 1, or 2 and 3) read rows k0 + 0..3 and k0 + 8..11, two chunks each;
// the XOR (bits 0, 1 and 3 of k) places those 16 chunks on all 64 banks.
//
// Wave w issues instructions w, w+NW, ...; where the rows of successive
// instructions differ by a whole number of XOR periods (16 rows), one
// per-lane offset plus a uniform stride per instruction covers them, else
// two offsets (even and odd instructions).
__device__ __forceinline__ int mn_swizzle(int k) { return 4 * (k & 3) + 2 * ((k >> 3) & 1); }
template <int ROWS, bool KMAJ, int BK, int NW>
struct OperandTile {
  static_assert(BK == 32 || BK == 64, "k-step of 32 or 64 elements");
  static constexpr int kBytes = ROWS * BK * 2;
  static constexpr int kInsts = kBytes / 1024;   // 1 KiB per load instruction
  static constexpr int kPer = kInsts / NW;
  static_assert(kPer >= 1 && kInsts % NW == 0, "tile too small for the wave count");
  static_assert(KMAJ || ROWS >= 128, "MN-major tiles need at least 16 chunks per row");
  static constexpr int kRowBytes = KMAJ ? BK * 2 : ROWS * 2;
  static constexpr int kRowsPerInst = 1024 / kRowBytes;
  static constexpr int kCpr = KMAJ ? BK / 8 : ROWS / 8;  // chunks per row
  static constexpr int kRpw = 16 / (BK / 8);             // K-major rows per bank sweep
  static constexpr int kStepRows = NW * kRowsPerInst;    // rows between a wave's instructions
  static constexpr bool kTwo = !KMAJ && kStepRows % 16 != 0;
  static_assert(KMAJ || kStepRows % 8 == 0, "MN-major swizzle: 8-row steps");
  static_assert(!kTwo || kPer % 2 == 0, "MN-major swizzle: even instruction count");

  uint32_t off;     // byte offset of this lane's chunk (instruction `wave`) from the tile origin
  uint32_t off2;    // kTwo: the same for instruction `wave` + NW
  uint32_t kchunk;  // K-major: first reduction index of the lane's chunk
  uint32_t ustep;   // byte stride between this wave's successive instructions (kTwo: of
                    // every second one)

  __device__ void init(int64_t ld, int wave, int lane) {
    const int r = kRowsPerInst * wave + lane / kCpr;
    const int c = KMAJ ? (lane % kCpr) ^ ((r / kRpw) % kCpr) : (lane % kCpr) ^ mn_swizzle(r);
    off = (uint32_t)((int64_t)r * ld + c * 8) * 2u;
    kchunk = (uint32_t)(c * 8);
    if (kTwo) {
      const int r2 = r + kStepRows;
      off2 = (uint32_t)((int64_t)r2 * ld + ((lane % kCpr) ^ mn_swizzle(r2)) * 8) * 2u;
    }
    ustep = (uint32_t)__builtin_amdgcn_readfirstlane((int)((kTwo ? 2 : 1) * kStepRows * ld * 2));
  }

  // Issue this wave's share of the tile's loads. `base` is the tile origin
  // for this k-step; `range` bytes from it are readable; `kv` reduction
  // elements are valid (K-major chunks past kv are zero-filled; MN-major
  // rows past kv fall outside `range`).
  __device__ void issue(const void* base, int64_t range, char* lds, int64_t kv, int wave) const {
    const i32x4_t rs = make_rsrc(base, range);
    const uint32_t l0 = lds_addr(lds) + (uint32_t)wave * 1024u;
    uint32_t v = off;
    if (KMAJ && kv < BK && (int64_t)kchunk >= kv) v = kOob;
    // Instruction u reads u * ustep bytes further on. The offset advances
    // through an opaque add, so the compiler keeps one offset register
    // instead of hoisting kPer of them out of the k-loop.
    if constexpr (kTwo) {
      uint32_t v2 = off2;
#pragma unroll
      for (int u = 0; u < kPer; u += 2) {
        load16_to_lds(rs, v, __builtin_amdgcn_readfirstlane(l0 + (uint32_t)(u * NW * 1024)));
        load16_to_lds(rs, v2, __builtin_amdgcn_readfirstlane(l0 + (uint32_t)((u + 1) * NW * 1024)));
        if (u + 2 < kPer) {
          v = add_opaque(v, ustep);
          v2 = add_opaque(v2, ustep);
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        load16_to_lds(rs, v, __builtin_amdgcn_readfirstlane(l0 + (uint32_t)(u * NW * 1024)));
        if (u + 1 < kPer) v = add_opaque(v, ustep);
      }
    }
  }
};

// Per-lane LDS byte offsets of the fragment reads of one operand: TS 16-row
// blocks starting at row `row0` of the tile, for each of the BK/32
// k-substeps of 32 elements. Lane l supplies index l % 16 of a block and
// reduction elements 8 (l / 16) .. +7 of the substep.
template <int ROWS, bool KMAJ, int TS, int BK>
struct FragReader {
  static constexpr int kRowBytes = KMAJ ? BK * 2 : ROWS * 2;
  static constexpr int kCpr = BK / 8;
  static constexpr int kRpw = 16 / kCpr;
  uint32_t base[KMAJ ? BK / 32 : TS];
  __device__ void init(int row0, int lane) {
    if (KMAJ) {
      // the K-major XOR repeats every 16 rows, so blocks differ by a stride
      const int r = row0 + (lane & 15);
#pragma unroll
      for (int ks = 0; ks < BK / 32; ++ks) {
        const int c = (4 * ks + (lane >> 4)) ^ ((r / kRpw) % kCpr);
        base[ks] = (uint32_t)(r * kRowBytes + c * 16);
      }
    } else {
      // mn_swizzle repeats every 16 rows and ignores bit 2, so the substep
      // (32 rows on) and the second read (4 rows on) are strides
      const int g = lane >> 4, s = lane & 15, j = s >> 2, q = s & 3;
      const int k = 8 * g + j;
#pragma unroll
      for (int t = 0; t < TS; ++t) {
        const int mn = row0 + 16 * t + 4 * q;
        const int c = (mn >> 3) ^ mn_swizzle(k);
        base[t] = (uint32_t)(k * kRowBytes + c * 16 + (mn & 7) * 2);
      }
    }
  }
  template <typename V>
  __device__ V read(const char* lds, int t, int ks) const {
    if (KMAJ) {
      return *reinterpret_cast<const V*>(lds + base[ks] + t * 16 * kRowBytes);
    } else {
      const char* p = lds + base[t] + 32 * ks * kRowBytes;
      const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
      const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 4 * kRowBytes));
      const s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      return __builtin_bit_cast(V, v);
    }
  }
};

struct GemmArgs {
  const void* a;  // fwd: X     dX: dOut   dW: X
  const void* b;  // fwd: W     dX: W      dW: dOut
  const int32_t* offsets;
  int32_t E;
  int64_t A, K, N;
  void* out;
  int32_t ntn;      // output tiles along the n dimension
  int32_t ntm;      // dW only: output tiles along K
  int64_t mtiles;   // m-tile slots enumerated by the grid (upper bound for fwd / dX)
  void* out2;       // fused GELU forward: gelu'(h), same layout as out
  const void* aux;  // fused GELU backward: gelu'(h), same layout as out
  int32_t chunk;    // dW: rows per reduction chunk (0: one chunk per expert)
  float* partial;   // dW: fp32 partial slabs [split chunks][K][N] when chunk > 0
  // SwiGLU forward: b2 = W_val (b = W_gate), out = hidden, out2 = gate,
  // out3 = value. SwiGLU backward: aux = gate, aux2 = value, out = dgate,
  // out2 = dvalue. Two-part dX: a2 / b2 = dOut / W of the second product.
  const void* a2;
  const void* b2;
  void* out3;
  const void* aux2;
  int32_t split_thr;  // dW: experts with more rows than this are split (when chunk > 0)
  int32_t slab_cap;   // dW: partial slabs the workspace holds (when chunk > 0)
  int32_t stagger;    // start delay of half the workgroups, 100 MHz ticks (0: none)
  // Paired dW with split experts: arrival counters, one per (split expert,
  // 256x256 output tile), tagged with done_epoch; the last chunk of a tile
  // to arrive sums its slabs (fold_split_tile). Null: a reduce pass does.
  unsigned long long* done;
  unsigned long long done_epoch;
};

// Epilogues: plain store; forward GELU (out = gelu(h), out2 = gelu'(h), h
// itself is not stored); backward GELU (out = C * aux, aux = gelu'(h));
// SwiGLU forward (gate and value tiles of one output tile computed side by
// side: out = silu(gate) * value, out2 = gate, out3 = value); SwiGLU
// backward (C = dhidden: out = dgate, out2 = dvalue from aux = gate, aux2 =
// value); two-part dX (plain store, C = dOut @ W^T + dOut2 @ W2^T over one
// concatenated reduction).
enum GemmEpilogue {
  kEpiPlain = 0,
  kEpiGelu = 1,
  kEpiGeluGrad = 2,
  kEpiSwiGLU = 3,
  kEpiSwiGLUGrad = 4,
  kEpiDualK = 5
};

// Logical tile -> (m-tile, n-tile): groups of kGroupM m-tiles, m fastest
// inside a group, so neighbouring logical tiles reuse both A and B panels.
constexpr int kGroupM = 8;
__device__ __forceinline__ void tile_coords(int64_t logical, int64_t mtiles, int ntn, int64_t& mt,
                                            int& nt) {
  const int64_t per_group = (int64_t)kGroupM * ntn;
  const int64_t grp = logical / per_group;
  const int64_t rem = logical - grp * per_group;
  const int64_t gm0 = grp * kGroupM;
  const int64_t gsz = (mtiles - gm0) < kGroupM ? (mtiles - gm0) : kGroupM;
  mt = gm0 + rem % gsz;
  nt = (int)(rem / gsz);
}

// Row-tiled modes (forward, dX): logical tile -> (expert, m-tile within the
// expert, n-tile). Expert e's tiles are the block [P_e * ntn, P_{e+1} * ntn)
// of the logical order (P = s_pref, its m-tile prefix), so that tiles
// which run at the same time share the expert's weight panels. Inside the
// block the expert's m-tiles form ceil(mt_e / kGroupM) groups of balanced
// sizes (never crossing into the next expert, and with no stub group for
// an expert one m-tile past a multiple of kGroupM), each walked m fastest.
__device__ __forceinline__ void expert_tile_coords(int64_t logical, const int32_t* s_pref, int E,
                                                   int ntn, int& e_out, int64_t& mtl, int& nt) {
  const int64_t mt_global = logical / ntn;
  int lo = 0, hi = E - 1;  // largest e with s_pref[e] <= mt_global
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= mt_global) lo = mid;
    else hi = mid - 1;
  }
  const int64_t mt_e = s_pref[lo + 1] - s_pref[lo];
  const int64_t l = logical - (int64_t)s_pref[lo] * ntn;
  const int64_t ng = ceil_div(mt_e, (int64_t)kGroupM);
  const int64_t base = mt_e / ng, rem = mt_e % ng;  // rem groups of base + 1, then base
  const int64_t big = rem * (base + 1) * ntn;       // tiles in the larger groups
  int64_t gi, gsz, gm0;
  if (l < big) {
    gi = l / ((base + 1) * ntn);
    gsz = base + 1;
    gm0 = gi * (base + 1);
  } else {
    gi = (l - big) / (base * ntn);
    gsz = base;
    gm0 = rem * (base + 1) + gi * base;
    gi += rem;
  }
  const int64_t r = l - gm0 * ntn;
  e_out = lo;
  mtl = gm0 + r % gsz;
  nt = (int)(r / gsz);
}

// Start of the logical-tile range of the workgroups before `before` (of G):
// the proportional share, moved to the nearest expert boundary when that
// is within 1/16 of one XCD's share (so an XCD's range holds whole experts
// where the routing allows it, without unbalancing the XCDs).
__device__ __forceinline__ int64_t xcd_range_start(int64_t total, int64_t before, int64_t G,
                                                   const int32_t* s_pref, int E, int ntn) {
  const int64_t b = total * before / G;
  if (b <= 0 || b >= total) return b;
  const int64_t mt = b / ntn;
  int lo = 0, hi = E - 1;  // largest e with s_pref[e] <= mt
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= mt) lo = mid;
    else hi = mid - 1;
  }
  const int64_t e0 = (int64_t)s_pref[lo] * ntn, e1 = (int64_t)s_pref[lo + 1] * ntn;
  const int64_t near = (b - e0 <= e1 - b) ? e0 : e1;
  const int64_t tol = total / 8 / 16;
  const int64_t dist = near > b ? near - b : b - near;
  return dist <= tol ? near : b;
}

// Operand pointers, strides and valid extents of one output tile, for
// elements of storage type U (uint16_t: bf16 / fp16; float).
template <typename U>
struct TileJobT {
  const U* pa;  // A operand origin (tile rows, reduction 0)
  const U* pb;  // B operand origin (tile columns, reduction 0)
  int64_t lda, ldb;
  int64_t rows_valid, cols_valid;  // output rows / columns from the tile origin
  int64_t kred;                    // reduction length
  U* po;
  int64_t ldo;
  U* po2;          // second output (GELU: gelu'(h); SwiGLU: gate / dvalue)
  U* po3;          // SwiGLU forward: value output
  const U* paux;   // GELU backward: gelu'(h); SwiGLU backward: gate
  const U* paux2;  // SwiGLU backward: value
  const U* pa2;    // two-part dX: second A operand origin
  const U* pb2;    // SwiGLU forward: value weights; two-part dX: second W
  int64_t kred1;   // two-part dX: reduction length of the first part
  float* pf;       // dW of a split expert: fp32 partial slab origin (or null)
  const float* pf0;  // split dW: the tile's origin in the expert's first slab
  int32_t nch;       // split dW: the expert's reduction chunks
  int64_t done_idx;  // split dW: the tile's arrival counter
};
typedef TileJobT<uint16_t> TileJob;

// Operands and extents of logical output tile `logical` (< mtiles * ntn).
// For the row-tiled modes s_pref must hold the m-tile prefix of the experts
// (build_m_prefix) and `mtiles` its total.
// SwiGLU forward tiles are BN wide in the MFMA (gate and value halves) and
// BN / 2 wide in the output.
template <int MODE, int BM, int BN, int EPI = kEpiPlain, typename U = uint16_t>
__device__ __forceinline__ void setup_job(const GemmArgs& g, const int32_t* s_pref, int64_t mtiles,
                                          int64_t logical, TileJobT<U>& j) {
  j.po2 = nullptr;
  j.po3 = nullptr;
  j.paux = nullptr;
  j.paux2 = nullptr;
  j.pa2 = nullptr;
  j.pb2 = nullptr;
  j.kred1 = 0;
  j.pf = nullptr;
  j.pf0 = nullptr;
  j.nch = 1;
  j.done_idx = 0;
  int64_t mt = 0;
  int nt = 0;
  if (MODE == kDw) tile_coords(logical, mtiles, g.ntn, mt, nt);
  if (MODE == kDw) {
    // m-tile = (reduction chunk, K tile); s_pref / s_split: build_chunk_prefix.
    const int32_t* s_split = s_pref + (NT_MAX_EXPERTS + 1);
    const int64_t cg = mt / g.ntm;
    const int mtl = (int)(mt % g.ntm);
    int e;
    int64_t r0, r1, c;
    find_m_tile(g.offsets, g.E, g.A, s_pref, cg, e, r0, r1, c);
    // Uniform across the workgroup (read from HBM / LDS): keep them scalar.
    e = __builtin_amdgcn_readfirstlane(e);
    r0 = (int64_t)__builtin_amdgcn_readfirstlane((int)r0);
    r1 = (int64_t)__builtin_amdgcn_readfirstlane((int)r1);
    c = (int64_t)__builtin_amdgcn_readfirstlane((int)c);
    const int nch = s_pref[e + 1] - s_pref[e];
    int64_t c0 = r0, c1 = r1;
    if (nch >= 2) {
      c0 = r0 + c * g.chunk;
      c1 = c0 + g.chunk < r1 ? c0 + g.chunk : r1;
    }
    j.kred = c1 - c0;
    j.pa = static_cast<const U*>(g.a) + c0 * g.K + (int64_t)mtl * BM;
    j.lda = g.K;
    j.pb = static_cast<const U*>(g.b) + c0 * g.N + (int64_t)nt * BN;
    j.ldb = g.N;
    j.rows_valid = g.K - (int64_t)mtl * BM;
    j.cols_valid = g.N - (int64_t)nt * BN;
    const int64_t tile_off = (int64_t)mtl * BM * g.N + (int64_t)nt * BN;
    j.po = static_cast<U*>(g.out) + (int64_t)e * g.K * g.N + tile_off;
    j.ldo = g.N;
    if (nch >= 2) {
      j.pf = g.partial + (int64_t)(s_split[e] + c) * g.K * g.N + tile_off;
      j.pf0 = g.partial + (int64_t)s_split[e] * g.K * g.N + tile_off;
      j.nch = nch;
      // s_split[e] is unique per split expert (they hold two or more slabs)
      j.done_idx = ((int64_t)s_split[e] * g.ntm + mtl) * g.ntn + nt;
    }
  } else {
    int e;
    int64_t r0, r1, mtl;
    expert_tile_coords(logical, s_pref, g.E, g.ntn, e, mtl, nt);
    expert_rows(g.offsets, e, g.A, r0, r1);
    e = __builtin_amdgcn_readfirstlane(e);
    nt = __builtin_amdgcn_readfirstlane(nt);
    r0 = (int64_t)__builtin_amdgcn_readfirstlane((int)r0);
    r1 = (int64_t)__builtin_amdgcn_readfirstlane((int)r1);
    mtl = (int64_t)__builtin_amdgcn_readfirstlane((int)mtl);
    const int64_t row0 = r0 + mtl * BM;
    j.rows_valid = r1 - row0;
    if (MODE == kFwd) {
      constexpr int64_t BNO = EPI == kEpiSwiGLU ? BN / 2 : BN;  // output columns per tile
      const int64_t wofs = (int64_t)e * g.K * g.N + (int64_t)nt * BNO;
      const int64_t oofs = row0 * g.N + (int64_t)nt * BNO;
      j.pa = static_cast<const U*>(g.a) + row0 * g.K;
      j.lda = g.K;
      j.pb = static_cast<const U*>(g.b) + wofs;
      j.ldb = g.N;
      j.cols_valid = g.N - (int64_t)nt * BNO;
      j.kred = g.K;
      j.po = static_cast<U*>(g.out) + oofs;
      j.ldo = g.N;
      if (g.out2) j.po2 = static_cast<U*>(g.out2) + oofs;
      if (EPI == kEpiSwiGLU) {
        j.pb2 = static_cast<const U*>(g.b2) + wofs;
        j.po3 = static_cast<U*>(g.out3) + oofs;
      }
    } else {  // kDx
      const int64_t oofs = row0 * g.K + (int64_t)nt * BN;
      j.pa = static_cast<const U*>(g.a) + row0 * g.N;
      j.lda = g.N;
      j.pb = static_cast<const U*>(g.b) + (int64_t)e * g.K * g.N + (int64_t)nt * BN * g.N;
      j.ldb = g.N;
      j.cols_valid = g.K - (int64_t)nt * BN;
      j.kred = g.N;
      j.po = static_cast<U*>(g.out) + oofs;
      j.ldo = g.K;
      if (g.aux) j.paux = static_cast<const U*>(g.aux) + oofs;
      if (EPI == kEpiSwiGLUGrad) {
        j.paux2 = static_cast<const U*>(g.aux2) + oofs;
        j.po2 = static_cast<U*>(g.out2) + oofs;
      }
      if (EPI == kEpiDualK) {
        j.pa2 = static_cast<const U*>(g.a2) + row0 * g.N;
        j.pb2 = static_cast<const U*>(g.b2) + (int64_t)e * g.K * g.N +
                (int64_t)nt * BN * g.N;
        j.kred1 = g.N;
        j.kred = 2 * g.N;
      }
    }
  }
}

// Global loads of one k-step of both operands of a tile into an LDS stage.
// DUAL 1 (SwiGLU forward): the B tile is two BN/2-column halves, gate
// weights then value weights, for the same output columns. DUAL 2 (two-part
// dX): k-steps below kred1 / BK read (pa, pb), the rest (pa2, pb2).
template <int BM, int BN, bool AK, bool BKM, int BK, int NW, int DUAL = 0>
struct StageLoader {
  typedef OperandTile<BM, AK, BK, NW> TA;
  typedef OperandTile<DUAL == 1 ? BN / 2 : BN, BKM, BK, NW> TB;
  static constexpr int kBBytes = (DUAL == 1 ? 2 : 1) * TB::kBytes;
  static constexpr int kBK = BK;
  static constexpr bool kAK = AK;
  static constexpr bool kBKM = BKM;
  static constexpr int kLoads = TA::kPer + (DUAL == 1 ? 2 : 1) * TB::kPer;  // per wave
  TA ta;
  TB tb;
  const uint16_t* pa;
  const uint16_t* pb;
  const uint16_t* pa2;
  const uint16_t* pb2;
  int64_t lda, ldb, rv, cv, kred, kred1;
  int wave;
  __device__ void init(const TileJob& j, int wave_, int lane) {
    constexpr int kCols = DUAL == 1 ? BN / 2 : BN;
    pa = j.pa;
    pb = j.pb;
    pa2 = j.pa2;
    pb2 = j.pb2;
    lda = j.lda;
    ldb = j.ldb;
    rv = j.rows_valid < BM ? j.rows_valid : BM;
    cv = j.cols_valid < kCols ? j.cols_valid : kCols;
    kred = j.kred;
    kred1 = j.kred1;
    wave = wave_;
    ta.init(lda, wave, lane);
    tb.init(ldb, wave, lane);
  }
  // Issue this wave's loads of k-step kt into the stage at `lds` (A tile
  // first, then the B tile).
  __device__ void issue(int64_t kt, char* lds) const {
    const uint16_t* a = pa;
    const uint16_t* b = pb;
    int64_t kl = kt * BK, klen = kred;
    if (DUAL == 2) {
      klen = kred1;
      if (kl >= kred1) {
        a = pa2;
        b = pb2;
        kl -= kred1;
        klen = kred - kred1;
      }
    }
    const int64_t kleft = klen - kl;
    const int64_t kv = kleft < BK ? kleft : BK;
    // Readable bytes from each tile origin: up to the last valid element.
    const int64_t ra = AK ? ((rv - 1) * lda + kv) * 2 : ((kv - 1) * lda + rv) * 2;
    const int64_t rb = BKM ? ((cv - 1) * ldb + kv) * 2 : ((kv - 1) * ldb + cv) * 2;
    ta.issue(a + (AK ? kl : kl * lda), ra, lds, kv, wave);
    tb.issue(b + (BKM ? kl : kl * ldb), rb, lds + TA::kBytes, kv, wave);
    if (DUAL == 1) tb.issue(pb2 + (BKM ? kl : kl * ldb), rb, lds + TA::kBytes + TB::kBytes, kv, wave);
  }
};

// Epilogue straight from the accumulators (AccTile layout): each lane
// stores 4 consecutive columns (8 bytes) per block, rounded once (RNE).
template <typename T, int TM, int TN>
__device__ __forceinline__ void store_tile(const AccTile<TM, TN>& acc, const TileJob& j, int m0,
                                           int n0, int lane) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int m = m0 + i * 32 + acc_row(gq, lane);
      if (m >= j.rows_valid) continue;
      uint16_t* prow = j.po + (int64_t)m * j.ldo;
#pragma unroll
      for (int jn = 0; jn < TN; ++jn) {
        const int n = n0 + jn * 32 + acc_col(gq, lane);
        if (n >= j.cols_valid) continue;
        const f32x4_t& a = acc[i][jn][gq];
        uint2 pk;
        pk.x = pack2<T>(a[0], a[1]);
        pk.y = pack2<T>(a[2], a[3]);
        *reinterpret_cast<uint2*>(prow + n) = pk;
      }
    }
}

// GELU, erf form, for 16-bit outputs: gelu(x) = x * Phi(x) and
// gelu'(x) = Phi(x) + x * phi(x), with Phi the standard normal CDF,
// Phi(x) = erfc(-x/sqrt2)/2, and phi(x) = exp(-x^2/2)/sqrt(2 pi).
// erfc(z), z >= 0, is the Chebyshev fit of Press et al., Numerical Recipes
// ("erfcc": t = 1/(1 + z/2), erfc(z) = t exp(-z^2 + P(t)), fractional error
// below 1.2e-7 everywhere), evaluated with the hardware exp2 and reciprocal:
// far below the half-ulp of bf16 / fp16 and about half the instructions of
// the library erff. The fp32 / fp64 elementwise path uses erf / exp.
__device__ __forceinline__ float erfc_nonneg(float z, float& ez2) {
  constexpr float kLog2e = 1.4426950408889634f;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.5f, z, 1.0f));
  float p = 0.17087277f;
  p = fmaf(p, t, -0.82215223f);
  p = fmaf(p, t, 1.48851587f);
  p = fmaf(p, t, -1.13520398f);
  p = fmaf(p, t, 0.27886807f);
  p = fmaf(p, t, -0.18628806f);
  p = fmaf(p, t, 0.09678418f);
  p = fmaf(p, t, 0.37409196f);
  p = fmaf(p, t, 1.00002368f);
  p = fmaf(p, t, -1.26551223f);
  ez2 = __builtin_amdgcn_exp2f(-z * z * kLog2e);           // exp(-z^2)
  return t * ez2 * __builtin_amdgcn_exp2f(p * kLog2e);
}
__device__ __forceinline__ float norm_cdf(float x, float& ez2) {
  const float c = 0.5f * erfc_nonneg(fabsf(x) * 0.70710678118654752f, ez2);
  return x >= 0.f ? 1.0f - c : c;
}
// gelu and gelu' of the two 16-bit values of `w` through the erfc fit.
template <typename T>
__device__ __forceinline__ void gelu2_formula(uint32_t w, uint32_t& r, uint32_t& r2) {
  const float x0 = elem<T>::load((uint16_t)(w & 0xffffu));
  const float x1 = elem<T>::load((uint16_t)(w >> 16));
  float e0, e1;
  const float c0 = norm_cdf(x0, e0), c1 = norm_cdf(x1, e1);
  r = pack2<T>(x0 * c0, x1 * c1);
  r2 = pack2<T>(fmaf(x0, e0 * 0.39894228040143268f, c0), fmaf(x1, e1 * 0.39894228040143268f, c1));
}

// gelu and gelu' of the 2 NW bf16 values of `w`: one LDS read each from the
// generated table (kGeluTab, correctly rounded for 2^-16 <= |x| < 8); the
// rare values outside that range take the erfc fit. All 2 NW reads are
// issued before the first result is used.
template <int NW>
__device__ __forceinline__ void gelu_table(const uint32_t (&w)[NW], const uint32_t* tab,
                                           uint32_t (&r)[NW], uint32_t (&r2)[NW]) {
  // Both halves of a word at once (packed 16-bit integer ops). The entry of
  // x = (-1)^s (kGeluTabLo + m) (bf16 bits) is word 2m + s. In a 16-bit lane
  // 2 bits(x) loses the sign bit, so 2 bits(x) + s - 2 kGeluTabLo is that
  // index, wrapping below the range; clamped, it addresses the table.
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const char* tb = reinterpret_cast<const char*>(tab);
  uint32_t t[2 * NW];
  bool out = false;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    const u16x2 x = __builtin_bit_cast(u16x2, w[q]);
    const u16x2 i = (x << 1) + (x >> 15) - (u16x2)(2 * kGeluTabLo);
    const u16x2 c = __builtin_elementwise_min(i, (u16x2)(2 * kGeluTabN - 1));
    out |= __builtin_bit_cast(uint32_t, i) != __builtin_bit_cast(uint32_t, c);
    const uint32_t o = __builtin_bit_cast(uint32_t, c);
    t[2 * q] = *reinterpret_cast<const uint32_t*>(tb + 4 * (o & 0xffffu));
    t[2 * q + 1] = *reinterpret_cast<const uint32_t*>(tb + 4 * (o >> 16));
  }
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    r[q] = __builtin_amdgcn_perm(t[2 * q + 1], t[2 * q], 0x05040100u);   // low halves
    r2[q] = __builtin_amdgcn_perm(t[2 * q + 1], t[2 * q], 0x07060302u);  // high halves
  }
  if (out) {
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const bool o0 = (w[q] & 0x7fffu) - kGeluTabLo >= kGeluTabN;
      const bool o1 = ((w[q] >> 16) & 0x7fffu) - kGeluTabLo >= kGeluTabN;
      if (o0 || o1) {
        uint32_t f, f2;
        gelu2_formula<bf16>(w[q], f, f2);
        const uint32_t keep = (o0 ? 0u : 0xffffu) | (o1 ? 0u : 0xffff0000u);
        r[q] = (r[q] & keep) | (f & ~keep);
        r2[q] = (r2[q] & keep) | (f2 & ~keep);
      }
    }
  }
}

// SwiGLU pieces in fp32, in the order torch evaluates silu and its
// backward: silu(x) = x * sigma(x), silu'(x) = sigma(x) (1 + x (1 - sigma(x))),
// sigma(x) = 1 / (1 + e^-x). Every tensor the reference's unfused graph
// stores is rounded to T where it would be (round<T>).
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return elem<T>::load(elem<T>::store(x));
}
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}
// hidden = round(round(silu(g)) * v) for rounded g, v.
template <typename T>
__device__ __forceinline__ float swiglu_hidden(float g, float v) {
  return round_to<T>(round_to<T>(g * sigmoid_f(g)) * v);
}
// dgate, dvalue from rounded dhidden, gate, value.
template <typename T>
__device__ __forceinline__ void swiglu_grad(float dh, float g, float v, float& dg, float& dv) {
  const float sg = sigmoid_f(g);
  dv = round_to<T>(dh * round_to<T>(g * sg));
  const float ds = round_to<T>(dh * v);
  dg = round_to<T>((ds * sg) * (1.0f + g * (1.0f - sg)));
}

// Stores 8 consecutive 16-bit outputs `v` (already rounded) at byte offset
// `off` of the tile's output (descriptor `ro`; `ro2` for the second GELU
// output), applying the epilogue:
//   kEpiGelu:     out = gelu(v), out2 = gelu'(v)   (v = h, not stored;
//                 through `tab` when TAB, else the erfc fit)
//   kEpiGeluGrad: out = v * gv                     (v = dA, gv = gelu'(h),
//                 loaded by the caller ahead of time)
//   kEpiSwiGLUGrad: out = dgate, out2 = dvalue     (v = dhidden, gv = gate,
//                 gv2 = value)
template <typename T, int EPI, bool TAB>
__device__ __forceinline__ void epilogue8(uint4 v, __amdgpu_buffer_rsrc_t ro,
                                          __amdgpu_buffer_rsrc_t ro2, uint32_t off, uint4 gv,
                                          uint4 gv2, const uint32_t* tab) {
  if (EPI == kEpiPlain || EPI == kEpiDualK) {
    store16(ro, off, v);
    return;
  }
  if (EPI == kEpiSwiGLUGrad) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
    const uint32_t vw[4] = {gv2.x, gv2.y, gv2.z, gv2.w};
    uint32_t rg[4], rv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float dg0, dv0, dg1, dv1;
      swiglu_grad<T>(elem<T>::load((uint16_t)(w[q] & 0xffffu)),
                     elem<T>::load((uint16_t)(gw[q] & 0xffffu)),
                     elem<T>::load((uint16_t)(vw[q] & 0xffffu)), dg0, dv0);
      swiglu_grad<T>(elem<T>::load((uint16_t)(w[q] >> 16)), elem<T>::load((uint16_t)(gw[q] >> 16)),
                     elem<T>::load((uint16_t)(vw[q] >> 16)), dg1, dv1);
      rg[q] = pack2<T>(dg0, dg1);
      rv[q] = pack2<T>(dv0, dv1);
    }
    store16(ro, off, make_uint4(rg[0], rg[1], rg[2], rg[3]));
    store16(ro2, off, make_uint4(rv[0], rv[1], rv[2], rv[3]));
    return;
  }
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t r[4], r2[4];
  if (EPI == kEpiGelu) {
    if constexpr (TAB) {
      gelu_table<4>(w, tab, r, r2);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) gelu2_formula<T>(w[q], r[q], r2[q]);
    }
    store16(ro, off, make_uint4(r[0], r[1], r[2], r[3]));
    store16(ro2, off, make_uint4(r2[0], r2[1], r2[2], r2[3]));
  } else {
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float d0 = elem<T>::load((uint16_t)(w[q] & 0xffffu));
      const float d1 = elem<T>::load((uint16_t)(w[q] >> 16));
      const float g0 = elem<T>::load((uint16_t)(gw[q] & 0xffffu));
      const float g1 = elem<T>::load((uint16_t)(gw[q] >> 16));
      r[q] = pack2<T>(d0 * g0, d1 * g1);
    }
    store16(ro, off, make_uint4(r[0], r[1], r[2], r[3]));
  }
}

// Epilogue through LDS for 64- or 128-column wave blocks (TN = 2 or 4):
// each 32-row sub-tile is rounded (RNE), written to this wave's LDS scratch
// (pitch 32*TN*2 + 16 bytes: one 8-byte write instruction covers 16 rows x
// 16 bytes, which then fall on distinct banks), and read back 16 bytes per
// lane so that every store instruction writes whole 128- or 256-byte row
// segments. `scratch` is epi_bytes<TN, ROWS>() bytes private to the wave;
// LDS operations of one wave complete in order, so no barrier is needed (a
// wavefront fence keeps the compiler from reusing a lane's earlier reads).
// With ROWS = 16 the sub-tile goes through in two halves (blocks 0, 1 hold
// rows 0-15, blocks 2, 3 rows 16-31), halving the scratch.
template <int TN>
constexpr int epi_pitch() { return 64 * TN + 16; }
template <int TN, int ROWS>
constexpr int epi_bytes() { return ROWS * epi_pitch<TN>(); }
// Scratch row that `lane` reads back (16 bytes, chunk lane % (4 TN)) in
// read instruction q. 64-column blocks: 8 lanes per 128-byte row, and the
// two 8-lane halves of each 16-lane LDS cycle take rows 8 apart, which the
// pitch puts 32 banks apart (rows r and r + 1 would share 4 banks, a
// second pass for every read). 128-column blocks: 16 lanes read one whole
// 256-byte row.
template <int TN>
__device__ __forceinline__ int epi_read_row(int q, int lane) {
  if constexpr (TN == 2)
    return (16 * (q >> 1) + (q & 1)) | (lane & 8) | ((lane >> 3) & 6);
  else
    return 4 * q + (lane >> 4);
}
// Store instructions one wave issues in store_tile_lds.
template <int EPI, int ROWS, int TM, int TN>
constexpr int epi_stores() {
  return TM * (32 / ROWS) * (ROWS / (64 / (TN * 4))) *
         (EPI == kEpiGelu || EPI == kEpiSwiGLUGrad ? 2 : 1);
}
template <typename T, int EPI, bool TAB, int ROWS, int TM, int TN>
__device__ __forceinline__ void store_tile_lds(const AccTile<TM, TN>& acc, const TileJob& j,
                                               int m0, int n0, int lane, char* scratch,
                                               const uint32_t* tab) {
  static_assert(TN == 2 || TN == 4, "64- or 128-column wave blocks");
  static_assert(ROWS == 32 || ROWS == 16, "32 or 16 scratch rows");
  constexpr int kPitch = epi_pitch<TN>();
  constexpr int kPasses = 32 / ROWS;
  constexpr int kLanesPerRow = TN * 4;       // 16-byte chunks per row
  constexpr int kRowsPerRead = 64 / kLanesPerRow;
  constexpr int kReads = kPasses * (ROWS / kRowsPerRead);  // 16-byte chunks per lane per sub-tile
  // kEpiGeluGrad: the gelu'(h) chunk that a lane needs for chunk c of
  // sub-tile i+1 is loaded as soon as chunk c of sub-tile i is stored, so
  // its latency hides behind the rest of sub-tile i (kReads chunks in flight,
  // 4 registers each).
  // kEpiSwiGLUGrad loads two inputs (gate and value) the same way.
  constexpr bool kAux = EPI == kEpiGeluGrad || EPI == kEpiSwiGLUGrad;
  constexpr bool kAux2 = EPI == kEpiSwiGLUGrad;
  // In-tile bounds and offsets fit 32 bits (m < 256, ldo < 2^22); 64-bit
  // row indices would be hoisted out of the tile loop and spilled.
  const int rv = (int)(j.rows_valid < 256 ? j.rows_valid : 256);
  const int cv = (int)(j.cols_valid < 256 ? j.cols_valid : 256);
  const uint32_t ldo = (uint32_t)j.ldo;
  uint4 aux[kReads], aux2[kReads];
  // Inputs through buffer descriptors: lanes outside the tile read zeros.
  const __amdgpu_buffer_rsrc_t ra = out_rsrc(kAux ? j.paux : j.po);
  const __amdgpu_buffer_rsrc_t ra2 = out_rsrc(kAux2 ? j.paux2 : j.po);
  auto load_aux = [&](int i, int ps, int q) {
    const int m = m0 + i * 32 + ps * ROWS + epi_read_row<TN>(q, lane);
    const int n = n0 + (lane % kLanesPerRow) * 8;
    const uint32_t off = (m < rv && n < cv) ? ((uint32_t)m * ldo + (uint32_t)n) * 2u : kOob;
    aux[ps * (ROWS / kRowsPerRead) + q] = load16(ra, off);
    aux2[ps * (ROWS / kRowsPerRead) + q] = kAux2 ? load16(ra2, off) : make_uint4(0u, 0u, 0u, 0u);
  };
  if constexpr (kAux) {
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps)
#pragma unroll
      for (int q = 0; q < ROWS / kRowsPerRead; ++q) load_aux(0, ps, q);
  }
  const __amdgpu_buffer_rsrc_t ro = out_rsrc(j.po);
  const __amdgpu_buffer_rsrc_t ro2 =
      out_rsrc(EPI == kEpiGelu || EPI == kEpiSwiGLUGrad ? j.po2 : j.po);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      // the blocks of this pass's rows: all four, or blocks 2 ps and 2 ps + 1
#pragma unroll
      for (int jn = 0; jn < TN; ++jn)
#pragma unroll
        for (int h = 0; h < 4 / kPasses; ++h) {
          const int gq = ps * (4 / kPasses) + h;
          const int c = jn * 32 + acc_col(gq, lane);
          const f32x4_t& a = acc[i][jn][gq];
          uint2 pk;
          pk.x = pack2<T>(a[0], a[1]);
          pk.y = pack2<T>(a[2], a[3]);
          *reinterpret_cast<uint2*>(scratch + (acc_row(gq, lane) % ROWS) * kPitch + c * 2) = pk;
        }
      // Each lane reads back rows other lanes wrote. The compiler models
      // lanes as threads, so without a fence it may forward a lane's earlier
      // read of the same scratch address where that lane wrote nothing (it
      // did so where only some lanes wrote each pass). A wavefront-scope
      // fence emits no instruction (a wave's LDS operations complete in
      // order) and forbids that.
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
      auto chunk_off = [&](int q, uint4& v) -> uint32_t {
        const int rr = epi_read_row<TN>(q, lane);
        const int ch = lane % kLanesPerRow;
        v = *reinterpret_cast<const uint4*>(scratch + rr * kPitch + ch * 16);
        const int m = m0 + i * 32 + ps * ROWS + rr;
        const int n = n0 + ch * 8;
        return (m < rv && n < cv) ? ((uint32_t)m * ldo + (uint32_t)n) * 2u : kOob;
      };
      // GELU through the table: GQ chunks at a time, all 16 GQ table reads of
      // a lane issued before the first result is used, so the latency (and
      // the bank conflicts) of the random lookups overlap. Measured on the
      // C2 layer: GQ = 4 -7.5 us per step, GQ = 2 no gain, against one chunk.
      constexpr int GQ = 4;
      if constexpr (EPI == kEpiGelu && TAB && (ROWS / kRowsPerRead) % GQ == 0) {
#pragma unroll
        for (int q = 0; q < ROWS / kRowsPerRead; q += GQ) {
          uint4 v[GQ];
          uint32_t off[GQ], w[4 * GQ], r[4 * GQ], r2[4 * GQ];
#pragma unroll
          for (int h = 0; h < GQ; ++h) {
            off[h] = chunk_off(q + h, v[h]);
            w[4 * h] = v[h].x; w[4 * h + 1] = v[h].y; w[4 * h + 2] = v[h].z; w[4 * h + 3] = v[h].w;
          }
          gelu_table<4 * GQ>(w, tab, r, r2);
#pragma unroll
          for (int h = 0; h < GQ; ++h) {
            store16(ro, off[h], make_uint4(r[4 * h], r[4 * h + 1], r[4 * h + 2], r[4 * h + 3]));
            store16(ro2, off[h], make_uint4(r2[4 * h], r2[4 * h + 1], r2[4 * h + 2], r2[4 * h + 3]));
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < ROWS / kRowsPerRead; ++q) {
          uint4 v;
          const uint32_t off = chunk_off(q, v);
          epilogue8<T, EPI, TAB>(v, ro, ro2, off, aux[ps * (ROWS / kRowsPerRead) + q],
                                 aux2[ps * (ROWS / kRowsPerRead) + q], tab);
          if constexpr (kAux) {
            if (i + 1 < TM) load_aux(i + 1, ps, q);
          }
        }
      }
    }
  }
}

// Epilogue of the 8-wave kernel with split duties (plain, two-part and
// GELU epilogues): waves NW/2..NW-1 issue every global store of the tile
// and never wait for them, so the stores drain behind the next tile's
// k-loop (vmcnt is per wave and retires in issue order: a wave that also
// issued the operand loads would wait for its stores at its next load
// wait). Each round every wave rounds split_rows() rows of one of its
// 32-row sub-tiles (all of it, or a 16-row half) into its LDS scratch region
// (for the GELU epilogue it also computes gelu and gelu' of the rounded
// values there, so that VALU work is shared by all the waves, and writes
// both into two regions); after a barrier storer wave w reads back its own
// region(s) and those of wave w - NW/2 (16 bytes per lane, whole 128-byte
// row segments) and stores them; a second barrier frees the scratch for the
// next round.
// `scratch` holds split_scratch_bytes<TN, EPI>(NW) bytes.
//
// Rows per round: whole 32-row sub-tiles where eight waves' regions fit in
// the idle 64 KiB stage (plain and two-part epilogues on 64-column wave
// blocks: 36 KiB), halving the rounds and their barriers; 16-row halves for
// the GELU epilogue's two regions and 128-column wave blocks. Measured on
// MI355X, bit-identical: C2 layer step 0.9947 -> 0.9879 ms (mean of four
// alternations), C4 level.
template <int TN, int EPI = kEpiPlain>
constexpr int split_rows() { return (EPI == kEpiGelu || TN == 4) ? 16 : 32; }
template <int TN, int EPI = kEpiPlain>
constexpr int split_scratch_bytes(int nw) {
  return (EPI == kEpiGelu ? 2 : 1) * nw * split_rows<TN, EPI>() * epi_pitch<TN>();
}
template <typename T, int TM, int TN, int WGN, int WM, int WN, int NW, int EPI = kEpiPlain,
          bool TAB = false>
__device__ __forceinline__ void store_tile_split(const AccTile<TM, TN>& acc, const TileJob& j,
                                                 int wave, int lane, char* scratch,
                                                 const uint32_t* tab = nullptr) {
  static_assert(TN == 2 || TN == 4, "64- or 128-column wave blocks");
  static_assert(EPI == kEpiPlain || EPI == kEpiDualK || EPI == kEpiGelu,
                "plain, two-part or GELU epilogue");
  constexpr bool kGelu = EPI == kEpiGelu;
  constexpr int ROWS = split_rows<TN, EPI>();
  constexpr int kPitch = epi_pitch<TN>();
  constexpr int kRegion = ROWS * kPitch;  // one wave's rows of a round
  constexpr int kOut2 = NW * kRegion;     // GELU: gelu' regions follow the gelu ones
  constexpr int kLanesPerRow = TN * 4;
  constexpr int kRowsPerRead = 64 / kLanesPerRow;
  constexpr int kQ = ROWS / kRowsPerRead;
  constexpr int NL = NW / 2;
  const bool storer = wave >= NL;
  // In-tile bounds and offsets fit 32 bits (m < 256, ldo < 2^22).
  const int rv = (int)(j.rows_valid < 256 ? j.rows_valid : 256);
  const int cv = (int)(j.cols_valid < 256 ? j.cols_valid : 256);
  const uint32_t ldo = (uint32_t)j.ldo;
  char* mine = scratch + wave * kRegion;
  const __amdgpu_buffer_rsrc_t ro = out_rsrc(j.po);
  const __amdgpu_buffer_rsrc_t ro2 = out_rsrc(kGelu ? j.po2 : j.po);
  constexpr int kG = ROWS / 8;  // 16x16 blocks per 32-column block in one round
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int ps = 0; ps < 32 / ROWS; ++ps) {
      // blocks ps kG .. ps kG + kG - 1 of each column block: every lane
      // holds 4 kG values of a row of this round per column block
      uint32_t w[2 * TN * kG];
#pragma unroll
      for (int jn = 0; jn < TN; ++jn)
#pragma unroll
        for (int h = 0; h < kG; ++h) {
          const f32x4_t& a = acc[i][jn][ps * kG + h];
          w[2 * (kG * jn + h)] = pack2<T>(a[0], a[1]);
          w[2 * (kG * jn + h) + 1] = pack2<T>(a[2], a[3]);
        }
      auto put = [&](int jn, int h, char* region, uint32_t lo, uint32_t hi) {
        const int gq = ps * kG + h;
        const int c = jn * 32 + acc_col(gq, lane);
        *reinterpret_cast<uint2*>(region + (acc_row(gq, lane) % ROWS) * kPitch + c * 2) =
            make_uint2(lo, hi);
      };
      if constexpr (kGelu) {
        // gelu and gelu' of the rounded h (h itself is not stored)
        uint32_t g1[2 * TN * kG], g2[2 * TN * kG];
        if constexpr (TAB) {
          gelu_table<2 * TN * kG>(w, tab, g1, g2);
        } else {
#pragma unroll
          for (int q = 0; q < 2 * TN * kG; ++q) gelu2_formula<T>(w[q], g1[q], g2[q]);
        }
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
          for (int h = 0; h < kG; ++h) {
            const int q = kG * jn + h;
            put(jn, h, mine, g1[2 * q], g1[2 * q + 1]);
            put(jn, h, mine + kOut2, g2[2 * q], g2[2 * q + 1]);
          }
      } else {
#pragma unroll
        for (int jn = 0; jn < TN; ++jn)
#pragma unroll
          for (int h = 0; h < kG; ++h) {
            const int q = kG * jn + h;
            put(jn, h, mine, w[2 * q], w[2 * q + 1]);
          }
      }
      __syncthreads();
      if (storer) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int src = h == 0 ? wave - NL : wave;
          const int sm0 = (src / WGN) * WM + i * 32 + ps * ROWS;
          const int sn0 = (src % WGN) * WN;
          const char* sp = scratch + src * kRegion;
#pragma unroll
          for (int q = 0; q < kQ; ++q) {
            const int rr = epi_read_row<TN>(q, lane);
            const int ch = lane % kLanesPerRow;
            const int m = sm0 + rr;
            const int n = sn0 + ch * 8;
            const uint32_t off =
                (m < rv && n < cv) ? ((uint32_t)m * ldo + (uint32_t)n) * 2u : kOob;
            store16(ro, off, *reinterpret_cast<const uint4*>(sp + rr * kPitch + ch * 16));
            if constexpr (kGelu)
              store16(ro2, off, *reinterpret_cast<const uint4*>(sp + kOut2 + rr * kPitch + ch * 16));
          }
        }
      }
      __syncthreads();
    }
  }
}

// fp32 partial of a split dW tile: each lane stores its 4 consecutive
// columns of a row as one 16-byte write; the reduce pass rounds later.
template <int TM, int TN>
__device__ __forceinline__ void store_partial(const AccTile<TM, TN>& acc, const TileJob& j,
                                              int m0, int n0, int lane) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int m = m0 + i * 32 + acc_row(gq, lane);
      if (m >= j.rows_valid) continue;
      float* prow = j.pf + (int64_t)m * j.ldo;
#pragma unroll
      for (int jn = 0; jn < TN; ++jn) {
        const int n = n0 + jn * 32 + acc_col(gq, lane);
        if (n >= j.cols_valid) continue;
        const f32x4_t& a = acc[i][jn][gq];
        *reinterpret_cast<float4*>(prow + n) = make_float4(a[0], a[1], a[2], a[3]);
      }
    }
}

// On 128-register wave tiles every accumulator register is zeroed by an
// instruction of its own that the compiler cannot see through. With a
// literal (or one shared) zero it specialises the peeled first k-step into
// MFMAs on a common zero operand whose results land in other registers than
// the loop's, and the reshuffle took those kernels to 256 registers and
// spills. Smaller tiles keep their accumulators in AGPRs, where the opaque
// (VGPR) zeros cost more than they save.
__device__ __forceinline__ float opaque_zero() {
  float z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}
template <typename T, int TM, int TN>
__device__ __forceinline__ void zero_acc(AccTile<TM, TN>& acc) {
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if constexpr (TM * TN >= 8)
          acc[i][j][g] = f32x4_t{opaque_zero(), opaque_zero(), opaque_zero(), opaque_zero()};
        else
          acc[i][j][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
}

// Persistent grouped GEMM. Each workgroup of WGM x WGN waves walks a range
// of BM x BN output tiles; each wave owns a (BM/WGM) x (BN/WGN) block of
// 16x16 MFMA blocks (AccTile). The MFMA is issued with the B fragment as its
// first operand, so each lane's accumulator holds 4 consecutive output
// columns of one output row. K advances BK per iteration through a ring of NS LDS
// stages: the loads of stage kt+NS-1 are issued right after the barrier of
// iteration kt and have NS-1 iterations of MFMAs to land. The first stages
// of a workgroup's next tile are issued before the current tile's results
// are stored, so their latency hides behind the epilogue.
//
// Tiles are dealt to XCDs in contiguous ranges (workgroup b runs on XCD
// b % 8), so tiles that share operand panels share that XCD's L2; inside a
// range, tile_coords walks groups of kGroupM m-tiles with m fastest.
// LDS of one tile configuration (declared by the kernels that run it).
template <typename T, int MODE, int BM, int BN, int WGM, int WGN, int BK, int NS, int EPI,
          bool SPLIT>
struct GemmLds {
  static constexpr int kDual = EPI == kEpiSwiGLU ? 1 : (EPI == kEpiDualK ? 2 : 0);
  static constexpr int NL = SPLIT ? WGM * WGN / 2 : WGM * WGN;
  typedef StageLoader<BM, BN, MODE != kDw, MODE == kDx, BK, NL, kDual> Loader;
  static constexpr int kStage = Loader::TA::kBytes + Loader::kBBytes;
  static constexpr int kSmem = NS * kStage;
  // fwd / dX: m-tile prefix of the experts; dW: chunk prefix and split prefix.
  static constexpr int kPref = (MODE == kDw ? 2 : 1) * (NT_MAX_EXPERTS + 1);
  // bf16 GELU epilogue of the 256-row tiles: the gelu / gelu' table in LDS
  // (the 128-row tiles run two workgroups per CU, which the table would not
  // leave room for). It sits below the stages, at an LDS address under 64 KiB,
  // so its base folds into the lookups' immediate offset.
  static constexpr bool kTab = EPI == kEpiGelu && std::is_same<T, bf16>::value && BM == 256;
  static constexpr int kTabOff = kTab ? (kGeluTabWords * 4 + 1023) / 1024 * 1024 : 0;
};

// The next of `limit` items from a counter tagged with the launch's epoch:
// high 40 bits the epoch, low 24 the number of claims so far. A claim is one
// atomic add. An add that finds a word from before this launch (another
// epoch: an earlier launch's count, or any other leftover data) installs
// this launch's epoch with one claim taken, by compare-and-swap; if another
// workgroup installed it first, the claim is counted again by an add. So the
// counters need no clearing before a launch, and only the first claims of a
// launch can take more than one atomic.
constexpr int kClaimBits = 24;
__device__ int64_t claim_tagged(unsigned long long* ctr, unsigned long long epoch,
                                int64_t limit) {
  constexpr unsigned long long kCount = (1ull << kClaimBits) - 1;
  unsigned long long v = atomicAdd(ctr, 1ull);
  while ((v >> kClaimBits) != epoch) {
    const unsigned long long cur =
        __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((cur >> kClaimBits) == epoch) {
      v = atomicAdd(ctr, 1ull);
    } else if (atomicCAS(ctr, cur, (epoch << kClaimBits) | 1ull) == cur) {
      return limit > 0 ? 0 : -1;
    }
  }
  const int64_t cnt = (int64_t)(v & kCount);
  return cnt < limit ? cnt : -1;
}

// Split dW tile of a paired launch, after its fp32 partial is stored: every
// wave publishes its stores at agent scope (the slabs are read by a
// workgroup on any XCD), then one thread counts the chunk on the tile's
// counter. The last of the expert's nch chunks to arrive sums the nch slabs
// in chunk order, the order and arithmetic of dw_reduce_kernel, and writes
// the dW tile (8 columns per thread and step; K and N are multiples of 8).
// `s_flag` is an LDS slot.
template <typename T>
__device__ void fold_split_tile(const GemmArgs& g, const TileJob& j, int64_t* s_flag) {
  __threadfence();  // this wave's partial stores complete and written back
  __syncthreads();
  if (threadIdx.x == 0) {
    // release (after the barrier: every wave's stores), count, and on the
    // last arrival acquire, before the flag hands the slabs to every wave
    __threadfence();
    const bool last = claim_tagged(g.done + j.done_idx, g.done_epoch, j.nch) == j.nch - 1;
    if (last) __threadfence();
    *s_flag = last ? 1 : 0;
  }
  __syncthreads();
  if (*s_flag == 0) return;
  __threadfence();  // acquire in every wave that reads the other chunks' partials
  const int64_t KN = g.K * g.N;
  const int rows = (int)(j.rows_valid < 256 ? j.rows_valid : 256);
  const int vecs = (int)((j.cols_valid < 256 ? j.cols_valid : 256) / 8);
  typename elem<T>::storage* out = reinterpret_cast<typename elem<T>::storage*>(j.po);
  for (int idx = threadIdx.x; idx < rows * vecs; idx += blockDim.x) {
    const int m = idx / vecs, n = (idx % vecs) * 8;
    const float* src = j.pf0 + (int64_t)m * g.N + n;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < j.nch; ++c) {
      const float4 u = *reinterpret_cast<const float4*>(src + (int64_t)c * KN);
      const float4 v = *reinterpret_cast<const float4*>(src + (int64_t)c * KN + 4);
      acc[0] += u.x; acc[1] += u.y; acc[2] += u.z; acc[3] += u.w;
      acc[4] += v.x; acc[5] += v.y; acc[6] += v.z; acc[7] += v.w;
    }
    uint4 r;
    r.x = (uint32_t)elem<T>::store(acc[0]) | ((uint32_t)elem<T>::store(acc[1]) << 16);
    r.y = (uint32_t)elem<T>::store(acc[2]) | ((uint32_t)elem<T>::store(acc[3]) << 16);
    r.z = (uint32_t)elem<T>::store(acc[4]) | ((uint32_t)elem<T>::store(acc[5]) << 16);
    r.w = (uint32_t)elem<T>::store(acc[6]) | ((uint32_t)elem<T>::store(acc[7]) << 16);
    *reinterpret_cast<uint4*>(out + (int64_t)m * j.ldo + n) = r;
  }
}

// The tile loop of workgroup `wg` of `G` that share this GEMM (the kernel's
// body; gg_pair_kernel runs two of them side by side).
template <typename T, int MODE, int BM, int BN, int WGM, int WGN, int BK, int NS, int EPI,
          bool SPLIT, bool DYN = false>
__device__ __forceinline__ void gemm_tiles(const GemmArgs& g, int64_t wg, int64_t G, char* smem,
                                           int32_t* s_pref, uint32_t* s_gtab,
                                           unsigned long long* dyn = nullptr,
                                           int64_t* s_next = nullptr,
                                           unsigned long long epoch = 0) {
  constexpr int NW = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 32, TN = WN / 32;
  static_assert(TM >= 1 && TN >= 1, "wave tile below one MFMA tile");
  static_assert(NS >= 2, "at least two LDS stages");
  // Only the 64-deep k-step is built and tested: 32-deep k-steps with 2 to 4
  // stages give the same bits (measured on MI355X) but were 7-13% slower at
  // C4 and slower at C3.
  static_assert(BK == 64, "k-step depth 64");
  constexpr bool kAK = MODE != kDw;   // A operand K-major?
  constexpr bool kBKm = MODE == kDx;  // B operand K-major?
  constexpr int kDual = EPI == kEpiSwiGLU ? 1 : (EPI == kEpiDualK ? 2 : 0);
  static_assert(kDual != 1 || (MODE == kFwd && TN % 2 == 0), "SwiGLU: forward, gate|value halves");
  static_assert(kDual != 2 || MODE == kDx, "two-part reduction: dX only");
  // Split duties (SPLIT; 8 waves, plain epilogues): waves 0..NW/2-1 issue
  // every operand load, the others every output store (store_tile_split).
  constexpr bool kSplit = SPLIT;
  static_assert(!SPLIT || (NW == 8 && MODE != kDw && kDual != 1 &&
                           (EPI == kEpiPlain || EPI == kEpiDualK || EPI == kEpiGelu) &&
                           (WN / 32 == 2 || WN / 32 == 4)),
                "split duties: 8-wave plain, two-part or GELU epilogues");
  constexpr int NL = kSplit ? NW / 2 : NW;  // waves that issue operand loads
  typedef StageLoader<BM, BN, kAK, kBKm, BK, NL, kDual> Loader;
  constexpr int kStage = Loader::TA::kBytes + Loader::kBBytes;
  constexpr int kLoadsPerStage = Loader::kLoads;  // per loading wave
  constexpr bool kTab = GemmLds<T, MODE, BM, BN, WGM, WGN, BK, NS, EPI, SPLIT>::kTab;

  int64_t mtiles;
  if (MODE != kDw) {
    build_m_prefix(g.offsets, g.E, g.A, BM, s_pref);
    mtiles = s_pref[g.E];
  } else {
    build_chunk_prefix(g.offsets, g.E, g.A, g.chunk, g.split_thr, g.slab_cap, s_pref,
                       s_pref + (NT_MAX_EXPERTS + 1));
    mtiles = (int64_t)s_pref[g.E] * g.ntm;
  }
  const int64_t total = mtiles * g.ntn;
  constexpr int kXcd = 8;
  const int xcd = (int)(wg % kXcd);
  const int64_t q = G / kXcd, r = G % kXcd;
  const int64_t before = xcd * q + (xcd < r ? xcd : r);
  const int64_t nbx = q + (xcd < r ? 1 : 0);  // workgroups on this XCD
  // Row-tiled modes snap the XCD ranges to expert boundaries where they can.
  const int64_t t_end = MODE == kDw ? total * (before + nbx) / G
                                    : xcd_range_start(total, before + nbx, G, s_pref, g.E, g.ntn);
  int64_t logical = (MODE == kDw ? total * before / G
                                 : xcd_range_start(total, before, G, s_pref, g.E, g.ntn)) +
                    wg / kXcd;
  // Dynamic order (DYN): the tiles form kXcd contiguous parts;
  // workgroup wg takes the next tile of its XCD's part from the epoch-tagged
  // counter dyn[p] (claim_tagged), then those of the following parts. One
  // thread claims, the LDS slot *s_next publishes it at a barrier.
  auto claim = [&]() -> int64_t {
    for (int i = 0; i < kXcd; ++i) {
      const int p = (xcd + i) % kXcd;
      const int64_t p0 = total * p / kXcd, p1 = total * (p + 1) / kXcd;
      if (p1 <= p0) continue;
      const int64_t c = claim_tagged(dyn + p, epoch, p1 - p0);
      if (c >= 0) return p0 + c;
    }
    return -1;
  };
  // The claimed index is the same for the whole workgroup: keep it scalar.
  auto uniform = [](int64_t v) -> int64_t {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  if constexpr (DYN) {
    if (threadIdx.x == 0) *s_next = claim();
    __syncthreads();
    logical = uniform(*s_next);
    if (logical < 0) return;
  } else {
    (void)claim;
    (void)uniform;
    if (logical >= t_end) return;
  }

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave / WGN, wn = wave % WGN;
  if constexpr (kTab) {
    // Published by the barrier of the first k-step (or the one before the
    // first epilogue).
    for (int i = threadIdx.x; i < kGeluTabWords; i += NW * kWave) s_gtab[i] = kGeluTab[i];
  }
  // B fragments: one reader over the BN-column tile, or (SwiGLU) one per
  // half: sub-tiles j < TN/2 are gate columns, the others the value columns
  // of the same outputs.
  constexpr int kBRows = kDual == 1 ? BN / 2 : BN;
  constexpr int kBTs = kDual == 1 ? TN / 2 : TN;
  constexpr int kAB = 2 * TM, kBB = 2 * TN;  // 16-row A and 16-column B blocks
  constexpr int kKS = BK / 32;               // 32-deep substeps per k-step
  FragReader<BM, kAK, kAB, BK> fa;
  FragReader<kBRows, kBKm, 2 * kBTs, BK> fb;
  fa.init(wm * WM, lane);
  fb.init(wn * (WN * kBRows / BN), lane);

  const bool loader = !kSplit || wave < NL;
  TileJob job;
  setup_job<MODE, BM, BN, EPI>(g, s_pref, mtiles, logical, job);
  Loader ld;
  ld.init(job, wave, lane);
  int64_t nk = ceil_div(job.kred, BK);
  if (loader) {
#pragma unroll
    for (int s0 = 0; s0 < NS - 1; ++s0)
      if (s0 < nk) ld.issue(s0, smem + s0 * kStage);
  }

  typedef typename mfma_op<T>::vec vec;
  AccTile<TM, TN> acc;
  // The operand with fewer blocks per wave ("held") is read a substep ahead
  // into a second register set; the other one streams, each block read two
  // blocks ahead of its MFMAs, across the substeps of the k-step (3 blocks
  // of registers instead of 2 x 2 TM). Scheduling fences keep that order, so
  // the LDS latency hides behind the MFMAs of the blocks before.
  constexpr bool kStreamA = TM >= TN;
  constexpr int kHeld = kStreamA ? kBB : kAB;
  constexpr int kStr = kStreamA ? kAB : kBB;
  auto compute = [&](const char* sa, const char* sb) {
    auto read_a = [&](int ib, int ks) { return fa.template read<vec>(sa, ib, ks); };
    auto read_b = [&](int jb, int ks) {
      if (kDual == 1 && jb >= 2 * kBTs)
        return fb.template read<vec>(sb + Loader::TB::kBytes, jb - 2 * kBTs, ks);
      return fb.template read<vec>(sb, jb, ks);
    };
    auto read_held = [&](int h, int ks) { return kStreamA ? read_b(h, ks) : read_a(h, ks); };
    auto read_str = [&](int n) {
      return kStreamA ? read_a(n % kStr, n / kStr) : read_b(n % kStr, n / kStr);
    };
    vec held[2][kHeld];
#pragma unroll
    for (int h = 0; h < kHeld; ++h) held[0][h] = read_held(h, 0);
    vec s0 = read_str(0), s1 = read_str(1);
#pragma unroll
    for (int n = 0; n < kKS * kStr; ++n) {
      const int ks = n / kStr, x = n % kStr, cur = ks & 1;
      if (x == 0 && ks + 1 < kKS) {
#pragma unroll
        for (int h = 0; h < kHeld; ++h) held[cur ^ 1][h] = read_held(h, ks + 1);
      }
      vec s2 = s1;
      if (n + 2 < kKS * kStr) s2 = read_str(n + 2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int h = 0; h < kHeld; ++h) {
        const int ib = kStreamA ? x : h, jb = kStreamA ? h : x;
        f32x4_t& c = acc[ib >> 1][jb >> 1][2 * (ib & 1) + (jb & 1)];
        c = kStreamA ? mfma_op<T>::run(held[cur][h], s0, c) : mfma_op<T>::run(s0, held[cur][h], c);
      }
      __builtin_amdgcn_sched_barrier(0);
      s0 = s1;
      s1 = s2;
    }
  };

  // The LDS-staged epilogue issues kStores store instructions per wave after
  // the next tile's first stages; the first wait of that tile lets them stay
  // in flight.
  // SwiGLU stores three outputs of TN/2 sub-tiles each (gate, value, hidden).
  constexpr int TNO = kDual == 1 ? TN / 2 : TN;
  constexpr bool kLdsEpi = TNO == 2 || TNO == 4;
  constexpr int kRows = !kLdsEpi || NW * epi_bytes<TNO, 32>() <= kStage ? 32 : 16;
  constexpr int kStoresAll =
      !kLdsEpi ? 0
               : (kDual == 1 ? 3 * epi_stores<kEpiPlain, kRows, TM, TNO>()
                             : epi_stores<EPI, kRows, TM, TN>());
  // Beyond the counter's range the next tile simply waits for the stores.
  constexpr bool kDrain = (NS - 2) * kLoadsPerStage + kStoresAll < 64;
  constexpr int kStores = kDrain ? kStoresAll : 0;
  bool stores_out = false;
  while (true) {
    zero_acc<T>(acc);
    // Ring pipeline. Iteration kt waits until its own stage has landed (the
    // loads of up to NS-2 younger stages may stay in flight: vector memory
    // operations retire in issue order), and the barrier then publishes the
    // stage to every wave and retires every wave's reads of the slot that
    // is refilled next.
    int slot = 0;
    for (int64_t kt = 0; kt < nk; ++kt) {
      const int64_t younger = nk - 1 - kt;  // stages issued after this one (capped below)
      if (!loader) {
        // storer waves have no loads to wait for (only their stores)
      } else if (kt == 0 && stores_out) {
        if (younger >= NS - 2) {
          wait_vmcnt<(NS - 2) * kLoadsPerStage + kStores>();
        } else if (NS > 3 && younger == 2) {
          wait_vmcnt<(NS > 3 ? 2 : 0) * kLoadsPerStage + kStores>();
        } else if (NS > 2 && younger == 1) {
          wait_vmcnt<(NS > 2 ? 1 : 0) * kLoadsPerStage + kStores>();
        } else {
          wait_vmcnt<kStores>();
        }
      } else if (younger >= NS - 2) {
        wait_vmcnt<(NS - 2) * kLoadsPerStage>();
      } else if (NS > 3 && younger == 2) {
        wait_vmcnt<(NS > 3 ? 2 : 0) * kLoadsPerStage>();
      } else if (NS > 2 && younger == 1) {
        wait_vmcnt<(NS > 2 ? 1 : 0) * kLoadsPerStage>();
      } else {
        wait_vmcnt<0>();
      }
      __syncthreads();
      if (loader && kt + NS - 1 < nk) {
        int fill = slot + NS - 1;
        if (fill >= NS) fill -= NS;
        ld.issue(kt + NS - 1, smem + fill * kStage);
      }
      const char* cur = smem + slot * kStage;
      compute(cur, cur + Loader::TA::kBytes);
      slot = slot + 1 == NS ? 0 : slot + 1;
    }
    // Every wave is done with the stages; start the next tile's loads, then
    // store this tile.
    int64_t next = logical + nbx;
    if constexpr (DYN) {
      if (threadIdx.x == 0) *s_next = claim();
    }
    __syncthreads();
    if constexpr (DYN) next = uniform(*s_next);
    const bool more = DYN ? next >= 0 : next < t_end;
    TileJob nj;
    if (more) {
      setup_job<MODE, BM, BN, EPI>(g, s_pref, mtiles, next, nj);
      ld.init(nj, wave, lane);
      nk = ceil_div(nj.kred, BK);
      if (loader) {
#pragma unroll
        for (int s0 = 0; s0 < NS - 1; ++s0)
          if (s0 < nk) ld.issue(s0, smem + s0 * kStage);
      }
    }
    static_assert(kLdsEpi || EPI == kEpiPlain, "fused epilogues use the LDS-staged store");
    stores_out = false;
    if (MODE == kDw && job.pf != nullptr) {
      store_partial(acc, job, wm * WM, wn * WN, lane);
      if (g.done != nullptr) {
        // the fold's fields are set up again here, not kept live across the k-loop
        TileJob fj;
        setup_job<MODE, BM, BN, EPI>(g, s_pref, mtiles, logical, fj);
        fold_split_tile<T>(g, fj, s_next);
      }
    } else if constexpr (kDual == 1) {
      // gate and value rounded as the unfused GEMMs would store them, then
      // hidden = round(round(silu(gate)) * value); three LDS-staged stores.
      static_assert(NW * epi_bytes<TNO, kRows>() <= kStage, "epilogue scratch fits one stage");
      char* scr = smem + (NS - 1) * kStage + wave * epi_bytes<TNO, kRows>();
      const int n0 = wn * (WN / 2);
      AccTile<TM, TNO> part;
      TileJob jo = job;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jn = 0; jn < TNO; ++jn)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              acc[i][jn][gq][v] = round_to<T>(acc[i][jn][gq][v]);
              acc[i][jn + TNO][gq][v] = round_to<T>(acc[i][jn + TNO][gq][v]);
              part[i][jn][gq][v] = acc[i][jn][gq][v];
            }
      jo.po = job.po2;
      store_tile_lds<T, kEpiPlain, false, kRows>(part, jo, wm * WM, n0, lane, scr, s_gtab);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jn = 0; jn < TNO; ++jn)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) part[i][jn][gq] = acc[i][jn + TNO][gq];
      jo.po = job.po3;
      store_tile_lds<T, kEpiPlain, false, kRows>(part, jo, wm * WM, n0, lane, scr, s_gtab);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jn = 0; jn < TNO; ++jn)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              part[i][jn][gq][v] = swiglu_hidden<T>(acc[i][jn][gq][v], acc[i][jn + TNO][gq][v]);
      store_tile_lds<T, kEpiPlain, false, kRows>(part, job, wm * WM, n0, lane, scr, s_gtab);
      stores_out = kDrain && more;
    } else if constexpr (kSplit) {
      static_assert(split_scratch_bytes<TN, EPI>(NW) <= kStage, "split scratch fits one stage");
      store_tile_split<T, TM, TN, WGN, WM, WN, NW, EPI, kTab>(acc, job, wave, lane,
                                                              smem + (NS - 1) * kStage, s_gtab);
    } else if constexpr (kLdsEpi) {
      // The ring's last slot is idle until the next tile's first iteration.
      static_assert(NW * epi_bytes<TN, kRows>() <= kStage, "epilogue scratch fits one stage");
      store_tile_lds<T, EPI, kTab, kRows>(acc, job, wm * WM, wn * WN, lane,
                                          smem + (NS - 1) * kStage + wave * epi_bytes<TN, kRows>(),
                                          s_gtab);
      stores_out = kDrain && more;
    } else {
      store_tile<T>(acc, job, wm * WM, wn * WN, lane);
    }
    if (!more) break;
    job = nj;
    logical = next;
  }
}

// Every tile of a short-reduction GEMM takes the same time, so without a
// delay all CUs reach their epilogues together and the chip writes in bursts
// at HBM speed while the matrix cores wait. Half of each XCD's workgroups
// (odd blockIdx / 8) start `ticks` late, a bounded wait on the constant
// 100 MHz counter, and their stores then overlap the other half's main loops.
__device__ __forceinline__ void stagger_wait(int32_t ticks) {
  if (ticks > 0 && ((blockIdx.x / 8) & 1)) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < (uint64_t)ticks) __builtin_amdgcn_s_sleep(8);
  }
}

template <typename T, int MODE, int BM, int BN, int WGM, int WGN, int BK, int NS, int EPI,
          bool SPLIT>
__global__ void __launch_bounds__(WGM * WGN * kWave)
gg_mfma_kernel(GemmArgs g) {
  stagger_wait(g.stagger);
  typedef GemmLds<T, MODE, BM, BN, WGM, WGN, BK, NS, EPI, SPLIT> L;
  // [GELU table | stages]; the stages stay 1 KiB aligned.
  __shared__ __attribute__((aligned(1024))) char lds[L::kTabOff + L::kSmem];
  __shared__ int32_t s_pref[L::kPref];
  gemm_tiles<T, MODE, BM, BN, WGM, WGN, BK, NS, EPI, SPLIT>(
      g, blockIdx.x, gridDim.x, lds + L::kTabOff, s_pref, reinterpret_cast<uint32_t*>(lds));
}

// A dW and a dX-type GEMM in one launch, side by side: workgroups [0, nw)
// walk the dW's tiles (gw, static ranges), then every workgroup takes dX
// tiles (gx) in the dynamic order, so the workgroups that started on the dX
// keep the device busy while the dW's run, and any imbalance in the dW (a
// skewed expert's chunks) is absorbed. Both on 256x256 tiles with 8 waves;
// nw is a multiple of 8, so the dW part keeps the XCD mapping (workgroup b
// runs on XCD b % 8). dyn: kXcd claim counters (claim_tagged, with this
// launch's epoch).
template <typename T, int EPIX, bool SPLITX>
__global__ void __launch_bounds__(8 * kWave)
gg_pair_kernel(GemmArgs gw, GemmArgs gx, int32_t nw, unsigned long long* dyn,
               unsigned long long epoch) {
  typedef GemmLds<T, kDw, 256, 256, 2, 4, 64, 2, kEpiPlain, false> LW;
  typedef GemmLds<T, kDx, 256, 256, 2, 4, 64, 2, EPIX, SPLITX> LX;
  static_assert(!LX::kTab, "no GELU table in the pair kernel");
  __shared__ __attribute__((aligned(1024))) char smem[LW::kSmem > LX::kSmem ? LW::kSmem : LX::kSmem];
  __shared__ int32_t s_pref[LW::kPref > LX::kPref ? LW::kPref : LX::kPref];
  __shared__ uint32_t s_gtab[1];
  __shared__ int64_t s_next;
  if ((int32_t)blockIdx.x < nw) {
    gemm_tiles<T, kDw, 256, 256, 2, 4, 64, 2, kEpiPlain, false>(gw, blockIdx.x, nw, smem, s_pref,
                                                               s_gtab, nullptr, &s_next);
    __syncthreads();  // LDS is reused by the dX tiles below
  } else {
    stagger_wait(gx.stagger);  // of the workgroups that start on the dX
  }
  gemm_tiles<T, kDx, 256, 256, 2, 4, 64, 2, EPIX, SPLITX, true>(gx, blockIdx.x, gridDim.x, smem,
                                                              s_pref, s_gtab, dyn, &s_next, epoch);
}

// ------------------------------------------------------- generic FMA kernel

template <typename T>
struct acc_type {
  typedef float type;
};
template <>
struct acc_type<double> {
  typedef double type;
};

template <typename T>
__device__ __forceinline__ typename acc_type<T>::type to_acc(typename elem<T>::storage v) {
  return elem<T>::load(v);
}
template <>
__device__ __forceinline__ double to_acc<double>(double v) {
  return v;
}
template <typename T>
__device__ __forceinline__ typename elem<T>::storage from_acc(typename acc_type<T>::type v) {
  return elem<T>::store(v);
}
template <>
__device__ __forceinline__ double from_acc<double>(double v) {
  return v;
}

// ------------------------------------------------------ fp32 MFMA GEMM
// fp32 operands on v_mfma_f32_32x32x2_f32 (64 MACs per lane, 2048 per
// instruction). Tiles of 128x128 outputs, 32-deep k-steps, 4 waves of
// 64x64 (2x2 MFMA tiles each), two workgroups per CU (2 x 32 KiB LDS
// stages each). The same tile scheduler and operand roles as the bf16/fp16
// kernel; direct-to-LDS 16-byte loads, a two-stage ring.
//
// Reduction order inside a k-step: lanes 0..31 (the MFMA's k-slot 0) take
// k = 0..15 of the step and lanes 32..63 (k-slot 1) k = 16..31; MFMA j
// adds the products of k = j and k = 16 + j. A lane's 16 k values of one
// row are then contiguous, so a K-major operand is read from LDS as four
// 16-byte reads per row.
//
// LDS layouts (16-byte chunks XOR-swizzled so that every fragment read is
// conflict-free):
//   K-major (reduction contiguous in memory): row r (of 128) = 32 floats =
//     8 chunks, chunk c at position c ^ ((r >> 1) & 7); read 16 bytes a lane.
//   MN-major: k-row k (of 32) = 128 floats = 32 chunks, chunk c at position
//     c ^ (8 * (k >> 4)); read 4 bytes a lane (the two half-waves read
//     k-rows 16 apart, which the swizzle puts in opposite bank halves).
constexpr int kF32BM = 128, kF32BN = 128, kF32BK = 32, kF32Waves = 4;

template <bool KMAJ>
struct F32Tile {
  static constexpr int kBytes = 128 * kF32BK * 4;       // 16 KiB
  static constexpr int kPer = kBytes / 1024 / kF32Waves;  // load instructions per wave
  uint32_t off;    // instruction 0: this lane's byte offset from the k-step origin
  uint32_t ustep;  // byte step between this wave's instructions
  uint32_t kofs;   // K-major: k of this lane's chunk within the step
  int wave;
  // K-major: instruction i = 4u + w covers rows 8i .. 8i+7 (rows 32u + 8w +
  // lane/8: the swizzle does not depend on u). MN-major: instruction i = 4w
  // + u covers k-rows 2i, 2i+1 (k-rows 8w + 2u + lane/32: the swizzle does
  // not depend on u).
  __device__ void init(int64_t ld, int wave_, int lane) {
    wave = wave_;
    if (KMAJ) {
      const int r = 8 * wave + lane / 8;
      const int c = (lane % 8) ^ ((r >> 1) & 7);
      off = (uint32_t)((int64_t)r * ld * 4 + c * 16);
      ustep = (uint32_t)(32 * ld * 4);
      kofs = (uint32_t)(4 * c);
    } else {
      const int k = 8 * wave + lane / 32;
      const int c = (lane % 32) ^ (8 * (k >> 4));
      off = (uint32_t)((int64_t)k * ld * 4 + c * 16);
      ustep = (uint32_t)(2 * ld * 4);
      kofs = 0;
    }
  }
  __device__ uint32_t lds_of(int u) const {
    return (uint32_t)((KMAJ ? 4 * u + wave : 4 * wave + u) * 1024);
  }
  // Loads of the k-step whose origin is `base` (`range` readable bytes) with
  // `kv` valid reduction indices into the tile at `lds`.
  __device__ void issue(const float* base, int64_t range, char* lds, int64_t kv) const {
    const i32x4_t rs = make_rsrc(base, range);
    const uint32_t l0 = lds_addr(lds);
    uint32_t v = off;
    if (KMAJ && kv < kF32BK && (int64_t)kofs >= kv) v = kOob;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      load16_to_lds(rs, v, __builtin_amdgcn_readfirstlane(l0 + lds_of(u)));
      if (u + 1 < kPer) v = add_opaque(v, ustep);
    }
  }
};

template <bool KMAJ>
struct F32Frag {
  uint32_t base[2];  // per 32-row sub-tile t
  __device__ void init(int row0, int lane) {
    const int h = lane >> 5;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r = row0 + 32 * t + (lane & 31);
      if (KMAJ) base[t] = (uint32_t)(r * 128 + ((4 * h) ^ ((r >> 1) & 7)) * 16);
      else base[t] = (uint32_t)(16 * h * 512 + ((r >> 2) ^ (8 * h)) * 16 + (r & 3) * 4);
    }
  }
  // K-major: floats for MFMAs 4q .. 4q+3 of sub-tile t.
  __device__ f32x4_t read4(const char* lds, int t, int q) const {
    // chunk (4h + q) ^ s == ((4h) ^ s) ^ q for q < 4 and s < 8
    const uint32_t a = base[t] ^ (uint32_t)(q * 16);
    return *reinterpret_cast<const f32x4_t*>(lds + a);
  }
  // MN-major: the float for MFMA j of sub-tile t (k-row 16h + j).
  __device__ float read1(const char* lds, int t, int j) const {
    return *reinterpret_cast<const float*>(lds + base[t] + j * 512);
  }
};

template <int MODE, int EPI>
__global__ void __launch_bounds__(kF32Waves * kWave, 2)
gg_f32_mfma_kernel(GemmArgs g) {
  constexpr bool kAK = MODE != kDw;   // A operand K-major?
  constexpr bool kBKm = MODE == kDx;  // B operand K-major?
  typedef F32Tile<kAK> TA;
  typedef F32Tile<kBKm> TB;
  constexpr int kStage = TA::kBytes + TB::kBytes;
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage];
  __shared__ int32_t s_pref[2 * (NT_MAX_EXPERTS + 1)];

  int64_t mtiles;
  if (MODE != kDw) {
    build_m_prefix(g.offsets, g.E, g.A, kF32BM, s_pref);
    mtiles = s_pref[g.E];
  } else {
    build_chunk_prefix(g.offsets, g.E, g.A, 0, 0, 0, s_pref, s_pref + (NT_MAX_EXPERTS + 1));
    mtiles = (int64_t)s_pref[g.E] * g.ntm;
  }
  const int64_t logical = blockIdx.x;
  if (logical >= mtiles * g.ntn) return;
  TileJobT<float> job;
  setup_job<MODE, kF32BM, kF32BN, EPI, float>(g, s_pref, mtiles, logical, job);

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave / 2, wn = wave % 2;
  TA ta;
  TB tb;
  ta.init(job.lda, wave, lane);
  tb.init(job.ldb, wave, lane);
  F32Frag<kAK> fa;
  F32Frag<kBKm> fb;
  fa.init(wm * 64, lane);
  fb.init(wn * 64, lane);
  const int64_t rv = job.rows_valid < kF32BM ? job.rows_valid : kF32BM;
  const int64_t cv = job.cols_valid < kF32BN ? job.cols_valid : kF32BN;

  // Stage kt. A two-part dX reduction takes nk1 = ceil(kred1 / BK) k-steps
  // of (pa, pb), then those of (pa2, pb2): each part starts a k-step.
  const int64_t nk1 = EPI == kEpiDualK ? ceil_div(job.kred1, kF32BK) : 0;
  auto issue = [&](int64_t kt, char* lds) {
    const float* a = job.pa;
    const float* b = job.pb;
    int64_t kl = kt * kF32BK, klen = job.kred;
    if (EPI == kEpiDualK) {
      klen = job.kred1;
      if (kt >= nk1) {
        a = job.pa2;
        b = job.pb2;
        kl = (kt - nk1) * kF32BK;
        klen = job.kred - job.kred1;
      }
    }
    const int64_t kleft = klen - kl;
    const int64_t kv = kleft < kF32BK ? kleft : kF32BK;
    const int64_t ra = kAK ? ((rv - 1) * job.lda + kv) * 4 : ((kv - 1) * job.lda + rv) * 4;
    const int64_t rb = kBKm ? ((cv - 1) * job.ldb + kv) * 4 : ((kv - 1) * job.ldb + cv) * 4;
    ta.issue(a + (kAK ? kl : kl * job.lda), ra, lds, kv);
    tb.issue(b + (kBKm ? kl : kl * job.ldb), rb, lds + TA::kBytes, kv);
  };

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int64_t nk =
      EPI == kEpiDualK ? nk1 + ceil_div(job.kred - job.kred1, kF32BK) : ceil_div(job.kred, kF32BK);
  if (nk > 0) issue(0, smem);
  for (int64_t kt = 0; kt < nk; ++kt) {
    wait_vmcnt<0>();
    __syncthreads();
    const char* st = smem + (kt & 1) * kStage;
    if (kt + 1 < nk) issue(kt + 1, smem + ((kt + 1) & 1) * kStage);
    const char* sa = st;
    const char* sb = st + TA::kBytes;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float av[2][4], bv[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (kAK) {
          const f32x4_t x = fa.read4(sa, t, q);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) av[t][jj] = x[jj];
        } else {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) av[t][jj] = fa.read1(sa, t, 4 * q + jj);
        }
        if (kBKm) {
          const f32x4_t x = fb.read4(sb, t, q);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) bv[t][jj] = x[jj];
        } else {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) bv[t][jj] = fb.read1(sb, t, 4 * q + jj);
        }
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[j][jj], av[i][jj], acc[i][j], 0, 0, 0);
    }
  }

  // acc[i][j][v] = C[m][n], m = 64 wm + 32 i + lane % 32, n = 64 wn + 32 j +
  // 8 (v / 4) + 4 (lane / 32) + v % 4: four consecutive columns per group.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = wm * 64 + i * 32 + (lane & 31);
    if (m >= job.rows_valid) continue;
    float* prow = job.po + (int64_t)m * job.ldo;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int n = wn * 64 + j * 32 + 8 * gq + 4 * (lane >> 5);
        if (n >= job.cols_valid) continue;
        const f32x4_t v = {acc[i][j][4 * gq], acc[i][j][4 * gq + 1], acc[i][j][4 * gq + 2],
                           acc[i][j][4 * gq + 3]};
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t*>(prow + n));
      }
  }
}

constexpr int kGT = 64;  // generic tile
constexpr int kGK = 16;

template <typename T, int MODE>
__global__ void __launch_bounds__(256)
gg_generic_kernel(GemmArgs g) {
  typedef typename elem<T>::storage S;
  typedef typename acc_type<T>::type AT;
  __shared__ AT s_a[kGK][kGT + 1];
  __shared__ AT s_b[kGK][kGT + 1];
  __shared__ int32_t s_pref[NT_MAX_EXPERTS + 1];

  const S* X = static_cast<const S*>(g.a);
  const S* Bm = static_cast<const S*>(g.b);
  S* out = static_cast<S*>(g.out);
  // Two-part dX: reduction indices N .. 2N-1 read (a2, b2).
  const bool dual = MODE == kDx && g.a2 != nullptr;
  const S* X2 = static_cast<const S*>(g.a2);
  const S* B2 = static_cast<const S*>(g.b2);
  const int64_t bid = blockIdx.x;
  const int nt = (int)(bid % g.ntn);
  const int64_t mt = bid / g.ntn;

  int e;
  int64_t r0, r1, m0, rows_valid, cols_valid, kred;
  if (MODE == kDw) {
    e = (int)(mt / g.ntm);
    m0 = (mt % g.ntm) * kGT;
    expert_rows(g.offsets, e, g.A, r0, r1);
    kred = r1 - r0;
    rows_valid = g.K - m0;
    cols_valid = g.N - (int64_t)nt * kGT;
  } else {
    int64_t mtl;
    if (!map_m_tile(g.offsets, g.E, g.A, kGT, mt, s_pref, e, r0, r1, mtl)) return;
    m0 = r0 + mtl * kGT;
    rows_valid = r1 - m0;
    cols_valid = (MODE == kFwd ? g.N : g.K) - (int64_t)nt * kGT;
    kred = MODE == kFwd ? g.K : (dual ? 2 * g.N : g.N);
  }
  const int64_t n0 = (int64_t)nt * kGT;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  AT acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0;

  for (int64_t k0 = 0; k0 < kred; k0 += kGK) {
    for (int q = threadIdx.x; q < kGK * kGT; q += 256) {
      const int kk = q / kGT, m = q % kGT;
      const int64_t kg = k0 + kk;
      AT va = 0, vb = 0;
      const bool second = dual && kg >= g.N;
      const int64_t kx = second ? kg - g.N : kg;
      if (kg < kred && m < rows_valid) {
        if (MODE == kFwd) va = to_acc<T>(X[(m0 + m) * g.K + kg]);
        else if (MODE == kDx) va = to_acc<T>((second ? X2 : X)[(m0 + m) * g.N + kx]);
        else va = to_acc<T>(X[(r0 + kg) * g.K + m0 + m]);
      }
      if (kg < kred && m < cols_valid) {
        const int64_t n = n0 + m;
        if (MODE == kFwd) vb = to_acc<T>(Bm[(int64_t)e * g.K * g.N + kg * g.N + n]);
        else if (MODE == kDx)
          vb = to_acc<T>((second ? B2 : Bm)[(int64_t)e * g.K * g.N + n * g.N + kx]);
        else vb = to_acc<T>(Bm[(r0 + kg) * g.N + n]);
      }
      s_a[kk][m] = va;
      s_b[kk][m] = vb;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kGK; ++kk) {
      AT av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = s_a[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = s_b[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = ty * 4 + i, n = tx * 4 + j;
      if (m < rows_valid && n < cols_valid) {
        int64_t idx;
        if (MODE == kFwd) idx = (m0 + m) * g.N + n0 + n;
        else if (MODE == kDx) idx = (m0 + m) * g.K + n0 + n;
        else idx = (int64_t)e * g.K * g.N + (m0 + m) * g.N + n0 + n;
        out[idx] = from_acc<T>(acc[i][j]);
      }
    }
}

// ---------------------------------------------------------------- host side

bool mfma_ok(int dtype, int64_t K, int64_t N, const void* p0, const void* p1, const void* p2) {
  if (dtype != NT_BF16 && dtype != NT_F16) return false;
  if (K % 8 != 0 || N % 8 != 0) return false;
  const uintptr_t al = reinterpret_cast<uintptr_t>(p0) | reinterpret_cast<uintptr_t>(p1) |
                       reinterpret_cast<uintptr_t>(p2);
  return al % 16 == 0;
}

// CUs of the device that `s` launches on (the null stream: the current
// device). Concurrent first calls may both query; they store the same value.
int device_cus(hipStream_t s) {
  static std::atomic<int> cache[64];
  hipDevice_t dev = 0;
  if (hipStreamGetDevice(s, &dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Tile bookkeeping shared by the launchers: n-tiles, m-tile slots and the
// grid size (one workgroup per tile).
template <int MODE>
int64_t plan_tiles(GemmArgs& g, int64_t out_cols, int BM, int BN) {
  g.ntn = (int32_t)ceil_div(out_cols, BN);
  if (MODE == kDw) {
    g.ntm = (int32_t)ceil_div(g.K, BM);
    // Chunks: at most one per expert plus A / chunk (upper bound).
    const int64_t chunks = g.chunk > 0 ? g.E + g.A / g.chunk : g.E;
    g.mtiles = chunks * g.ntm;
  } else {
    g.ntm = 0;
    g.mtiles = ceil_div(g.A, BM) + g.E;  // upper bound: each expert's last tile may be partial
  }
  return g.mtiles * g.ntn;
}

// Workgroups of `kernel` that fit on one CU at once.
template <typename K>
int blocks_per_cu(K kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1)
    n = 1;
  return n;
}

// Start delay (100 MHz ticks) for half the workgroups of a forward / dX
// launch whose tiles are short (reduction <= 1024) and many (at least 4 per
// CU): the time the whole chip needs to move one round of the epilogue's
// traffic (outputs written plus auxiliary tiles read) at ~6 TB/s. Measured
// on C2's routed inputs, warm and interleaved, against no delay: GELU
// up-projection 226 -> 200 us, plain up-projection 163 -> 149 us, plain dX
// (reduction 512) 165 -> 152 us, GELU dX 199 -> 185 us. Half or 1.5 times
// this delay gained less, 3 times lost; at longer reductions or fewer tiles
// the delay only lengthens the tail. The GELU epilogues (table or gelu'
// reads on top of the stores) with at least 6 tiles per CU take 1.5 times
// the delay (measured on the 16x16x32 kernels, three alternations: C2
// layer step 0.9333-0.9352 -> 0.9253-0.9283 ms, C3 and C5 level; 1.5 times
// for every launch with 6 tiles per CU made C3 1% slower, 2 times was
// slower at C2).
int32_t stagger_ticks(int mode, int epi, int64_t red, int64_t tiles, int64_t cus, int BM, int BN) {
  if (mode == kDw || red > 1024 || tiles < 4 * cus) return 0;
  int tensors = 1;  // output tiles written plus input tiles read by the epilogue
  if (epi == kEpiGelu || epi == kEpiGeluGrad) tensors = 2;
  if (epi == kEpiSwiGLU) tensors = 3;
  if (epi == kEpiSwiGLUGrad) tensors = 4;
  const int64_t bytes = (int64_t)tensors * BM * (epi == kEpiSwiGLU ? BN / 2 : BN) * 2 * cus;
  const bool gelu_many = tensors == 2 && tiles >= 6 * cus;
  return (int32_t)(bytes / 60000 * (gelu_many ? 3 : 2) / 2);  // bytes / 6 TB/s, in 10 ns ticks
}

template <int MODE, int EPI, int BM, int BN, int WGM, int WGN, int BK, int NS, bool SPLIT = false>
int launch_mfma(int dtype, GemmArgs g, int64_t out_cols, hipStream_t s) {
  const int64_t tiles = plan_tiles<MODE>(g, out_cols, BM, EPI == kEpiSwiGLU ? BN / 2 : BN);
  if (tiles == 0) return NT_OK;
  if (tiles > INT32_MAX) return NT_ERR_TOO_LARGE;
  {
    const int64_t red = MODE == kFwd ? g.K : (EPI == kEpiDualK ? 2 * g.N : g.N);
    const int64_t real_tiles = ceil_div(g.A, BM) * g.ntn;  // without the empty slots
    g.stagger = stagger_ticks(MODE, EPI, red, real_tiles, device_cus(s), BM, BN);
  }
  constexpr int threads = WGM * WGN * kWave;
  auto kb = gg_mfma_kernel<bf16, MODE, BM, BN, WGM, WGN, BK, NS, EPI, SPLIT>;
  // Occupancy of this instantiation (bf16 and fp16 share resource usage).
  static const int per_cu = blocks_per_cu(kb, threads);
  // Persistent: at most one resident wave of workgroups; each walks tiles.
  const int64_t nblocks = std::min<int64_t>(tiles, (int64_t)device_cus(s) * per_cu);
  const dim3 grid((unsigned)nblocks);
  if (dtype == NT_BF16) {
    hipLaunchKernelGGL(kb, grid, dim3(threads), 0, s, g);
  } else if constexpr (EPI == kEpiGelu && SPLIT) {
    // The GELU forward runs split only in bf16 (gelu_split), so no fp16 form
    // of it is built.
    return NT_ERR_DTYPE;
  } else {
    hipLaunchKernelGGL((gg_mfma_kernel<f16, MODE, BM, BN, WGM, WGN, BK, NS, EPI, SPLIT>), grid,
                       dim3(threads), 0, s, g);
  }
  return launch_status();
}

// Tile shape (measured on MI355X over the configs' shapes): 256x256 with 8
// waves unless that leaves fewer than 1.5 tiles per CU, then 128x128 with 4
// waves (two workgroups per CU). Plain 256x256 forward / dX tiles with a
// reduction of at least kSplitMinRed split load and store duties between the
// waves (measured: C4 +5%, C2 down-projection -10 us; shorter reductions and
// the GELU epilogue were slower split).
constexpr int64_t kSplitMinRed = 1024;
// GELU forward with split duties only for long reductions and the bf16
// table (measured on routed inputs, bit-identical either way: C4
// up-projection, K = 4096, 3885 -> 3840 us; C2, K = 512, 199 -> 282 us,
// where the short k-loop cannot hide the storer waves' doubled store
// rounds). fp16 evaluates gelu through the erfc fit, about four times the
// table's VALU work per element; on half the waves that work outlasts the
// next tile's loads (C5 up-projection, K = 2048: 2568-2593 us split,
// 2105-2118 us with every wave in the epilogue).
bool gelu_split(int dtype, int64_t red) { return dtype == NT_BF16 && red >= 2048; }
template <int MODE, int EPI>
int launch_mfma_auto(int dtype, GemmArgs g, int64_t out_cols, hipStream_t s) {
  const int64_t chunks = g.chunk > 0 ? g.E + g.A / g.chunk : g.E;
  const int64_t tiles256 = MODE == kDw
                               ? chunks * ceil_div(g.K, 256) * ceil_div(out_cols, 256)
                               : ceil_div(g.A, 256) * ceil_div(out_cols, 256);
  // SwiGLU forward: 256 rows x (128 gate | 128 value) columns, waves 4 x 2,
  // so that each wave holds the gate and value tiles of the same outputs.
  if constexpr (EPI == kEpiSwiGLU) {
    (void)tiles256;
    return launch_mfma<MODE, EPI, 256, 256, 4, 2, 64, 2>(dtype, g, out_cols, s);
  } else {
    if (tiles256 * 2 >= (int64_t)device_cus(s) * 3) {
      if constexpr (MODE != kDw && (EPI == kEpiPlain || EPI == kEpiDualK)) {
        const int64_t red = MODE == kFwd ? g.K : (EPI == kEpiDualK ? 2 * g.N : g.N);
        if (red >= kSplitMinRed)
          return launch_mfma<MODE, EPI, 256, 256, 2, 4, 64, 2, true>(dtype, g, out_cols, s);
      }
      if constexpr (MODE == kFwd && EPI == kEpiGelu) {
        if (gelu_split(dtype, g.K))
          return launch_mfma<MODE, EPI, 256, 256, 2, 4, 64, 2, true>(dtype, g, out_cols, s);
      }
      return launch_mfma<MODE, EPI, 256, 256, 2, 4, 64, 2>(dtype, g, out_cols, s);
    }
    return launch_mfma<MODE, EPI, 128, 128, 2, 2, 64, 2>(dtype, g, out_cols, s);
  }
}

// Elementwise GELU for the generic path (fp32 / fp64, or shapes the MFMA
// kernel does not take). Forward: io holds h on entry and gelu(h) on exit,
// g receives gelu'(h). Backward: io holds dA on entry and dA * g on exit.
template <typename T, bool GRAD>
__global__ void __launch_bounds__(256) gelu_elementwise_kernel(void* io_, void* g_, int64_t n) {
  typedef typename elem<T>::storage S;
  typedef typename acc_type<T>::type AT;
  S* io = static_cast<S*>(io_);
  S* g = static_cast<S*>(g_);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    if (GRAD) {
      io[i] = from_acc<T>(to_acc<T>(io[i]) * to_acc<T>(g[i]));
    } else {
      const AT x = to_acc<T>(io[i]);
      const AT cdf = AT(0.5) * (AT(1) + erf(x * AT(0.70710678118654752440)));
      const AT pdf = exp(AT(-0.5) * x * x) * AT(0.39894228040143267794);
      g[i] = from_acc<T>(cdf + x * pdf);
      io[i] = from_acc<T>(x * cdf);
    }
  }
}

template <bool GRAD>
int launch_gelu_elementwise(int dtype, void* io, void* g, int64_t n, hipStream_t s) {
  if (n == 0) return NT_OK;
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(n, 256), (int64_t)device_cus(s) * 16));
  switch (dtype) {
    case NT_F32: hipLaunchKernelGGL((gelu_elementwise_kernel<float, GRAD>), grid, dim3(256), 0, s, io, g, n); break;
    case NT_F64: hipLaunchKernelGGL((gelu_elementwise_kernel<double, GRAD>), grid, dim3(256), 0, s, io, g, n); break;
    case NT_F16: hipLaunchKernelGGL((gelu_elementwise_kernel<f16, GRAD>), grid, dim3(256), 0, s, io, g, n); break;
    case NT_BF16: hipLaunchKernelGGL((gelu_elementwise_kernel<bf16, GRAD>), grid, dim3(256), 0, s, io, g, n); break;
    default: return NT_ERR_DTYPE;
  }
  return launch_status();
}

// Elementwise SwiGLU for the generic path. Forward: h = silu(g) * v from
// the stored gate and value. Backward: io holds dhidden on entry and
// dvalue on exit, dg receives dgate. Same roundings as the MFMA epilogues
// for 16-bit types; fp32 / fp64 keep full precision throughout.
template <typename T, bool GRAD>
__global__ void __launch_bounds__(256)
swiglu_elementwise_kernel(void* io_, void* dg_, const void* g_, const void* v_, int64_t n) {
  typedef typename elem<T>::storage S;
  typedef typename acc_type<T>::type AT;
  S* io = static_cast<S*>(io_);
  S* dg = static_cast<S*>(dg_);
  const S* gp = static_cast<const S*>(g_);
  const S* vp = static_cast<const S*>(v_);
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const AT g = to_acc<T>(gp[i]);
    const AT v = to_acc<T>(vp[i]);
    const AT sg = AT(1) / (AT(1) + exp(-g));
    const AT silu = to_acc<T>(from_acc<T>(g * sg));
    if (GRAD) {
      const AT dh = to_acc<T>(io[i]);
      const AT ds = to_acc<T>(from_acc<T>(dh * v));
      dg[i] = from_acc<T>((ds * sg) * (AT(1) + g * (AT(1) - sg)));
      io[i] = from_acc<T>(dh * silu);
    } else {
      io[i] = from_acc<T>(silu * v);
    }
  }
}
template <bool GRAD>
int launch_swiglu_elementwise(int dtype, void* io, void* dg, const void* g, const void* v,
                              int64_t n, hipStream_t s) {
  if (n == 0) return NT_OK;
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(n, 256), (int64_t)device_cus(s) * 16));
  switch (dtype) {
    case NT_F32: hipLaunchKernelGGL((swiglu_elementwise_kernel<float, GRAD>), grid, dim3(256), 0, s, io, dg, g, v, n); break;
    case NT_F64: hipLaunchKernelGGL((swiglu_elementwise_kernel<double, GRAD>), grid, dim3(256), 0, s, io, dg, g, v, n); break;
    case NT_F16: hipLaunchKernelGGL((swiglu_elementwise_kernel<f16, GRAD>), grid, dim3(256), 0, s, io, dg, g, v, n); break;
    case NT_BF16: hipLaunchKernelGGL((swiglu_elementwise_kernel<bf16, GRAD>), grid, dim3(256), 0, s, io, dg, g, v, n); break;
    default: return NT_ERR_DTYPE;
  }
  return launch_status();
}

// Split dW: dW[e] = sum over its chunks, in chunk order, of the fp32
// partial slabs, rounded once. Only experts with two or more chunks; the
// others were written by the GEMM. Grid: (element blocks, E).
template <typename T>
__global__ void __launch_bounds__(256)
dw_reduce_kernel(const int32_t* __restrict__ offsets, int32_t E, int64_t A, int32_t R,
                 int32_t thr, int32_t cap,
                 const float* __restrict__ partial, int64_t KN,
                 typename elem<T>::storage* __restrict__ dW) {
  __shared__ int32_t s_info[2];
  const int e = blockIdx.y;
  {
    // Experts in one chunk were written by the GEMM: leave before the
    // prefix (the common case for balanced routing). Uniform per block.
    int64_t a, b;
    expert_rows(offsets, e, A, a, b);
    if (dw_chunks(b - a, R, thr) < 2) return;
  }
  if (threadIdx.x < kWave) {
    // More split chunks than slabs (overlapping expert ranges): the GEMM
    // ran every expert unsplit (build_chunk_prefix) and wrote dW itself.
    if (split_total(offsets, E, A, R, thr) > cap) R = 0;
    const int lane = lane_id();
    int before = 0;
    for (int s0 = 0; s0 < e; s0 += kWave) {
      const int ee = s0 + lane;
      int v = 0;
      if (ee < e) {
        int64_t a, b;
        expert_rows(offsets, ee, A, a, b);
        v = dw_chunks(b - a, R, thr);
        v = v >= 2 ? v : 0;
      }
      before += wave_sum_int(v);
    }
    if (lane == 0) {
      int64_t a, b;
      expert_rows(offsets, e, A, a, b);
      s_info[0] = before;
      s_info[1] = dw_chunks(b - a, R, thr);
    }
  }
  __syncthreads();
  const int nch = s_info[1];
  if (nch < 2) return;
  const float* base = partial + (int64_t)s_info[0] * KN;
  typename elem<T>::storage* out = dW + (int64_t)e * KN;
  for (int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8; i < KN;
       i += (int64_t)gridDim.x * blockDim.x * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nch; ++c) {
      const float4 u = *reinterpret_cast<const float4*>(base + (int64_t)c * KN + i);
      const float4 v = *reinterpret_cast<const float4*>(base + (int64_t)c * KN + i + 4);
      acc[0] += u.x; acc[1] += u.y; acc[2] += u.z; acc[3] += u.w;
      acc[4] += v.x; acc[5] += v.y; acc[6] += v.z; acc[7] += v.w;
    }
    uint4 r;
    r.x = (uint32_t)elem<T>::store(acc[0]) | ((uint32_t)elem<T>::store(acc[1]) << 16);
    r.y = (uint32_t)elem<T>::store(acc[2]) | ((uint32_t)elem<T>::store(acc[3]) << 16);
    r.z = (uint32_t)elem<T>::store(acc[4]) | ((uint32_t)elem<T>::store(acc[5]) << 16);
    r.w = (uint32_t)elem<T>::store(acc[6]) | ((uint32_t)elem<T>::store(acc[7]) << 16);
    *reinterpret_cast<uint4*>(out + i) = r;
  }
}

// Rows per expert chunk used to estimate a dW launch's tile count for its
// tile-shape choice: at least twice the mean expert size and 1024, and
// large enough that the fp32 partial slabs (fewer than 2A/R of them) fit
// kDwBudget bytes. 0: no expert can split.
constexpr int64_t kDwBudget = int64_t(256) << 20;
int32_t dw_chunk_rows(int64_t A, int64_t K, int64_t N, int32_t E) {
  const int64_t slab = K * N * 4;
  if (A <= 0 || slab <= 0 || E <= 0) return 0;
  if (slab >= kDwBudget) return 0;  // R would exceed 2A: no expert can split
  int64_t R = ceil_div(2 * A * slab, kDwBudget);
  R = std::max<int64_t>(R, 2 * ceil_div(A, E));
  R = round_up(std::max<int64_t>(R, 1024), 64);
  if (R >= A) return 0;
  return (int32_t)R;
}

// Split of every dW launch, paired or not (the same split gives the same
// summation order, so the paired and separate calls agree bit for bit).
// W = A * (128x128 tiles per expert) / (two workgroups per CU) is a
// workgroup's share of the reduction rows. An expert with more than
// thr = 5W/4 rows is cut into chunks of R = W/2 rows (at least 1024, and at
// least what keeps the slabs within kDwBudget), so no tile is much longer
// than a share: with skewed routing (C3: the head expert has 8x the mean
// rows) one whole-expert tile would otherwise outlast everything else.
// Balanced routing stays unsplit.
// The split is planned for MI355X's 256 CUs on every device: it fixes the
// summation order, so dW bits and the workspace size do not depend on the
// device that runs the launch.
constexpr int64_t kDwSplitCus = 256;
struct DwSplit {
  int32_t R = 0;    // rows per chunk of a split expert (0: no split)
  int32_t thr = 0;  // experts with more rows than this are split
};
DwSplit dw_split(int64_t A, int64_t K, int64_t N, int32_t E) {
  DwSplit p;
  const int64_t slab = K * N * 4;
  if (A <= 0 || slab <= 0 || E <= 0 || slab >= kDwBudget) return p;
  const int64_t W = ceil_div(A * ceil_div(K, 128) * ceil_div(N, 128), 2 * kDwSplitCus);
  int64_t R = std::max<int64_t>(ceil_div(W, 2), 1024);
  R = round_up(std::max<int64_t>(R, ceil_div(2 * A * slab, kDwBudget)), 64);
  const int64_t thr = std::max<int64_t>(round_up(ceil_div(5 * W, 4), 64), R);
  if (thr >= A) return p;
  p.R = (int32_t)R;
  p.thr = (int32_t)thr;
  return p;
}
// Upper bound on the partial slabs: at most A / (thr + 1) experts are split
// (more than thr rows each), and their ceil(M_e / R) chunks add up to at
// most A / R plus one per split expert.
int64_t dw_slabs(int64_t A, DwSplit p) {
  if (p.R <= 0) return 0;
  return A / p.R + A / ((int64_t)p.thr + 1) + 1;
}

// Tile shape of a dW launch (not paired): 256x256 tiles when the experts'
// tiles (with dw_chunk_rows chunks) give at least 1.5 per CU, else 128x128
// tiles, two workgroups per CU (the rule launch_mfma_auto applies).
bool dw_big_tiles(int64_t A, int64_t K, int64_t N, int32_t E, hipStream_t s) {
  const int32_t R0 = dw_chunk_rows(A, K, N, E);
  const int64_t chunks = R0 > 0 ? E + A / R0 : E;
  return chunks * ceil_div(K, 256) * ceil_div(N, 256) * 2 >= device_cus(s) * 3;
}

// Workspace of the dW entry points: kCtrBytes of tile-claim counters
// (paired launches), the fp32 partial slabs of split experts, then the
// paired launch's arrival counters of their 256x256 tiles (fold_split_tile),
// indexed by the expert's first slab.
constexpr size_t kCtrBytes = 256;
size_t dw_ws_bytes(int64_t A, int64_t K, int64_t N, int32_t E) {
  const size_t slabs = (size_t)dw_slabs(A, dw_split(A, K, N, E));
  return slabs * (size_t)(K * N * 4) + slabs * (size_t)(ceil_div(K, 256) * ceil_div(N, 256) * 8);
}

// fp32 MFMA kernel: 16-byte aligned operands and outputs, K and N multiples
// of 4 (whole 16-byte chunks along every row).
bool f32_mfma_ok(const GemmArgs& g, bool dual) {
  if (g.K % 4 != 0 || g.N % 4 != 0) return false;
  uintptr_t al = reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b) |
                 reinterpret_cast<uintptr_t>(g.out);
  if (dual) al |= reinterpret_cast<uintptr_t>(g.a2) | reinterpret_cast<uintptr_t>(g.b2);
  return al % 16 == 0;
}

template <int MODE, int EPI>
int launch_f32_mfma(GemmArgs g, int64_t out_cols, hipStream_t s) {
  g.chunk = 0;
  const int64_t tiles = plan_tiles<MODE>(g, out_cols, kF32BM, kF32BN);
  if (tiles == 0) return NT_OK;
  if (tiles > INT32_MAX) return NT_ERR_TOO_LARGE;
  hipLaunchKernelGGL((gg_f32_mfma_kernel<MODE, EPI>), dim3((unsigned)tiles),
                     dim3(kF32Waves * kWave), 0, s, g);
  return launch_status();
}

template <int MODE>
int launch_generic(int dtype, GemmArgs g, int64_t out_cols, hipStream_t s);

template <int MODE, int EPI>
int launch_mode(int dtype, GemmArgs g, int64_t out_cols, bool mfma, hipStream_t s) {
  if (mfma) return launch_mfma_auto<MODE, EPI>(dtype, g, out_cols, s);
  if constexpr (EPI == kEpiSwiGLU) {
    // Generic path: the gate and value GEMMs, then the elementwise SwiGLU.
    GemmArgs gg = g;
    gg.out = g.out2;
    gg.out2 = nullptr;
    int st = launch_mode<MODE, kEpiPlain>(dtype, gg, out_cols, false, s);
    if (st != NT_OK) return st;
    gg.b = g.b2;
    gg.out = g.out3;
    st = launch_mode<MODE, kEpiPlain>(dtype, gg, out_cols, false, s);
    if (st != NT_OK) return st;
    return launch_swiglu_elementwise<false>(dtype, g.out, nullptr, g.out2, g.out3,
                                            g.A * out_cols, s);
  }
  if constexpr (EPI == kEpiSwiGLUGrad) {
    // Generic path: dhidden into the dvalue buffer, then the elementwise
    // backward (dgate -> out, dvalue over dhidden).
    GemmArgs gg = g;
    gg.out = g.out2;
    gg.aux = nullptr;
    int st = launch_mode<MODE, kEpiPlain>(dtype, gg, out_cols, false, s);
    if (st != NT_OK) return st;
    return launch_swiglu_elementwise<true>(dtype, g.out2, g.out, g.aux, g.aux2, g.A * out_cols,
                                           s);
  }
  int st;
  if (dtype == NT_F32 && f32_mfma_ok(g, EPI == kEpiDualK)) {
    st = launch_f32_mfma<MODE, EPI == kEpiDualK ? kEpiDualK : kEpiPlain>(g, out_cols, s);
  } else {
    st = launch_generic<MODE>(dtype, g, out_cols, s);
  }
  if (st != NT_OK || (EPI != kEpiGelu && EPI != kEpiGeluGrad)) return st;
  // Generic path: the GELU epilogue as a second, elementwise pass over the
  // output rows (rows past offsets[E] hold unspecified values either way).
  const int64_t n = g.A * out_cols;
  if (EPI == kEpiGelu) return launch_gelu_elementwise<false>(dtype, g.out, g.out2, n, s);
  return launch_gelu_elementwise<true>(dtype, g.out, const_cast<void*>(g.aux), n, s);
}

// The VALU kernel (any dtype, any shape; two-part dX when g.a2 is set).
template <int MODE>
int launch_generic(int dtype, GemmArgs g, int64_t out_cols, hipStream_t s) {
  g.ntn = (int32_t)ceil_div(out_cols, kGT);
  int64_t nblocks;
  if (MODE == kDw) {
    g.ntm = (int32_t)ceil_div(g.K, kGT);
    nblocks = (int64_t)g.E * g.ntm * g.ntn;
  } else {
    g.ntm = 0;
    nblocks = (ceil_div(g.A, kGT) + g.E) * (int64_t)g.ntn;
  }
  if (nblocks == 0) return NT_OK;
  if (nblocks > INT32_MAX) return NT_ERR_TOO_LARGE;
  const dim3 grid((unsigned)nblocks);
  switch (dtype) {
    case NT_F32: hipLaunchKernelGGL((gg_generic_kernel<float, MODE>), grid, dim3(256), 0, s, g); break;
    case NT_F64: hipLaunchKernelGGL((gg_generic_kernel<double, MODE>), grid, dim3(256), 0, s, g); break;
    case NT_F16: hipLaunchKernelGGL((gg_generic_kernel<f16, MODE>), grid, dim3(256), 0, s, g); break;
    case NT_BF16: hipLaunchKernelGGL((gg_generic_kernel<bf16, MODE>), grid, dim3(256), 0, s, g); break;
    default: return NT_ERR_DTYPE;
  }
  return launch_status();
}

// Argument check of one grouped GEMM of `mode`: fwd out[A,N] = a[A,K] b[E,K,N];
// dX out[A,K] = a[A,N] b[E,K,N]^T; dW out[E,K,N] = a[A,K]^T b[A,N]. Pointers
// of empty tensors may be null.
int check_gemm(int dtype, int32_t E, int64_t A, int64_t K, int64_t N, const void* a,
               const void* b, const int32_t* offsets, const void* out, int mode = kFwd) {
  if (dtype_bytes(dtype) == 0) return NT_ERR_DTYPE;
  if (E < 1 || A < 0 || K < 0 || N < 0) return NT_ERR_INVALID_ARG;
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
  if (offsets == nullptr) return NT_ERR_INVALID_ARG;
  const int64_t a_cols = mode == kDx ? N : K;
  const int64_t b_elems = mode == kDw ? A * N : K * N;
  const int64_t out_elems = mode == kDw ? K * N : A * (mode == kDx ? K : N);
  if ((A * a_cols > 0 && a == nullptr) || (b_elems > 0 && b == nullptr) ||
      (out_elems > 0 && out == nullptr))
    return NT_ERR_INVALID_ARG;
  if (A > INT32_MAX) return NT_ERR_TOO_LARGE;
  // Tile operand and output offsets are 32-bit byte offsets: 256 rows of
  // the widest operand row must stay below 2 GiB.
  if (K > (int64_t{1} << 22) - 256 || N > (int64_t{1} << 22) - 256) return NT_ERR_TOO_LARGE;
  return NT_OK;
}

}  // namespace
}  // namespace nt

namespace nt {
namespace {

// dX-type GEMM (plain, or with the GELU backward when act_grad is set) and
// dW; the C entry points below wrap them.
template <int EPI>
int dx_impl(int dtype, const void* W, const int32_t* offsets, const void* dOut,
            const void* act_grad, int32_t E, int64_t A, int64_t K, int64_t N, void* dX,
            hipStream_t stream) {
  if (A == 0 || K == 0) return NT_OK;
  GemmArgs g{dOut, W, offsets, E, A, K, N, dX, 0, 0, 0, nullptr, act_grad, 0, nullptr};
  bool mfma = mfma_ok(dtype, K, N, dOut, W, dX);
  if (EPI == kEpiGeluGrad) mfma = mfma && reinterpret_cast<uintptr_t>(act_grad) % 16 == 0;
  return launch_mode<kDx, EPI>(dtype, g, K, mfma, stream);
}

int launch_dw_reduce(int dtype, const int32_t* offsets, int32_t E, int64_t A, int64_t K,
                     int64_t N, DwSplit sp, const float* partial, void* dW, hipStream_t stream) {
  const int64_t KN = K * N;
  const int32_t cap = (int32_t)dw_slabs(A, sp);
  const dim3 grid((unsigned)std::min<int64_t>(ceil_div(KN, 256 * 8), 64), (unsigned)E);
  if (dtype == NT_BF16)
    hipLaunchKernelGGL((dw_reduce_kernel<bf16>), grid, dim3(256), 0, stream, offsets, E, A, sp.R,
                       sp.thr, cap, partial, KN, static_cast<uint16_t*>(dW));
  else
    hipLaunchKernelGGL((dw_reduce_kernel<f16>), grid, dim3(256), 0, stream, offsets, E, A, sp.R,
                       sp.thr, cap, partial, KN, static_cast<uint16_t*>(dW));
  return launch_status();
}

int dw_impl(int dtype, const void* X, const int32_t* offsets, const void* dOut, int32_t E,
            int64_t A, int64_t K, int64_t N, void* dW, void* ws, size_t ws_bytes,
            hipStream_t stream) {
  if (K == 0 || N == 0) return NT_OK;
  GemmArgs g{X, dOut, offsets, E, A, K, N, dW, 0, 0, 0, nullptr, nullptr, 0, nullptr};
  const bool mfma = mfma_ok(dtype, K, N, X, dOut, dW);
  if (!mfma) return launch_mode<kDw, kEpiPlain>(dtype, g, N, false, stream);
  // Split long reductions (skewed experts) when the caller's workspace holds
  // the partial slabs; without it every expert is one chunk.
  const DwSplit sp = dw_split(A, K, N, E);
  const bool split = sp.R > 0 && ws != nullptr && ws_bytes >= kCtrBytes + dw_ws_bytes(A, K, N, E) &&
                     reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  float* partial = split ? reinterpret_cast<float*>(static_cast<char*>(ws) + kCtrBytes) : nullptr;
  if (split) {
    g.chunk = sp.R;
    g.split_thr = sp.thr;
    g.slab_cap = (int32_t)dw_slabs(A, sp);
    g.partial = partial;
  }
  // 128x128 tiles: three stages, one workgroup per CU (measured on C3's
  // routing against two stages at two workgroups per CU: 166-170 -> 161-165
  // us per dW, bit-identical; four stages no better).
  const int st = dw_big_tiles(A, K, N, E, stream)
                     ? launch_mfma<kDw, kEpiPlain, 256, 256, 2, 4, 64, 2>(dtype, g, N, stream)
                     : launch_mfma<kDw, kEpiPlain, 128, 128, 2, 2, 64, 3>(dtype, g, N, stream);
  if (st != NT_OK || !split) return st;
  return launch_dw_reduce(dtype, offsets, E, A, K, N, sp, partial, dW, stream);
}

// dW = X^T dOut and a dX-type GEMM (gx, epilogue EPIX) over the same
// (A, K, N), which share nothing but their inputs. When the dW alone has too
// few 256x256 tiles to fill the device (it would run on 128x128 tiles, at
// about two thirds of the per-CU rate), both run in one launch of
// gg_pair_kernel: the dW on 256x256 tiles, one per workgroup, and the dX's
// tiles on the remaining workgroups, which the dW's workgroups join when
// their own tiles are done (gg_pair_kernel). Measured at C2: 358 -> 309 us
// with the GELU backward, 271 -> 245 us without. Results are bit-identical
// to the two separate calls (every output tile is reduced in the same
// order).
constexpr int32_t kPairMaxExperts = 16;
constexpr int kXcdParts = 8;  // claim counters of a paired launch (one per XCD part)

__global__ void zero_u64_kernel(unsigned long long* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

// Epochs of the paired launches' claim counters: 40 bits, a different
// value per launch in this process, starting from a value drawn from the
// clock and this library's load address (so leftover data from another
// process is unlikely to carry it), never 0.
unsigned long long next_claim_epoch() {
  constexpr unsigned long long kMask = (1ull << (64 - kClaimBits)) - 1;
  static std::atomic<unsigned long long> next{
      (static_cast<unsigned long long>(
           std::chrono::steady_clock::now().time_since_epoch().count()) *
           0x9E3779B97F4A7C15ull ^
       reinterpret_cast<uintptr_t>(&next)) &
      kMask};
  unsigned long long e = next.fetch_add(1, std::memory_order_relaxed) & kMask;
  if (e == 0) e = next.fetch_add(1, std::memory_order_relaxed) & kMask;
  return e;
}

template <int EPIX>
int pair_dw_dx(int dtype, const void* X, const int32_t* offsets, const void* dOut, int32_t E,
               int64_t A, int64_t K, int64_t N, void* dW, void* ws, size_t ws_bytes,
               GemmArgs gx, bool dx_mfma, hipStream_t stream) {
  const int64_t cus = device_cus(stream);
  const bool mfma_dw = mfma_ok(dtype, K, N, X, dOut, dW);
  const DwSplit sp = mfma_dw ? dw_split(A, K, N, E) : DwSplit();
  const bool aligned = ws != nullptr && reinterpret_cast<uintptr_t>(ws) % 16 == 0;
  const bool split = sp.R > 0 && aligned && ws_bytes >= kCtrBytes + dw_ws_bytes(A, K, N, E);
  // Workgroups for the dW: one per tile of the experts' full reductions. A
  // skewed expert split into chunks adds tiles that the same workgroups
  // walk (the persistent loop counts the tiles on the device); sizing for
  // the host's upper bound on chunks would leave workgroups idle.
  const int64_t dw_tiles = (int64_t)E * ceil_div(K, 256) * ceil_div(N, 256);
  const int64_t nw = round_up(dw_tiles, 8);
  // Few experts only: with many (C3: 64, Zipf-skewed) the total work is
  // small next to one 256x256 dW tile over a whole chunk of a heavy expert,
  // which then becomes the critical path (measured: C3 1.37 -> 1.53 ms per
  // layer step paired), while 128x128 tiles balance it.
  const bool pair = mfma_dw && dx_mfma && A > 0 && K > 0 && N > 0 && aligned &&
                    ws_bytes >= kCtrBytes && E <= kPairMaxExperts && dw_tiles * 2 < cus * 3 &&
                    nw <= cus - cus / 4 && cus % 8 == 0 &&
                    // claim counts stay below 2^kClaimBits: every tile once, plus
                    // at most one failed claim per part per claim call
                    ((ceil_div(A, 256) + E) * ceil_div(K, 256) + 64) * 9 <
                        (int64_t{1} << kClaimBits);
  if (!pair) {
    const int st = dw_impl(dtype, X, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, stream);
    if (st != NT_OK) return st;
    return launch_mode<kDx, EPIX>(dtype, gx, K, dx_mfma, stream);
  }
  GemmArgs gw{X, dOut, offsets, E, A, K, N, dW, 0, 0, 0, nullptr, nullptr, 0, nullptr};
  float* partial = split ? reinterpret_cast<float*>(static_cast<char*>(ws) + kCtrBytes) : nullptr;
  unsigned long long* dyn = static_cast<unsigned long long*>(ws);
  const unsigned long long epoch = next_claim_epoch();
  if (split) {
    gw.chunk = sp.R;
    gw.split_thr = sp.thr;
    gw.slab_cap = (int32_t)dw_slabs(A, sp);
    gw.partial = partial;
    // the split tiles sum their slabs in the launch (no reduce pass)
    gw.done = reinterpret_cast<unsigned long long*>(partial + dw_slabs(A, sp) * K * N);
    gw.done_epoch = epoch;
  }
  // Under stream capture the graph replays this launch with the epoch it
  // was captured with, so the counters would still hold the previous
  // replay's final counts under that same epoch (every dX claim would fail,
  // no split tile would be the last to arrive). A captured call clears them
  // first, with a fill kernel that is part of the graph (a memset node is
  // avoided: such nodes have given wrong results on replays here).
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap == hipStreamCaptureStatusActive) {
    hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(256), 0, stream, dyn, (int64_t)kXcdParts);
    if (split) {
      const int64_t ndone = (int64_t)dw_slabs(A, sp) * ceil_div(K, 256) * ceil_div(N, 256);
      hipLaunchKernelGGL(zero_u64_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(ndone, 256), 1024)),
                         dim3(256), 0, stream, gw.done, ndone);
    }
    const int st = launch_status();
    if (st != NT_OK) return st;
  }
  plan_tiles<kDw>(gw, N, 256, 256);
  plan_tiles<kDx>(gx, K, 256, 256);
  gx.stagger = stagger_ticks(kDx, EPIX, EPIX == kEpiDualK ? 2 * N : N,
                             ceil_div(A, 256) * ceil_div(K, 256), cus, 256, 256);
  // split duties for the dX as launch_mfma_auto would choose them
  constexpr bool kPlain = EPIX == kEpiPlain || EPIX == kEpiDualK;
  const bool splitx = kPlain && (EPIX == kEpiDualK ? 2 * N : N) >= kSplitMinRed;
  const dim3 grid((unsigned)cus);
  const dim3 block(8 * kWave);
  const int32_t nw32 = (int32_t)nw;
  if (dtype == NT_BF16) {
    if (splitx) {
      if constexpr (kPlain)
        hipLaunchKernelGGL((gg_pair_kernel<bf16, EPIX, true>), grid, block, 0, stream, gw, gx, nw32, dyn, epoch);
    } else {
      hipLaunchKernelGGL((gg_pair_kernel<bf16, EPIX, false>), grid, block, 0, stream, gw, gx, nw32, dyn, epoch);
    }
  } else {
    if (splitx) {
      if constexpr (kPlain)
        hipLaunchKernelGGL((gg_pair_kernel<f16, EPIX, true>), grid, block, 0, stream, gw, gx, nw32, dyn, epoch);
    } else {
      hipLaunchKernelGGL((gg_pair_kernel<f16, EPIX, false>), grid, block, 0, stream, gw, gx, nw32, dyn, epoch);
    }
  }
  return launch_status();
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

size_t nt_grouped_gemm_workspace_bytes(int dtype, int32_t E, int64_t A, int64_t K, int64_t N) {
  if (dtype != NT_BF16 && dtype != NT_F16) return 0;
  if (E < 1 || A < 0 || K < 0 || N < 0) return 0;
  return kCtrBytes + dw_ws_bytes(A, K, N, E);
}

int nt_grouped_gemm(int dtype, const void* X, const int32_t* offsets, const void* W, int32_t E,
                    int64_t A, int64_t K, int64_t N, void* out, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, X, W, offsets, out);
  if (st != NT_OK) return st;
  if (A == 0 || N == 0) return NT_OK;
  GemmArgs g{X, W, offsets, E, A, K, N, out, 0, 0, 0, nullptr, nullptr, 0, nullptr};
  return launch_mode<kFwd, kEpiPlain>(dtype, g, N, mfma_ok(dtype, K, N, X, W, out), stream);
}

int nt_grouped_gemm_gelu(int dtype, const void* X, const int32_t* offsets, const void* W,
                         int32_t E, int64_t A, int64_t K, int64_t N, void* act, void* act_grad,
                         void* ws, size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, X, W, offsets, act);
  if (st != NT_OK) return st;
  if (act_grad == nullptr && A > 0 && N > 0) return NT_ERR_INVALID_ARG;
  if (A == 0 || N == 0) return NT_OK;
  GemmArgs g{X, W, offsets, E, A, K, N, act, 0, 0, 0, act_grad, nullptr, 0, nullptr};
  const bool mfma =
      mfma_ok(dtype, K, N, X, W, act) && reinterpret_cast<uintptr_t>(act_grad) % 16 == 0;
  return launch_mode<kFwd, kEpiGelu>(dtype, g, N, mfma, stream);
}

int nt_grouped_gemm_dx(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                       int32_t E, int64_t A, int64_t K, int64_t N, void* dX, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dX, kDx);
  if (st != NT_OK) return st;
  return dx_impl<kEpiPlain>(dtype, W, offsets, dOut, nullptr, E, A, K, N, dX, stream);
}

int nt_grouped_gemm_dx_gelu(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                            const void* act_grad, int32_t E, int64_t A, int64_t K, int64_t N,
                            void* dH, void* ws, size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dH, kDx);
  if (st != NT_OK) return st;
  if (act_grad == nullptr && A > 0 && K > 0) return NT_ERR_INVALID_ARG;
  return dx_impl<kEpiGeluGrad>(dtype, W, offsets, dOut, act_grad, E, A, K, N, dH, stream);
}

int nt_grouped_gemm_swiglu(int dtype, const void* X, const int32_t* offsets, const void* W_gate,
                           const void* W_val, int32_t E, int64_t A, int64_t K, int64_t N,
                           void* hidden, void* gate, void* value, void* ws, size_t ws_bytes,
                           hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, X, W_gate, offsets, hidden);
  if (st != NT_OK) return st;
  if (A > 0 && N > 0 && (gate == nullptr || value == nullptr || (K > 0 && W_val == nullptr)))
    return NT_ERR_INVALID_ARG;
  if (A == 0 || N == 0) return NT_OK;
  GemmArgs g{X, W_gate, offsets, E, A, K, N, hidden, 0, 0, 0, gate, nullptr, 0, nullptr,
             nullptr, W_val, value, nullptr};
  const uintptr_t al = reinterpret_cast<uintptr_t>(W_val) | reinterpret_cast<uintptr_t>(gate) |
                       reinterpret_cast<uintptr_t>(value);
  const bool mfma = mfma_ok(dtype, K, N, X, W_gate, hidden) && al % 16 == 0;
  return launch_mode<kFwd, kEpiSwiGLU>(dtype, g, N, mfma, stream);
}

int nt_grouped_gemm_dx_swiglu(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                              const void* gate, const void* value, int32_t E, int64_t A,
                              int64_t K, int64_t N, void* dgate, void* dvalue, void* ws,
                              size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dgate, kDx);
  if (st != NT_OK) return st;
  if (A > 0 && K > 0 && (dvalue == nullptr || gate == nullptr || value == nullptr))
    return NT_ERR_INVALID_ARG;
  if (A == 0 || K == 0) return NT_OK;
  GemmArgs g{dOut, W, offsets, E, A, K, N, dgate, 0, 0, 0, dvalue, gate, 0, nullptr,
             nullptr, nullptr, nullptr, value};
  const uintptr_t al = reinterpret_cast<uintptr_t>(dvalue) | reinterpret_cast<uintptr_t>(gate) |
                       reinterpret_cast<uintptr_t>(value);
  const bool mfma = mfma_ok(dtype, K, N, dOut, W, dgate) && al % 16 == 0;
  return launch_mode<kDx, kEpiSwiGLUGrad>(dtype, g, K, mfma, stream);
}

int nt_grouped_gemm_dx2(int dtype, const void* W1, const void* W2, const int32_t* offsets,
                        const void* dOut1, const void* dOut2, int32_t E, int64_t A, int64_t K,
                        int64_t N, void* dX, void* ws, size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, dOut1, W1, offsets, dX, kDx);
  if (st != NT_OK) return st;
  if (A > 0 && N > 0 && K > 0 && (W2 == nullptr || dOut2 == nullptr)) return NT_ERR_INVALID_ARG;
  if (A == 0 || K == 0) return NT_OK;
  GemmArgs g{dOut1, W1, offsets, E, A, K, N, dX, 0, 0, 0, nullptr, nullptr, 0, nullptr,
             dOut2, W2, nullptr, nullptr};
  // The MFMA path switches operands at a k-step boundary: N a multiple of 64.
  const uintptr_t al = reinterpret_cast<uintptr_t>(W2) | reinterpret_cast<uintptr_t>(dOut2);
  const bool mfma = mfma_ok(dtype, K, N, dOut1, W1, dX) && al % 16 == 0 && N % 64 == 0;
  return launch_mode<kDx, kEpiDualK>(dtype, g, K, mfma, stream);
}

int nt_grouped_gemm_dw_dx_swiglu(int dtype, const void* hidden, const void* W,
                                 const int32_t* offsets, const void* dOut, const void* gate,
                                 const void* value, int32_t E, int64_t A, int64_t K, int64_t N,
                                 void* dW, void* dgate, void* dvalue, void* ws, size_t ws_bytes,
                                 hipStream_t stream) {
  int st = check_gemm(dtype, E, A, K, N, hidden, dOut, offsets, dW, kDw);
  if (st != NT_OK) return st;
  if (A == 0 || K == 0)
    return dw_impl(dtype, hidden, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, stream);
  st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dgate, kDx);
  if (st != NT_OK) return st;
  if (dvalue == nullptr || gate == nullptr || value == nullptr) return NT_ERR_INVALID_ARG;
  GemmArgs gx{dOut, W, offsets, E, A, K, N, dgate, 0, 0, 0, dvalue, gate, 0, nullptr,
              nullptr, nullptr, nullptr, value};
  const uintptr_t al = reinterpret_cast<uintptr_t>(dvalue) | reinterpret_cast<uintptr_t>(gate) |
                       reinterpret_cast<uintptr_t>(value);
  const bool dx_mfma = mfma_ok(dtype, K, N, dOut, W, dgate) && al % 16 == 0;
  return pair_dw_dx<kEpiSwiGLUGrad>(dtype, hidden, offsets, dOut, E, A, K, N, dW, ws, ws_bytes,
                                    gx, dx_mfma, stream);
}

int nt_grouped_gemm_dw_dx2(int dtype, const void* X, const void* W1, const void* W2,
                           const int32_t* offsets, const void* dOut1, const void* dOut2,
                           int32_t E, int64_t A, int64_t K, int64_t N, void* dW1, void* dX,
                           void* ws, size_t ws_bytes, hipStream_t stream) {
  int st = check_gemm(dtype, E, A, K, N, X, dOut1, offsets, dW1, kDw);
  if (st != NT_OK) return st;
  if (A == 0 || K == 0)
    return dw_impl(dtype, X, offsets, dOut1, E, A, K, N, dW1, ws, ws_bytes, stream);
  st = check_gemm(dtype, E, A, K, N, dOut1, W1, offsets, dX, kDx);
  if (st != NT_OK) return st;
  if (N > 0 && (W2 == nullptr || dOut2 == nullptr)) return NT_ERR_INVALID_ARG;
  GemmArgs gx{dOut1, W1, offsets, E, A, K, N, dX, 0, 0, 0, nullptr, nullptr, 0, nullptr,
              dOut2, W2, nullptr, nullptr};
  const uintptr_t al = reinterpret_cast<uintptr_t>(W2) | reinterpret_cast<uintptr_t>(dOut2);
  const bool dx_mfma = mfma_ok(dtype, K, N, dOut1, W1, dX) && al % 16 == 0 && N % 64 == 0;
  return pair_dw_dx<kEpiDualK>(dtype, X, offsets, dOut1, E, A, K, N, dW1, ws, ws_bytes, gx,
                               dx_mfma, stream);
}

int nt_grouped_gemm_dw(int dtype, const void* X, const int32_t* offsets, const void* dOut,
                       int32_t E, int64_t A, int64_t K, int64_t N, void* dW, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
  int st = check_gemm(dtype, E, A, K, N, X, dOut, offsets, dW, kDw);
  if (st != NT_OK) return st;
  return dw_impl(dtype, X, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, stream);
}

int nt_grouped_gemm_dw_dx(int dtype, const void* X, const void* W, const int32_t* offsets,
                          const void* dOut, int32_t E, int64_t A, int64_t K, int64_t N, void* dW,
                          void* dX, void* ws, size_t ws_bytes, hipStream_t stream) {
  int st = check_gemm(dtype, E, A, K, N, X, dOut, offsets, dW, kDw);
  if (st != NT_OK) return st;
  // No rows (or no dX columns): only the dW (zero for empty experts).
  if (A == 0 || K == 0) return dw_impl(dtype, X, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, stream);
  st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dX, kDx);
  if (st != NT_OK) return st;
  GemmArgs gx{dOut, W, offsets, E, A, K, N, dX, 0, 0, 0, nullptr, nullptr, 0, nullptr};
  return pair_dw_dx<kEpiPlain>(dtype, X, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, gx,
                               mfma_ok(dtype, K, N, dOut, W, dX), stream);
}

int nt_grouped_gemm_dw_dx_gelu(int dtype, const void* act, const void* W, const int32_t* offsets,
                               const void* dOut, const void* act_grad, int32_t E, int64_t A,
                               int64_t K, int64_t N, void* dW, void* dH, void* ws,
                               size_t ws_bytes, hipStream_t stream) {
  int st = check_gemm(dtype, E, A, K, N, act, dOut, offsets, dW, kDw);
  if (st != NT_OK) return st;
  if (A == 0 || K == 0)
    return dw_impl(dtype, act, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, stream);
  st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dH, kDx);
  if (st != NT_OK) return st;
  if (act_grad == nullptr) return NT_ERR_INVALID_ARG;
  GemmArgs gx{dOut, W, offsets, E, A, K, N, dH, 0, 0, 0, nullptr, act_grad, 0, nullptr};
  const bool dx_mfma = mfma_ok(dtype, K, N, dOut, W, dH) &&
                       reinterpret_cast<uintptr_t>(act_grad) % 16 == 0;
  return pair_dw_dx<kEpiGeluGrad>(dtype, act, offsets, dOut, E, A, K, N, dW, ws, ws_bytes, gx,
                                  dx_mfma, stream);
}

}  // extern "C"
