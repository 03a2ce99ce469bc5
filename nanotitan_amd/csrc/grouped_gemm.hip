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

#include "common.hpp"

namespace nt {
namespace {

enum GemmMode { kFwd = 0, kDx = 1, kDw = 2 };

constexpr int kGemmThreads = 256;

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

template <typename T>
struct mfma_op;
template <>
struct mfma_op<bf16> {
  typedef bf16x8_t vec;
  __device__ static f32x16_t run(vec a, vec b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct mfma_op<f16> {
  typedef f16x8_t vec;
  __device__ static f32x16_t run(vec a, vec b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // elements; 144 B rows keep 16-B reads conflict-free

// Operand tiles are fetched with raw buffer loads: one wave-uniform
// descriptor per tile and k-step (base address + byte range), a 32-bit
// per-lane offset, and the hardware's range check returning zeros for any
// offset past the range. Lanes whose slot is outside the tile get kOob.
// No branches or selects around the loads, and no 64-bit address registers.
constexpr uint32_t kBufConfig = 0x00020000u;  // gfx9 buffer descriptor word 3
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int32_t n = (int32_t)(bytes <= 0 ? 0 : (bytes > 0x7ffffff0 ? 0x7ffffff0 : bytes));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, (int)kBufConfig);
}

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// K-contiguous operand: element (row, kk) at p[row*ld + kk]; `rows` valid
// rows, `kleft` valid kk from this k-step on. One 16-byte chunk (8 elements
// along kk) per slot.
template <int ROWS>
struct LoaderK {
  static constexpr int kChunks = ROWS * kBK / 8 / kGemmThreads;
  static constexpr int kLoads = kChunks;   // buffer loads per tile
  static constexpr int kStores = kChunks;  // LDS writes per tile
  uint4 r[kChunks];
  __device__ void load(const uint16_t* p, int64_t ld, int64_t rows, int64_t kleft) {
    const int64_t kv = kleft < kBK ? kleft : kBK;
    const int64_t rv = rows < ROWS ? rows : ROWS;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p, ((rv - 1) * ld + kv) * 2);
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int q = threadIdx.x + i * kGemmThreads;
      const int row = q / (kBK / 8);
      const int kc = (q % (kBK / 8)) * 8;
      const uint32_t off = kc < kv ? (uint32_t)(row * ld + kc) * 2u : kOob;
      r[i] = buf_load16(rs, off);
    }
  }
  __device__ void store(uint16_t* s) const {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int q = threadIdx.x + i * kGemmThreads;
      const int row = q / (kBK / 8);
      const int kc = (q % (kBK / 8)) * 8;
      *reinterpret_cast<uint4*>(s + row * kLdsStride + kc) = r[i];
    }
  }
};

// M-contiguous operand: element (row, kk) at p[kk*ld + row]; `rows` valid
// rows (columns in memory), `kleft` valid kk. Each slot is a 4 (kk) x 8 (row)
// block: four 16-byte loads, transposed in registers into eight 8-byte LDS
// writes (row-major, kk contiguous). Consecutive lanes take consecutive kk
// blocks of the same rows, so each group of 16 lanes writes 128 contiguous
// LDS bytes of one row (bank-conflict free); across the wave the four row
// groups read 64 contiguous bytes of every HBM row they touch.
template <int ROWS>
struct LoaderM {
  static constexpr int kBlocks = ROWS * kBK / 32 / kGemmThreads;
  static_assert(kBlocks >= 1, "tile too small for one 4x8 block per thread");
  static constexpr int kLoads = 4 * kBlocks;
  static constexpr int kStores = 8 * kBlocks;
  uint4 r[kBlocks][4];
  __device__ void load(const uint16_t* p, int64_t ld, int64_t rows, int64_t kleft) {
    const int64_t kv = kleft < kBK ? kleft : kBK;
    const int64_t cv = rows < ld ? rows : ld;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p, ((kv - 1) * ld + cv) * 2);
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      const int q = threadIdx.x + i * kGemmThreads;
      const int kb = (q % (kBK / 4)) * 4;
      const int mb = (q / (kBK / 4)) * 8;
      const bool ok = mb < cv;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const uint32_t off = ok ? (uint32_t)((kb + rr) * ld + mb) * 2u : kOob;
        r[i][rr] = buf_load16(rs, off);
      }
    }
  }
  __device__ void store(uint16_t* s) const {
#pragma unroll
    for (int i = 0; i < kBlocks; ++i) {
      const int q = threadIdx.x + i * kGemmThreads;
      const int kb = (q % (kBK / 4)) * 4;
      const int mb = (q / (kBK / 4)) * 8;
      const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&r[i][0]);
      const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&r[i][1]);
      const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&r[i][2]);
      const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&r[i][3]);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        // Element 2w: low halves; element 2w+1: high halves.
        uint2 lo, hi;
        lo.x = __builtin_amdgcn_perm(w1[w], w0[w], 0x05040100u);
        lo.y = __builtin_amdgcn_perm(w3[w], w2[w], 0x05040100u);
        hi.x = __builtin_amdgcn_perm(w1[w], w0[w], 0x07060302u);
        hi.y = __builtin_amdgcn_perm(w3[w], w2[w], 0x07060302u);
        *reinterpret_cast<uint2*>(s + (mb + 2 * w) * kLdsStride + kb) = lo;
        *reinterpret_cast<uint2*>(s + (mb + 2 * w + 1) * kLdsStride + kb) = hi;
      }
    }
  }
};

template <bool KCONTIG, int ROWS>
struct LoaderSel;
template <int ROWS>
struct LoaderSel<true, ROWS> {
  typedef LoaderK<ROWS> type;
};
template <int ROWS>
struct LoaderSel<false, ROWS> {
  typedef LoaderM<ROWS> type;
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
};

// Workgroup ids are dealt to the 8 XCDs round-robin; renumber them so each
// XCD receives a contiguous range of logical tiles (tiles that share operand
// panels then share that XCD's L2).
__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t G) {
  constexpr int kXcd = 8;
  const int64_t q = G / kXcd, r = G % kXcd;
  const int64_t x = bid % kXcd, s = bid / kXcd;
  return x * q + (x < r ? x : r) + s;
}

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

// Persistent: one or two workgroups per CU loop over output tiles. Tiles are
// dealt to XCDs in contiguous ranges (neighbouring tiles share operand panels
// in that XCD's L2), and a tile's output stores drain while the next tile
// computes. Each tile is BM x BN, computed by 4 waves (2 x 2); each wave owns a
// (BM/2) x (BN/2) block of 32x32 MFMA tiles. The MFMA is issued with the B
// fragment as its first operand, so each lane's accumulator holds 4
// consecutive output columns of one output row (packable 8-byte groups).
// K advances 64 per iteration through two LDS stages (one barrier per
// iteration); the epilogue stages the bf16/fp16 tile through LDS and writes
// 16-byte row chunks.
template <typename T, int MODE, int BM, int BN>
__global__ void __launch_bounds__(kGemmThreads)
__attribute__((amdgpu_waves_per_eu(1, BM * BN >= 256 * 128 ? 1 : 2)))
gg_mfma_kernel(GemmArgs g) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int kStageA = BM * kLdsStride;
  constexpr int kStage = (BM + BN) * kLdsStride;
  constexpr int kEpiStride = BN + 8;
  constexpr int kLdsElems = (2 * kStage > BM * kEpiStride) ? 2 * kStage : BM * kEpiStride;
  __shared__ __attribute__((aligned(16))) uint16_t smem[kLdsElems];
  __shared__ int32_t s_pref[NT_MAX_EXPERTS + 1];

  constexpr bool kAK = MODE != kDw;   // A operand K-contiguous?
  constexpr bool kBK_ = MODE == kDx;  // B operand K-contiguous?
  typedef typename LoaderSel<kAK, BM>::type LA;
  typedef typename LoaderSel<kBK_, BN>::type LB;

  int64_t mtiles = g.mtiles;
  if (MODE != kDw) {
    build_m_prefix(g.offsets, g.E, g.A, BM, s_pref);
    mtiles = s_pref[g.E];
  }
  const int64_t total = mtiles * g.ntn;
  // Blocks are dealt to the 8 XCDs round-robin (block b runs on XCD b % 8).
  // XCD x owns a contiguous range of tiles, sized by how many blocks it has;
  // its blocks walk that range in step. With one tile per block (large
  // tiles, non-persistent launch) this reduces to a renumbering.
  constexpr int kXcd = 8;
  const int64_t G = gridDim.x;
  const int xcd = blockIdx.x % kXcd;
  const int64_t q = G / kXcd, r = G % kXcd;
  const int64_t before = xcd * q + (xcd < r ? xcd : r);
  const int64_t nbx = q + (xcd < r ? 1 : 0);
  const int64_t t_end = total * (before + nbx) / G;
  for (int64_t logical = total * before / G + blockIdx.x / kXcd; logical < t_end;
       logical += nbx) {
  const uint16_t* pa;
  const uint16_t* pb;
  int64_t lda, ldb, rows_valid, cols_valid, kred;
  uint16_t* po;
  int64_t ldo;

  int64_t mt;
  int nt;
  tile_coords(logical, mtiles, g.ntn, mt, nt);

  if (MODE == kDw) {
    const int e = (int)(mt / g.ntm);
    const int mtl = (int)(mt % g.ntm);
    int64_t r0, r1;
    expert_rows(g.offsets, e, g.A, r0, r1);
    kred = r1 - r0;
    pa = static_cast<const uint16_t*>(g.a) + r0 * g.K + (int64_t)mtl * BM;
    lda = g.K;
    pb = static_cast<const uint16_t*>(g.b) + r0 * g.N + (int64_t)nt * BN;
    ldb = g.N;
    rows_valid = g.K - (int64_t)mtl * BM;
    cols_valid = g.N - (int64_t)nt * BN;
    po = static_cast<uint16_t*>(g.out) + (int64_t)e * g.K * g.N + (int64_t)mtl * BM * g.N +
         (int64_t)nt * BN;
    ldo = g.N;
  } else {
    int e;
    int64_t r0, r1, mtl;
    find_m_tile(g.offsets, g.E, g.A, s_pref, mt, e, r0, r1, mtl);
    const int64_t row0 = r0 + mtl * BM;
    rows_valid = r1 - row0;
    if (MODE == kFwd) {
      pa = static_cast<const uint16_t*>(g.a) + row0 * g.K;
      lda = g.K;
      pb = static_cast<const uint16_t*>(g.b) + (int64_t)e * g.K * g.N + (int64_t)nt * BN;
      ldb = g.N;
      cols_valid = g.N - (int64_t)nt * BN;
      kred = g.K;
      po = static_cast<uint16_t*>(g.out) + row0 * g.N + (int64_t)nt * BN;
      ldo = g.N;
    } else {  // kDx
      pa = static_cast<const uint16_t*>(g.a) + row0 * g.N;
      lda = g.N;
      pb = static_cast<const uint16_t*>(g.b) + (int64_t)e * g.K * g.N + (int64_t)nt * BN * g.N;
      ldb = g.N;
      cols_valid = g.K - (int64_t)nt * BN;
      kred = g.N;
      po = static_cast<uint16_t*>(g.out) + row0 * g.K + (int64_t)nt * BN;
      ldo = g.K;
    }
  }

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int wm = wave >> 1, wn = wave & 1;

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  LA la;
  LB lb;
  const int64_t nk = ceil_div(kred, kBK);
  // Operand pointers advance along the reduction dimension.
  const int64_t a_kstep = kAK ? kBK : kBK * lda;
  const int64_t b_kstep = kBK_ ? kBK : kBK * ldb;
  if (nk > 0) {
    la.load(pa, lda, rows_valid, kred);
    lb.load(pb, ldb, cols_valid, kred);
    la.store(smem);
    lb.store(smem + kStageA);
  }
  __syncthreads();
  typedef typename mfma_op<T>::vec vec;
  // Fragments for k-step ks+1 are read from LDS while the MFMAs of k-step
  // ks run (two register sets), hiding LDS latency inside one wave.
  auto compute = [&](const uint16_t* sa, const uint16_t* sb) {
    const uint16_t* pa_l = sa + (wm * WM + (lane & 31)) * kLdsStride + (lane >> 5) * 8;
    const uint16_t* pb_l = sb + (wn * WN + (lane & 31)) * kLdsStride + (lane >> 5) * 8;
    vec av[2][TM], bv[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) av[0][i] = *reinterpret_cast<const vec*>(pa_l + i * 32 * kLdsStride);
#pragma unroll
    for (int j = 0; j < TN; ++j) bv[0][j] = *reinterpret_cast<const vec*>(pb_l + j * 32 * kLdsStride);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < kBK / 16) {
        const int kof = (ks + 1) * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i)
          av[cur ^ 1][i] = *reinterpret_cast<const vec*>(pa_l + i * 32 * kLdsStride + kof);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bv[cur ^ 1][j] = *reinterpret_cast<const vec*>(pb_l + j * 32 * kLdsStride + kof);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma_op<T>::run(bv[cur][j], av[cur][i], acc[i][j]);
      // Keep each k-step's reads ahead of its MFMAs, and the MFMAs of step
      // ks ahead of the reads for step ks+2 (no reordering across).
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Steady state (branch-free body): load tile kt+1 into registers, compute
  // tile kt from LDS, store tile kt+1 into the other LDS stage, one barrier.
  for (int64_t kt = 0; kt + 1 < nk; ++kt) {
    const int64_t kleft = kred - (kt + 1) * kBK;
    // The next tile's buffer loads go out first; their latency is covered
    // by this tile's MFMAs, and the LDS stores come after them.
    la.load(pa + (kt + 1) * a_kstep, lda, rows_valid, kleft);
    lb.load(pb + (kt + 1) * b_kstep, ldb, cols_valid, kleft);
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t* sa = smem + (kt & 1) * kStage;
    compute(sa, sa + kStageA);
    uint16_t* nxt = smem + ((kt + 1) & 1) * kStage;
    la.store(nxt);
    lb.store(nxt + kStageA);
    __syncthreads();
  }
  if (nk > 0) {
    const uint16_t* sa = smem + ((nk - 1) & 1) * kStage;
    compute(sa, sa + kStageA);
  }
  __syncthreads();

  // Epilogue. acc[i][j][v] = C[m][n] with m = wm*WM + 32i + lane%32 and
  // n = wn*WN + 32j + 8*(v/4) + 4*(lane/32) + v%4: each lane packs 4
  // consecutive columns into 8 bytes of the LDS staging tile.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int m = wm * WM + i * 32 + (lane & 31);
        const int n = wn * WN + j * 32 + 8 * gq + 4 * (lane >> 5);
        uint2 pk;
        pk.x = (uint32_t)elem<T>::store(acc[i][j][4 * gq + 0]) |
               ((uint32_t)elem<T>::store(acc[i][j][4 * gq + 1]) << 16);
        pk.y = (uint32_t)elem<T>::store(acc[i][j][4 * gq + 2]) |
               ((uint32_t)elem<T>::store(acc[i][j][4 * gq + 3]) << 16);
        *reinterpret_cast<uint2*>(smem + m * kEpiStride + n) = pk;
      }
  __syncthreads();
  constexpr int kChunksPerRow = BN / 8;
#pragma unroll 4
  for (int q = threadIdx.x; q < BM * kChunksPerRow; q += kGemmThreads) {
    const int row = q / kChunksPerRow;
    const int c = (q % kChunksPerRow) * 8;
    if (row < rows_valid && c < cols_valid)
      *reinterpret_cast<uint4*>(po + (int64_t)row * ldo + c) =
          *reinterpret_cast<const uint4*>(smem + row * kEpiStride + c);
  }
  __syncthreads();  // the staging tile is read before the next tile reuses LDS
  // 256x256 tiles are launched one per workgroup: a single pass, so nothing
  // is carried (or hoisted) across tiles.
  if constexpr (BM * BN >= 256 * 256) break;
  }
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
    kred = MODE == kFwd ? g.K : g.N;
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
      if (kg < kred && m < rows_valid) {
        if (MODE == kFwd) va = to_acc<T>(X[(m0 + m) * g.K + kg]);
        else if (MODE == kDx) va = to_acc<T>(X[(m0 + m) * g.N + kg]);
        else va = to_acc<T>(X[(r0 + kg) * g.K + m0 + m]);
      }
      if (kg < kred && m < cols_valid) {
        const int64_t n = n0 + m;
        if (MODE == kFwd) vb = to_acc<T>(Bm[(int64_t)e * g.K * g.N + kg * g.N + n]);
        else if (MODE == kDx) vb = to_acc<T>(Bm[(int64_t)e * g.K * g.N + n * g.N + kg]);
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

// Compute units of the current device (cached per device id).
int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

template <int MODE, int BM, int BN>
int launch_mfma(int dtype, GemmArgs g, int64_t out_cols, hipStream_t s) {
  g.ntn = (int32_t)ceil_div(out_cols, BN);
  if (MODE == kDw) {
    g.ntm = (int32_t)ceil_div(g.K, BM);
    g.mtiles = (int64_t)g.E * g.ntm;
  } else {
    g.ntm = 0;
    g.mtiles = ceil_div(g.A, BM) + g.E;
  }
  const int64_t tiles = g.mtiles * g.ntn;
  if (tiles == 0) return NT_OK;
  if (tiles > INT32_MAX) return NT_ERR_TOO_LARGE;
  // 256x256 tiles: one tile per workgroup (a tile loop would push the
  // 512-register kernel into spills); smaller tiles: persistent workgroups,
  // one (256x128) or two (128x128) per CU.
  const int per_cu = BM * BN >= 256 * 128 ? 1 : 2;
  const int64_t nblocks = BM * BN >= 256 * 256
                              ? tiles
                              : std::min<int64_t>(tiles, (int64_t)device_cus() * per_cu);
  const dim3 grid((unsigned)nblocks);
  if (dtype == NT_BF16)
    hipLaunchKernelGGL((gg_mfma_kernel<bf16, MODE, BM, BN>), grid, dim3(kGemmThreads), 0, s, g);
  else
    hipLaunchKernelGGL((gg_mfma_kernel<f16, MODE, BM, BN>), grid, dim3(kGemmThreads), 0, s, g);
  return launch_status();
}

// Tile shape: 256x256 when the problem has enough tiles to fill the 256 CUs
// a few times over, otherwise smaller tiles for more parallelism.
template <int MODE>
int launch_mfma_auto(int dtype, GemmArgs g, int64_t out_cols, hipStream_t s) {
  const int64_t rows = MODE == kDw ? g.K * g.E : g.A;
  auto tiles = [&](int bm, int bn) { return ceil_div(rows, bm) * ceil_div(out_cols, bn); };
  if (tiles(256, 256) >= 1024) return launch_mfma<MODE, 256, 256>(dtype, g, out_cols, s);
  if (tiles(256, 128) >= 768) return launch_mfma<MODE, 256, 128>(dtype, g, out_cols, s);
  return launch_mfma<MODE, 128, 128>(dtype, g, out_cols, s);
}

template <int MODE>
int launch_mode(int dtype, GemmArgs g, int64_t out_cols, bool mfma, hipStream_t s) {
  if (mfma) return launch_mfma_auto<MODE>(dtype, g, out_cols, s);
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

int check_gemm(int dtype, int32_t E, int64_t A, int64_t K, int64_t N, const void* a,
               const void* b, const int32_t* offsets, const void* out) {
  if (dtype_bytes(dtype) == 0) return NT_ERR_DTYPE;
  if (E < 1 || A < 0 || K < 0 || N < 0) return NT_ERR_INVALID_ARG;
  if (E > NT_MAX_EXPERTS) return NT_ERR_TOO_MANY_EXPERTS;
  if (offsets == nullptr) return NT_ERR_INVALID_ARG;
  if ((A > 0 && K > 0 && a == nullptr) || (K > 0 && N > 0 && b == nullptr)) return NT_ERR_INVALID_ARG;
  if (out == nullptr && ((A > 0 && (K > 0 || N > 0)) || (K > 0 && N > 0))) return NT_ERR_INVALID_ARG;
  if (A > INT32_MAX) return NT_ERR_TOO_LARGE;
  return NT_OK;
}

}  // namespace
}  // namespace nt

using namespace nt;

extern "C" {

size_t nt_grouped_gemm_workspace_bytes(int dtype, int32_t E, int64_t A, int64_t K, int64_t N) {
  (void)dtype;
  (void)E;
  (void)A;
  (void)K;
  (void)N;
  return 0;
}

int nt_grouped_gemm(int dtype, const void* X, const int32_t* offsets, const void* W, int32_t E,
                    int64_t A, int64_t K, int64_t N, void* out, void* ws, size_t ws_bytes,
                    hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, X, W, offsets, out);
  if (st != NT_OK) return st;
  if (A == 0 || N == 0) return NT_OK;
  GemmArgs g{X, W, offsets, E, A, K, N, out, 0, 0, 0};
  return launch_mode<kFwd>(dtype, g, N, mfma_ok(dtype, K, N, X, W, out), stream);
}

int nt_grouped_gemm_dx(int dtype, const void* W, const int32_t* offsets, const void* dOut,
                       int32_t E, int64_t A, int64_t K, int64_t N, void* dX, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, dOut, W, offsets, dX);
  if (st != NT_OK) return st;
  if (A == 0 || K == 0) return NT_OK;
  GemmArgs g{dOut, W, offsets, E, A, K, N, dX, 0, 0, 0};
  return launch_mode<kDx>(dtype, g, K, mfma_ok(dtype, K, N, dOut, W, dX), stream);
}

int nt_grouped_gemm_dw(int dtype, const void* X, const int32_t* offsets, const void* dOut,
                       int32_t E, int64_t A, int64_t K, int64_t N, void* dW, void* ws,
                       size_t ws_bytes, hipStream_t stream) {
  (void)ws;
  (void)ws_bytes;
  int st = check_gemm(dtype, E, A, K, N, X, dOut, offsets, dW);
  if (st != NT_OK) return st;
  if (K == 0 || N == 0) return NT_OK;
  GemmArgs g{X, dOut, offsets, E, A, K, N, dW, 0, 0, 0};
  return launch_mode<kDw>(dtype, g, N, mfma_ok(dtype, K, N, X, dOut, dW), stream);
}

}  // extern "C"
