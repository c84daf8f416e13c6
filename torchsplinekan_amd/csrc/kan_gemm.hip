// Dense contraction engine for the KAN forward and backward on gfx950 MFMA.
//
// The three contractions of a KANLinear step all run through this file with
// different operand layouts (A = augmented basis [H | silu(x)],
// W = augmented weight [coef*scaler | base_weight], D = grad_output):
//   forward  Y[n,o]  = sum_k A[n,k] W[o,k]     (NT: both K-contiguous)
//   params   G[o,k]  = sum_n D[n,o] A[n,k]     (TN: both M/N-contiguous)
//   input    E[n,k]  = sum_o D[n,o] W[o,k]     (NN)
// They replace the cuBLAS calls of csrc/kan_cuda.cu:521-529, 579-604.
//
// fp32 runs on gemm_pipe_kernel, a software-pipelined v_mfma_f32_32x32x2f32
// main loop, in one of three tile configurations picked per problem by a
// cost model (pick_cfg_f32):
//   big    256x256 block tile, 8 waves of 128x64 (two waves per SIMD), one
//          block per CU;
//   small  128x128 block tile, 4 waves of 64x64, two blocks per CU (for
//          problems with too few big tiles to fill the chip);
//   narrow 256x64 block tile, 4 waves of 64x64, for outputs of at most 64
//          columns.
// A 256x256 tile over 4 waves of 128x128 (one wave per SIMD) can be forced
// for comparison.
// fp64 runs on gemm_kernel: 128x128 tile, 2x2 waves, v_mfma_f64_16x16x4f64.
//
// Operand slabs (BK deep) are staged through LDS with double buffering.  Each
// operand keeps its global layout in LDS:
//   K-contiguous operand  -> LDS [rows][BK+4]; a lane reads 4 consecutive k
//                            with one 16-byte ds_read.  Within each k-group
//                            of the MFMA the k order is permuted identically
//                            for A and B (step s, lane group q uses
//                            k = KG*g + 4q + s), which leaves the sum unchanged;
//   MN-contiguous operand -> LDS [BK][rows+4]; a lane reads one element.
// Pipeline of gemm_pipe_kernel, per K slab kt (NG k-groups of 8):
//   group 0 issues the LDS stores of slab kt+1 (held in registers) and the
//   global loads of slab kt+2, interleaved one-for-one with its MFMAs by
//   scheduling-group barriers; every group reads the fragments of the next
//   group from LDS while its own MFMAs run; the barrier that publishes slab
//   kt+1 sits before the last group's MFMAs, which then cover the first
//   fragment reads of slab kt+1.  The loop body is branch-free: whole tiles
//   (every row, column and k in range, 16-byte aligned operands) take vector
//   loads, edge tiles take a separately compiled loop with clamped scalar
//   loads and zero fill.
// Scheduling: the linear workgroup id is remapped so that each XCD (dispatch
// is round-robin over 8 XCDs) receives a contiguous range of tiles, visited
// in groups of 8 row-tiles so that tiles running together on one XCD share
// operand slabs in its L2.  Optional split-K writes partial products to
// separate slices of C (reduced by the caller in a fixed order).

#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "kan_common.h"
#include "kan_spline.h"

namespace kan {
namespace {

constexpr int kPadK = 4;
constexpr int kPadMN = 4;
constexpr int kGroupM = 8;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

// MFMA shapes: operand fragment of lane (row, kq) and accumulator layout.
template <typename T, int MF>
struct Mfma;

template <>
struct Mfma<float, 32> {  // v_mfma_f32_32x32x2f32
  typedef f32x16 acc_t;
  static constexpr int kKG = 8;
  static constexpr int kNAcc = 16;
  __device__ static __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane) { return lane & 31; }
  __device__ static __forceinline__ int kq(int lane) { return lane >> 5; }
  __device__ static __forceinline__ int kofs(int g, int q) { return 8 * g + 4 * q; }
  __device__ static __forceinline__ int out_row(int lane, int v) {
    return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
  }
  __device__ static __forceinline__ int out_col(int lane) { return lane & 31; }
};

template <>
struct Mfma<double, 16> {  // v_mfma_f64_16x16x4f64
  typedef f64x4 acc_t;
  static constexpr int kKG = 16;
  static constexpr int kNAcc = 4;
  __device__ static __forceinline__ acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane) { return lane & 15; }
  __device__ static __forceinline__ int kq(int lane) { return lane >> 4; }
  __device__ static __forceinline__ int kofs(int g, int q) { return 16 * g + 4 * q; }
  // the f64 instruction interleaves rows across the four accumulators
  __device__ static __forceinline__ int out_row(int lane, int v) { return (lane >> 4) + 4 * v; }
  __device__ static __forceinline__ int out_col(int lane) { return lane & 15; }
};

// Kernel configuration: block tile BM x BN, K slab BK, WM x WN waves,
// MFMA shape MF, minimum resident blocks per CU.
template <typename T_, int BM_, int BN_, int BK_, int WM_, int WN_, int MF_, int MINB_>
struct Cfg {
  typedef T_ T;
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, MF = MF_;
  static constexpr int MINB = MINB_;
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / MF, FN = TN / MF;
  static_assert(FM * MF == TM && FN * MF == TN, "wave tile must be whole MFMA tiles");
  static_assert(BK % Mfma<T, MF>::kKG == 0, "slab must be whole k-groups");
};

// 256 x 256 block tiles: 8 waves of 128 x 64 (two per SIMD: while one wave
// of a SIMD waits at the slab barrier or on its fragment reads, the other
// issues MFMAs), or 4 waves of 128 x 128 (one per SIMD; only when forced).
using CfgF32Big = Cfg<float, 256, 256, 32, 2, 4, 32, 1>;
using CfgF32Big4 = Cfg<float, 256, 256, 32, 2, 2, 32, 1>;
using CfgF32Small = Cfg<float, 128, 128, 32, 2, 2, 32, 2>;
// Narrow outputs (N <= 64, e.g. a 64-wide layer): 4 waves stacked along M,
// 64 x 64 each, so no wave computes padding columns.
using CfgF32Narrow = Cfg<float, 256, 64, 32, 4, 1, 32, 1>;
using CfgF64 = Cfg<double, 128, 128, 16, 2, 2, 16, 1>;
// fp64, 256 x 128 block tiles: 8 waves of 64 x 64, two per SIMD (while one
// wave waits at the slab barrier the other issues MFMAs)
using CfgF64Big = Cfg<double, 256, 128, 16, 4, 2, 16, 1>;
// fp64 on the software-pipelined kernel: 128 x 128 tiles, 32-deep slabs (two
// k-groups), 8 waves of 64 x 32 (two per SIMD); 147 KB of LDS, one block per CU
using CfgF64Pipe = Cfg<double, 128, 128, 32, 2, 4, 16, 1>;
// fp64 on the pipelined kernel with 64 x 64 tiles: 4 waves of 32 x 32, two
// blocks per CU (73 KB of LDS each), for products with a side of at most 64
// (a 64-wide layer's products fill half of a 128 x 128 tile)
using CfgF64Small = Cfg<double, 64, 64, 32, 2, 2, 16, 2>;

// Configurations that run on gemm_pipe_kernel (the rest on gemm_kernel).
template <class C>
struct RunsPipe {
  static constexpr bool value = std::is_same<typename C::T, float>::value || C::BK == 32;
};

template <typename T>
struct GemmParams {
  const T* A;
  const T* B;
  T* C;
  int64_t M, N, K;
  int64_t lda, ldb, ldc;
  int64_t k_per_split;
  int64_t split_stride;
  int tiles_m, tiles_n, splits;
  int vec;  // operands 16-byte aligned with leading dimensions % 4 == 0
  int buf;  // a whole slab's byte offsets fit 31 bits (buffer-resource loads)
};

// LDS footprint of one operand slab.
template <int ROWS, int BK, bool KCONT>
struct Slab {
  static constexpr int kStride = KCONT ? (BK + kPadK) : (ROWS + kPadMN);
  static constexpr int kElems = KCONT ? ROWS * (BK + kPadK) : BK * (ROWS + kPadMN);
};

// Tile owned by this block: output origin, split and K range.
struct TileCoords {
  int64_t m0, n0, kbeg, kend;
  int split, nkt;
};

template <class C, typename T>
__device__ __forceinline__ TileCoords tile_coords(const GemmParams<T>& p) {
  const int total = p.tiles_m * p.tiles_n * p.splits;
  const int pid = xcd_remap(blockIdx.x, total);
  const int per_split = p.tiles_m * p.tiles_n;
  TileCoords tc;
  tc.split = pid / per_split;
  const int t = pid - tc.split * per_split;
  const int group = kGroupM * p.tiles_n;
  const int first_m = (t / group) * kGroupM;
  const int gm = min(p.tiles_m - first_m, kGroupM);
  const int tm = first_m + (t % group) % gm;
  const int tn = (t % group) / gm;
  tc.m0 = (int64_t)tm * C::BM;
  tc.n0 = (int64_t)tn * C::BN;
  tc.kbeg = (int64_t)tc.split * p.k_per_split;
  tc.kend = min(p.K, tc.kbeg + p.k_per_split);
  tc.nkt = tc.kend > tc.kbeg ? (int)ceil_div(tc.kend - tc.kbeg, C::BK) : 0;
  return tc;
}

// Global -> register staging of one operand slab (ROWS x BK), in chunks of 4
// elements along the contiguous dimension.
template <typename T, int ROWS, int BK, bool KCONT, int NT>
struct SlabLoader {
  static constexpr int kChunks = ROWS * BK / 4;
  static constexpr int kPer = kChunks / NT;
  static_assert(kPer * NT == kChunks, "slab must split evenly over the block");
  Vec4<T> reg[kPer];

  __device__ __forceinline__ void coords(int c, int64_t row0, int64_t k0, int64_t& r,
                                         int64_t& kk) const {
    if (KCONT) {
      r = row0 + c / (BK / 4);
      kk = k0 + 4 * (c % (BK / 4));
    } else {
      kk = k0 + c / (ROWS / 4);
      r = row0 + 4 * (c % (ROWS / 4));
    }
  }

  // Whole slab in bounds and aligned: one 16-byte load per chunk.
  __device__ __forceinline__ void load_full(const T* __restrict__ src, int64_t ld, int64_t row0,
                                            int64_t k0) {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      int64_t r, kk;
      coords(threadIdx.x + p * NT, row0, k0, r, kk);
      reg[p] = *reinterpret_cast<const Vec4<T>*>(KCONT ? src + r * ld + kk : src + kk * ld + r);
    }
  }

  // Whole slab through a buffer resource (fp32).  A lane's byte offset
  // within a slab is the same for every slab, and its chunks p lie a
  // wave-uniform stride apart, so a load takes no per-lane address
  // arithmetic: base (scalar, per slab) + voff (lane, set once) + p * stride
  // (scalar soffset).  Needs NT to be a multiple of the chunks per row.
  uint32_t voff;
  static constexpr int64_t kStep = KCONT ? NT / (BK / 4) : NT / (ROWS / 4);  // rows (k) per p
  __device__ __forceinline__ void init_buf(int64_t ld) {
    static_assert(KCONT ? NT % (BK / 4) == 0 : NT % (ROWS / 4) == 0, "uniform chunk stride");
    int64_t r, kk;
    coords(threadIdx.x, 0, 0, r, kk);
    voff = (uint32_t)((KCONT ? r * ld + kk : kk * ld + r) * (int64_t)sizeof(T));
  }
  __device__ __forceinline__ void load_buf(const T* __restrict__ src, int64_t ld, int64_t row0,
                                           int64_t k0) {
    static_assert(sizeof(T) == 4, "128-bit buffer loads of 4 fp32 values");
    const T* base = KCONT ? src + row0 * ld + k0 : src + k0 * ld + row0;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<T*>(base), (short)0, -1, 0x00020000 /* gfx9 raw buffer, 32-bit data */);
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
          rs, (int)voff, (int)((int64_t)p * kStep * ld * (int64_t)sizeof(T)), 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) reg[p].v[j] = __uint_as_float(v[j]);
    }
  }

  // Edge slab (rows < rows, k < kend; k0 < kend and rows >= 1): every lane
  // loads from an address clamped into the operand and selects zero where
  // the element lies outside it, so the loop has no divergent branches.
  __device__ __forceinline__ void load_guarded(const T* __restrict__ src, int64_t ld, int64_t row0,
                                               int64_t rows, int64_t k0, int64_t kend) {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      int64_t r, kk;
      coords(threadIdx.x + p * NT, row0, k0, r, kk);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t rr = KCONT ? r : r + j;
        const int64_t kj = KCONT ? kk + j : kk;
        const bool in = (rr < rows) && (kj < kend);
        const int64_t rc = rr < rows ? rr : rows - 1;
        const int64_t kc = kj < kend ? kj : kend - 1;
        const T v = KCONT ? src[rc * ld + kc] : src[kc * ld + rc];
        reg[p].v[j] = in ? v : T(0);
      }
    }
  }

  __device__ __forceinline__ void store(T* __restrict__ lds) const {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int c = threadIdx.x + p * NT;
      int off;
      if (KCONT) off = (c / (BK / 4)) * Slab<ROWS, BK, true>::kStride + 4 * (c % (BK / 4));
      else off = (c / (ROWS / 4)) * Slab<ROWS, BK, false>::kStride + 4 * (c % (ROWS / 4));
      *reinterpret_cast<Vec4<T>*>(lds + off) = reg[p];
    }
  }
};

// MFMA operand fragment: the 4 k values (one per MFMA step) of one row.
template <typename T, int ROWS, int BK, bool KCONT>
__device__ __forceinline__ void read_frag(const T* __restrict__ lds, int row, int kofs,
                                          T (&f)[4]) {
  if (KCONT) {
    const Vec4<T> v = *reinterpret_cast<const Vec4<T>*>(lds + row * Slab<ROWS, BK, true>::kStride + kofs);
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = v.v[s];
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = lds[(kofs + s) * Slab<ROWS, BK, false>::kStride + row];
  }
}

// Fragments of an MN-contiguous operand for all F of a wave's MFMA tiles
// at once, with the tiles' rows interleaved: tile t's row r is the wave's
// row F r + t (a permutation of the rows, undone where the output is
// stored), so the F values a lane needs at one k are contiguous in the
// [BK][rows + 4] layout and come from one 8- or 16-byte read instead of F
// scalar reads.  f[t][s] = value of tile t at k = kofs + s.
template <typename T, int ROWS, int BK, int F>
__device__ __forceinline__ void read_frag_il(const T* __restrict__ lds, int row0, int kofs,
                                             T (&f)[F][4]) {
  static_assert(F == 2 || F == 4, "2 or 4 tiles per wave");
  constexpr int kS = Slab<ROWS, BK, false>::kStride;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if constexpr (F == 4) {
      const Vec4<T> v = *reinterpret_cast<const Vec4<T>*>(lds + (kofs + s) * kS + row0);
#pragma unroll
      for (int t = 0; t < 4; ++t) f[t][s] = v.v[t];
    } else {
      typedef T T2 __attribute__((ext_vector_type(2)));
      const T2 v = *reinterpret_cast<const T2*>(lds + (kofs + s) * kS + row0);
      f[0][s] = v[0];
      f[1][s] = v[1];
    }
  }
}

// Writes the wave's accumulators to C (+ split slice), bounds-checked.  AIL /
// BIL: the rows / columns of the MFMA tiles are interleaved (read_frag_il).
template <class C, typename Acc, bool AIL = false, bool BIL = false>
__device__ __forceinline__ void store_tile(const GemmParams<typename C::T>& p, const TileCoords& tc,
                                           const Acc (&acc)[C::FM][C::FN], int wm, int wn,
                                           int lane) {
  typedef Mfma<typename C::T, C::MF> M;
  typename C::T* Cp = p.C + (int64_t)tc.split * p.split_stride;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int cl = M::out_col(lane);
      const int64_t col = tc.n0 + wn * C::TN + (BIL ? C::FN * cl + j : j * C::MF + cl);
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < M::kNAcc; ++v) {
        const int rl = M::out_row(lane, v);
        const int64_t row = tc.m0 + wm * C::TM + (AIL ? C::FM * rl + i : i * C::MF + rl);
        if (row < p.M) Cp[row * p.ldc + col] = acc[i][j][v];
      }
    }
  }
}

// ---- fp64: double-buffered LDS slabs, one fragment set per k-group --------

template <class C, bool AK, bool BKC>
__global__ __launch_bounds__(C::kThreads, C::MINB) void gemm_kernel(GemmParams<typename C::T> p) {
  typedef typename C::T T;
  typedef Mfma<T, C::MF> M;
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, NT = C::kThreads;
  constexpr int FM = C::FM, FN = C::FN, NG = BK / M::kKG;
  typedef Slab<BM, BK, AK> SA;
  typedef Slab<BN, BK, BKC> SB;
  __shared__ __align__(16) T lds_a[2][SA::kElems];
  __shared__ __align__(16) T lds_b[2][SB::kElems];

  const TileCoords tc = tile_coords<C>(p);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int rl = M::row(lane), q = M::kq(lane);

  typename M::acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < M::kNAcc; ++v) acc[i][j][v] = T(0);

  SlabLoader<T, BM, BK, AK, NT> la;
  SlabLoader<T, BN, BK, BKC, NT> lb;
  const bool full = p.vec && (tc.m0 + BM <= p.M) && (tc.n0 + BN <= p.N) &&
                    ((tc.kend - tc.kbeg) % BK == 0);
  auto gload = [&](int slab) {
    const int64_t k0 = tc.kbeg + (int64_t)slab * BK;
    if (full) {
      la.load_full(p.A, p.lda, tc.m0, k0);
      lb.load_full(p.B, p.ldb, tc.n0, k0);
    } else {
      la.load_guarded(p.A, p.lda, tc.m0, p.M, k0, tc.kend);
      lb.load_guarded(p.B, p.ldb, tc.n0, p.N, k0, tc.kend);
    }
  };
  T fa[FM][4], fb[FN][4];
  // MN-contiguous operands: interleaved fragment reads (read_frag_il)
  constexpr bool AIL = !AK, BIL = !BKC;

  if (tc.nkt > 0) {
    gload(0);
    la.store(lds_a[0]);
    lb.store(lds_b[0]);
    __syncthreads();
    for (int kt = 0; kt < tc.nkt; ++kt) {
      const int cur = kt & 1;
      const bool more = kt + 1 < tc.nkt;
      if (more) gload(kt + 1);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if constexpr (AIL) {
          read_frag_il<T, BM, BK, FM>(lds_a[cur], wm * C::TM + FM * rl, M::kofs(g, q), fa);
        } else {
#pragma unroll
          for (int i = 0; i < FM; ++i)
            read_frag<T, BM, BK, AK>(lds_a[cur], wm * C::TM + i * C::MF + rl, M::kofs(g, q), fa[i]);
        }
        if constexpr (BIL) {
          read_frag_il<T, BN, BK, FN>(lds_b[cur], wn * C::TN + FN * rl, M::kofs(g, q), fb);
        } else {
#pragma unroll
          for (int j = 0; j < FN; ++j)
            read_frag<T, BN, BK, BKC>(lds_b[cur], wn * C::TN + j * C::MF + rl, M::kofs(g, q), fb[j]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = M::mma(fa[i][s], fb[j][s], acc[i][j]);
      }
      if (more) {
        la.store(lds_a[cur ^ 1]);
        lb.store(lds_b[cur ^ 1]);
      }
      __syncthreads();
    }
  }
  store_tile<C, typename M::acc_t, AIL, BIL>(p, tc, acc, wm, wn, lane);
}

// ---- fp32: software-pipelined main loop ------------------------------------

template <int N_>
struct IC {
  static constexpr int value = N_;
};

// max(0, |[A, B) intersect [LO, HI)|)
template <int A, int B, int LO, int HI>
struct Overlap {
  static constexpr int lo = A > LO ? A : LO;
  static constexpr int hi = B < HI ? B : HI;
  static constexpr int v = hi > lo ? hi - lo : 0;
};

// Scheduling-group barriers that spread R fragment reads, W LDS stores and L
// global loads (in that order) evenly over KMF MFMAs: MFMA i is followed by
// the memory operations [i*T/KMF, (i+1)*T/KMF) of the T = R+W+L.
template <int I, int KMF, int R, int W, int L>
struct SchedSeq {
  static __device__ __forceinline__ void run() {
    constexpr int T = R + W + L;
    constexpr int a = I * T / KMF, b = (I + 1) * T / KMF;
    constexpr int nr = Overlap<a, b, 0, R>::v;
    constexpr int nw = Overlap<a, b, R, R + W>::v;
    constexpr int nl = Overlap<a, b, R + W, T>::v;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    if constexpr (nr > 0) __builtin_amdgcn_sched_group_barrier(0x100, nr, 0);  // DS read
    if constexpr (nw > 0) __builtin_amdgcn_sched_group_barrier(0x200, nw, 0);  // DS write
    if constexpr (nl > 0) __builtin_amdgcn_sched_group_barrier(0x020, nl, 0);  // VMEM read
    SchedSeq<I + 1, KMF, R, W, L>::run();
  }
};
template <int KMF, int R, int W, int L>
struct SchedSeq<KMF, KMF, R, W, L> {
  static __device__ __forceinline__ void run() {}
};

// ---- fused input-gradient epilogue --------------------------------------
// For the input-side product E[n, c] = sum_o D[n, o] Waug[o, c] (columns
// c = i*R + r of the spline block, then I*R + i of the base block), the
// input gradient needs only
//   dx[n, i] = sum_r E[n, i*R + r] dB_r/dx(x[n, i]) + E[n, I*R + i] silu'(x[n, i]),
// so E is contracted in the GEMM epilogue instead of being written out.
// Each wave stages its accumulator block in LDS, one 32-row MFMA tile row at
// a time, and evaluates for every (sample, feature) whose columns meet the
// block the derivative window of span m (the k+1 columns m-k..m) and, for
// base columns, silu'.  Partial sums go to part[n, i, slot]:
//   slot 0  spline columns of feature i in the block holding column i*R,
//   slot 1  spline columns in the next block (0 if the feature fits in one),
//   slot 2  the base column (when the layer has a base branch).
// dx_finalize_kernel adds them in that fixed order.  A feature that fits in
// one block sums its window in the same order as basis_grad_kernel.
struct DxParams {
  const float* x;     // [M, I] samples (the rows of the product)
  const float* grid;  // [I, nk] knot rows
  float* part;        // [M, I, nslot] partial input gradients; compact route:
                      // [M, I, k+1] span-window values of E
  float* es;          // compact route: [M, I] base-column values of E
  int64_t I;
  int64_t ksp;        // I * R: first base column
  int R, nk, nslot;
};

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Column range of one wave block and the (sample, feature) items it owns.
struct DxBlock {
  int64_t c0, c_end, sp_end, fs, b0;
  int nfs, nbase;
  __device__ __host__ DxBlock(int64_t c0_, int64_t N, int64_t ksp, int R, int TN, bool base)
      : c0(c0_) {
    c_end = c0 + TN < N ? c0 + TN : N;
    sp_end = c_end < ksp ? c_end : ksp;
    fs = 0;
    nfs = 0;
    if (c0 < sp_end) {
      fs = c0 / R;
      nfs = (int)((sp_end - 1) / R - fs + 1);
    }
    b0 = c0 > ksp ? c0 : ksp;
    nbase = (base && b0 < c_end) ? (int)(c_end - b0) : 0;
  }
};

// LDS floats one wave's side buffer needs for a block: the knot rows of its
// spline features, then x for nb MFMA tile rows (32 samples each) of items.
__host__ __device__ inline int64_t dx_side_floats(const DxBlock& b, int nk, int nb) {
  return (((int64_t)b.nfs * nk + 3) & ~(int64_t)3) + (int64_t)32 * nb * (b.nfs + b.nbase);
}

// v / p for 0 <= v < 2^13 and 1 <= p <= 2^8, with rcp = 1.0f / p: the
// fraction of (v + 0.5) / p stays at least 0.5 / p from an integer, far above
// the float product's error, so the truncation is exact.
__device__ __forceinline__ int div_small(int v, float rcp) {
  return (int)(((float)v + 0.5f) * rcp);
}

template <class C, int K>
__device__ __forceinline__ void dx_epilogue(const GemmParams<float>& p, const DxParams& e,
                                            const TileCoords& tc,
                                            const f32x16 (&acc)[C::FM][C::FN], float* lds_stage,
                                            float* lds_side, int side_floats, int wave, int wm,
                                            int wn, int lane) {
  typedef Mfma<float, 32> M;
  constexpr int TN = C::TN, SW = C::TN + 1;  // staged row stride (odd: conflict-free columns)
  float* stage = lds_stage + wave * 32 * SW;
  const DxBlock blk(tc.n0 + (int64_t)wn * TN, p.N, e.ksp, e.R, TN, e.nslot == 3);
  const int per_row = blk.nfs + blk.nbase;
  if (per_row == 0) return;  // block lies past the last column
  // side buffer: knots of features fs.., then x[row, item] for nb tile rows
  float* kn = lds_side + wave * side_floats;
  const int nkn = blk.nfs * e.nk;
  float* xs = kn + ((nkn + 3) & ~3);
  static_assert(C::FM == 1 || C::FM == 2 || C::FM == 4, "tile rows per wave: 1, 2 or 4");
  int nb = C::FM;
  while (nb > 1 && dx_side_floats(blk, e.nk, nb) > side_floats) nb >>= 1;
  const float* gsrc = e.grid + blk.fs * e.nk;  // the block's knot rows are contiguous
  for (int b = lane; b < nkn; b += 64 * 4) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int idx = b + u * 64;
      v[u] = gsrc[idx < nkn ? idx : 0];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (b + u * 64 < nkn) kn[b + u * 64] = v[u];
  }
  const int64_t fbase = blk.b0 - e.ksp - blk.nfs;  // feature of base item idx: fbase + idx
  const int total = 32 * nb * per_row;  // x values per batch of nb tile rows
  const float rcp = 1.0f / (float)per_row;
  // tile rows are unrolled so the accumulator indices stay compile-time
#pragma unroll
  for (int iq = 0; iq < C::FM; ++iq) {
    const int q0 = iq & ~(nb - 1);
    const int64_t rbase = tc.m0 + (int64_t)wm * C::TM + q0 * 32;
    if (iq == q0) {
      // x for tile rows q0 .. q0+nb-1, sample-major: xs[rq * per_row + idx]
      // (consecutive lanes read consecutive features of one sample)
      for (int b = lane; b < total; b += 64 * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int el = b + u * 64;
          const int rq = div_small(el, rcp), idx = el - rq * per_row;
          const int64_t f = idx < blk.nfs ? blk.fs + idx : fbase + idx;
          const int64_t n = rbase + rq;
          const bool ok = el < total && n < p.M;
          v[u] = e.x[ok ? n * e.I + f : 0];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (b + u * 64 < total) xs[b + u * 64] = v[u];
      }
    }
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int v = 0; v < M::kNAcc; ++v)
        stage[M::out_row(lane, v) * SW + j * 32 + M::out_col(lane)] = acc[iq][j][v];
    wave_sync_lds();
    const float* xq = xs + (iq - q0) * 32 * per_row;
    // items (sample row, idx) of this tile row, idx fastest across lanes
    for (int it = lane; it < 32 * per_row; it += 64) {
      const int row = div_small(it, rcp), idx = it - row * per_row;
      const int64_t n = rbase + (iq - q0) * 32 + row;
      const float* srow = stage + row * SW;
      const float xv = xq[it];
      if (idx < blk.nfs) {
        const int64_t f = blk.fs + idx;
        const float* t = kn + idx * e.nk;
        const int64_t fc = f * e.R;
        float sum = 0.0f;
        const int m = knot_span(t, e.nk, xv);
        if (m >= 0) {
          float d[K + 1];
          span_derivs<K, float>(t, e.nk, m, xv, d);
#pragma unroll
          for (int jj = 0; jj <= K; ++jj) {
            const int r = m - K + jj;
            const int64_t col = fc + r;
            if (r >= 0 && r < e.R && col >= blk.c0 && col < blk.sp_end)
              sum += srow[col - blk.c0] * d[jj];
          }
        }
        if (n < p.M) {
          float* dst = e.part + (n * e.I + f) * e.nslot;
          if (fc >= blk.c0) {
            dst[0] = sum;
            if (fc + e.R <= blk.c0 + TN) dst[1] = 0.0f;
          } else {
            dst[1] = sum;
          }
        }
      } else {
        const int64_t col = blk.b0 + (idx - blk.nfs);
        const float g = srow[col - blk.c0] * silu_grad_of<float>(xv);
        if (n < p.M) e.part[(n * e.I + (col - e.ksp)) * e.nslot + 2] = g;
      }
    }
    wave_sync_lds();
  }
}

// Compact input-side product: of E's spline columns only the K+1 that the
// input gradient uses, those of the span window of x[n, i], are stored, as
// Ew[n, i, 0..K] (window slot jj = column m - K + jj of feature i, the
// columns inside 0..R-1 only), and the base columns as Es[n, i].  Base
// columns go from the accumulators straight to Es.  For the spline columns
// a wave block stages the knot rows of its features and x of its items
// (all its tile rows at once when the side buffer holds them), finds every
// item's span (four interleaved searches per lane) and keeps it in x's
// place; then per tile row it stages the accumulators in LDS and each item
// copies the window columns that lie in the block (a window that crosses a
// block boundary is completed by the neighbouring block; every slot is
// written by exactly one block).
template <class C, int K>
__device__ __forceinline__ void ecomp_epilogue(const GemmParams<float>& p, const DxParams& e,
                                               const TileCoords& tc,
                                               const f32x16 (&acc)[C::FM][C::FN],
                                               float* lds_stage, float* lds_side, int side_floats,
                                               int wave, int wm, int wn, int lane) {
  typedef Mfma<float, 32> M;
  constexpr int TN = C::TN, SW = C::TN + 1;  // staged row stride (odd: conflict-free columns)
  float* stage = lds_stage + wave * 32 * SW;
  const DxBlock blk(tc.n0 + (int64_t)wn * TN, p.N, e.ksp, e.R, TN, e.es != nullptr);
  if (blk.nbase > 0) {  // base columns of the block: accumulators -> Es
#pragma unroll
    for (int iq = 0; iq < C::FM; ++iq)
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        const int64_t col = blk.c0 + j * 32 + M::out_col(lane);
        if (col < e.ksp || col >= e.ksp + e.I) continue;
#pragma unroll
        for (int v = 0; v < M::kNAcc; ++v) {
          const int64_t row = tc.m0 + (int64_t)wm * C::TM + iq * 32 + M::out_row(lane, v);
          if (row < p.M) e.es[row * e.I + (col - e.ksp)] = acc[iq][j][v];
        }
      }
  }
  const int nfs = blk.nfs;
  if (nfs == 0) return;
  float* kn = lds_side + wave * side_floats;
  const int nkn = nfs * e.nk;
  float* xs = kn + ((nkn + 3) & ~3);
  static_assert(C::FM == 1 || C::FM == 2 || C::FM == 4, "tile rows per wave: 1, 2 or 4");
  int nb = C::FM;
  while (nb > 1 && (((int64_t)nkn + 3) & ~(int64_t)3) + (int64_t)32 * nb * nfs > side_floats)
    nb >>= 1;
  const float* gsrc = e.grid + blk.fs * e.nk;
  const float rcp = 1.0f / (float)nfs;
#pragma unroll
  for (int iq = 0; iq < C::FM; ++iq) {
    const int q0 = iq & ~(nb - 1);
    const int64_t rbase = tc.m0 + (int64_t)wm * C::TM + q0 * 32;
    const int total = 32 * nb * nfs;  // spline items of tile rows q0 .. q0 + nb - 1
    if (iq == q0) {
      // knot rows (first batch only; nfs * nk <= 256) and x, sample-major
      // xs[rq * nfs + idx], loaded together
      float kv[4];
      if (iq == 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) kv[u] = lane + 64 * u < nkn ? gsrc[lane + 64 * u] : 0.0f;
      }
      for (int b = lane; b < total; b += 64 * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int el = b + u * 64;
          const int rq = div_small(el, rcp), idx = el - rq * nfs;
          const int64_t n = rbase + rq;
          v[u] = (el < total && n < p.M) ? e.x[n * e.I + blk.fs + idx] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (b + u * 64 < total) xs[b + u * 64] = v[u];
      }
      if (iq == 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (lane + 64 * u < nkn) kn[lane + 64 * u] = kv[u];
      }
      wave_sync_lds();
      // spans through knot_spans (kan_spline.h), the routine
      // basis_grad_compact_kernel uses to read the window slots back; four
      // interleaved searches per lane, stored over x
      for (int b = lane; b < total; b += 64 * 4) {
        float xv[4];
        const float* tk[4];
        int ms[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int el = b + u * 64 < total ? b + u * 64 : total - 1;
          const int rq = div_small(el, rcp);
          xv[u] = xs[el];
          tk[u] = kn + (el - rq * nfs) * e.nk;
        }
        knot_spans<4, float>(tk, e.nk, xv, ms);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int m = ms[u];
          if (b + u * 64 < total) xs[b + u * 64] = __int_as_float(m);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int v = 0; v < M::kNAcc; ++v)
        stage[M::out_row(lane, v) * SW + j * 32 + M::out_col(lane)] = acc[iq][j][v];
    wave_sync_lds();
    const float* sq = xs + (iq - q0) * 32 * nfs;
    for (int it = lane; it < 32 * nfs; it += 64) {
      const int row = div_small(it, rcp), idx = it - row * nfs;
      const int64_t n = rbase + (iq - q0) * 32 + row;
      const int m = __float_as_int(sq[it]);
      if (n >= p.M || m < 0) continue;  // (no spline term: the window is not read)
      const float* srow = stage + row * SW;
      const int64_t f = blk.fs + idx;
      const int64_t c_lo = f * e.R + m - K;  // column of window slot 0
      float* dst = e.part + (n * e.I + f) * (K + 1);
#pragma unroll
      for (int jj = 0; jj <= K; ++jj) {
        const int r = m - K + jj;
        const int64_t col = c_lo + jj;
        if (r >= 0 && r < e.R && col >= blk.c0 && col < blk.sp_end) dst[jj] = srow[col - blk.c0];
      }
    }
    wave_sync_lds();
  }
}

template <class C, bool AK, bool BKC, int EPIK>
__global__ __launch_bounds__(C::kThreads, C::MINB) void gemm_pipe_kernel(
    GemmParams<typename C::T> p, DxParams e) {
  typedef typename C::T T;
  typedef Mfma<T, C::MF> M;
  // fp32 loads whole slabs through buffer resources; fp64 (a four-element
  // chunk is 32 bytes) through plain 16-byte loads
  constexpr bool kF32 = std::is_same<T, float>::value;
  constexpr int BM = C::BM, BN = C::BN, BK = C::BK, NT = C::kThreads;
  constexpr int FM = C::FM, FN = C::FN, NG = BK / M::kKG;
  static_assert(NG % 2 == 0, "slab must hold an even number of k-groups");
  typedef Slab<BM, BK, AK> SA;
  typedef Slab<BN, BK, BKC> SB;
  typedef SlabLoader<T, BM, BK, AK, NT> LA;
  typedef SlabLoader<T, BN, BK, BKC, NT> LB;
  // memory instructions (16 bytes each) per slab (stores, loads) and per
  // k-group (fragment reads); a chunk of four elements is kW of them
  constexpr int kW = (int)sizeof(T) / 4;
  constexpr int kDSW = (LA::kPer + LB::kPer) * kW;
  constexpr int kGLD = (LA::kPer + LB::kPer) * kW;
  // MN-contiguous operands take their fragments interleaved (read_frag_il):
  // F contiguous elements per k step for all of the wave's F tiles
  constexpr bool AIL = !AK, BIL = !BKC;
  constexpr int kRdA = AK ? FM * kW : 4 * ((FM * (int)sizeof(T) + 15) / 16);
  constexpr int kRdB = BKC ? FN * kW : 4 * ((FN * (int)sizeof(T) + 15) / 16);
  constexpr int kDSR = kRdA + kRdB;
  constexpr int kMF = 4 * FM * FN;  // MFMAs per k-group
  __shared__ __align__(16) T lds_a[2][SA::kElems];
  __shared__ __align__(16) T lds_b[2][SB::kElems];

  const TileCoords tc = tile_coords<C>(p);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int rl = M::row(lane), q = M::kq(lane);

  typename M::acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < M::kNAcc; ++v) acc[i][j][v] = T(0);

  LA la;
  LB lb;
  T fa[2][FM][4], fb[2][FN][4];
  auto fread = [&](const T* a_lds, const T* b_lds, int g, int slot) {
    if constexpr (AIL) {
      read_frag_il<T, BM, BK, FM>(a_lds, wm * C::TM + FM * rl, M::kofs(g, q), fa[slot]);
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        read_frag<T, BM, BK, AK>(a_lds, wm * C::TM + i * C::MF + rl, M::kofs(g, q), fa[slot][i]);
    }
    if constexpr (BIL) {
      read_frag_il<T, BN, BK, FN>(b_lds, wn * C::TN + FN * rl, M::kofs(g, q), fb[slot]);
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        read_frag<T, BN, BK, BKC>(b_lds, wn * C::TN + j * C::MF + rl, M::kofs(g, q), fb[slot][j]);
    }
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = M::mma(fa[slot][i][s], fb[slot][j][s], acc[i][j]);
  };
  // full_c: 1 = whole slabs through buffer resources, 0 = edge slabs
  // (guarded; also whole slabs whose offsets do not fit a buffer resource)
  auto gload = [&](int slab, auto full_c) {
    const int64_t k0 = tc.kbeg + (int64_t)slab * BK;
    if constexpr (decltype(full_c)::value == 1 && kF32) {
      la.load_buf(p.A, p.lda, tc.m0, k0);
      lb.load_buf(p.B, p.ldb, tc.n0, k0);
    } else if constexpr (decltype(full_c)::value == 1) {
      la.load_full(p.A, p.lda, tc.m0, k0);
      lb.load_full(p.B, p.ldb, tc.n0, k0);
    } else {
      la.load_guarded(p.A, p.lda, tc.m0, p.M, k0, tc.kend);
      lb.load_guarded(p.B, p.ldb, tc.n0, p.N, k0, tc.kend);
    }
  };
  // One slab.  STORE: registers of slab kt+1 -> the other LDS buffer;
  // LOAD: global loads of slab kt+2; NEXT: barrier + first fragments of kt+1.
  // par_c = kt & 1 as a constant (static LDS addresses) in the main loop;
  // IC<-1> takes it at run time (the last two slabs).
  auto slab = [&](int kt, auto store_c, auto load_c, auto next_c, auto full_c, auto par_c) {
    constexpr bool STORE = decltype(store_c)::value != 0;
    constexpr bool LOAD = decltype(load_c)::value != 0;
    constexpr bool NEXT = decltype(next_c)::value != 0;
    constexpr int kPar = decltype(par_c)::value;
    const int cur = kPar >= 0 ? kPar : (kt & 1);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      // The next group's fragment reads come first in program order: the
      // compiler cannot tell the two slab buffers apart (runtime index), so
      // reads placed after the stores of group 0 would wait for all of them.
      if (g + 1 < NG) {
        fread(lds_a[cur], lds_b[cur], g + 1, (g + 1) & 1);
      } else if (NEXT) {
        __syncthreads();
        fread(lds_a[cur ^ 1], lds_b[cur ^ 1], 0, 0);
      }
      if (g == 0) {
        if (STORE) {
          la.store(lds_a[cur ^ 1]);
          lb.store(lds_b[cur ^ 1]);
        }
        if (LOAD) gload(kt + 2, full_c);
      }
      mfmas(g & 1);
      if (g == 0 && STORE && LOAD) SchedSeq<0, kMF, kDSR, kDSW, kGLD>::run();
      else if (g == 0 && STORE) SchedSeq<0, kMF, kDSR, kDSW, 0>::run();
      else if (g + 1 < NG || NEXT) SchedSeq<0, kMF, kDSR, 0, 0>::run();
    }
  };
  auto run = [&](auto full_c) {
    if constexpr (decltype(full_c)::value == 1 && kF32) {
      la.init_buf(p.lda);
      lb.init_buf(p.ldb);
    }
    gload(0, full_c);
    la.store(lds_a[0]);
    lb.store(lds_b[0]);
    if (tc.nkt > 1) gload(1, full_c);
    __syncthreads();
    fread(lds_a[0], lds_b[0], 0, 0);
    int kt = 0;
    for (; kt + 2 < tc.nkt; ++kt) slab(kt, IC<1>(), IC<1>(), IC<1>(), full_c, IC<-1>());
    if (kt + 1 < tc.nkt) {
      slab(kt, IC<1>(), IC<0>(), IC<1>(), full_c, IC<-1>());
      ++kt;
    }
    slab(kt, IC<0>(), IC<0>(), IC<0>(), full_c, IC<-1>());
  };
  if (tc.nkt > 0) {
    const bool full = p.vec && (p.buf || !kF32) && (tc.m0 + BM <= p.M) && (tc.n0 + BN <= p.N) &&
                      ((tc.kend - tc.kbeg) % BK == 0);
    if (full) run(IC<1>());
    else run(IC<0>());
  }
  if constexpr (EPIK == 0) {
    (void)e;
    store_tile<C, typename M::acc_t, AIL, BIL>(p, tc, acc, wm, wn, lane);
  } else {
    static_assert(kF32, "the epilogues are fp32");
    static_assert(!AIL && !BIL, "the epilogues read the accumulators in tile order");
    static_assert(C::WM * C::WN * 32 * (C::TN + 1) <= 2 * SA::kElems,
                  "dx staging must fit in the A slab buffers");
    constexpr int kSide = 2 * SB::kElems / (C::WM * C::WN);
    static_assert(kSide + 512 <= 8192, "div_small covers the side buffer's indices");
    __syncthreads();  // every wave is done with the slab buffers
    if constexpr (EPIK > 0)
      dx_epilogue<C, EPIK>(p, e, tc, acc, &lds_a[0][0], &lds_b[0][0], kSide, wave, wm, wn, lane);
    else
      ecomp_epilogue<C, -EPIK>(p, e, tc, acc, &lds_a[0][0], &lds_b[0][0], kSide, wave, wm, wn,
                               lane);
  }
}

// dx[n, i] = (part[n, i, 0] + part[n, i, 1]) (+ part[n, i, 2])
__global__ void dx_finalize_kernel(const float* __restrict__ part, float* __restrict__ gx,
                                   int64_t count, int nslot) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    const float* q = part + e * nslot;
    float v = q[0] + q[1];
    if (nslot == 3) v += q[2];
    gx[e] = v;
  }
}

template <typename T>
bool vec_ok(const T* ptr, int64_t ld) {
  return ((reinterpret_cast<uintptr_t>(ptr) % (4 * sizeof(T))) == 0) && (ld % 4 == 0);
}

// ---- planning ----------------------------------------------------------------

// Cost model of the fp32 tile configurations, fitted to a sweep of every
// configuration and split count over the products of BASELINE's workloads
// (c2's first layer, c3's and c5's parameter products, c4's and c5's
// forward products) on MI355X.  The dispatcher spreads workgroups over CUs,
// so the busiest CU runs ceil(tiles / CUs) blocks one after another (two
// small blocks that share a CU run at half speed each, the same total);
// a block costs its MFMA work at the configuration's sustained efficiency
// plus a fixed start-up and write-out time.  The 128 x 128 tile loses most
// of its efficiency when it runs alone on a CU (one wave per SIMD: the slab
// barriers idle the MFMA pipes), which is why the earlier whole-wave model
// (eff 0.85 at two blocks per CU, a 256-k overhead) split c2's and c5's
// products onto small tiles that ran 10-30 % slower than the 256 x 256 tile
// with more splits, and c3's parameter product 4 ways instead of 8.
struct CfgModel {
  int bm, bn, bk;
  double eff;       // sustained fraction of the per-CU peak, blocks sharing CUs
  double eff_lone;  // the same when every block has a CU of its own
  double block_s;   // fixed seconds per block (start-up, epilogue)
};
constexpr CfgModel kModelF32[4] = {
    {256, 256, 32, 0.89, 0.89, 5e-6}, {128, 128, 32, 0.88, 0.40, 10e-6},
    {256, 64, 32, 0.75, 0.75, 5e-6}, {256, 256, 32, 0.89, 0.89, 5e-6}};
constexpr double kPeakPerCuF32 = 157.3e12 / 256.0;  // FP32 MFMA flop/s per CU
constexpr double kStreamBytesPerS = 5.0e12;          // split-K partial-sum traffic

// fp64: whole waves of resident blocks times one block's k range plus its
// configuration's start-up and write-out term.
struct CfgModelF64 {
  int bm, bn, bk, blocks_per_cu;
  double eff;
  double k_overhead;  // a block's start-up and write-out, in k of its own MFMA work
};
// (measured at c3's shapes: 0.81-0.83 of the FP64 peak for the 8-wave tile,
// 0.75-0.82 for the 4-wave one, whose parameter product lost most)
// (the pipelined 128 x 128 x 32 measured 0.91-0.95 of the FP64 peak at c3's
// three product shapes, where the other two measured 0.80-0.82; the
// pipelined 64 x 64 x 32 measured 0.65-0.68 on the products of a 64-wide
// layer, 16384 samples by 512 features, where the 128 x 128 tile, half of it
// past the 64 outputs, measured 0.31-0.33.  The pipelined tiles' start-up
// and write-out terms come from that layer's input-side product, K = 64:
// 16 us per 128 x 128 block against 7 us of MFMA work, 7 us per pair of
// 64 x 64 blocks against 4.5 us.)
constexpr CfgModelF64 kModelF64[4] = {
    {256, 128, 16, 1, 0.84, 256.0}, {128, 128, 16, 1, 0.80, 256.0},
    {128, 128, 32, 1, 0.93, 96.0}, {64, 64, 32, 2, 0.75, 48.0}};
constexpr double kPeakPerCuF64 = 78.6e12 / 256.0;

double split_traffic_s(int64_t M, int64_t N, int splits, size_t elem) {
  return splits > 1 ? 2.0 * (double)splits * (double)(M * N) * (double)elem / kStreamBytesPerS
                    : 0.0;
}

// Estimated seconds for M x N x K with `splits` K-slices on fp32 tiles of c,
// plus the split-K partial traffic (written once, read once by the sum).
double est_seconds(const CfgModel& c, int64_t M, int64_t N, int64_t K, int splits,
                   int64_t cus) {
  const int64_t tiles = ceil_div(M, c.bm) * ceil_div(N, c.bn) * splits;
  const int64_t per_cu = ceil_div(tiles, cus);
  const int64_t kper = round_up(ceil_div(K > 0 ? K : 1, splits), c.bk);
  const double eff = tiles <= cus ? c.eff_lone : c.eff;
  const double block = 2.0 * c.bm * c.bn * (double)kper / (kPeakPerCuF32 * eff) + c.block_s;
  return (double)per_cu * block + split_traffic_s(M, N, splits, 4);
}

double est_seconds_f64(const CfgModelF64& c, int64_t M, int64_t N, int64_t K, int splits,
                       int64_t cus) {
  const int64_t tiles = ceil_div(M, c.bm) * ceil_div(N, c.bn) * splits;
  const int64_t waves = ceil_div(tiles, cus * c.blocks_per_cu);
  const int64_t kper = round_up(ceil_div(K > 0 ? K : 1, splits), c.bk);
  const double block_s = 2.0 * c.bm * c.bn * ((double)kper + c.k_overhead) * c.blocks_per_cu /
                         (kPeakPerCuF64 * c.eff);
  return (double)waves * block_s + split_traffic_s(M, N, splits, 8);
}

// Forced fp32 tile configuration (route KAN_ROUTE_GEMM_TILE: 0 big, 1 small,
// 2 narrow, 3 the 4-wave 256x256), or -1 to leave the choice to the cost
// model.
int forced_cfg_f32() { return kan_hip_get_route(KAN_ROUTE_GEMM_TILE); }

// fp64 configuration (0 = 256 x 128 with 8 waves, 1 = 128 x 128 with 4,
// 2 = the pipelined 128 x 128 x 32, 3 = the pipelined 64 x 64 x 32) for a
// split count; the route forces 0 for "256", 1 for "128", 2 for "256x64"
// and 3 for "256w4" (the fp32 tiles' values).
int pick_cfg_f64(int64_t M, int64_t N, int64_t K, int splits, int64_t cus = 0) {
  const int forced = kan_hip_get_route(KAN_ROUTE_GEMM_TILE);
  if (forced >= 0 && forced <= 3) return forced;
  // The cost model chooses between the two pipelined tiles: the older ones
  // (0, 1) measured slower than one of them at every shape timed (c3's
  // products, a 64-wide layer's, PINN's), and are reached only by the route.
  if (cus <= 0) cus = device_cu_count();
  int best = 2;
  double best_t = est_seconds_f64(kModelF64[2], M, N, K, splits, cus);
  for (int c = 3; c <= 3; ++c) {
    const double t = est_seconds_f64(kModelF64[c], M, N, K, splits, cus);
    if (t < best_t) {
      best = c;
      best_t = t;
    }
  }
  return best;
}

// fp32 configuration (0 = big, 1 = small, 2 = narrow, 3 = 4-wave big, only
// when forced) for a given split count; the narrow one only where N fits its
// 64 columns.
int pick_cfg_f32(int64_t M, int64_t N, int64_t K, int splits, int64_t cus = 0) {
  const int forced = forced_cfg_f32();
  if (forced >= 0) return forced;
  if (cus <= 0) cus = device_cu_count();
  const int last = N <= 64 ? 2 : 1;
  int best = 0;
  double best_t = est_seconds(kModelF32[0], M, N, K, splits, cus);
  for (int c = 1; c <= last; ++c) {
    const double t = est_seconds(kModelF32[c], M, N, K, splits, cus);
    if (t < best_t) {
      best = c;
      best_t = t;
    }
  }
  return best;
}

template <class C, bool AK, bool BKC, int EPIK = 0>
int launch_cfg(GemmParams<typename C::T> p, int splits, hipStream_t st, const DxParams* dx = nullptr) {
  if (splits < 1) splits = 1;
  p.k_per_split = round_up(ceil_div(p.K > 0 ? p.K : 1, splits), C::BK);
  const int64_t tm = ceil_div(p.M, C::BM), tn = ceil_div(p.N, C::BN);
  const int64_t blocks = tm * tn * splits;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "gemm: problem too large (%lld tiles)", (long long)blocks);
  p.tiles_m = (int)tm;
  p.tiles_n = (int)tn;
  p.splits = splits;
  // whole-slab byte offsets (rows or k spanned by a slab times ld) in 31 bits
  auto span_ok = [](bool kcont, int rows, int64_t ld) {
    const int64_t span = kcont ? (int64_t)rows * ld + C::BK : (int64_t)C::BK * ld + rows;
    return span * (int64_t)sizeof(typename C::T) < (int64_t)1 << 31;
  };
  p.buf = span_ok(AK, C::BM, p.lda) && span_ok(BKC, C::BN, p.ldb);
  if constexpr (RunsPipe<C>::value) {
    DxParams e{};
    if (dx != nullptr) e = *dx;
    hipLaunchKernelGGL((gemm_pipe_kernel<C, AK, BKC, EPIK>), dim3((unsigned)blocks),
                       dim3(C::kThreads), 0, st, p, e);
  } else {
    (void)dx;
    hipLaunchKernelGGL((gemm_kernel<C, AK, BKC>), dim3((unsigned)blocks), dim3(C::kThreads), 0,
                       st, p);
  }
  return KAN_OK;
}

template <class C>
int launch_layout(int layout, const GemmParams<typename C::T>& p, int splits, hipStream_t st) {
  switch (layout) {
    case kLayoutNT: return launch_cfg<C, true, true>(p, splits, st);
    case kLayoutTN: return launch_cfg<C, false, false>(p, splits, st);
    case kLayoutNN: return launch_cfg<C, true, false>(p, splits, st);
    case kLayoutTT: return launch_cfg<C, false, true>(p, splits, st);
    default: return set_error(KAN_ERR_INVALID, "gemm: unknown layout %d", layout);
  }
}

// Every wave block's side buffer (knots + x of one tile row) fits in its
// share of the B slab buffers; exact, by walking the blocks of the row.
template <class C>
bool dx_cfg_fits(int64_t N, int64_t I, int R, int nk, bool has_base) {
  typedef Slab<C::BN, C::BK, true> SB;
  constexpr int64_t kSide = 2 * SB::kElems / (C::WM * C::WN);
  if (R > C::TN) return false;  // a feature's columns meet at most two blocks
  const int64_t ksp = I * R;
  for (int64_t c0 = 0; c0 < N; c0 += C::TN)
    if (dx_side_floats(DxBlock(c0, N, ksp, R, C::TN, has_base), nk, 1) > kSide) return false;
  return true;
}

template <class C>
int launch_dx_cfg(const GemmParams<float>& p, const DxParams& e, int k, hipStream_t st) {
  if (k == 1) return launch_cfg<C, true, true, 1>(p, 1, st, &e);
  if (k == 2) return launch_cfg<C, true, true, 2>(p, 1, st, &e);
  return launch_cfg<C, true, true, 3>(p, 1, st, &e);
}

// Every wave block's side buffer fits (the compact route has no bound on R:
// a window crossing blocks is completed by each of them).
template <class C>
bool ecomp_cfg_fits(int64_t N, int64_t I, int R, int nk, bool has_base) {
  typedef Slab<C::BN, C::BK, true> SB;
  constexpr int64_t kSide = 2 * SB::kElems / (C::WM * C::WN);
  const int64_t ksp = I * R;
  for (int64_t c0 = 0; c0 < N; c0 += C::TN) {
    const DxBlock b(c0, N, ksp, R, C::TN, has_base);
    if (b.nfs * nk > 256 ||
        (((int64_t)b.nfs * nk + 3) & ~(int64_t)3) + 32 * (int64_t)b.nfs > kSide)
      return false;
  }
  return true;
}

template <class C>
int launch_ecomp_cfg(const GemmParams<float>& p, const DxParams& e, int k, hipStream_t st) {
  if (k == 1) return launch_cfg<C, true, true, -1>(p, 1, st, &e);
  if (k == 2) return launch_cfg<C, true, true, -2>(p, 1, st, &e);
  return launch_cfg<C, true, true, -3>(p, 1, st, &e);
}


// ---------------------------------------------------------------------------
// Thin products: an output side of at most kThinMax (a classifier's or a
// PINN's output layer, and that layer's parameter product) or a contraction
// of at most kThinMax (the input-side product of such a layer).  MFMA tiles
// would be mostly padding there, and the product is bound by the traffic of
// its wide operand (with a short K, of C).  These kernels stream that operand
// with 16-byte loads and accumulate with FMAs in a fixed order (k ascending
// within a lane, then fixed partial-sum orders), so results are
// deterministic.  Element (m, n) of a layout is addressed through strides:
// A(m, k) = A[m * as_m + k * as_k], B(k, n) = B[k * bs_k + n * bs_n].
constexpr int kThinMax = 16;
constexpr int kThinThreads = 256;
constexpr int kThinChunk = 256;  // k rows (or k columns) of the thin operand staged at a time
constexpr int kThinUnroll = 8;   // wide-operand loads in flight per lane
constexpr int kThinRowChunk = 64;  // rows of A staged per wave (short contraction)

template <typename T>
struct ThinVec {
  static constexpr int kW = 16 / sizeof(T);  // elements per 16-byte vector
  typedef T type __attribute__((ext_vector_type(16 / sizeof(T))));
};

struct ThinStrides {
  int64_t as_m, as_k, bs_k, bs_n;
};
inline ThinStrides thin_strides(int layout, int64_t lda, int64_t ldb) {
  ThinStrides t;
  const bool ta = layout == kLayoutTN || layout == kLayoutTT;
  const bool tb = layout == kLayoutNT || layout == kLayoutTT;
  t.as_m = ta ? 1 : lda;
  t.as_k = ta ? lda : 1;
  t.bs_k = tb ? 1 : ldb;
  t.bs_n = tb ? ldb : 1;
  return t;
}

// LDS of the wide-rows kernel: the staged thin rows, then the partial sums of
// waves 1..3 (48 KB either way at P = 16)
template <typename T, int P>
struct ThinRowsLds {
  static constexpr int kW = ThinVec<T>::kW;
  static constexpr int kStage = kThinChunk * P;
  static constexpr int kRed = 3 * 64 * kW * P;
  static constexpr int kElems = kStage > kRed ? kStage : kRed;
};

// out(p, q) = sum_k X[k * ldx + q] * Y[k * ys_k + p * ys_p] over split s's k
// range, for p < np (<= P) and q < nq, written to C[s * sstride + p * cp +
// q * cq].  The wide operand X is contiguous along q.  A block's 4 waves take
// the same 64 * W wide indices (W per lane); the split's k range goes in
// chunks of kThinChunk rows whose thin values the block stages in LDS, and
// wave w takes the w-th quarter of each chunk.  The waves' sums are added in
// wave order through LDS.
template <typename T, int P, bool VEC>
__global__ __launch_bounds__(kThinThreads) void thin_wide_rows_kernel(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ys_k, int64_t ys_p,
    T* __restrict__ C, int64_t cp, int64_t cq, int64_t sstride, int np, int64_t nq, int64_t K,
    int64_t kper) {
  typedef ThinVec<T> TV;
  typedef ThinRowsLds<T, P> L;
  constexpr int W = TV::kW;
  __shared__ __align__(16) T lds[L::kElems];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t q0 = (int64_t)blockIdx.x * (64 * W) + lane * W;
  const int split = blockIdx.y;
  const int64_t kb = (int64_t)split * kper, ke = min(K, kb + kper);
  const bool whole_block = VEC && ((int64_t)blockIdx.x + 1) * (64 * W) <= nq;
  T acc[W][P];
#pragma unroll
  for (int j = 0; j < W; ++j)
#pragma unroll
    for (int pp = 0; pp < P; ++pp) acc[j][pp] = T(0);
  auto rows = [&](int64_t c0, int r0, int r1, auto whole_c) {
    constexpr bool kWhole = decltype(whole_c)::value;
    auto load_row = [&](int r, T (&x)[W]) {
      const T* src = X + (c0 + r) * ldx + q0;
      if constexpr (kWhole) {
        const typename TV::type v = *reinterpret_cast<const typename TV::type*>(src);
#pragma unroll
        for (int j = 0; j < W; ++j) x[j] = v[j];
      } else {
#pragma unroll
        for (int j = 0; j < W; ++j) x[j] = q0 + j < nq ? src[j] : T(0);
      }
    };
    auto fma_row = [&](int r, const T (&x)[W]) {
      const T* yr = lds + r * P;  // (the same address in every lane: a broadcast)
#pragma unroll
      for (int pp = 0; pp < P; ++pp) {
        const T y = yr[pp];
#pragma unroll
        for (int j = 0; j < W; ++j) acc[j][pp] += x[j] * y;
      }
    };
    const int rfull = r0 + (r1 - r0) / kThinUnroll * kThinUnroll;
    for (int r = r0; r < rfull; r += kThinUnroll) {
      T x[kThinUnroll][W];
#pragma unroll
      for (int u = 0; u < kThinUnroll; ++u) load_row(r + u, x[u]);
      // (row by row: the thin values of one row at a time in registers)
#pragma unroll
      for (int u = 0; u < kThinUnroll; ++u) {
        __builtin_amdgcn_sched_barrier(0);
        fma_row(r + u, x[u]);
      }
    }
    for (int r = rfull; r < r1; ++r) {
      T x[W];
      load_row(r, x);
      fma_row(r, x);
    }
  };
  for (int64_t c0 = kb; c0 < ke; c0 += kThinChunk) {
    const int nr = (int)min((int64_t)kThinChunk, ke - c0);
    __syncthreads();  // (the previous chunk's reads of the stage are done)
    for (int e = threadIdx.x; e < nr * P; e += kThinThreads) {
      const int r = e / P, pp = e - r * P;
      lds[e] = pp < np ? Y[(c0 + r) * ys_k + pp * ys_p] : T(0);
    }
    __syncthreads();
    const int quarter = (nr + 3) / 4;
    const int r0 = min(nr, wave * quarter), r1 = min(nr, r0 + quarter);
    if (whole_block) rows(c0, r0, r1, std::integral_constant<bool, VEC>());
    else rows(c0, r0, r1, std::false_type());
  }
  __syncthreads();  // (the stage is reused for the partial sums)
  if (wave > 0) {
    T* dst = lds + (wave - 1) * (64 * W * P) + lane;
#pragma unroll
    for (int j = 0; j < W; ++j)
#pragma unroll
      for (int pp = 0; pp < P; ++pp) dst[(j * P + pp) * 64] = acc[j][pp];
  }
  __syncthreads();
  if (wave != 0) return;
  // (one row of P values at a time: the loads need few registers)
#pragma unroll 1
  for (int w = 0; w < 3; ++w) {
    const T* src = lds + w * (64 * W * P) + lane;
#pragma unroll
    for (int j = 0; j < W; ++j) {
      T v[P];
#pragma unroll
      for (int pp = 0; pp < P; ++pp) v[pp] = src[(j * P + pp) * 64];
#pragma unroll
      for (int pp = 0; pp < P; ++pp) acc[j][pp] += v[pp];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  T* out = C + (int64_t)split * sstride;
#pragma unroll
  for (int j = 0; j < W; ++j) {
    if (q0 + j >= nq) continue;
#pragma unroll
    for (int pp = 0; pp < P; ++pp)
      if (pp < np) out[pp * cp + (q0 + j) * cq] = acc[j][pp];
  }
}

// out(p, q) = sum_k X[q * ldx + k] * Y[p * ys_p + k * ys_k] over split s's k
// range: the wide operand X is contiguous along k.  A block takes 16 wide
// indices (4 per wave, 16 lanes each) of one split; per chunk of kThinChunk
// columns it stages the thin rows Y(0..P-1, chunk) in LDS, and each lane
// covers W consecutive k per stripe of 16 lanes.  The 16 lanes' sums are added
// by a fixed butterfly.
template <typename T, int P, bool VEC>
__global__ __launch_bounds__(kThinThreads) void thin_wide_cols_kernel(
    const T* __restrict__ X, int64_t ldx, const T* __restrict__ Y, int64_t ys_k, int64_t ys_p,
    T* __restrict__ C, int64_t cp, int64_t cq, int64_t sstride, int np, int64_t nq, int64_t K,
    int64_t kper) {
  typedef ThinVec<T> TV;
  constexpr int W = TV::kW;
  constexpr int kStripes = kThinChunk / (16 * W);  // per lane and chunk
  __shared__ __align__(16) T ys[P * kThinChunk];
  const int lane = threadIdx.x & 63, sub = lane & 15;
  const int64_t q = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int split = blockIdx.y;
  const int64_t kb = (int64_t)split * kper, ke = min(K, kb + kper);
  const T* xr = X + min(q, nq - 1) * ldx;
  T acc[P];
#pragma unroll
  for (int pp = 0; pp < P; ++pp) acc[pp] = T(0);
  for (int64_t c0 = kb; c0 < ke; c0 += kThinChunk) {
    const int nc = (int)min((int64_t)kThinChunk, ke - c0);
    __syncthreads();  // (the previous chunk's reads of the stage are done)
    for (int e = threadIdx.x; e < P * kThinChunk; e += kThinThreads) {
      const int pp = e / kThinChunk, c = e - pp * kThinChunk;
      ys[e] = (pp < np && c < nc) ? Y[pp * ys_p + (c0 + c) * ys_k] : T(0);
    }
    __syncthreads();
    T x[kStripes][W];
    const bool whole = VEC && nc == kThinChunk;  // (block-uniform)
#pragma unroll
    for (int t = 0; t < kStripes; ++t) {
      const int c = (t * 16 + sub) * W;
      if (whole) {
        const typename TV::type v = *reinterpret_cast<const typename TV::type*>(xr + c0 + c);
#pragma unroll
        for (int j = 0; j < W; ++j) x[t][j] = v[j];
      } else {
#pragma unroll
        for (int j = 0; j < W; ++j) x[t][j] = c + j < nc ? xr[c0 + c + j] : T(0);
      }
    }
#pragma unroll
    for (int t = 0; t < kStripes; ++t) {
      const int c = (t * 16 + sub) * W;
#pragma unroll
      for (int pp = 0; pp < P; ++pp) {
        const typename TV::type y = *reinterpret_cast<const typename TV::type*>(ys + pp * kThinChunk + c);
#pragma unroll
        for (int j = 0; j < W; ++j) acc[pp] += x[t][j] * y[j];
      }
    }
  }
#pragma unroll
  for (int pp = 0; pp < P; ++pp) {
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc[pp] += __shfl_xor(acc[pp], off, 16);
  }
  if (q < nq && sub == 0) {
    T* out = C + (int64_t)split * sstride + q * cq;
#pragma unroll
    for (int pp = 0; pp < P; ++pp)
      if (pp < np) out[pp * cp] = acc[pp];
  }
}

// C[m, n] = sum_{k < K} A(m, k) B(k, n) for K <= kThinMax: a block's waves
// share 64 * W columns, whose B(0..K-1, ·) the block stages in LDS once and
// each lane then keeps in registers (W columns); a wave walks its row range in
// chunks of kThinRowChunk rows whose A values it stages in LDS.
template <typename T, bool VEC>
__global__ __launch_bounds__(kThinThreads) void thin_short_k_kernel(
    const T* __restrict__ A, ThinStrides st, const T* __restrict__ B, T* __restrict__ C,
    int64_t ldc, int64_t M, int64_t N, int K, int64_t rows_per_wave) {
  typedef ThinVec<T> TV;
  constexpr int W = TV::kW;
  __shared__ T as[kThinThreads / 64][kThinRowChunk * kThinMax];
  __shared__ T bs[kThinMax * 64 * W];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t nb = (int64_t)blockIdx.x * (64 * W), n0 = nb + lane * W;
  const int64_t m0 = ((int64_t)blockIdx.y * (kThinThreads / 64) + wave) * rows_per_wave;
  const int64_t m1 = min(M, m0 + rows_per_wave);
  // B(k, nb + c) at bs[k * 64W + c], loaded with consecutive threads on
  // consecutive addresses of whichever of k and n is contiguous in B
  for (int e = threadIdx.x; e < kThinMax * 64 * W; e += kThinThreads) {
    int k, c;
    if (st.bs_k == 1) {
      c = e / kThinMax;
      k = e - c * kThinMax;
    } else {
      k = e / (64 * W);
      c = e - k * (64 * W);
    }
    bs[k * (64 * W) + c] = (k < K && nb + c < N) ? B[k * st.bs_k + (nb + c) * st.bs_n] : T(0);
  }
  __syncthreads();
  T b[kThinMax][W];
#pragma unroll
  for (int k = 0; k < kThinMax; ++k)
#pragma unroll
    for (int j = 0; j < W; ++j) b[k][j] = bs[k * (64 * W) + lane * W + j];
  const bool whole = VEC && n0 + W <= N;
  T* aw = as[wave];
  for (int64_t mc = m0; mc < m1; mc += kThinRowChunk) {
    const int nr = (int)min((int64_t)kThinRowChunk, m1 - mc);
    // (wave-private stage: the wave's own loads and reads, in order)
    for (int e = lane; e < nr * kThinMax; e += 64) {
      const int r = e / kThinMax, k = e - r * kThinMax;
      aw[e] = k < K ? A[(mc + r) * st.as_m + k * st.as_k] : T(0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int r = 0; r < nr; ++r) {
      const T* ar = aw + r * kThinMax;  // (a broadcast read)
      T acc[W];
#pragma unroll
      for (int j = 0; j < W; ++j) acc[j] = T(0);
#pragma unroll
      for (int k = 0; k < kThinMax; ++k) {
        const T a = ar[k];
#pragma unroll
        for (int j = 0; j < W; ++j) acc[j] += a * b[k][j];
      }
      T* cr = C + (mc + r) * ldc + n0;
      if (whole) {
        typename TV::type v;
#pragma unroll
        for (int j = 0; j < W; ++j) v[j] = acc[j];
        *reinterpret_cast<typename TV::type*>(cr) = v;
      } else {
#pragma unroll
        for (int j = 0; j < W; ++j)
          if (n0 + j < N) cr[j] = acc[j];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Split count of a thin product (one side <= kThinMax, K > kThinMax): about
// 1024 waves over the wide side's 256-wide groups, at least 256 k per split.
// (Finer splits of a parameter product shortened the product but lengthened
// the fixed-order sum of its slices by more: at c2's output layer 17 + 29 us
// against 21 + 9 us.)
int thin_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t groups = ceil_div(max(M, N), (int64_t)256);
  int64_t s = ceil_div((int64_t)256, groups);
  s = min(s, K / 256);
  s = min(s, (int64_t)64);
  return (int)max(s, (int64_t)1);
}

template <typename T, int P>
int launch_thin_p(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda,
                  const T* B, int64_t ldb, T* C, int64_t ldc, int splits, int64_t sstride,
                  hipStream_t st) {
  constexpr int W = ThinVec<T>::kW;
  const ThinStrides t = thin_strides(layout, lda, ldb);
  const int64_t kper = ceil_div(K, (int64_t)splits);
  // thin side p, wide side q: X(.., q) the wide operand, Y(p, k) the thin one
  const bool thin_m = M <= N;
  const T* X = thin_m ? B : A;
  const T* Y = thin_m ? A : B;
  const int np = (int)(thin_m ? M : N);
  const int64_t nq = thin_m ? N : M;
  const int64_t x_q = thin_m ? t.bs_n : t.as_m, x_k = thin_m ? t.bs_k : t.as_k;
  const int64_t y_p = thin_m ? t.as_m : t.bs_n, y_k = thin_m ? t.as_k : t.bs_k;
  const int64_t cp = thin_m ? ldc : 1, cq = thin_m ? 1 : ldc;
  if (x_q == 1) {  // wide operand contiguous along the wide index
    const bool vec = aligned16(X) && x_k % W == 0;
    const dim3 grid((unsigned)ceil_div(nq, (int64_t)(64 * W)), (unsigned)splits);
    if (vec)
      hipLaunchKernelGGL((thin_wide_rows_kernel<T, P, true>), grid, dim3(kThinThreads), 0, st, X,
                         x_k, Y, y_k, y_p, C, cp, cq, sstride, np, nq, K, kper);
    else
      hipLaunchKernelGGL((thin_wide_rows_kernel<T, P, false>), grid, dim3(kThinThreads), 0, st, X,
                         x_k, Y, y_k, y_p, C, cp, cq, sstride, np, nq, K, kper);
  } else {  // contiguous along k
    const bool vec = aligned16(X) && x_q % W == 0 && kper % W == 0;
    const dim3 grid((unsigned)ceil_div(nq, (int64_t)16), (unsigned)splits);
    if (vec)
      hipLaunchKernelGGL((thin_wide_cols_kernel<T, P, true>), grid, dim3(kThinThreads), 0, st, X,
                         x_q, Y, y_k, y_p, C, cp, cq, sstride, np, nq, K, kper);
    else
      hipLaunchKernelGGL((thin_wide_cols_kernel<T, P, false>), grid, dim3(kThinThreads), 0, st, X,
                         x_q, Y, y_k, y_p, C, cp, cq, sstride, np, nq, K, kper);
  }
  return KAN_OK;
}

template <typename T>
int launch_thin(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda, const T* B,
                int64_t ldb, T* C, int64_t ldc, int splits, int64_t sstride, hipStream_t st) {
  constexpr int W = ThinVec<T>::kW;
  if (K <= kThinMax) {  // short contraction: bound by the writes of C
    const ThinStrides t = thin_strides(layout, lda, ldb);
    const bool vec = aligned16(C) && ldc % W == 0;
    const int64_t ncol = ceil_div(N, (int64_t)(64 * W));
    const int64_t rpw = ceil_div(M * ncol, (int64_t)4096);
    const int64_t wave_rows = ceil_div(M, rpw);
    const dim3 grid((unsigned)ncol, (unsigned)ceil_div(wave_rows, (int64_t)(kThinThreads / 64)));
    if (vec)
      hipLaunchKernelGGL((thin_short_k_kernel<T, true>), grid, dim3(kThinThreads), 0, st, A, t, B,
                         C, ldc, M, N, (int)K, rpw);
    else
      hipLaunchKernelGGL((thin_short_k_kernel<T, false>), grid, dim3(kThinThreads), 0, st, A, t,
                         B, C, ldc, M, N, (int)K, rpw);
    return KAN_OK;
  }
  const int64_t p = min(M, N);
  if (p <= 1) return launch_thin_p<T, 1>(layout, M, N, K, A, lda, B, ldb, C, ldc, splits, sstride, st);
  if (p <= 2) return launch_thin_p<T, 2>(layout, M, N, K, A, lda, B, ldb, C, ldc, splits, sstride, st);
  if (p <= 4) return launch_thin_p<T, 4>(layout, M, N, K, A, lda, B, ldb, C, ldc, splits, sstride, st);
  if (p <= 8) return launch_thin_p<T, 8>(layout, M, N, K, A, lda, B, ldb, C, ldc, splits, sstride, st);
  return launch_thin_p<T, 16>(layout, M, N, K, A, lda, B, ldb, C, ldc, splits, sstride, st);
}

inline bool gemm_is_thin(int64_t M, int64_t N, int64_t K) {
  return K <= kThinMax || M <= kThinMax || N <= kThinMax;
}
}  // namespace

// Split-K factor: the split count in 1..64 with the smallest estimated time
// (whole waves of resident blocks plus partial-sum traffic), keeping at least
// 8 slabs per split; any count, not only powers of two, so that the tiles of
// all splits fill their last wave of resident blocks.  Long-K products with few output tiles
// (the parameter product, sample reductions, small-batch inference) split.
template <typename T>
int gemm_pick_splits(int64_t M, int64_t N, int64_t K, int64_t max_slice_elems) {
  if (gemm_is_thin(M, N, K)) return K <= kThinMax ? 1 : thin_splits(M, N, K);
  const int64_t cus = device_cu_count();  // (once: the model is evaluated ~200 times)
  int best = 1;
  double best_t = 0.0;
  for (int s = 1; s <= 64; ++s) {
    if (s > 1 && max_slice_elems >= 0 && (int64_t)s * M * N > max_slice_elems) break;
    double t;
    if (std::is_same<T, float>::value) {
      if (s > 1 && K / s < 8 * kModelF32[0].bk) break;
      t = est_seconds(kModelF32[pick_cfg_f32(M, N, K, s, cus)], M, N, K, s, cus);
    } else {
      if (s > 1 && K / s < 8 * kModelF64[1].bk) break;
      t = est_seconds_f64(kModelF64[pick_cfg_f64(M, N, K, s, cus)], M, N, K, s, cus);
    }
    if (s == 1 || t < best_t * (1.0 - 1e-9)) {
      best = s;
      best_t = t;
    }
  }
  return best;
}

template <typename T>
int launch_gemm(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda, const T* B,
                int64_t ldb, T* C, int64_t ldc, int splits, int64_t split_stride,
                hipStream_t st) {
  if (M <= 0 || N <= 0) return KAN_OK;
  GemmParams<T> p;
  p.A = A;
  p.B = B;
  p.C = C;
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = ldc;
  p.split_stride = split_stride;
  p.vec = vec_ok(A, lda) && vec_ok(B, ldb);
  TimedLaunch timed(kClassContraction, st, 2.0 * (double)M * (double)N * (double)K);
  int rc;
  if (gemm_is_thin(M, N, K) && K > 0) {
    if (K <= kThinMax && splits > 1)
      return set_error(KAN_ERR_INVALID, "gemm: a contraction of K <= %d is not split", kThinMax);
    rc = launch_thin<T>(layout, M, N, K, A, lda, B, ldb, C, ldc, splits < 1 ? 1 : splits,
                        split_stride, st);
  } else if constexpr (std::is_same<T, float>::value) {
    const int cfg = pick_cfg_f32(M, N, K, splits < 1 ? 1 : splits);
    if (cfg == 0) rc = launch_layout<CfgF32Big>(layout, p, splits, st);
    else if (cfg == 3) rc = launch_layout<CfgF32Big4>(layout, p, splits, st);
    else if (cfg == 2) rc = launch_layout<CfgF32Narrow>(layout, p, splits, st);
    else rc = launch_layout<CfgF32Small>(layout, p, splits, st);
  } else {
    const int cfg = pick_cfg_f64(M, N, K, splits < 1 ? 1 : splits);
    if (cfg == 0) rc = launch_layout<CfgF64Big>(layout, p, splits, st);
    else if (cfg == 2) rc = launch_layout<CfgF64Pipe>(layout, p, splits, st);
    else if (cfg == 3) rc = launch_layout<CfgF64Small>(layout, p, splits, st);
    else rc = launch_layout<CfgF64>(layout, p, splits, st);
  }
  if (rc != KAN_OK) return rc;
  return check_launch("gemm");
}

namespace {
// C[m, n] = sum_s part[s][m, n], s in order (deterministic split-K result).
template <typename T>
__global__ void split_sum_kernel(const T* __restrict__ part, int splits, int64_t M, int64_t N,
                                 T* __restrict__ C, int64_t ldc) {
  const int64_t count = M * N, stride = M * N;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    T v = part[e];
    for (int s = 1; s < splits; ++s) v += part[s * stride + e];
    const int64_t m = e / N, n = e - m * N;
    C[m * ldc + n] = v;
  }
}

template <typename T>
__global__ void fill_rows_kernel(T* __restrict__ C, int64_t M, int64_t N, int64_t ldc) {
  const int64_t count = M * N;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t m = e / N, n = e - m * N;
    C[m * ldc + n] = T(0);
  }
}

inline unsigned flat_blocks(int64_t count) {
  int64_t b = ceil_div(count, 256);
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}
}  // namespace

template <typename T>
int64_t matmul_ws_elems(int layout, int64_t M, int64_t N, int64_t K, int64_t max_slice_elems) {
  (void)layout;
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const int s = gemm_pick_splits<T>(M, N, K, max_slice_elems);
  return s > 1 ? (int64_t)s * M * N : 0;
}

template <typename T>
int launch_matmul(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda,
                  const T* B, int64_t ldb, T* C, int64_t ldc, T* ws, hipStream_t st,
                  int64_t max_slice_elems) {
  if (M <= 0 || N <= 0) return KAN_OK;
  if (K <= 0) {
    hipLaunchKernelGGL(fill_rows_kernel<T>, dim3(flat_blocks(M * N)), dim3(256), 0, st, C, M, N,
                       ldc);
    return check_launch("matmul (K = 0)");
  }
  const int s = gemm_pick_splits<T>(M, N, K, max_slice_elems);
  if (s <= 1) return launch_gemm<T>(layout, M, N, K, A, lda, B, ldb, C, ldc, 1, 0, st);
  const int rc = launch_gemm<T>(layout, M, N, K, A, lda, B, ldb, ws, N, s, M * N, st);
  if (rc != KAN_OK) return rc;
  hipLaunchKernelGGL(split_sum_kernel<T>, dim3(flat_blocks(M * N)), dim3(256), 0, st, ws, s, M,
                     N, C, ldc);
  return check_launch("matmul split sum");
}

template int64_t matmul_ws_elems<float>(int, int64_t, int64_t, int64_t, int64_t);
template int64_t matmul_ws_elems<double>(int, int64_t, int64_t, int64_t, int64_t);
template int launch_matmul<float>(int, int64_t, int64_t, int64_t, const float*, int64_t,
                                  const float*, int64_t, float*, int64_t, float*, hipStream_t,
                                  int64_t);
template int launch_matmul<double>(int, int64_t, int64_t, int64_t, const double*, int64_t,
                                   const double*, int64_t, double*, int64_t, double*, hipStream_t,
                                   int64_t);

bool gemm_dx_supported(int64_t M, int64_t N, int64_t K, int64_t I, int G, int k, bool has_base) {
  if (k < 1 || k > 3) return false;
  const int R = G + k, nk = G + 2 * k + 1;
  const int cfg = pick_cfg_f32(M, N, K, 1);
  if (cfg == 0) return dx_cfg_fits<CfgF32Big>(N, I, R, nk, has_base);
  if (cfg == 3) return dx_cfg_fits<CfgF32Big4>(N, I, R, nk, has_base);
  return dx_cfg_fits<CfgF32Small>(N, I, R, nk, has_base);
}

// Input-side product fused with the input-gradient contraction (NT layout:
// A = D [M, K] row-major, B = Waug^T [N, K]): writes part [M, I, nslot]
// through dx_epilogue, then dx [M, I] = the fixed-order sum of the partials.
int launch_gemm_dx(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                   int64_t ldb, const float* x, const float* grid, int64_t I, int G, int k,
                   bool has_base, float* part, float* gx, hipStream_t st) {
  if (M <= 0 || I <= 0) return KAN_OK;
  if (!gemm_dx_supported(M, N, K, I, G, k, has_base))
    return set_error(KAN_ERR_LIMIT, "gemm_dx: layer shape not supported by the fused epilogue");
  GemmParams<float> p;
  p.A = A;
  p.B = B;
  p.C = nullptr;
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = 0;
  p.split_stride = 0;
  p.vec = vec_ok(A, lda) && vec_ok(B, ldb);
  DxParams e;
  e.x = x;
  e.grid = grid;
  e.part = part;
  e.I = I;
  e.R = G + k;
  e.ksp = I * e.R;
  e.nk = G + 2 * k + 1;
  e.es = nullptr;
  e.nslot = has_base ? 3 : 2;
  int rc;
  {
    TimedLaunch timed(kClassContraction, st, 2.0 * (double)M * (double)N * (double)K);
    const int cfg = pick_cfg_f32(M, N, K, 1);
    if (cfg == 0) rc = launch_dx_cfg<CfgF32Big>(p, e, k, st);
    else if (cfg == 3) rc = launch_dx_cfg<CfgF32Big4>(p, e, k, st);
    else rc = launch_dx_cfg<CfgF32Small>(p, e, k, st);
    if (rc != KAN_OK) return rc;
    rc = check_launch("gemm_dx");
    if (rc != KAN_OK) return rc;
  }
  const int64_t count = M * I;
  int64_t blocks = ceil_div(count, 256);
  if (blocks > 65536) blocks = 65536;
  TimedLaunch timed(kClassOther, st, 0.0);
  hipLaunchKernelGGL(dx_finalize_kernel, dim3((unsigned)blocks), dim3(256), 0, st, part, gx,
                     count, e.nslot);
  return check_launch("dx_finalize");
}

bool gemm_ecomp_supported(int64_t M, int64_t N, int64_t K, int64_t I, int G, int k,
                          bool has_base) {
  if (k < 1 || k > 3) return false;
  const int R = G + k, nk = G + 2 * k + 1;
  const int cfg = pick_cfg_f32(M, N, K, 1);
  if (cfg == 0) return ecomp_cfg_fits<CfgF32Big>(N, I, R, nk, has_base);
  if (cfg == 3) return ecomp_cfg_fits<CfgF32Big4>(N, I, R, nk, has_base);
  return ecomp_cfg_fits<CfgF32Small>(N, I, R, nk, has_base);
}

// Input-side product in compact form (NT layout: A = D [M, K], B = Waug^T
// [N, K]): the span-window values Ew [M, I, k+1] and the base columns Es
// [M, I] (has_base) through ecomp_epilogue; no [M, N] output.
int launch_gemm_ecomp(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda,
                      const float* B, int64_t ldb, const float* x, const float* grid, int64_t I,
                      int G, int k, bool has_base, float* ew, float* es, hipStream_t st) {
  if (M <= 0 || I <= 0) return KAN_OK;
  if (!gemm_ecomp_supported(M, N, K, I, G, k, has_base))
    return set_error(KAN_ERR_LIMIT, "gemm_ecomp: layer shape not supported by the compact epilogue");
  GemmParams<float> p;
  p.A = A;
  p.B = B;
  p.C = nullptr;
  p.M = M;
  p.N = N;
  p.K = K;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = 0;
  p.split_stride = 0;
  p.vec = vec_ok(A, lda) && vec_ok(B, ldb);
  DxParams e;
  e.x = x;
  e.grid = grid;
  e.part = ew;
  e.es = has_base ? es : nullptr;
  e.I = I;
  e.R = G + k;
  e.ksp = I * e.R;
  e.nk = G + 2 * k + 1;
  e.nslot = k + 1;
  TimedLaunch timed(kClassContraction, st, 2.0 * (double)M * (double)N * (double)K);
  const int cfg = pick_cfg_f32(M, N, K, 1);
  int rc;
  if (cfg == 0) rc = launch_ecomp_cfg<CfgF32Big>(p, e, k, st);
  else if (cfg == 3) rc = launch_ecomp_cfg<CfgF32Big4>(p, e, k, st);
  else rc = launch_ecomp_cfg<CfgF32Small>(p, e, k, st);
  if (rc != KAN_OK) return rc;
  return check_launch("gemm_ecomp");
}

template int launch_gemm<float>(int, int64_t, int64_t, int64_t, const float*, int64_t,
                                const float*, int64_t, float*, int64_t, int, int64_t,
                                hipStream_t);
template int launch_gemm<double>(int, int64_t, int64_t, int64_t, const double*, int64_t,
                                 const double*, int64_t, double*, int64_t, int, int64_t,
                                 hipStream_t);
template int gemm_pick_splits<float>(int64_t, int64_t, int64_t, int64_t);
template int gemm_pick_splits<double>(int64_t, int64_t, int64_t, int64_t);

}  // namespace kan
