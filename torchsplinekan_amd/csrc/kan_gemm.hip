// Dense contraction engine for the KAN forward and backward on gfx950 MFMA.
//
// The three contractions of a KANLinear step all run through this kernel
// with different operand layouts (A = augmented basis [H | silu(x)],
// W = augmented weight [coef*scaler | base_weight], D = grad_output):
//   forward  Y[n,o]  = sum_k A[n,k] W[o,k]     (NT: both K-contiguous)
//   params   G[o,k]  = sum_n D[n,o] A[n,k]     (TN: both M/N-contiguous)
//   input    E[n,k]  = sum_o D[n,o] W[o,k]     (NN)
// They replace the cuBLAS calls of csrc/kan_cuda.cu:521-529, 579-604.
//
// One kernel template, configured per dtype and layout (tile, waves, MFMA
// shape, pipelining), chosen by measurement on MI355X at the c3 shapes:
//   fp32 NT   128x128 tile, BK 32, 2x2 waves of 64x64, v_mfma_f32_32x32x2f32,
//             software-pipelined main loop;
//   fp32 TN/NN 256x128 tile, BK 16, 4x2 waves of 64x64, v_mfma_f32_16x16x4f32;
//   fp64      128x128 tile, BK 16, 2x2 waves, v_mfma_f64_16x16x4f64.
// Operand slabs (BK wide) are staged through LDS with double buffering: the
// next slab's global loads are in flight while the current slab feeds the
// MFMAs.  Each operand keeps its global layout in LDS:
//   K-contiguous operand  -> LDS [rows][BK+4]; a lane reads 4 consecutive k
//                            with one 16-byte ds_read.  Within each k-group
//                            of the MFMA the k order is permuted identically
//                            for A and B (step s, lane group q uses
//                            k = KG*g + 4q + s), which leaves the sum unchanged;
//   MN-contiguous operand -> LDS [BK][rows+4]; a lane reads one element.
// Tiles whose rows and K range are entirely in bounds (and whose operands are
// 16-byte aligned) take branch-free vector loads; edge tiles take a guarded
// path.  The pipelined loop keeps two register sets of MFMA fragments: the
// fragments of k-group g+1 are read from LDS while the MFMAs of group g run,
// and the hand-over to the next slab (LDS store, barrier, first fragment
// read) is issued ahead of the last group's MFMAs.
// Scheduling: the linear workgroup id is remapped so that each XCD (dispatch
// is round-robin over 8 XCDs) receives a contiguous range of tiles, visited
// in groups of 8 row-tiles so that tiles running together on one XCD share
// operand slabs in its L2.  Optional split-K writes partial products to
// separate slices of C (reduced by the caller in a fixed order).

#include "kan_common.h"

namespace kan {
namespace {

constexpr int kPadK = 4;
constexpr int kPadMN = 4;
constexpr int kNumXcd = 8;
constexpr int kGroupM = 8;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef double f64x4 __attribute__((ext_vector_type(4)));

// MFMA shapes: operand fragment of lane (row, kq) and accumulator layout.
template <typename T, int MF>
struct Mfma;

template <>
struct Mfma<float, 16> {  // v_mfma_f32_16x16x4f32
  typedef f32x4 acc_t;
  static constexpr int kKG = 16;    // k per fragment group (4 steps x 4)
  static constexpr int kNAcc = 4;
  __device__ static __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int row(int lane) { return lane & 15; }
  __device__ static __forceinline__ int kq(int lane) { return lane >> 4; }
  __device__ static __forceinline__ int kofs(int g, int q) { return 16 * g + 4 * q; }
  __device__ static __forceinline__ int out_row(int lane, int v) { return 4 * (lane >> 4) + v; }
  __device__ static __forceinline__ int out_col(int lane) { return lane & 15; }
};

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
// MFMA shape MF, pipelined main loop, minimum resident blocks per CU.
template <typename T_, int BM_, int BN_, int BK_, int WM_, int WN_, int MF_, bool PIPE_,
          int MINB_>
struct Cfg {
  typedef T_ T;
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_, MF = MF_;
  static constexpr bool PIPE = PIPE_;
  static constexpr int MINB = MINB_;
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / MF, FN = TN / MF;
  static_assert(FM * MF == TM && FN * MF == TN, "wave tile must be whole MFMA tiles");
  static_assert(BK % Mfma<T, MF>::kKG == 0, "slab must be whole k-groups");
};

using CfgF32NT = Cfg<float, 128, 128, 32, 2, 2, 32, true, 2>;
using CfgF32MN = Cfg<float, 256, 128, 16, 4, 2, 16, false, 1>;
using CfgF64 = Cfg<double, 128, 128, 16, 2, 2, 16, false, 1>;

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
};

// LDS footprint of one operand slab.
template <int ROWS, int BK, bool KCONT>
struct Slab {
  static constexpr int kStride = KCONT ? (BK + kPadK) : (ROWS + kPadMN);
  static constexpr int kElems = KCONT ? ROWS * (BK + kPadK) : BK * (ROWS + kPadMN);
};

// Bijective remap of the dispatch order so that each XCD receives a
// contiguous range of logical tile ids.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  const int per = total / kNumXcd, rem = total % kNumXcd;
  const int xcd = pid % kNumXcd, idx = pid / kNumXcd;
  return xcd * per + min(xcd, rem) + idx;
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

  // Edge slab: element-wise bounds (rows < rows, k < kend), zero fill.
  __device__ __forceinline__ void load_guarded(const T* __restrict__ src, int64_t ld, int64_t row0,
                                               int64_t rows, int64_t k0, int64_t kend, bool vec) {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      int64_t r, kk;
      coords(threadIdx.x + p * NT, row0, k0, r, kk);
      const bool full = KCONT ? ((r < rows) && (kk + 3 < kend)) : ((kk < kend) && (r + 3 < rows));
      if (vec && full) {
        reg[p] = *reinterpret_cast<const Vec4<T>*>(KCONT ? src + r * ld + kk : src + kk * ld + r);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          T v = T(0);
          if (KCONT) {
            if (r < rows && kk + j < kend) v = src[r * ld + kk + j];
          } else {
            if (kk < kend && r + j < rows) v = src[kk * ld + r + j];
          }
          reg[p].v[j] = v;
        }
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

  const int total = p.tiles_m * p.tiles_n * p.splits;
  const int pid = xcd_remap(blockIdx.x, total);
  const int per_split = p.tiles_m * p.tiles_n;
  const int split = pid / per_split;
  const int t = pid - split * per_split;
  const int group = kGroupM * p.tiles_n;
  const int first_m = (t / group) * kGroupM;
  const int gm = min(p.tiles_m - first_m, kGroupM);
  const int tm = first_m + (t % group) % gm;
  const int tn = (t % group) / gm;

  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int nkt = kend > kbeg ? (int)ceil_div(kend - kbeg, BK) : 0;

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
  const bool full = p.vec && (m0 + BM <= p.M) && (n0 + BN <= p.N) && ((kend - kbeg) % BK == 0);
  auto gload = [&](int slab) {
    const int64_t k0 = kbeg + (int64_t)slab * BK;
    if (full) {
      la.load_full(p.A, p.lda, m0, k0);
      lb.load_full(p.B, p.ldb, n0, k0);
    } else {
      la.load_guarded(p.A, p.lda, m0, p.M, k0, kend, p.vec != 0);
      lb.load_guarded(p.B, p.ldb, n0, p.N, k0, kend, p.vec != 0);
    }
  };
  T fa[2][FM][4], fb[2][FN][4];
  auto fread = [&](int buf, int g, int slot) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      read_frag<T, BM, BK, AK>(lds_a[buf], wm * C::TM + i * C::MF + rl, M::kofs(g, q), fa[slot][i]);
#pragma unroll
    for (int j = 0; j < FN; ++j)
      read_frag<T, BN, BK, BKC>(lds_b[buf], wn * C::TN + j * C::MF + rl, M::kofs(g, q), fb[slot][j]);
  };
  auto mfmas = [&](int slot) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = M::mma(fa[slot][i][s], fb[slot][j][s], acc[i][j]);
  };

  if (nkt > 0) {
    gload(0);
    la.store(lds_a[0]);
    lb.store(lds_b[0]);
    if (C::PIPE) {
      if (nkt > 1) gload(1);
      __syncthreads();
      fread(0, 0, 0);
      int slot = 0;
      for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          if (g + 1 < NG) {
            fread(cur, g + 1, slot ^ 1);
          } else if (kt + 1 < nkt) {
            // hand-over: slab kt+1 into the other buffer (last read during
            // slab kt-1, before the previous barrier), loads of slab kt+2
            la.store(lds_a[cur ^ 1]);
            lb.store(lds_b[cur ^ 1]);
            if (kt + 2 < nkt) gload(kt + 2);
            __syncthreads();
            fread(cur ^ 1, 0, slot ^ 1);
          }
          mfmas(slot);
          slot ^= 1;
        }
      }
    } else {
      __syncthreads();
      for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) gload(kt + 1);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          fread(cur, g, 0);
          mfmas(0);
        }
        if (more) {
          la.store(lds_a[cur ^ 1]);
          lb.store(lds_b[cur ^ 1]);
        }
        __syncthreads();
      }
    }
  }

  T* Cp = p.C + (int64_t)split * p.split_stride;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t col = n0 + wn * C::TN + j * C::MF + M::out_col(lane);
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < M::kNAcc; ++v) {
        const int64_t row = m0 + wm * C::TM + i * C::MF + M::out_row(lane, v);
        if (row < p.M) Cp[row * p.ldc + col] = acc[i][j][v];
      }
    }
  }
}

template <typename T>
bool vec_ok(const T* ptr, int64_t ld) {
  return ((reinterpret_cast<uintptr_t>(ptr) % (4 * sizeof(T))) == 0) && (ld % 4 == 0);
}

template <typename T>
struct Select;
template <>
struct Select<float> {
  typedef CfgF32NT NT;
  typedef CfgF32MN TN;
  typedef CfgF32MN NN;
};
template <>
struct Select<double> {
  typedef CfgF64 NT;
  typedef CfgF64 TN;
  typedef CfgF64 NN;
};

template <class C>
void tiles_of(int64_t M, int64_t N, int64_t* tm, int64_t* tn) {
  *tm = ceil_div(M, C::BM);
  *tn = ceil_div(N, C::BN);
}

template <class C, bool AK, bool BKC>
int launch_cfg(GemmParams<typename C::T> p, int splits, hipStream_t st) {
  if (splits < 1) splits = 1;
  p.k_per_split = round_up(ceil_div(p.K > 0 ? p.K : 1, splits), C::BK);
  int64_t tm, tn;
  tiles_of<C>(p.M, p.N, &tm, &tn);
  const int64_t blocks = tm * tn * splits;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "gemm: problem too large (%lld tiles)", (long long)blocks);
  p.tiles_m = (int)tm;
  p.tiles_n = (int)tn;
  p.splits = splits;
  hipLaunchKernelGGL((gemm_kernel<C, AK, BKC>), dim3((unsigned)blocks), dim3(C::kThreads), 0, st,
                     p);
  return KAN_OK;
}

}  // namespace

// Split-K factor for a TN (parameter-gradient) product: the smallest split
// that gives at least three waves of resident blocks, keeping >= 64 slabs
// of K per split; at most 8.
template <typename T>
int gemm_pick_splits(int64_t M, int64_t N, int64_t K) {
  typedef typename Select<T>::TN C;
  int64_t tm, tn;
  tiles_of<C>(M, N, &tm, &tn);
  const int64_t tiles = tm * tn;
  if (tiles <= 0) return 1;
  const int64_t slots = (int64_t)device_cu_count() * 2;
  int s = 1;
  while (s < 8 && tiles * s < 3 * slots && K / (2 * s) >= 64 * C::BK) s *= 2;
  return s;
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
  switch (layout) {
    case kLayoutNT: rc = launch_cfg<typename Select<T>::NT, true, true>(p, splits, st); break;
    case kLayoutTN: rc = launch_cfg<typename Select<T>::TN, false, false>(p, splits, st); break;
    case kLayoutNN: rc = launch_cfg<typename Select<T>::NN, true, false>(p, splits, st); break;
    default: return set_error(KAN_ERR_INVALID, "gemm: unknown layout %d", layout);
  }
  if (rc != KAN_OK) return rc;
  return check_launch("gemm");
}

template int launch_gemm<float>(int, int64_t, int64_t, int64_t, const float*, int64_t,
                                const float*, int64_t, float*, int64_t, int, int64_t,
                                hipStream_t);
template int launch_gemm<double>(int, int64_t, int64_t, int64_t, const double*, int64_t,
                                 const double*, int64_t, double*, int64_t, int, int64_t,
                                 hipStream_t);
template int gemm_pick_splits<float>(int64_t, int64_t, int64_t);
template int gemm_pick_splits<double>(int64_t, int64_t, int64_t);

}  // namespace kan
