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
// Tiling: 256 threads = 4 waves in a 2x2 arrangement; block tile 128x128,
// wave tile 64x64 = 4x4 MFMA tiles of 16x16 (v_mfma_f32_16x16x4f32, or
// v_mfma_f64_16x16x4f64 for fp64).  K advances in LDS-staged slabs of BK
// (32 fp32 / 16 fp64) with double buffering: the next slab's global loads are
// in flight while the current slab is consumed.  Each operand keeps its
// global layout in LDS:
//   K-contiguous operand  -> LDS [rows][BK+4]; a lane reads 4 consecutive k
//                            with one 16-byte ds_read (k permuted within each
//                            group of 16: MFMA step s, lane group q uses
//                            k = 16g + 4q + s, identically for A and B);
//   MN-contiguous operand -> LDS [BK][rows+4]; a lane reads one element.
// Row paddings are chosen so that both the staging writes and the MFMA
// operand reads are free of LDS bank conflicts.
// Scheduling: the linear workgroup id is remapped so that consecutive tiles
// land on the same XCD (workgroups are dealt round-robin over 8 XCDs), and
// tiles are visited in groups of 8 row-tiles so that the tiles an XCD runs
// together share operand slabs in its L2.  Optional split-K writes partial
// products to separate slices of C (reduced by the caller, deterministically).

#include "kan_common.h"

namespace kan {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kTileM = 128;
constexpr int kTileN = 128;
constexpr int kPadK = 4;
constexpr int kPadMN = 4;
constexpr int kNumXcd = 8;
constexpr int kGroupM = 8;

template <typename T>
struct Mfma;

template <>
struct Mfma<float> {
  typedef float acc_t __attribute__((ext_vector_type(4)));
  static constexpr int kBK = 32;
  __device__ static __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  // Row (within the 16x16 tile) of accumulator element v of lane group q;
  // the column is the lane's index within its group of 16.
  __device__ static __forceinline__ int out_row(int q, int v) { return 4 * q + v; }
};

template <>
struct Mfma<double> {
  typedef double acc_t __attribute__((ext_vector_type(4)));
  static constexpr int kBK = 16;
  __device__ static __forceinline__ acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  // The f64 instruction interleaves rows across the four accumulators.
  __device__ static __forceinline__ int out_row(int q, int v) { return q + 4 * v; }
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
template <typename T, int ROWS, int BK, bool KCONT, bool VEC>
struct SlabLoader {
  static constexpr int kChunks = ROWS * BK / 4;
  static constexpr int kPer = kChunks / kGemmThreads;
  static_assert(kPer * kGemmThreads == kChunks, "slab must split evenly over the block");
  Vec4<T> reg[kPer];

  // src points at the operand; row0/rows bound the M (or N) extent;
  // k0/kend bound the K extent of this slab.
  __device__ __forceinline__ void load(const T* __restrict__ src, int64_t ld, int64_t row0,
                                       int64_t rows, int64_t k0, int64_t kend) {
#pragma unroll
    for (int p = 0; p < kPer; ++p) {
      const int c = threadIdx.x + p * kGemmThreads;
      int64_t r, kk;
      if (KCONT) {
        r = row0 + c / (BK / 4);
        kk = k0 + 4 * (c % (BK / 4));
      } else {
        kk = k0 + c / (ROWS / 4);
        r = row0 + 4 * (c % (ROWS / 4));
      }
      // element j of the chunk is at (r, kk + j) for KCONT, (r + j, kk) otherwise
      bool full;
      if (KCONT) full = (r < rows) && (kk + 3 < kend);
      else full = (kk < kend) && (r + 3 < rows);
      if (VEC && full) {
        const T* p4 = KCONT ? src + r * ld + kk : src + kk * ld + r;
        reg[p] = *reinterpret_cast<const Vec4<T>*>(p4);
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
      const int c = threadIdx.x + p * kGemmThreads;
      int off;
      if (KCONT) off = (c / (BK / 4)) * Slab<ROWS, BK, true>::kStride + 4 * (c % (BK / 4));
      else off = (c / (ROWS / 4)) * Slab<ROWS, BK, false>::kStride + 4 * (c % (ROWS / 4));
      *reinterpret_cast<Vec4<T>*>(lds + off) = reg[p];
    }
  }
};

// MFMA operand fragment of one 16-row block for the 4 steps of k-group g.
template <typename T, int ROWS, int BK, bool KCONT>
__device__ __forceinline__ void read_frag(const T* __restrict__ lds, int row, int g, int q,
                                          T (&f)[4]) {
  if (KCONT) {
    const Vec4<T> v = *reinterpret_cast<const Vec4<T>*>(
        lds + row * Slab<ROWS, BK, true>::kStride + 16 * g + 4 * q);
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = v.v[s];
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) f[s] = lds[(16 * g + 4 * q + s) * Slab<ROWS, BK, false>::kStride + row];
  }
}

template <typename T, bool AK, bool BKC, bool VEC>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_kernel(GemmParams<T> p) {
  constexpr int BK = Mfma<T>::kBK;
  using SA = Slab<kTileM, BK, AK>;
  using SB = Slab<kTileN, BK, BKC>;
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

  const int64_t m0 = (int64_t)tm * kTileM;
  const int64_t n0 = (int64_t)tn * kTileN;
  const int64_t kbeg = (int64_t)split * p.k_per_split;
  const int64_t kend = min(p.K, kbeg + p.k_per_split);
  const int nkt = kend > kbeg ? (int)ceil_div(kend - kbeg, BK) : 0;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int q = lane >> 4, rl = lane & 15;

  typename Mfma<T>::acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = T(0);

  SlabLoader<T, kTileM, BK, AK, VEC> la;
  SlabLoader<T, kTileN, BK, BKC, VEC> lb;

  if (nkt > 0) {
    la.load(p.A, p.lda, m0, p.M, kbeg, kend);
    lb.load(p.B, p.ldb, n0, p.N, kbeg, kend);
    la.store(lds_a[0]);
    lb.store(lds_b[0]);
  }
  __syncthreads();

  for (int kt = 0; kt < nkt; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) {
      const int64_t k0 = kbeg + (int64_t)(kt + 1) * BK;
      la.load(p.A, p.lda, m0, p.M, k0, kend);
      lb.load(p.B, p.ldb, n0, p.N, k0, kend);
    }
    const T* sa = lds_a[cur];
    const T* sb = lds_b[cur];
#pragma unroll
    for (int g = 0; g < BK / 16; ++g) {
      T fa[4][4], fb[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) read_frag<T, kTileM, BK, AK>(sa, wm * 64 + i * 16 + rl, g, q, fa[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) read_frag<T, kTileN, BK, BKC>(sb, wn * 64 + j * 16 + rl, g, q, fb[j]);
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<T>::mma(fa[i][s], fb[j][s], acc[i][j]);
    }
    if (more) {
      la.store(lds_a[cur ^ 1]);
      lb.store(lds_b[cur ^ 1]);
    }
    __syncthreads();
  }

  // Epilogue: lane holds column rl and rows out_row(q, 0..3) of each 16x16 tile.
  T* C = p.C + (int64_t)split * p.split_stride;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + wn * 64 + j * 16 + rl;
      if (col >= p.N) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = m0 + wm * 64 + i * 16 + Mfma<T>::out_row(q, v);
        if (row < p.M) C[row * p.ldc + col] = acc[i][j][v];
      }
    }
  }
}

template <typename T>
bool vec_ok(const T* ptr, int64_t ld) {
  return ((reinterpret_cast<uintptr_t>(ptr) % (4 * sizeof(T))) == 0) && (ld % 4 == 0);
}

template <typename T, bool AK, bool BKC>
void launch_layout(const GemmParams<T>& p, bool vec, unsigned blocks, hipStream_t st) {
  if (vec)
    hipLaunchKernelGGL((gemm_kernel<T, AK, BKC, true>), dim3(blocks), dim3(kGemmThreads), 0, st, p);
  else
    hipLaunchKernelGGL((gemm_kernel<T, AK, BKC, false>), dim3(blocks), dim3(kGemmThreads), 0, st, p);
}

}  // namespace

template <typename T>
int gemm_pick_splits(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = ceil_div(M, kTileM) * ceil_div(N, kTileN);
  if (tiles <= 0) return 1;
  const int64_t slots = (int64_t)device_cu_count() * (sizeof(T) == 4 ? 2 : 1);
  if (tiles >= 8 * slots) return 1;
  const int64_t bk = Mfma<T>::kBK;
  int best = 1;
  double best_eff = 0.0;
  for (int s = 1; s <= 8; ++s) {
    if (s > 1 && K / s < 16 * bk) break;
    const double work = (double)(tiles * s) / (double)slots;
    const double waves = (double)ceil_div(tiles * s, slots);
    const double eff = work / waves;
    if (eff > best_eff + 0.05) {
      best_eff = eff;
      best = s;
    }
  }
  return best;
}

template <typename T>
int launch_gemm(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda, const T* B,
                int64_t ldb, T* C, int64_t ldc, int splits, int64_t split_stride,
                hipStream_t st) {
  if (M <= 0 || N <= 0) return KAN_OK;
  if (splits < 1) splits = 1;
  constexpr int BK = Mfma<T>::kBK;
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
  p.k_per_split = round_up(ceil_div(K > 0 ? K : 1, splits), BK);
  p.split_stride = split_stride;
  const int64_t tm = ceil_div(M, kTileM), tn = ceil_div(N, kTileN);
  const int64_t blocks = tm * tn * splits;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "gemm: problem too large (%lld tiles)", (long long)blocks);
  p.tiles_m = (int)tm;
  p.tiles_n = (int)tn;
  p.splits = splits;
  const bool vec = vec_ok(A, lda) && vec_ok(B, ldb);
  TimedLaunch timed(kClassContraction, st, 2.0 * (double)M * (double)N * (double)K);
  switch (layout) {
    case kLayoutNT: launch_layout<T, true, true>(p, vec, (unsigned)blocks, st); break;
    case kLayoutTN: launch_layout<T, false, false>(p, vec, (unsigned)blocks, st); break;
    case kLayoutNN: launch_layout<T, true, false>(p, vec, (unsigned)blocks, st); break;
    default: return set_error(KAN_ERR_INVALID, "gemm: unknown layout %d", layout);
  }
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
