// B-spline basis kernels for gfx950: the basis H[n, I, R], its input-gradient
// contraction gx = sum_r gH * dB_r/dx, and the small packing kernels that
// build the augmented operands of the contraction GEMMs.
//
// Conventions (identical to the reference's native path,
// csrc/kan_cuda.cu:188-271, and to spline_kan/reference_backend.py:69-94 for
// finite inputs):
//   * spans are half-open [t_m, t_{m+1}); x == t_{nk-1} uses the last
//     non-degenerate span;
//   * x outside [t_0, t_{nk-1}] (and NaN) gives an all-zero row;
//   * a zero knot difference contributes zero (repeated knots allowed).
//
// Work mapping: a workgroup owns a block of up to 64 consecutive features
// (their knot rows are staged in LDS) and a range of samples.  A wave
// computes 64 (sample, feature) items per step; each lane writes its dense
// R-row into an LDS stage, and the wave then stores the stage with
// consecutive lanes on consecutive addresses, so global stores of the
// [n, I, R] rows are fully coalesced.  x reads are coalesced along features.

#include "kan_common.h"
#include "kan_spline.h"

namespace kan {
namespace {

constexpr int kBasisThreads = 256;  // upper bound; a block has sh.waves waves

// Dense Cox-de Boor recurrence over the whole knot row (legacy basis
// implementation 0).  Operation order follows compute_basis
// (spline_kan/reference_backend.py:69-94): alpha = (x - t_r)/dl,
// beta = (t_{r+d+1} - x)/dr, B = alpha*B_r + beta*B_{r+1}, with contraction
// into FMA disabled so that the rounding sequence is the same.
// Writes the degree-`deg` values into out[0 .. nk-2-deg].
template <typename T>
__device__ void dense_recurrence(const T* __restrict__ t, int nk, T x, int deg, T* out) {
#pragma clang fp contract(off)
  T buf[kMaxKnots];
  const int n0 = nk - 1;
  for (int r = 0; r < n0; ++r) {
    const bool in = (x >= t[r]) && (x < t[r + 1]);
    const bool last = (r == n0 - 1) && (x >= t[r]) && (x <= t[r + 1]);
    buf[r] = (in || last) ? T(1) : T(0);
  }
  int cur = n0;
  for (int d = 1; d <= deg; ++d) {
    const int nn = cur - 1;
    for (int r = 0; r < nn; ++r) {
      const T dl = t[r + d] - t[r];
      const T dr = t[r + d + 1] - t[r + 1];
      const T alpha = (dl != T(0)) ? (x - t[r]) / dl : T(0);
      const T beta = (dr != T(0)) ? (t[r + d + 1] - x) / dr : T(0);
      const T lhs = alpha * buf[r];
      const T rhs = beta * buf[r + 1];
      buf[r] = lhs + rhs;
    }
    cur = nn;
  }
  for (int r = 0; r < cur; ++r) out[r] = buf[r];
}

// Dense derivative (legacy implementation 0), compute_basis_derivative order
// (spline_kan/reference_backend.py:115-125): k*(Hm_r/d1 - Hm_{r+1}/d2).
template <typename T>
__device__ void dense_derivative(const T* __restrict__ t, int nk, T x, int k, T* out) {
#pragma clang fp contract(off)
  T lower[kMaxKnots];
  dense_recurrence<T>(t, nk, x, k - 1, lower);
  const int R = nk - k - 1;
  for (int r = 0; r < R; ++r) {
    const T d1 = t[r + k] - t[r];
    const T d2 = t[r + k + 1] - t[r + 1];
    const T t1 = (d1 != T(0)) ? lower[r] / d1 : T(0);
    const T t2 = (d2 != T(0)) ? lower[r + 1] / d2 : T(0);
    out[r] = T(k) * (t1 - t2);
  }
}

// c / R for small non-negative c (c < 2^16) via a float reciprocal; exact
// because the fractional part of (c + 0.5)/R is at least 0.5/R away from an
// integer while the product's error is below 1e-3.
__device__ __forceinline__ int small_div(int c, float inv_r) {
  return (int)(((float)c + 0.5f) * inv_r);
}

struct BasisShape {
  int64_t n;
  int I, G;
  int fb;     // features per block (<= 64)
  int subs;   // samples per wave step (64 / fb)
  int iters;  // wave steps per block
  int waves;  // waves per block
  int vec;    // 16-byte vector path for the staged rows (alignment holds)
  int64_t ld_aux;  // row stride of silu(x) (basis) or of its gradient (basis_grad)
  int nfb;    // feature blocks (ceil(I / fb))
  const void* scale;  // optional [n, I] factor of every item's output (T)
};

// Block of a basis launch: feature block f and sample-row group g.  The
// launch is a 1-D grid of nfb x (row groups) workgroups whose ids are
// remapped (xcd_remap) so that each XCD takes a contiguous range of logical
// blocks, feature block fastest.  An XCD then streams whole consecutive
// sample rows of the [n, ld] rows; with the 2-D grid dealt round-robin, XCD
// j took feature blocks j and j + 8 of every row, a strided eighth of the
// whole buffer.  Measured at c3: basis 0.757 -> 0.713 ms, basis_grad 0.839
// -> 0.810 ms.
struct BasisBlock {
  int f;
  int64_t g;
};
__device__ __forceinline__ BasisBlock basis_block(const BasisShape& sh) {
  const int id = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  return {id % sh.nfb, (int64_t)(id / sh.nfb)};
}

// 16-byte vector of T.
template <typename T>
struct V16 {
  static constexpr int kN = 16 / sizeof(T);
  typedef T type __attribute__((ext_vector_type(16 / sizeof(T))));
};

template <typename T>
__device__ __forceinline__ T* stage_knots(unsigned char* smem, const T* __restrict__ grid,
                                          int i0, int fbv, int nk) {
  T* knots = reinterpret_cast<T*>(smem);
  const T* src = grid + (int64_t)i0 * nk;
  for (int e = threadIdx.x; e < fbv * nk; e += blockDim.x) knots[e] = src[e];
  return knots;
}

// Copies cnt elements between a staged row in LDS and global memory, with
// 16-byte vectors when both sides are aligned (vec), element-wise otherwise.
template <typename T, bool TO_GLOBAL>
__device__ __forceinline__ void move_row(T* __restrict__ gmem, T* __restrict__ lds, int cnt,
                                         int lane, bool vec) {
  typedef typename V16<T>::type VT;
  constexpr int kV = V16<T>::kN;
  int done = 0;
  if (vec) {
    const int nv = cnt / kV;
    for (int c = lane; c < nv; c += 64) {
      if (TO_GLOBAL) reinterpret_cast<VT*>(gmem)[c] = reinterpret_cast<const VT*>(lds)[c];
      else reinterpret_cast<VT*>(lds)[c] = reinterpret_cast<const VT*>(gmem)[c];
    }
    done = nv * kV;
  }
  for (int c = done + lane; c < cnt; c += 64) {
    if (TO_GLOBAL) gmem[c] = lds[c];
    else lds[c] = gmem[c];
  }
}

// Record of a lane with no window (zero row): every r is outside it.
constexpr int kNoWindow = -(1 << 20);

// Writes one staged sample segment (fbv features x R values, contiguous in
// the output) from the per-item window records: item f has its K+1 values
// at vals[f*(K+1) ..] for r = r0[f] .. r0[f]+K, zero elsewhere.  Each lane
// forms whole 16-byte vectors of the segment (when vec), so the stores are
// coalesced; window entries that are not real basis functions (r < 0 or
// r >= R near the ends of the knot vector) are never addressed.
template <int K, typename T>
__device__ __forceinline__ void write_window_segment(T* __restrict__ gmem,
                                                     const T* __restrict__ vals,
                                                     const int* __restrict__ r0, int fbv, int R,
                                                     float inv_r, int lane, bool vec) {
  typedef typename V16<T>::type VT;
  constexpr int kV = V16<T>::kN;
  const int cnt = fbv * R;
  auto value = [&](int idx) -> T {
    const int f = small_div(idx, inv_r);
    const int j = idx - f * R - r0[f];
    const int jc = j < 0 ? 0 : (j > K ? K : j);
    const T v = vals[f * (K + 1) + jc];
    return j == jc ? v : T(0);
  };
  int done = 0;
  if (vec) {
    const int nv = cnt / kV;
    for (int c = lane; c < nv; c += 64) {
      VT o;
#pragma unroll
      for (int e = 0; e < kV; ++e) o[e] = value(c * kV + e);
      reinterpret_cast<VT*>(gmem)[c] = o;
    }
    done = nv * kV;
  }
  for (int c = done + lane; c < cnt; c += 64) gmem[c] = value(c);
}

// Wave-scope barrier: orders this wave's LDS writes before its following
// LDS reads (and vice versa) at the compiler level; LDS instructions of one
// wave complete in issue order.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave steps per block are bounded so that a wave's x values for all of its
// steps are loaded into registers before the first step is computed.
constexpr int kMaxIters = 8;

// H rows (and optionally silu(x)) for a block of features x samples.
// Each wave loads the x values of all of its steps up front.  Per step, the
// wave stages its items and writes each sample segment with coalesced
// 16-byte stores.  Staging:
//   REC (impl 1, large R): each item's window record (span start and K+1
//     values); segments are formed from the records (write_window_segment),
//     so the dense rows are never staged: K+2 LDS writes per item instead
//     of R, and a small LDS footprint;
//   dense stage (impl 1, small R): a dense R-row per item (the subs sample
//     segments exactly as they lie in the output), zeroed once, after which
//     each step clears only the item's previous window before writing the
//     new one, and copied out (move_row);
//   impl 0 (dense recurrence): the dense R-row, fully written each step.
// Only the knot staging needs a block barrier; the stages are private to
// their waves.  DER > 0 (impl 1 only) writes the order-DER derivatives.
// Grid sizes above this take impl 1's window records; at or below it the
// dense stage is cheaper (fewer VALU operations per output element).
constexpr int kWindowRecordMinR = 25;

template <int K, typename T, int IMPL, int DER = 0, bool REC = false>
__global__ __launch_bounds__(kBasisThreads) void basis_kernel(
    const T* __restrict__ x, const T* __restrict__ grid, T* __restrict__ out, int64_t ld,
    T* __restrict__ silu_out, BasisShape sh) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nk = sh.G + 2 * K + 1, R = sh.G + K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const BasisBlock bb = basis_block(sh);
  const int i0 = bb.f * sh.fb;
  const int fbv = min(sh.fb, sh.I - i0);
  const int sub = lane / sh.fb, fi = lane - sub * sh.fb;
  const bool lane_ok = sub < sh.subs && fi < fbv;
  const int64_t step = (int64_t)sh.waves * sh.subs;
  const int64_t nbase = bb.g * sh.iters * step + (int64_t)wave * sh.subs;
  T xs[kMaxIters];
#pragma unroll
  for (int it = 0; it < kMaxIters; ++it) {
    const int64_t nn = nbase + it * step + sub;
    xs[it] = (it < sh.iters && lane_ok && nn < sh.n) ? x[nn * sh.I + i0 + fi] : T(0);
  }
  T* knots = stage_knots<T>(smem, grid, i0, fbv, nk);
  T* region = knots + round_up((int64_t)sh.fb * nk, 4);
  // REC: K+1 window values per lane, followed by the lanes' window starts;
  // otherwise a dense R-row per lane
  T* stage = region + wave * 64 * (REC ? K + 1 : R);
  int* rec_r0 = reinterpret_cast<int*>(region + sh.waves * 64 * (K + 1)) + wave * 64;
  const T* t = knots + fi * nk;
  if (IMPL == 1 && !REC) {  // zero the wave's dense stage once
    typedef typename V16<T>::type VT;
    constexpr int kV = V16<T>::kN;
    const int cnt = 64 * R;
    if (((64 * R) % kV) == 0) {
      for (int c = lane; c < cnt / kV; c += 64) reinterpret_cast<VT*>(stage)[c] = VT{};
    } else {
      for (int c = lane; c < cnt; c += 64) stage[c] = T(0);
    }
  }
  __syncthreads();
  T* row = stage + lane * (REC ? K + 1 : R);
  const bool vec = sh.vec != 0;
  const float inv_r = 1.0f / (float)R;
  int prev_m = -1;  // dense stage: span of the window this lane wrote last
#pragma unroll
  for (int it = 0; it < kMaxIters; ++it) {
    if (it >= sh.iters) break;
    const int64_t nb = nbase + it * step;
    const int64_t nn = nb + sub;
    const bool ok = lane_ok && nn < sh.n;
    const T xv = xs[it];
    if (IMPL == 1) {
      const int m = ok ? knot_span(t, nk, xv) : -1;
      T v[K + 1];
#pragma unroll
      for (int j = 0; j <= K; ++j) v[j] = T(0);
      if (m >= 0) span_window<K, DER, T>(t, nk, m, xv, v);
      if (sh.scale != nullptr && m >= 0) {
        const T w = static_cast<const T*>(sh.scale)[nn * sh.I + i0 + fi];
#pragma unroll
        for (int j = 0; j <= K; ++j) v[j] *= w;
      }
      if (REC) {
#pragma unroll
        for (int j = 0; j <= K; ++j) row[j] = v[j];
        rec_r0[lane] = m >= 0 ? m - K : kNoWindow;
      } else {
        if (prev_m >= 0) {
#pragma unroll
          for (int j = 0; j <= K; ++j) {
            const int r = prev_m - K + j;
            if (r >= 0 && r < R) row[r] = T(0);
          }
        }
        if (m >= 0) {
#pragma unroll
          for (int j = 0; j <= K; ++j) {
            const int r = m - K + j;
            if (r >= 0 && r < R) row[r] = v[j];
          }
        }
        prev_m = m;
      }
    } else {
      if (ok) {
        dense_recurrence<T>(t, nk, xv, K, row);
      } else {
        for (int r = 0; r < R; ++r) row[r] = T(0);
      }
    }
    if (silu_out != nullptr && ok) silu_out[nn * sh.ld_aux + i0 + fi] = silu_of<T>(xv);
    wave_sync();
    for (int s = 0; s < sh.subs; ++s) {
      const int64_t ns = nb + s;
      if (ns >= sh.n) break;
      T* dst = out + ns * ld + (int64_t)i0 * R;
      if (REC)
        write_window_segment<K, T>(dst, stage + s * sh.fb * (K + 1), rec_r0 + s * sh.fb, fbv, R,
                                   inv_r, lane, vec);
      else
        move_row<T, true>(dst, stage + s * sh.fb * R, fbv * R, lane, vec);
    }
    wave_sync();
  }
}

// gx[n, i] = sum_r g[n, i*R + r] * dB_r/dx (+ gbase[n, i] * silu'(x)).
// The gradient segments are staged into LDS with coalesced 16-byte loads;
// each lane then reads the k+1 values of its span window (impl 1) or its
// whole row (impl 0).
// DER selects the derivative order contracted by impl 1 (0 = values).
template <int K, typename T, int IMPL, int DER = 1>
__global__ __launch_bounds__(kBasisThreads) void basis_grad_kernel(
    const T* __restrict__ x, const T* __restrict__ grid, const T* __restrict__ g, int64_t ld,
    const T* __restrict__ gbase, T* __restrict__ gx, BasisShape sh) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nk = sh.G + 2 * K + 1, R = sh.G + K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const BasisBlock bb = basis_block(sh);
  const int i0 = bb.f * sh.fb;
  const int fbv = min(sh.fb, sh.I - i0);
  T* knots = stage_knots<T>(smem, grid, i0, fbv, nk);
  T* stage = knots + round_up((int64_t)sh.fb * nk, 4) + wave * 64 * R;
  __syncthreads();

  const int sub = lane / sh.fb, fi = lane - sub * sh.fb;
  const bool lane_ok = sub < sh.subs && fi < fbv;
  const T* t = knots + fi * nk;
  const int64_t step = (int64_t)sh.waves * sh.subs;
  int64_t nbase = bb.g * sh.iters * step + (int64_t)wave * sh.subs;
  const T* row = stage + lane * R;
  const bool vec = sh.vec != 0;

  for (int it = 0; it < sh.iters; ++it, nbase += step) {
    for (int s = 0; s < sh.subs; ++s) {
      const int64_t ns = nbase + s;
      if (ns >= sh.n) break;
      move_row<T, false>(const_cast<T*>(g) + ns * ld + (int64_t)i0 * R, stage + s * sh.fb * R,
                         fbv * R, lane, vec);
    }
    const int64_t nn = nbase + sub;
    const bool ok = lane_ok && nn < sh.n;
    const T xv = ok ? x[nn * sh.I + i0 + fi] : T(0);
    const T gb = (ok && gbase != nullptr) ? gbase[nn * sh.ld_aux + i0 + fi] : T(0);
    __syncthreads();
    if (ok) {
      T acc = T(0);
      if (IMPL == 1) {
        const int m = knot_span(t, nk, xv);
        if (m >= 0) {
          T d[K + 1];
          span_window<K, DER, T>(t, nk, m, xv, d);
#pragma unroll
          for (int j = 0; j <= K; ++j) {
            const int r = m - K + j;
            if (r >= 0 && r < R) acc += row[r] * d[j];
          }
        }
      } else {
        T d[kMaxKnots];
        dense_derivative<T>(t, nk, xv, K, d);
        for (int r = 0; r < R; ++r) acc += row[r] * d[r];
      }
      if (gbase != nullptr) acc += gb * silu_deriv_of<T>(xv, DER);
      if (sh.scale != nullptr) acc *= static_cast<const T*>(sh.scale)[nn * sh.I + i0 + fi];
      gx[nn * sh.I + i0 + fi] = acc;
    }
    __syncthreads();
  }
}

// aug[n, i*R + r] = basis[n, i, r]; aug[n, I*R + i] = silu(x[n, i]).
template <typename T>
__global__ void pack_basis_kernel(const T* __restrict__ basis, const T* __restrict__ x,
                                  T* __restrict__ aug, int64_t ld, int64_t n, int64_t I,
                                  int64_t R, bool has_base) {
  const int64_t IR = I * R;
  const int64_t row_len = IR + (has_base ? I : 0);
  const int64_t total = n * row_len;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = e / row_len, c = e - r * row_len;
    aug[r * ld + c] = c < IR ? basis[r * IR + c] : silu_of<T>(x[r * I + (c - IR)]);
  }
}

// V consecutive elements through one 16-byte access (V > 1) or one element
template <typename T, int V>
__device__ __forceinline__ void pg_load(const T* __restrict__ p, T (&e)[V]) {
  if constexpr (V == 1) {
    e[0] = *p;
  } else {
    typedef T vt __attribute__((ext_vector_type(V)));
    const vt v = *reinterpret_cast<const vt*>(p);
#pragma unroll
    for (int j = 0; j < V; ++j) e[j] = v[j];
  }
}

template <typename T, int V>
__device__ __forceinline__ void pg_store(T* __restrict__ p, const T (&e)[V]) {
  if constexpr (V == 1) {
    *p = e[0];
  } else {
    typedef T vt __attribute__((ext_vector_type(V)));
    vt v;
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = e[j];
    *reinterpret_cast<vt*>(p) = v;
  }
}

// waug[o, i*R + r] = sw[o,i,r] * scaler[o,i]; waug[o, I*R + i] = bw[o,i];
// padding columns are zeroed.
template <typename T>
__device__ __forceinline__ T waug_value(const T* __restrict__ sw, const T* __restrict__ scaler,
                                        const T* __restrict__ bw, int64_t o, int c, int i, int r,
                                        int64_t I, int64_t IR, int R) {
  if (c < IR) {
    const T v = sw[o * IR + c];
    return scaler != nullptr ? v * scaler[o * I + i] : v;
  }
  if (bw != nullptr && c < IR + I) return bw[o * I + (c - IR)];
  return T(0);
}

// waug[o, c] for one row o (blockIdx.y, strided) and V consecutive columns
// per thread: 16 bytes and one store where the output is 16-byte aligned
// (rows then start aligned too: ld % 4 == 0), else V = 1.  A thread divides
// by R once; its next columns step the (feature, r) pair.
template <typename T, int V>
__global__ __launch_bounds__(256) void build_waug_kernel(
    const T* __restrict__ sw, const T* __restrict__ scaler, const T* __restrict__ bw,
    T* __restrict__ waug, int64_t ld, int64_t O, int64_t I, int64_t R) {
  const int64_t IR = I * R;
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * V;
  if (c0 >= ld) return;
  const int Ri = (int)R;
  const int f0 = c0 / Ri, r0 = c0 - f0 * Ri;
  for (int64_t o = blockIdx.y; o < O; o += gridDim.y) {
    T v[V];
    int f = f0, r = r0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      v[j] = waug_value<T>(sw, scaler, bw, o, c0 + j, f, r, I, IR, Ri);
      if (++r == Ri) {
        r = 0;
        ++f;
      }
    }
    pg_store<T, V>(waug + o * ld + c0, v);
  }
}

// Transposed augmented weight, waug_t[c, o] = waug[o, c] for the kaug
// columns c of [coef*scaler | base_weight], so that the input-side product
// E = D waug runs with both operands K-contiguous.  The product is formed as
// in build_waug_kernel (same rounding).  64x64 tiles are transposed through
// LDS so that reads (along c) and writes (along o) are both coalesced.
template <typename T>
__global__ __launch_bounds__(256) void build_waug_t_kernel(
    const T* __restrict__ sw, const T* __restrict__ scaler, const T* __restrict__ bw,
    T* __restrict__ waug_t, int64_t O, int64_t I, int64_t R, int64_t kaug) {
  __shared__ T tile[64][65];
  const int64_t c0 = (int64_t)blockIdx.x * 64, o0 = (int64_t)blockIdx.y * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t IR = I * R;
  const int Ri = (int)R, ci = (int)(c0 + tx);  // kaug < 2^31
  const int f = ci / Ri, r = ci - f * Ri;
#pragma unroll 4
  for (int j = 0; j < 16; ++j) {
    const int64_t o = o0 + ty + 4 * j;
    tile[ty + 4 * j][tx] =
        o < O && ci < kaug ? waug_value<T>(sw, scaler, bw, o, ci, f, r, I, IR, Ri) : T(0);
  }
  __syncthreads();
#pragma unroll 4
  for (int j = 0; j < 16; ++j) {
    const int64_t c = c0 + ty + 4 * j, o = o0 + tx;
    if (c < kaug && o < O) waug_t[c * O + o] = tile[tx][ty + 4 * j];
  }
}

// Parameter gradients from the (split) products G = D^T [H | s]:
//   gsw = scaler * G_H, gscaler = sum_r sw * G_H, gbw = G_s
// (csrc/kan_cuda.cu:576-598).  Split partials are summed in fixed order.
// A block owns kPairs consecutive (o, i) edges of one output row o: their
// kPairs*R partial values are contiguous, so the loads are coalesced.  The
// pass is a pure stream (splits + 1 reads and one write per element), so
// each thread keeps kPgUnroll vectors of V elements in flight per split;
// V = 16 bytes when the rows, split slices and pointers allow it, else 1;
// the host picks V only where V divides I*R, so V divides every block's
// np*R (= I*R - i0*R, with i0 a multiple of kPairs) and there is no tail.
// The per-edge sum over r goes through LDS rows of odd stride (conflict-free
// for the one-thread-per-edge reads), in r order.
constexpr int kPairs = 128;
constexpr int kPgThreads = 256;
constexpr int kPgUnroll = 2;

template <typename T, int V>
__global__ __launch_bounds__(kPgThreads) void param_grads_kernel(
    const T* __restrict__ part, int splits, int64_t split_stride, int64_t ld,
    const T* __restrict__ sw, const T* __restrict__ scaler, T* __restrict__ gsw,
    T* __restrict__ gscaler, T* __restrict__ gbw, int64_t O, int64_t I, int64_t R,
    int64_t blocks_per_row) {
  extern __shared__ __align__(16) unsigned char smem_pg[];
  const int rs = (int)(R | 1);  // LDS row stride
  T* prod = reinterpret_cast<T*>(smem_pg);
  T* sc = prod + kPairs * rs;
  const int64_t o = blockIdx.x / blocks_per_row;
  const int64_t i0 = (blockIdx.x - o * blocks_per_row) * (int64_t)kPairs;
  const int np = (int)min((int64_t)kPairs, I - i0);
  const int cnt = np * (int)R;
  const T* src = part + o * ld + i0 * R;
  const int64_t ebase = (o * I + i0) * R;
  const float inv_r = 1.0f / (float)R;
  if (gsw != nullptr || gscaler != nullptr) {
    if ((int)threadIdx.x < np)
      sc[threadIdx.x] = scaler != nullptr ? scaler[o * I + i0 + threadIdx.x] : T(1);
    __syncthreads();
    constexpr int kStep = kPgUnroll * kPgThreads * V;
    for (int c0 = (int)threadIdx.x * V; c0 < cnt; c0 += kStep) {
      T g[kPgUnroll][V], w[kPgUnroll][V];
#pragma unroll
      for (int u = 0; u < kPgUnroll; ++u) {
        const int c = c0 + u * kPgThreads * V;
        if (c < cnt) {
          pg_load<T, V>(src + c, g[u]);
          if (gscaler != nullptr) pg_load<T, V>(sw + ebase + c, w[u]);
        }
      }
      for (int s = 1; s < splits; ++s) {
        T h[kPgUnroll][V];
#pragma unroll
        for (int u = 0; u < kPgUnroll; ++u) {
          const int c = c0 + u * kPgThreads * V;
          if (c < cnt) pg_load<T, V>(src + s * split_stride + c, h[u]);
        }
#pragma unroll
        for (int u = 0; u < kPgUnroll; ++u) {
          const int c = c0 + u * kPgThreads * V;
          if (c < cnt) {
#pragma unroll
            for (int j = 0; j < V; ++j) g[u][j] += h[u][j];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kPgUnroll; ++u) {
        const int c = c0 + u * kPgThreads * V;
        if (c >= cnt) continue;
        T out[V];
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const int pr = small_div(c + j, inv_r);
          out[j] = sc[pr] * g[u][j];
          if (gscaler != nullptr) prod[pr * rs + (c + j - pr * (int)R)] = w[u][j] * g[u][j];
        }
        if (gsw != nullptr) {
          if (scaler != nullptr) pg_store<T, V>(gsw + ebase + c, out);
          else pg_store<T, V>(gsw + ebase + c, g[u]);
        }
      }
    }
    if (gscaler != nullptr) {
      __syncthreads();
      if ((int)threadIdx.x < np) {
        const T* row = prod + threadIdx.x * rs;
        T acc = T(0);
        for (int r = 0; r < (int)R; ++r) acc += row[r];
        gscaler[o * I + i0 + threadIdx.x] = acc;
      }
    }
  }
  if (gbw != nullptr && (int)threadIdx.x < np) {
    const T* bp = part + o * ld + I * R + i0 + threadIdx.x;
    T g = bp[0];
    for (int s = 1; s < splits; ++s) g += bp[s * split_stride];
    gbw[o * I + i0 + threadIdx.x] = g;
  }
}

// basis_grad_kernel for one sample per wave step (subs == 1) with 16-byte
// rows: the next step's gradient segment (and x, gbase) is loaded into
// registers while the current step is computed, and the stage hand-off uses
// wave-scope syncs only, so every wave keeps a segment load in flight.
// PV = 16-byte vectors per lane (the segment of fbv * R values is at most
// 64 * PV vectors).  Same arithmetic, in the same order, as basis_grad_kernel
// with impl 1.
template <int K, typename T, int DER, int PV>
__global__ __launch_bounds__(kBasisThreads) void basis_grad_pf_kernel(
    const T* __restrict__ x, const T* __restrict__ grid, const T* __restrict__ g, int64_t ld,
    const T* __restrict__ gbase, T* __restrict__ gx, BasisShape sh) {
  typedef typename V16<T>::type VT;
  constexpr int kV = V16<T>::kN;
  extern __shared__ __align__(16) unsigned char smem[];
  const int nk = sh.G + 2 * K + 1, R = sh.G + K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const BasisBlock bb = basis_block(sh);
  const int i0 = bb.f * sh.fb;
  const int fbv = min(sh.fb, sh.I - i0);
  T* knots = stage_knots<T>(smem, grid, i0, fbv, nk);
  T* stage = knots + round_up((int64_t)sh.fb * nk, 4) + wave * 64 * R;
  // the segment is segv whole vectors plus rem (< kV) trailing elements,
  // which a ragged last feature block can leave
  const int seg = fbv * R;
  const int segv = seg / kV, rem = seg - segv * kV;
  const bool lane_ok = lane < fbv;
  const int fi = lane_ok ? lane : 0;
  const T* t = knots + fi * nk;
  const int64_t step = sh.waves;
  int64_t nn = bb.g * sh.iters * step + wave;
  const T* row = stage + lane * R;
  VT pf[PV];
  T tail = T(0), xn = T(0), gbn = T(0);
  // loads of sample ns (clamped into the operand; rows past n are never used)
  auto issue = [&](int64_t ns) {
    const int64_t nc = ns < sh.n ? ns : sh.n - 1;
    const T* base = g + nc * ld + (int64_t)i0 * R;
    const VT* src = reinterpret_cast<const VT*>(base);
    if (segv > 0) {
#pragma unroll
      for (int j = 0; j < PV; ++j) {
        const int c = lane + 64 * j;
        pf[j] = src[c < segv ? c : segv - 1];
      }
    }
    if (rem > 0) tail = base[segv * kV + (lane < rem ? lane : 0)];
    xn = x[nc * sh.I + i0 + fi];
    gbn = gbase != nullptr ? gbase[nc * sh.ld_aux + i0 + fi] : T(0);
  };
  issue(nn);
  __syncthreads();  // knot rows staged
  for (int it = 0; it < sh.iters; ++it, nn += step) {
    wave_sync();  // the previous step's reads of the stage are done
#pragma unroll
    for (int j = 0; j < PV; ++j) {
      const int c = lane + 64 * j;
      if (c < segv) reinterpret_cast<VT*>(stage)[c] = pf[j];
    }
    if (lane < rem) stage[segv * kV + lane] = tail;
    const T xv = xn, gb = gbn;
    wave_sync();
    if (it + 1 < sh.iters && nn + step < sh.n) issue(nn + step);
    if (lane_ok && nn < sh.n) {
      T acc = T(0);
      const int m = knot_span(t, nk, xv);
      if (m >= 0) {
        T d[K + 1];
        span_window<K, DER, T>(t, nk, m, xv, d);
#pragma unroll
        for (int j = 0; j <= K; ++j) {
          const int r = m - K + j;
          if (r >= 0 && r < R) acc += row[r] * d[j];
        }
      }
      if (gbase != nullptr) acc += gb * silu_deriv_of<T>(xv, DER);
      if (sh.scale != nullptr) acc *= static_cast<const T*>(sh.scale)[nn * sh.I + i0 + lane];
      gx[nn * sh.I + i0 + lane] = acc;
    }
  }
}

// basis_grad for large grids (impl 1, R >= kWindowRecordMinR): each lane
// loads only the K+1 gradient values of its span window straight from
// global memory; the other R - K - 1 values of the item's row are never
// read, so the bytes fetched per item are the window's cache lines instead
// of the whole row.  No gradient staging in LDS (only the knot rows), so a
// CU holds many waves to cover the load latency; the next step's x is
// loaded while the current step is computed.  Same products in the same
// order as basis_grad_pf_kernel (a window entry outside 0..R-1 adds +0).
template <int K, typename T, int DER>
__global__ __launch_bounds__(kBasisThreads) void basis_grad_window_kernel(
    const T* __restrict__ x, const T* __restrict__ grid, const T* __restrict__ g, int64_t ld,
    const T* __restrict__ gbase, T* __restrict__ gx, BasisShape sh) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nk = sh.G + 2 * K + 1, R = sh.G + K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const BasisBlock bb = basis_block(sh);
  const int i0 = bb.f * sh.fb;
  const int fbv = min(sh.fb, sh.I - i0);
  T* knots = stage_knots<T>(smem, grid, i0, fbv, nk);
  const int sub = lane / sh.fb, fi = lane - sub * sh.fb;
  const bool lane_ok = sub < sh.subs && fi < fbv;
  const T* t = knots + (lane_ok ? fi : 0) * nk;
  const int64_t step = (int64_t)sh.waves * sh.subs;
  int64_t nn = bb.g * sh.iters * step + (int64_t)wave * sh.subs + sub;
  const int64_t col = (int64_t)i0 + (lane_ok ? fi : 0);
  T xn = (lane_ok && nn < sh.n) ? x[nn * sh.I + col] : T(0);
  __syncthreads();  // knot rows staged
  for (int it = 0; it < sh.iters; ++it, nn += step) {
    const bool ok = lane_ok && nn < sh.n;
    const T xv = xn;
    const int m = ok ? knot_span(t, nk, xv) : -1;
    const T* grow = g + nn * ld + col * R;  // dereferenced only inside the window
    T gw[K + 1];
#pragma unroll
    for (int j = 0; j <= K; ++j) {
      const int r = m - K + j;
      gw[j] = (m >= 0 && r >= 0 && r < R) ? grow[r] : T(0);
    }
    const T gb = (ok && gbase != nullptr) ? gbase[nn * sh.ld_aux + col] : T(0);
    const int64_t nx = nn + step;
    xn = (it + 1 < sh.iters && lane_ok && nx < sh.n) ? x[nx * sh.I + col] : T(0);
    if (ok) {
      T acc = T(0);
      if (m >= 0) {
        T d[K + 1];
        span_window<K, DER, T>(t, nk, m, xv, d);
#pragma unroll
        for (int j = 0; j <= K; ++j) acc += gw[j] * d[j];
      }
      if (gbase != nullptr) acc += gb * silu_grad_of<T>(xv);
      gx[nn * sh.I + col] = acc;
    }
  }
}

// Input gradient from the compact input-side product: Ew [n, I, K+1]
// (window slot j of item (n, i)) and Es [n, I].  The same products in the
// same order as basis_grad_window_kernel (a slot outside 0..R-1 adds +0), so
// the result equals the route through the full E.  An item's slots lie at a
// fixed place whatever its span, so the next step's window values, base
// value and x are all loaded while the current step is computed (one
// 16-byte load for the window with k = 3).
template <int K>
__global__ __launch_bounds__(kBasisThreads) void basis_grad_compact_kernel(
    const float* __restrict__ x, const float* __restrict__ grid, const float* __restrict__ ew,
    const float* __restrict__ es, float* __restrict__ gx, BasisShape sh) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int nk = sh.G + 2 * K + 1, R = sh.G + K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const BasisBlock bb = basis_block(sh);
  const int i0 = bb.f * sh.fb;
  const int fbv = min(sh.fb, sh.I - i0);
  float* knots = stage_knots<float>(smem, grid, i0, fbv, nk);
  const int sub = lane / sh.fb, fi = lane - sub * sh.fb;
  const bool lane_ok = sub < sh.subs && fi < fbv;
  const float* t = knots + (lane_ok ? fi : 0) * nk;
  const int64_t step = (int64_t)sh.waves * sh.subs;
  int64_t nn = bb.g * sh.iters * step + (int64_t)wave * sh.subs + sub;
  const int64_t col = (int64_t)i0 + (lane_ok ? fi : 0);
  typedef float f4 __attribute__((ext_vector_type(4)));
  float xn = 0.0f, bn = 0.0f, wn[K + 1];
  auto fetch = [&](int64_t n_, bool ok_) {
    const int64_t e = n_ * sh.I + col;
    xn = ok_ ? x[e] : 0.0f;
    if constexpr (K == 3) {
      const f4 v = ok_ ? *reinterpret_cast<const f4*>(ew + e * 4) : f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 4; ++j) wn[j] = v[j];
    } else {
#pragma unroll
      for (int j = 0; j <= K; ++j) wn[j] = ok_ ? ew[e * (K + 1) + j] : 0.0f;
    }
    bn = (ok_ && es != nullptr) ? es[e] : 0.0f;
  };
  fetch(nn, lane_ok && nn < sh.n);
  __syncthreads();  // knot rows staged
  for (int it = 0; it < sh.iters; ++it, nn += step) {
    const bool ok = lane_ok && nn < sh.n;
    const float xv = xn, gb = bn;
    float gw[K + 1];
#pragma unroll
    for (int j = 0; j <= K; ++j) gw[j] = wn[j];
    const int64_t nx = nn + step;
    fetch(nx, it + 1 < sh.iters && lane_ok && nx < sh.n);
    if (ok) {
      const int m = knot_span(t, nk, xv);
      float acc = 0.0f;
      if (m >= 0) {
        float d[K + 1];
        span_window<K, 1, float>(t, nk, m, xv, d);
#pragma unroll
        for (int j = 0; j <= K; ++j) {
          const int r = m - K + j;
          acc += (r >= 0 && r < R ? gw[j] : 0.0f) * d[j];
        }
      }
      if (es != nullptr) acc += gb * silu_grad_of<float>(xv);
      gx[nn * sh.I + col] = acc;
    }
  }
}

// Register vectors per lane the prefetching kernel needs (0 = not eligible).
template <typename T>
int grad_pf_vectors(const BasisShape& sh, int R) {
  if (sh.subs != 1 || !sh.vec) return 0;
  constexpr int kV = 16 / (int)sizeof(T);
  const int per_lane = (int)ceil_div((int64_t)sh.fb * R / kV, 64);
  if (per_lane <= 4) return 4;
  if (per_lane <= 8) return 8;
  if (per_lane <= 18) return 18;
  return 0;
}

BasisShape make_shape(int64_t n, int64_t I, int G, int R, size_t elem, int64_t ld,
                      const void* rows_ptr, int64_t* blocks_y, bool dense_stage = true) {
  BasisShape sh;
  sh.n = n;
  sh.I = (int)I;
  sh.G = G;
  sh.ld_aux = ld;
  sh.fb = (int)(I < 64 ? I : 64);
  sh.nfb = (int)ceil_div(I, sh.fb);
  sh.scale = nullptr;
  sh.subs = 64 / sh.fb;
  sh.waves = 4;
  // a dense R-row stage per lane bounds the waves of a block by LDS
  while (dense_stage && sh.waves > 1 && (size_t)sh.waves * 64 * R * elem > 48 * 1024)
    sh.waves /= 2;
  // 16-byte vectors: the output rows, each block's feature offset and each
  // staged sample segment must all start 16-byte aligned.
  const int64_t v = 16 / (int64_t)elem;
  sh.vec = ((reinterpret_cast<uintptr_t>(rows_ptr) % 16) == 0) && (ld % v == 0) &&
           (((int64_t)sh.fb * R) % v == 0);
  const int64_t per_step = (int64_t)sh.waves * sh.subs;
  const int64_t steps = ceil_div(n, per_step);
  // Aim for ~4 steps per block (at most kMaxIters), but keep enough blocks
  // to fill the chip.
  const int64_t fblocks = ceil_div(I, sh.fb);
  int64_t iters = 4;
  static_assert(kMaxIters >= 4, "basis_kernel holds up to kMaxIters steps of x per wave");
  while (iters > 1 && fblocks * ceil_div(steps, iters) < 8192) iters /= 2;
  sh.iters = (int)iters;
  *blocks_y = ceil_div(steps, iters);
  return sh;
}

template <typename T>
size_t basis_smem(const BasisShape& sh, int nk, int R) {
  return sizeof(T) * (round_up((int64_t)sh.fb * nk, 4) + (int64_t)sh.waves * 64 * R);
}

// LDS of basis_kernel with impl 1: knots, K+1 window values and the window
// start per lane.
template <typename T>
size_t basis_window_smem(const BasisShape& sh, int nk, int k) {
  return sizeof(T) * (round_up((int64_t)sh.fb * nk, 4) + (int64_t)sh.waves * 64 * (k + 1)) +
         sizeof(int) * (size_t)sh.waves * 64;
}

inline int gs_blocks(int64_t total) {
  int64_t b = ceil_div(total, 256);
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace

template <typename T>
int launch_basis(const T* x, const T* grid, T* out, int64_t ld_out, T* silu_out, int64_t n,
                 int64_t I, int G, int k, int impl, hipStream_t st, int64_t ld_silu) {
  if (n == 0 || I == 0) return KAN_OK;
  const int R = G + k, nk = G + 2 * k + 1;
  const bool rec = impl == 1 && R >= kWindowRecordMinR;
  int64_t by = 0;
  BasisShape sh = make_shape(n, I, G, R, sizeof(T), ld_out, out, &by, !rec);
  if (ld_silu >= 0) sh.ld_aux = ld_silu;
  if (sh.nfb * by > 2147483647LL) return set_error(KAN_ERR_LIMIT, "basis: too many samples (%lld)", (long long)n);
  const dim3 grid_dim((unsigned)(sh.nfb * by));
  const size_t smem = rec ? basis_window_smem<T>(sh, nk, k) : basis_smem<T>(sh, nk, R);
  // algorithmic bytes: read x, write the R basis values (+ silu) per item
  TimedLaunch timed(kClassBasis, st,
                    (double)sizeof(T) * (double)n * (double)I * (1.0 + R + (silu_out ? 1 : 0)));
#define KAN_BASIS_LAUNCH(KK, IM, RC)                                                     \
  hipLaunchKernelGGL((basis_kernel<KK, T, IM, 0, RC>), grid_dim, dim3(64 * sh.waves), smem, \
                     st, x, grid, out, ld_out, silu_out, sh)
  if (rec) {
    if (k == 1) KAN_BASIS_LAUNCH(1, 1, true);
    else if (k == 2) KAN_BASIS_LAUNCH(2, 1, true);
    else KAN_BASIS_LAUNCH(3, 1, true);
  } else if (impl == 1) {
    if (k == 1) KAN_BASIS_LAUNCH(1, 1, false);
    else if (k == 2) KAN_BASIS_LAUNCH(2, 1, false);
    else KAN_BASIS_LAUNCH(3, 1, false);
  } else {
    if (k == 1) KAN_BASIS_LAUNCH(1, 0, false);
    else if (k == 2) KAN_BASIS_LAUNCH(2, 0, false);
    else KAN_BASIS_LAUNCH(3, 0, false);
  }
#undef KAN_BASIS_LAUNCH
  return check_launch("basis");
}

// Prefetching contraction (impl 1, order DER) when the shape allows it; returns
// false (nothing launched) otherwise.
template <typename T, int DER>
bool launch_grad_pf(const T* x, const T* grid, const T* gH, int64_t ld_g, const T* gbase, T* gx,
                    int64_t n, int64_t I, int G, int k, hipStream_t st, int* rc,
                    int64_t ld_base = -1, const T* scale = nullptr) {
  if (k < DER) return false;
  const int R = G + k, nk = G + 2 * k + 1;
  int64_t by = 0;
  BasisShape sh = make_shape(n, I, G, R, sizeof(T), ld_g, gH, &by);
  if (ld_base >= 0) sh.ld_aux = ld_base;
  sh.scale = scale;
  const int pv = grad_pf_vectors<T>(sh, R);
  if (pv == 0) return false;
  // two steps per block: more blocks in flight, each still overlapping one load
  const int64_t steps = ceil_div(n, (int64_t)sh.waves);
  sh.iters = 2;
  by = ceil_div(steps, (int64_t)sh.iters);
  if (sh.nfb * by > 2147483647LL) {
    *rc = set_error(KAN_ERR_LIMIT, "basis_grad: too many samples");
    return true;
  }
  const dim3 grid_dim((unsigned)(sh.nfb * by));
  const size_t smem = basis_smem<T>(sh, nk, R);
#define KAN_BGPF(KK, PVV)                                                                         \
  hipLaunchKernelGGL((basis_grad_pf_kernel<KK, T, DER, PVV>), grid_dim, dim3(64 * sh.waves), smem, \
                     st, x, grid, gH, ld_g, gbase, gx, sh)
#define KAN_BGPF_K(KK)                    \
  do {                                    \
    if (pv == 4) KAN_BGPF(KK, 4);         \
    else if (pv == 8) KAN_BGPF(KK, 8);    \
    else KAN_BGPF(KK, 18);                \
  } while (0)
  if (k == 1) {
    if constexpr (DER <= 1) KAN_BGPF_K(1);
  } else if (k == 2) {
    if constexpr (DER <= 2) KAN_BGPF_K(2);
  } else {
    KAN_BGPF_K(3);
  }
#undef KAN_BGPF_K
#undef KAN_BGPF
  *rc = check_launch("basis_grad");
  return true;
}

// Input gradient from the compact input-side product (fp32, local basis):
// gx[n, i] = sum_j Ew[n, i, j] dB_{m-k+j}/dx + Es[n, i] silu'(x).
int launch_basis_grad_compact(const float* x, const float* grid, const float* ew,
                              const float* es, float* gx, int64_t n, int64_t I, int G, int k,
                              hipStream_t st) {
  if (n == 0 || I == 0) return KAN_OK;
  if (k < 1 || k > 3) return set_error(KAN_ERR_INVALID, "basis_grad_compact: spline order 1..3");
  if ((reinterpret_cast<uintptr_t>(ew) & 15) != 0)
    return set_error(KAN_ERR_INVALID, "basis_grad_compact: window values must be 16-byte aligned");
  const int R = G + k, nk = G + 2 * k + 1;
  // algorithmic bytes: read x, the k+1 window values (+ base), write gx
  TimedLaunch timed(kClassBasisGrad, st,
                    4.0 * (double)n * (double)I * (2.0 + (k + 1) + (es ? 1 : 0)));
  int64_t by = 0;
  BasisShape sh = make_shape(n, I, G, R, sizeof(float), 0, ew, &by, false);
  if (sh.nfb * by > 2147483647LL) return set_error(KAN_ERR_LIMIT, "basis_grad: too many samples");
  const dim3 grid_dim((unsigned)(sh.nfb * by));
  const size_t smem = sizeof(float) * (size_t)round_up((int64_t)sh.fb * nk, 4);
#define KAN_BGC(KK)                                                                           \
  hipLaunchKernelGGL((basis_grad_compact_kernel<KK>), grid_dim, dim3(64 * sh.waves), smem, st, \
                     x, grid, ew, es, gx, sh)
  if (k == 1) KAN_BGC(1);
  else if (k == 2) KAN_BGC(2);
  else KAN_BGC(3);
#undef KAN_BGC
  return check_launch("basis_grad_compact");
}

template <typename T>
int launch_basis_grad(const T* x, const T* grid, const T* gH, int64_t ld_g, const T* gbase,
                      T* gx, int64_t n, int64_t I, int G, int k, int impl, hipStream_t st,
                      int64_t ld_base) {
  if (n == 0 || I == 0) return KAN_OK;
  const int R = G + k, nk = G + 2 * k + 1;
  // algorithmic bytes: read x and the R gradient values (+ base), write gx
  TimedLaunch timed(kClassBasisGrad, st,
                    (double)sizeof(T) * (double)n * (double)I * (2.0 + R + (gbase ? 1 : 0)));
  int rc = KAN_OK;
  if (impl == 1 && R >= kWindowRecordMinR) {
    int64_t by = 0;
    BasisShape sh = make_shape(n, I, G, R, sizeof(T), ld_g, gH, &by, false);
    if (ld_base >= 0) sh.ld_aux = ld_base;
    if (sh.nfb * by > 2147483647LL) return set_error(KAN_ERR_LIMIT, "basis_grad: too many samples");
    const dim3 grid_dim((unsigned)(sh.nfb * by));
    const size_t smem = sizeof(T) * (size_t)round_up((int64_t)sh.fb * nk, 4);
#define KAN_BGW(KK)                                                                        \
  hipLaunchKernelGGL((basis_grad_window_kernel<KK, T, 1>), grid_dim, dim3(64 * sh.waves), \
                     smem, st, x, grid, gH, ld_g, gbase, gx, sh)
    if (k == 1) KAN_BGW(1);
    else if (k == 2) KAN_BGW(2);
    else KAN_BGW(3);
#undef KAN_BGW
    return check_launch("basis_grad");
  }
  if (impl == 1 && launch_grad_pf<T, 1>(x, grid, gH, ld_g, gbase, gx, n, I, G, k, st, &rc,
                                        ld_base))
    return rc;
  int64_t by = 0;
  BasisShape sh = make_shape(n, I, G, R, sizeof(T), ld_g, gH, &by);
  if (ld_base >= 0) sh.ld_aux = ld_base;
  if (sh.nfb * by > 2147483647LL) return set_error(KAN_ERR_LIMIT, "basis_grad: too many samples");
  const dim3 grid_dim((unsigned)(sh.nfb * by));
  const size_t smem = basis_smem<T>(sh, nk, R);
#define KAN_BGRAD_LAUNCH(KK, IM)                                                             \
  hipLaunchKernelGGL((basis_grad_kernel<KK, T, IM>), grid_dim, dim3(64 * sh.waves), smem, st, \
                     x, grid, gH, ld_g, gbase, gx, sh)
  if (impl == 1) {
    if (k == 1) KAN_BGRAD_LAUNCH(1, 1);
    else if (k == 2) KAN_BGRAD_LAUNCH(2, 1);
    else KAN_BGRAD_LAUNCH(3, 1);
  } else {
    if (k == 1) KAN_BGRAD_LAUNCH(1, 0);
    else if (k == 2) KAN_BGRAD_LAUNCH(2, 0);
    else KAN_BGRAD_LAUNCH(3, 0);
  }
#undef KAN_BGRAD_LAUNCH
  return check_launch("basis_grad");
}

namespace {
template <typename T>
__global__ void zero_fill_kernel(T* __restrict__ out, int64_t count) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x)
    out[e] = T(0);
}

// out[e] = silu^(q)(x[e]) * w1[e] * w2[e] (factors optional)
template <typename T>
__global__ void silu_deriv_kernel(const T* __restrict__ x, const T* __restrict__ w1,
                                  const T* __restrict__ w2, T* __restrict__ out, int64_t count,
                                  int q) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    T v = silu_deriv_of<T>(x[e], q);
    if (w1 != nullptr) v *= w1[e];
    if (w2 != nullptr) v *= w2[e];
    out[e] = v;
  }
}
}  // namespace

template <typename T>
int launch_silu_deriv(const T* x, const T* w1, const T* w2, T* out, int64_t count, int order,
                      hipStream_t st) {
  if (count == 0) return KAN_OK;
  if (order < 0 || order > kMaxSiluOrder)
    return set_error(KAN_ERR_INVALID, "silu_deriv: order must lie in 0..%d, got %d",
                     kMaxSiluOrder, order);
  TimedLaunch timed(kClassOther, st,
                    (double)sizeof(T) * (double)count * (2.0 + (w1 ? 1 : 0) + (w2 ? 1 : 0)));
  hipLaunchKernelGGL(silu_deriv_kernel<T>, dim3(gs_blocks(count)), dim3(256), 0, st, x, w1, w2,
                     out, count, order);
  return check_launch("silu_deriv");
}

template int launch_silu_deriv<float>(const float*, const float*, const float*, float*, int64_t,
                                      int, hipStream_t);
template int launch_silu_deriv<double>(const double*, const double*, const double*, double*,
                                       int64_t, int, hipStream_t);

template <typename T>
int launch_basis_deriv(const T* x, const T* grid, const T* scale, T* out, int64_t n, int64_t I,
                       int G, int k, int order, hipStream_t st) {
  if (n == 0 || I == 0) return KAN_OK;
  const int R = G + k, nk = G + 2 * k + 1;
  if (order > k) {  // a degree-k piecewise polynomial: zero almost everywhere
    hipLaunchKernelGGL(zero_fill_kernel<T>, dim3(gs_blocks(n * I * R)), dim3(256), 0, st, out,
                       n * I * R);
    return check_launch("basis_deriv (zero)");
  }
  const bool rec = R >= kWindowRecordMinR;
  int64_t by = 0;
  BasisShape sh = make_shape(n, I, G, R, sizeof(T), I * R, out, &by, !rec);
  sh.scale = scale;
  if (sh.nfb * by > 2147483647LL) return set_error(KAN_ERR_LIMIT, "basis_deriv: too many samples");
  const dim3 grid_dim((unsigned)(sh.nfb * by));
  const size_t smem = rec ? basis_window_smem<T>(sh, nk, k) : basis_smem<T>(sh, nk, R);
  TimedLaunch timed(kClassBasis, st, (double)sizeof(T) * (double)n * (double)I * (1.0 + R));
#define KAN_BDER_LAUNCH(KK, DD)                                                                \
  do {                                                                                         \
    if (rec)                                                                                   \
      hipLaunchKernelGGL((basis_kernel<KK, T, 1, DD, true>), grid_dim, dim3(64 * sh.waves),    \
                         smem, st, x, grid, out, (int64_t)I * R, (T*)nullptr, sh);             \
    else                                                                                       \
      hipLaunchKernelGGL((basis_kernel<KK, T, 1, DD, false>), grid_dim, dim3(64 * sh.waves),   \
                         smem, st, x, grid, out, (int64_t)I * R, (T*)nullptr, sh);             \
  } while (0)
  if (k == 1) {
    if (order == 0) KAN_BDER_LAUNCH(1, 0);
    else KAN_BDER_LAUNCH(1, 1);
  } else if (k == 2) {
    if (order == 0) KAN_BDER_LAUNCH(2, 0);
    else if (order == 1) KAN_BDER_LAUNCH(2, 1);
    else KAN_BDER_LAUNCH(2, 2);
  } else {
    if (order == 0) KAN_BDER_LAUNCH(3, 0);
    else if (order == 1) KAN_BDER_LAUNCH(3, 1);
    else if (order == 2) KAN_BDER_LAUNCH(3, 2);
    else KAN_BDER_LAUNCH(3, 3);
  }
#undef KAN_BDER_LAUNCH
  return check_launch("basis_deriv");
}

template <typename T>
int launch_basis_deriv_contract(const T* x, const T* grid, const T* gH, const T* gbase,
                                const T* scale, T* gx, int64_t n, int64_t I, int G, int k,
                                int order, hipStream_t st) {
  if (n == 0 || I == 0) return KAN_OK;
  const int R = G + k, nk = G + 2 * k + 1;
  if (order > k) {  // the spline part is zero; the base part (if any) remains
    if (gbase != nullptr) return launch_silu_deriv<T>(x, gbase, scale, gx, n * I, order, st);
    hipLaunchKernelGGL(zero_fill_kernel<T>, dim3(gs_blocks(n * I)), dim3(256), 0, st, gx, n * I);
    return check_launch("basis_deriv_contract (zero)");
  }
  TimedLaunch timed(kClassBasisGrad, st,
                    (double)sizeof(T) * (double)n * (double)I *
                        (2.0 + R + (gbase ? 1 : 0) + (scale ? 1 : 0)));
  int rc = KAN_OK;
  const int64_t lb = I;  // gbase is [n, I]
  if ((order == 0 &&
       launch_grad_pf<T, 0>(x, grid, gH, I * R, gbase, gx, n, I, G, k, st, &rc, lb, scale)) ||
      (order == 1 &&
       launch_grad_pf<T, 1>(x, grid, gH, I * R, gbase, gx, n, I, G, k, st, &rc, lb, scale)) ||
      (order == 2 &&
       launch_grad_pf<T, 2>(x, grid, gH, I * R, gbase, gx, n, I, G, k, st, &rc, lb, scale)) ||
      (order == 3 &&
       launch_grad_pf<T, 3>(x, grid, gH, I * R, gbase, gx, n, I, G, k, st, &rc, lb, scale)))
    return rc;
  int64_t by = 0;
  BasisShape sh = make_shape(n, I, G, R, sizeof(T), I * R, gH, &by);
  sh.ld_aux = I;
  sh.scale = scale;
  if (sh.nfb * by > 2147483647LL) return set_error(KAN_ERR_LIMIT, "basis_deriv_contract: too many samples");
  const dim3 grid_dim((unsigned)(sh.nfb * by));
  const size_t smem = basis_smem<T>(sh, nk, R);
#define KAN_BDC_LAUNCH(KK, DD)                                                                  \
  hipLaunchKernelGGL((basis_grad_kernel<KK, T, 1, DD>), grid_dim, dim3(64 * sh.waves), smem, st, \
                     x, grid, gH, (int64_t)I * R, gbase, gx, sh)
  if (k == 1) {
    if (order == 0) KAN_BDC_LAUNCH(1, 0);
    else KAN_BDC_LAUNCH(1, 1);
  } else if (k == 2) {
    if (order == 0) KAN_BDC_LAUNCH(2, 0);
    else if (order == 1) KAN_BDC_LAUNCH(2, 1);
    else KAN_BDC_LAUNCH(2, 2);
  } else {
    if (order == 0) KAN_BDC_LAUNCH(3, 0);
    else if (order == 1) KAN_BDC_LAUNCH(3, 1);
    else if (order == 2) KAN_BDC_LAUNCH(3, 2);
    else KAN_BDC_LAUNCH(3, 3);
  }
#undef KAN_BDC_LAUNCH
  return check_launch("basis_deriv_contract");
}

template int launch_basis_deriv<float>(const float*, const float*, const float*, float*,
                                       int64_t, int64_t, int, int, int, hipStream_t);
template int launch_basis_deriv<double>(const double*, const double*, const double*, double*,
                                        int64_t, int64_t, int, int, int, hipStream_t);
template int launch_basis_deriv_contract<float>(const float*, const float*, const float*,
                                                const float*, const float*, float*, int64_t,
                                                int64_t, int, int, int, hipStream_t);
template int launch_basis_deriv_contract<double>(const double*, const double*, const double*,
                                                 const double*, const double*, double*, int64_t,
                                                 int64_t, int, int, int, hipStream_t);

template <typename T>
int launch_pack_basis(const T* basis, const T* x, T* aug, int64_t ld_aug, int64_t n, int64_t I,
                      int64_t R, bool has_base, hipStream_t st) {
  const int64_t total = n * (I * R + (has_base ? I : 0));
  if (total == 0) return KAN_OK;
  TimedLaunch timed(kClassOther, st, 0.0);
  hipLaunchKernelGGL((pack_basis_kernel<T>), dim3(gs_blocks(total)), dim3(256), 0, st, basis, x,
                     aug, ld_aug, n, I, R, has_base);
  return check_launch("pack_basis");
}

template <typename T>
int launch_build_waug(const T* sw, const T* scaler, const T* bw, T* waug, int64_t ld, int64_t O,
                      int64_t I, int64_t R, hipStream_t st) {
  if (O * ld == 0) return KAN_OK;
  if (ld > (1LL << 30)) return set_error(KAN_ERR_LIMIT, "build_weight_aug: rows too long");
  constexpr int V = 16 / (int)sizeof(T);
  const bool vec = (reinterpret_cast<uintptr_t>(waug) & 15) == 0 && ld % V == 0;
  const unsigned gy = (unsigned)std::min<int64_t>(O, 65535);
  TimedLaunch timed(kClassOther, st, 0.0);
  if (vec)
    hipLaunchKernelGGL((build_waug_kernel<T, V>), dim3((unsigned)ceil_div(ld, 256 * V), gy),
                       dim3(256), 0, st, sw, scaler, bw, waug, ld, O, I, R);
  else
    hipLaunchKernelGGL((build_waug_kernel<T, 1>), dim3((unsigned)ceil_div(ld, 256), gy), dim3(256),
                       0, st, sw, scaler, bw, waug, ld, O, I, R);
  return check_launch("build_weight_aug");
}

template <typename T>
int launch_build_waug_t(const T* sw, const T* scaler, const T* bw, T* waug_t, int64_t kaug,
                        int64_t O, int64_t I, int64_t R, hipStream_t st) {
  if (kaug * O == 0) return KAN_OK;
  const int64_t bx = ceil_div(kaug, 64), by = ceil_div(O, 64);
  if (bx > 2147483647LL || by > 65535) return set_error(KAN_ERR_LIMIT, "build_waug_t: too large");
  TimedLaunch timed(kClassOther, st, 0.0);
  hipLaunchKernelGGL((build_waug_t_kernel<T>), dim3((unsigned)bx, (unsigned)by), dim3(256), 0, st,
                     sw, scaler, bw, waug_t, O, I, R, kaug);
  return check_launch("build_weight_aug_t");
}

template <typename T>
int launch_param_grads(const T* part, int splits, int64_t split_stride, int64_t ld, const T* sw,
                       const T* scaler, T* gsw, T* gscaler, T* gbw, int64_t O, int64_t I,
                       int64_t R, hipStream_t st) {
  if (O * I == 0) return KAN_OK;
  const int64_t per_row = ceil_div(I, kPairs);
  const int64_t blocks = O * per_row;
  if (blocks > 2147483647LL) return set_error(KAN_ERR_LIMIT, "param_grads: too many edges");
  // 16-byte vectors when every row start, split slice and edge run is aligned
  constexpr int V = 16 / (int)sizeof(T);
  auto al = [](const void* q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool vec = ld % V == 0 && split_stride % V == 0 && (I * R) % V == 0 && al(part) &&
                   al(sw) && al(gsw);
  const size_t lds = sizeof(T) * (size_t)kPairs * (size_t)((R | 1) + 1);
  TimedLaunch timed(kClassOther, st, 0.0);
  if (vec)
    hipLaunchKernelGGL((param_grads_kernel<T, V>), dim3((unsigned)blocks), dim3(kPgThreads), lds,
                       st, part, splits, split_stride, ld, sw, scaler, gsw, gscaler, gbw, O, I, R,
                       per_row);
  else
    hipLaunchKernelGGL((param_grads_kernel<T, 1>), dim3((unsigned)blocks), dim3(kPgThreads), lds,
                       st, part, splits, split_stride, ld, sw, scaler, gsw, gscaler, gbw, O, I, R,
                       per_row);
  return check_launch("param_grads");
}

#define KAN_INST(T)                                                                          \
  template int launch_basis<T>(const T*, const T*, T*, int64_t, T*, int64_t, int64_t, int, int, \
                               int, hipStream_t, int64_t);                                   \
  template int launch_basis_grad<T>(const T*, const T*, const T*, int64_t, const T*, T*,       \
                                    int64_t, int64_t, int, int, int, hipStream_t, int64_t);  \
  template int launch_pack_basis<T>(const T*, const T*, T*, int64_t, int64_t, int64_t,        \
                                    int64_t, bool, hipStream_t);                             \
  template int launch_build_waug<T>(const T*, const T*, const T*, T*, int64_t, int64_t,       \
                                    int64_t, int64_t, hipStream_t);                          \
  template int launch_build_waug_t<T>(const T*, const T*, const T*, T*, int64_t, int64_t,     \
                                      int64_t, int64_t, hipStream_t);                        \
  template int launch_param_grads<T>(const T*, int, int64_t, int64_t, const T*, const T*, T*, \
                                     T*, T*, int64_t, int64_t, int64_t, hipStream_t);
KAN_INST(float)
KAN_INST(double)
#undef KAN_INST

}  // namespace kan
