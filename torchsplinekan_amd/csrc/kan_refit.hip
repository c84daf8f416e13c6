// Gram matrices of the least-squares refit of a layer's spline curves onto a
// new knot grid (KANLinear.update_grid and extend_grid).  For input feature i
// and samples x[b, i], with bn = the order-k basis on the new grid (Rn values)
// and bo = the basis on the old grid (Ro values):
//   G[i] = sum_b bn(b) bn(b)^T      [Rn, Rn]   (normal matrix A^T A)
//   C[i] = sum_b bn(b) bo(b)^T      [Rn, Ro]   (cross term)
// The refit right-hand side of the reference, A^T y_old with
// y_old[o, b, i] = sum_s coef[o, i, s] bo_s(b), equals C[i] coef[o, i, :]^T,
// so the [O, B, I] curve tensor of spline_kan/reference_backend.py:483-484 and
// kan_linear.py:580-581 is never formed: the samples are streamed once and
// each contributes (k+1)^2 products to G and to C.
//
// Work mapping: one workgroup per feature.  The workgroup's threads own the
// entries of G's upper band (|r - s| <= k, the only non-zero ones) and of C.
// Samples are taken 256 at a time: each thread evaluates one sample's spans
// and values on both grids (knot rows in LDS) and stages them in LDS; then
// every thread adds, for each entry it owns, the chunk's contributions in
// sample order.  Each entry is summed by one thread in a fixed order, in
// float64, so the result is deterministic.

#include "kan_common.h"
#include "kan_spline.h"

namespace kan {
namespace {

constexpr int kRefitThreads = 256;
// Entries owned per thread: ceil((Rn (k+1) + Rn Ro) / 256) <= ceil((70*4 + 70*70) / 256) = 21.
constexpr int kRefitMaxOwn = 21;

// MO = entries owned per thread (compile time, so the accumulators stay in
// registers); the launcher picks the smallest MO that covers the matrices.
template <int K, typename T, int MO>
__global__ __launch_bounds__(kRefitThreads) void refit_gram_kernel(
    const T* __restrict__ xt, const T* __restrict__ grid_old, const T* __restrict__ grid_new,
    double* __restrict__ gram, double* __restrict__ cross, int64_t n, int Go, int Gn) {
  __shared__ T knots_o[kMaxKnots];
  __shared__ T knots_n[kMaxKnots];
  __shared__ int span_n[kRefitThreads];
  __shared__ int span_o[kRefitThreads];
  __shared__ double val_n[kRefitThreads][K + 1];
  __shared__ double val_o[kRefitThreads][K + 1];
  const int i = blockIdx.x;
  const int t = threadIdx.x;
  const int nko = Go + 2 * K + 1, nkn = Gn + 2 * K + 1;
  const int Ro = Go + K, Rn = Gn + K;
  if (t < nko) knots_o[t] = grid_old[(int64_t)i * nko + t];
  if (t < nkn) knots_n[t] = grid_new[(int64_t)i * nkn + t];

  // owned entries: e < Rn*(K+1) is G[r, r+d] (d = e % (K+1)), else C[r, s]
  const int eg_count = Rn * (K + 1);
  const int e_total = eg_count + Rn * Ro;
  int er[MO], es[MO];
  bool is_g[MO];
  double acc[MO];
#pragma unroll
  for (int j = 0; j < MO; ++j) {
    const int e = t + kRefitThreads * j;
    acc[j] = 0.0;
    is_g[j] = e < eg_count;
    if (e < eg_count) {
      er[j] = e / (K + 1);
      es[j] = er[j] + e % (K + 1);
    } else if (e < e_total) {
      er[j] = (e - eg_count) / Ro;
      es[j] = (e - eg_count) % Ro;
    } else {
      er[j] = -1 - 2 * K;  // never inside a span window
      es[j] = 0;
    }
  }
  // G is written as a full symmetric matrix: clear it before the band lands
  double* Gi = gram + (int64_t)i * Rn * Rn;
  for (int e = t; e < Rn * Rn; e += kRefitThreads) Gi[e] = 0.0;
  __syncthreads();

  const T* xi = xt + (int64_t)i * n;
  for (int64_t b0 = 0; b0 < n; b0 += kRefitThreads) {
    const int64_t b = b0 + t;
    int mn = -1, mo = -1;
    T vn[K + 1], vo[K + 1];
    if (b < n) {
      const T xv = xi[b];
      mn = knot_span(knots_n, nkn, xv);
      if (mn >= 0) span_values<K, T>(knots_n, nkn, mn, xv, vn);
      mo = knot_span(knots_o, nko, xv);
      if (mo >= 0) span_values<K, T>(knots_o, nko, mo, xv, vo);
    }
    span_n[t] = mn;
    span_o[t] = mo;
#pragma unroll
    for (int j = 0; j <= K; ++j) {
      // window slots that are not real basis functions carry zero
      const int rn = mn - K + j, ro = mo - K + j;
      val_n[t][j] = (mn >= 0 && rn >= 0 && rn < Rn) ? (double)vn[j] : 0.0;
      val_o[t][j] = (mo >= 0 && ro >= 0 && ro < Ro) ? (double)vo[j] : 0.0;
    }
    __syncthreads();
    const int cnt = (int)min((int64_t)kRefitThreads, n - b0);
    for (int s = 0; s < cnt; ++s) {
      const int m_n = span_n[s];
      if (m_n < 0) continue;
      const int m_o = span_o[s];
#pragma unroll
      for (int j = 0; j < MO; ++j) {
        const int ir = er[j] - (m_n - K);
        if (ir < 0 || ir > K) continue;
        if (is_g[j]) {
          const int is = es[j] - (m_n - K);
          if (is <= K) acc[j] += val_n[s][ir] * val_n[s][is];
        } else if (m_o >= 0) {
          const int is = es[j] - (m_o - K);
          if (is >= 0 && is <= K) acc[j] += val_n[s][ir] * val_o[s][is];
        }
      }
    }
    __syncthreads();
  }

  double* Ci = cross + (int64_t)i * Rn * Ro;
#pragma unroll
  for (int j = 0; j < MO; ++j) {
    const int e = t + kRefitThreads * j;
    if (e >= e_total) continue;
    if (is_g[j]) {
      if (es[j] < Rn) {
        Gi[er[j] * Rn + es[j]] = acc[j];
        Gi[es[j] * Rn + er[j]] = acc[j];
      }
    } else {
      Ci[er[j] * Ro + es[j]] = acc[j];
    }
  }
}

}  // namespace

template <typename T>
int launch_refit_gram(const T* xt, const T* grid_old, const T* grid_new, double* gram,
                      double* cross, int64_t n, int64_t I, int Go, int Gn, int k,
                      hipStream_t st) {
  if (I == 0) return KAN_OK;
  const int64_t Rn = Gn + k, Ro = Go + k;
  if (Rn * (k + 1) + Rn * Ro > (int64_t)kRefitThreads * kRefitMaxOwn)
    return set_error(KAN_ERR_LIMIT, "refit_gram: basis too large (Rn=%lld, Ro=%lld)",
                     (long long)Rn, (long long)Ro);
  if (I > 2147483647LL) return set_error(KAN_ERR_LIMIT, "refit_gram: too many features");
  TimedLaunch timed(kClassOther, st, 0.0);
  const int64_t own = ceil_div(Rn * (k + 1) + Rn * Ro, kRefitThreads);
#define KAN_REFIT_LAUNCH(KK, MO)                                                              \
  hipLaunchKernelGGL((refit_gram_kernel<KK, T, MO>), dim3((unsigned)I), dim3(kRefitThreads), 0, \
                     st, xt, grid_old, grid_new, gram, cross, n, Go, Gn)
#define KAN_REFIT_BY_OWN(KK)                   \
  if (own <= 1) KAN_REFIT_LAUNCH(KK, 1);       \
  else if (own <= 2) KAN_REFIT_LAUNCH(KK, 2);  \
  else if (own <= 4) KAN_REFIT_LAUNCH(KK, 4);  \
  else if (own <= 8) KAN_REFIT_LAUNCH(KK, 8);  \
  else KAN_REFIT_LAUNCH(KK, kRefitMaxOwn)
  if (k == 1) {
    KAN_REFIT_BY_OWN(1);
  } else if (k == 2) {
    KAN_REFIT_BY_OWN(2);
  } else {
    KAN_REFIT_BY_OWN(3);
  }
#undef KAN_REFIT_BY_OWN
#undef KAN_REFIT_LAUNCH
  return check_launch("refit_gram");
}

template int launch_refit_gram<float>(const float*, const float*, const float*, double*, double*,
                                      int64_t, int64_t, int, int, int, hipStream_t);
template int launch_refit_gram<double>(const double*, const double*, const double*, double*,
                                       double*, int64_t, int64_t, int, int, int, hipStream_t);

}  // namespace kan
