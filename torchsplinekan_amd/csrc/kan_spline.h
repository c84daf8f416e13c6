// Device helpers of the local B-spline evaluation, shared by the basis
// kernels (kan_basis.hip) and the refit kernels (kan_refit.hip): span search
// and the non-zero values / first derivatives of the order-K functions on a
// span, read from a knot row t[0..nk-1] (normally staged in LDS).
#pragma once

#include "kan_common.h"

namespace kan {

// Span search.  For W values x[u] on knot rows t[u] of nk knots each, m[u]
// is the span index with t[m] <= x < t[m+1] (x == t[nk-1]: the last
// non-degenerate span), or -1 when x lies outside [t[0], t[nk-1]] or is NaN
// (the conventions of find_span, csrc/kan_cuda.cu:207-221).  Inside the
// knots the index is found by greedy binary lifting: starting from 0, add
// each power of two below nk - 1, largest first, wherever the knot reached
// is still <= x.  On a sorted row that gives the largest m <= nk - 2 with
// t[m] <= x.  The step count depends on nk alone, so lanes never diverge,
// and W independent searches interleave for latency.  Every kernel finds its
// spans through this one routine, so kernels that exchange span-indexed data
// (the compact input-side product writes window slots that
// basis_grad_compact_kernel reads) agree on any knot row, sorted or not.
__host__ __device__ __forceinline__ int lift_top_step(int nk) {
  return nk > 2 ? 1 << (31 - __builtin_clz((unsigned)(nk - 2))) : 0;
}

template <int W, typename T>
__host__ __device__ __forceinline__ void knot_spans(const T* const (&t)[W], int nk,
                                                    const T (&x)[W], int (&m)[W]) {
  const int last = nk - 2;
#pragma unroll
  for (int u = 0; u < W; ++u) m[u] = 0;
  for (int step = lift_top_step(nk); step > 0; step >>= 1) {
#pragma unroll
    for (int u = 0; u < W; ++u) {
      const int c = m[u] + step;
      const T knot = t[u][c <= last ? c : last];   // in range whether or not c is
      if (c <= last && knot <= x[u]) m[u] = c;
    }
  }
#pragma unroll
  for (int u = 0; u < W; ++u) {
    const T top = t[u][nk - 1];
    if (!(x[u] >= t[u][0]) || x[u] > top) {
      m[u] = -1;
    } else if (x[u] == top) {
      int q = last;
      while (q > 0 && t[u][q] == top) --q;
      m[u] = q;
    }
  }
}

template <typename T>
__host__ __device__ __forceinline__ int knot_span(const T* t, int nk, T x) {
  const T* const rows[1] = {t};
  const T xs[1] = {x};
  int m[1];
  knot_spans<1, T>(rows, nk, xs, m);
  return m[0];
}

template <typename T>
__device__ __forceinline__ T knot_at(const T* __restrict__ t, int nk, int idx) {
  idx = idx < 0 ? 0 : (idx > nk - 1 ? nk - 1 : idx);
  return t[idx];
}

// The D+1 degree-D functions that are non-zero on span m,
//   v[j] = B_{m-D+j, D}(x),  j = 0..D,
// by the triangular scheme of Piegl & Tiller (The NURBS Book, A2.2) with a
// zero-denominator guard.  Window entries that are not real basis functions
// (near the ends of the knot vector) read clamped knots and are discarded by
// the caller; every real function only depends on in-range knots.
// Same recurrence as local_basis, csrc/kan_cuda.cu:230-271.
template <int D, typename T>
__device__ __forceinline__ void span_values(const T* __restrict__ t, int nk, int m, T x,
                                            T (&v)[D + 1]) {
  T left[D + 1], right[D + 1];
  v[0] = T(1);
#pragma unroll
  for (int j = 1; j <= D; ++j) {
    left[j] = x - knot_at(t, nk, m + 1 - j);
    right[j] = knot_at(t, nk, m + j) - x;
    T saved = T(0);
#pragma unroll
    for (int r = 0; r < j; ++r) {
      const T den = right[r + 1] + left[j - r];
      const T tmp = den != T(0) ? v[r] / den : T(0);
      v[r] = saved + right[r + 1] * tmp;
      saved = left[j - r] * tmp;
    }
    v[j] = saved;
  }
}

// First derivatives of the K+1 degree-K functions active on span m:
//   dB_{r,K} = K * ( B_{r,K-1}/(t_{r+K}-t_r) - B_{r+1,K-1}/(t_{r+K+1}-t_{r+1}) ),
// r = m-K+j, from the degree-(K-1) values on the same span.
// Formula of csrc/kan_cuda.cu:238-255 / spline_kan/reference_backend.py:99-125.
template <int K, typename T>
__device__ __forceinline__ void span_derivs(const T* __restrict__ t, int nk, int m, T x,
                                            T (&d)[K + 1]) {
  T lower[K];
  span_values<K - 1, T>(t, nk, m, x, lower);
#pragma unroll
  for (int j = 0; j <= K; ++j) {
    const int r = m - K + j;
    T a = T(0), b = T(0);
    if (j >= 1) {
      const T den = knot_at(t, nk, r + K) - knot_at(t, nk, r);
      if (den != T(0)) a = lower[j - 1] / den;
    }
    if (j <= K - 1) {
      const T den = knot_at(t, nk, r + K + 1) - knot_at(t, nk, r + 1);
      if (den != T(0)) b = lower[j] / den;
    }
    d[j] = T(K) * (a - b);
  }
}

// Order-Q derivatives (1 <= Q <= K) of the K+1 degree-K functions active on
// span m, d[j] = D^Q B_{m-K+j, K}(x): the degree K-Q values on span m, then Q
// steps of the derivative recurrence (p = K-Q+1 .. K)
//   D^q B_{r,p} = p * ( D^(q-1) B_{r,p-1} / (t_{r+p} - t_r)
//                     - D^(q-1) B_{r+1,p-1} / (t_{r+p+1} - t_{r+1}) ),
// each term zero where its knot difference is zero.  This is the exact
// derivative of the piecewise polynomial that autograd finds through the
// differentiable recurrence of spline_kan/reference_backend.py:69-125
// (The NURBS Book, eq. 2.9 and A2.3).  Q = 1 is span_derivs, operation for
// operation.
template <int K, int Q, typename T>
__device__ __forceinline__ void span_derivs_n(const T* __restrict__ t, int nk, int m, T x,
                                              T (&d)[K + 1]) {
  static_assert(Q >= 1 && Q <= K, "derivative order must lie in 1..K");
  T cur[K + 1];
  {
    T low[K - Q + 1];
    span_values<K - Q, T>(t, nk, m, x, low);
#pragma unroll
    for (int j = 0; j <= K - Q; ++j) cur[j] = low[j];
  }
#pragma unroll
  for (int p = K - Q + 1; p <= K; ++p) {
    T nxt[K + 1];
#pragma unroll
    for (int j = 0; j <= p; ++j) {
      const int r = m - p + j;
      T a = T(0), b = T(0);
      if (j >= 1) {
        const T den = knot_at(t, nk, r + p) - knot_at(t, nk, r);
        if (den != T(0)) a = cur[j - 1] / den;
      }
      if (j <= p - 1) {
        const T den = knot_at(t, nk, r + p + 1) - knot_at(t, nk, r + 1);
        if (den != T(0)) b = cur[j] / den;
      }
      nxt[j] = T(p) * (a - b);
    }
#pragma unroll
    for (int j = 0; j <= p; ++j) cur[j] = nxt[j];
  }
#pragma unroll
  for (int j = 0; j <= K; ++j) d[j] = cur[j];
}

// Values (Q = 0) or order-Q derivatives of the window on span m.
template <int K, int Q, typename T>
__device__ __forceinline__ void span_window(const T* __restrict__ t, int nk, int m, T x,
                                            T (&d)[K + 1]) {
  if constexpr (Q == 0) span_values<K, T>(t, nk, m, x, d);
  else span_derivs_n<K, Q, T>(t, nk, m, x, d);
}

}  // namespace kan
