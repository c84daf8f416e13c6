// Regulariser of one layer from its edge means a[o, i] (the KAN paper's
// activation penalty, eqs. 20-21):
//   reg = mu1 * T + mu2 * H,   T = sum a,   H = -sum p log p,
//   p = max(a / max(T, tiny), tiny)          (tiny: the smallest normal number)
// and its gradient with respect to a, with the clamps' zero-gradient masks:
//   d reg / d a_j = mu1 + mu2 * ( -(log p_j + 1) m_j / tc + c U / tc^2 ),
//   tc = max(T, tiny), m_j = [a_j / tc >= tiny], c = [T >= tiny],
//   U = sum_i (log p_i + 1) m_i a_i.
// This is what autograd takes through the reference's expression
// (spline_kan/reference_backend.py:149-170): about 10 elementwise and
// reduction launches forward and 20 backward per layer, replaced here by
// three forward launches and one backward.  Sums are accumulated in double
// over fixed per-block ranges and added in block order, so results are
// deterministic; elementwise terms use the input type's arithmetic as the
// reference does.
//
// Workspace (doubles): part[P] block sums of a, hu[2P] block sums of p log p
// and of U's terms, then the stats {T, tc, U, c} the backward reads.

#include "kan_common.h"

namespace kan {

namespace {

constexpr int kRegThreads = 256;
constexpr int kRegMaxBlocks = 256;

template <typename T>
__device__ __forceinline__ T tiny_of();
template <>
__device__ __forceinline__ float tiny_of<float>() {
  return 1.17549435e-38f;
}
template <>
__device__ __forceinline__ double tiny_of<double>() {
  return 2.2250738585072014e-308;
}

__device__ __forceinline__ float log_of(float v) { return logf(v); }
__device__ __forceinline__ double log_of(double v) { return log(v); }

// Fixed-order block sum of the threads' values (kRegThreads of them).
__device__ __forceinline__ double block_sum(double v, double* red) {
  red[threadIdx.x] = v;
  __syncthreads();
#pragma unroll
  for (int s = kRegThreads / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] += red[threadIdx.x + s];
    __syncthreads();
  }
  const double r = red[0];
  __syncthreads();
  return r;
}

// the range of block b: [b * chunk, min(n, (b + 1) * chunk))
struct RegRange {
  int64_t lo, hi;
  __device__ RegRange(int64_t n, int64_t chunk, int b) {
    lo = (int64_t)b * chunk;
    hi = lo + chunk < n ? lo + chunk : n;
  }
};

template <typename T>
__global__ void __launch_bounds__(kRegThreads)
reg_sum_kernel(const T* __restrict__ a, int64_t n, int64_t chunk, double* __restrict__ part) {
  __shared__ double red[kRegThreads];
  const RegRange rg(n, chunk, blockIdx.x);
  double acc = 0.0;
  for (int64_t e = rg.lo + threadIdx.x; e < rg.hi; e += kRegThreads) acc += (double)a[e];
  const double s = block_sum(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// T (the input type) of the block sums, added in block order by every block
template <typename T>
__device__ __forceinline__ T total_of(const double* __restrict__ part, int nb) {
  double t = 0.0;
  for (int b = 0; b < nb; ++b) t += part[b];
  return (T)t;
}

template <typename T>
__global__ void __launch_bounds__(kRegThreads)
reg_entropy_kernel(const T* __restrict__ a, int64_t n, int64_t chunk,
                   const double* __restrict__ part, double* __restrict__ hu) {
  __shared__ double red[kRegThreads];
  const T total = total_of<T>(part, gridDim.x);
  const T tiny = tiny_of<T>();
  const T tc = total > tiny ? total : tiny;
  const RegRange rg(n, chunk, blockIdx.x);
  double h = 0.0, u = 0.0;
  for (int64_t e = rg.lo + threadIdx.x; e < rg.hi; e += kRegThreads) {
    const T q = a[e] / tc;
    const T p = q > tiny ? q : tiny;
    const T lp = log_of(p);
    h += (double)(p * lp);
    if (q >= tiny) u += (double)((lp + T(1)) * a[e]);
  }
  const double hs = block_sum(h, red);
  const double us = block_sum(u, red);
  if (threadIdx.x == 0) {
    hu[2 * blockIdx.x] = hs;
    hu[2 * blockIdx.x + 1] = us;
  }
}

template <typename T>
__global__ void reg_final_kernel(const double* __restrict__ part, const double* __restrict__ hu,
                                 int nb, double mu1, double mu2, T* __restrict__ reg,
                                 double* __restrict__ stats) {
  if (threadIdx.x != 0) return;
  const T total = total_of<T>(part, nb);
  const T tiny = tiny_of<T>();
  const T tc = total > tiny ? total : tiny;
  double h = 0.0, u = 0.0;
  for (int b = 0; b < nb; ++b) {
    h += hu[2 * b];
    u += hu[2 * b + 1];
  }
  const T ent = -(T)h;
  reg[0] = (T)mu1 * total + (T)mu2 * ent;
  stats[0] = (double)total;
  stats[1] = (double)tc;
  stats[2] = u;
  stats[3] = total >= tiny ? 1.0 : 0.0;
}

template <typename T>
__global__ void __launch_bounds__(kRegThreads)
reg_grad_kernel(const T* __restrict__ g, const T* __restrict__ a, int64_t n,
                const double* __restrict__ stats, double mu1, double mu2, T* __restrict__ ga) {
  const T tiny = tiny_of<T>();
  const T tc = (T)stats[1];
  // c U / tc^2, divided twice (tc^2 underflows where the total is tiny; c = 0
  // for an all-zero layer, whose gradient is then mu1)
  const T cu = stats[3] != 0.0 ? ((T)stats[2] / tc) / tc : T(0);
  const T gv = g[0], m1 = (T)mu1, m2 = (T)mu2;
  for (int64_t e = blockIdx.x * (int64_t)kRegThreads + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * kRegThreads) {
    const T q = a[e] / tc;
    const T p = q > tiny ? q : tiny;
    const T lp1 = q >= tiny ? log_of(p) + T(1) : T(0);
    ga[e] = gv * (m1 + m2 * (cu - lp1 / tc));
  }
}

inline int reg_blocks(int64_t n) {
  int64_t b = ceil_div(n, (int64_t)kRegThreads * 8);
  if (b > kRegMaxBlocks) b = kRegMaxBlocks;
  return (int)(b < 1 ? 1 : b);
}

}  // namespace

size_t edge_reg_ws_bytes(int64_t n) {
  return sizeof(double) * (3 * (size_t)reg_blocks(n) + 4);
}

template <typename T>
int launch_edge_reg(const T* a, int64_t n, double mu1, double mu2, T* reg, double* ws,
                    hipStream_t st) {
  const int nb = reg_blocks(n);
  const int64_t chunk = ceil_div(n > 0 ? n : 1, (int64_t)nb);
  double* part = ws;
  double* hu = ws + nb;
  double* stats = ws + 3 * nb;
  hipLaunchKernelGGL(reg_sum_kernel<T>, dim3(nb), dim3(kRegThreads), 0, st, a, n, chunk, part);
  hipLaunchKernelGGL(reg_entropy_kernel<T>, dim3(nb), dim3(kRegThreads), 0, st, a, n, chunk, part,
                     hu);
  hipLaunchKernelGGL(reg_final_kernel<T>, dim3(1), dim3(64), 0, st, part, hu, nb, mu1, mu2, reg,
                     stats);
  return check_launch("edge_regularization");
}

template <typename T>
int launch_edge_reg_backward(const T* g, const T* a, int64_t n, double mu1, double mu2,
                             const double* ws, T* ga, hipStream_t st) {
  if (n == 0) return KAN_OK;
  const int nb = reg_blocks(n);
  int64_t blocks = ceil_div(n, (int64_t)kRegThreads);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(reg_grad_kernel<T>, dim3((unsigned)blocks), dim3(kRegThreads), 0, st, g, a,
                     n, ws + 3 * nb, mu1, mu2, ga);
  return check_launch("edge_regularization_backward");
}

template int launch_edge_reg<float>(const float*, int64_t, double, double, float*, double*,
                                    hipStream_t);
template int launch_edge_reg<double>(const double*, int64_t, double, double, double*, double*,
                                     hipStream_t);
template int launch_edge_reg_backward<float>(const float*, const float*, int64_t, double, double,
                                             const double*, float*, hipStream_t);
template int launch_edge_reg_backward<double>(const double*, const double*, int64_t, double,
                                              double, const double*, double*, hipStream_t);

}  // namespace kan
