// Fused edge statistic of the activation regulariser,
//     a[o,i] = (1/n) sum_m |phi[m,o,i]|,
//     phi[m,o,i] = s[m,i] bw[o,i] + sum_r H[m,i,r] W[o,i,r],
// and its backward, without materialising the [n, O, I] edge tensor
// (replaces csrc/kan_reg_cuda.cu:34-238).
//
// Per edge the computation is a dot product of the augmented vectors
// h = [s, H_0..H_{R-1}] and w = [bw, W_0..W_{R-1}] (length R+1).  All three
// kernels evaluate phi with the same fused multiply-add chain in the same
// order (c = 0..R), so sign(phi) is identical in forward and backward.
//   forward      thread (o, i): w in registers, h rows of 64 samples staged
//                in LDS and read as wave-wide broadcasts.
//   params grad  thread (o, i): dw[c] += g * h[c], g = ga[o,i] sign(phi) / n.
//   inputs grad  thread (m, i): h in registers, w rows of 64 outputs staged
//                in LDS; dh[c] += g * w[c].
// Sums over samples may be split across workgroups; each split writes its own
// partial slice and a finalize kernel adds the slices in fixed order, so the
// result is deterministic (no atomics).  sign(0) = 0 (kan_reg_cuda.cu:25-28).

#include <type_traits>

#include "kan_common.h"

namespace kan {
namespace {

constexpr int kEdgeThreads = 256;
constexpr int kEdgeTile = 64;

template <typename T>
__device__ __forceinline__ T sign_of(T v) {
  return (T)((v > T(0)) - (v < T(0)));
}

__device__ __forceinline__ int small_div_e(int c, float inv) {
  return (int)(((float)c + 0.5f) * inv);
}

// Stages h rows [s, H_0..H_{R-1}] of samples [m0, m0+tn) for feature i.
template <typename T, int RP>
__device__ __forceinline__ void stage_h(T (*hs)[RP], const T* __restrict__ s,
                                       const T* __restrict__ H, int64_t m0, int tn, int I, int i,
                                       int R) {
  const int R1 = R + 1;
  const float inv = 1.0f / (float)R1;
  for (int e = threadIdx.x; e < tn * R1; e += blockDim.x) {
    const int tt = small_div_e(e, inv);
    const int c = e - tt * R1;
    const int64_t m = m0 + tt;
    T v;
    if (c == 0) v = s != nullptr ? s[m * I + i] : T(0);
    else v = H[(m * I + i) * R + (c - 1)];
    hs[tt][c] = v;
  }
}

template <typename T, int RP>
__device__ __forceinline__ T edge_phi(const T* __restrict__ h, const T (&w)[RP], int R1) {
  T phi = T(0);
#pragma unroll
  for (int c = 0; c < RP; ++c)
    if (c < R1) phi = fma(h[c], w[c], phi);
  return phi;
}

// stage_h for optional operands: a null s or H stages zeros.
template <typename T, int RP>
__device__ __forceinline__ void stage_h_opt(T (*hs)[RP], const T* __restrict__ s,
                                           const T* __restrict__ H, int64_t m0, int tn, int I,
                                           int i, int R) {
  const int R1 = R + 1;
  const float inv = 1.0f / (float)R1;
  for (int e = threadIdx.x; e < tn * R1; e += blockDim.x) {
    const int tt = small_div_e(e, inv);
    const int c = e - tt * R1;
    const int64_t m = m0 + tt;
    T v = T(0);
    if (c == 0) {
      if (s != nullptr) v = s[m * I + i];
    } else if (H != nullptr) {
      v = H[(m * I + i) * R + (c - 1)];
    }
    hs[tt][c] = v;
  }
}

template <typename T, int RP>
__global__ __launch_bounds__(kEdgeThreads) void edge_forward_kernel(
    const T* __restrict__ s, const T* __restrict__ H, const T* __restrict__ bw,
    const T* __restrict__ W, T* __restrict__ out, int64_t n, int I, int O, int R,
    int64_t per_split, bool final_out) {
  __shared__ __align__(16) T hs[kEdgeTile][RP];
  const int i = blockIdx.y;
  const int o = blockIdx.x * kEdgeThreads + threadIdx.x;
  const bool valid = o < O;
  const int R1 = R + 1;
  const int64_t e = (int64_t)o * I + i;
  T w[RP];
#pragma unroll
  for (int c = 0; c < RP; ++c) {
    T v = T(0);
    if (valid && c < R1) v = (c == 0) ? (bw != nullptr ? bw[e] : T(0)) : W[e * R + (c - 1)];
    w[c] = v;
  }
  const int64_t mb = (int64_t)blockIdx.z * per_split;
  const int64_t me = min(n, mb + per_split);
  T acc = T(0);
  for (int64_t m0 = mb; m0 < me; m0 += kEdgeTile) {
    const int tn = (int)min((int64_t)kEdgeTile, me - m0);
    stage_h<T, RP>(hs, s, H, m0, tn, I, i, R);
    __syncthreads();
    if (valid) {
      for (int tt = 0; tt < tn; ++tt) acc += fabs(edge_phi<T, RP>(hs[tt], w, R1));
    }
    __syncthreads();
  }
  if (!valid) return;
  if (final_out) out[e] = acc / (T)n;
  else out[(int64_t)blockIdx.z * ((int64_t)O * I) + e] = acc;
}

template <typename T>
__global__ void edge_forward_finalize(const T* __restrict__ part, T* __restrict__ a, int splits,
                                      int64_t count, int64_t n) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    T v = part[e];
    for (int s = 1; s < splits; ++s) v += part[s * count + e];
    a[e] = v / (T)n;
  }
}

// Parameter gradients: thread (o, i), sum over samples of g * h.
// final_out: write dbw/dW directly; otherwise write the split's partial
// [R+1] vector per edge into part.
// SUB: the contraction rows come from (s2, H2) (either may be null = zero)
// while sign(phi) still comes from (s, H) and (bw, W): the double backward
// of the statistic contracts the incoming gradients with the same sign
// pattern.
template <typename T, int RP, bool SUB = false>
__global__ __launch_bounds__(kEdgeThreads) void edge_param_grad_kernel(
    const T* __restrict__ ga, const T* __restrict__ s, const T* __restrict__ H,
    const T* __restrict__ bw, const T* __restrict__ W, T* __restrict__ dbw, T* __restrict__ dW,
    T* __restrict__ part, int64_t n, int I, int O, int R, int64_t per_split, bool final_out,
    const T* __restrict__ s2 = nullptr, const T* __restrict__ H2 = nullptr) {
  __shared__ __align__(16) T hs[kEdgeTile][RP];
  __shared__ __align__(16) T hs2[SUB ? kEdgeTile : 1][RP];
  const int i = blockIdx.y;
  const int o = blockIdx.x * kEdgeThreads + threadIdx.x;
  const bool valid = o < O;
  const int R1 = R + 1;
  const int64_t e = (int64_t)o * I + i;
  T w[RP], dw[RP];
#pragma unroll
  for (int c = 0; c < RP; ++c) {
    T v = T(0);
    if (valid && c < R1) v = (c == 0) ? (bw != nullptr ? bw[e] : T(0)) : W[e * R + (c - 1)];
    w[c] = v;
    dw[c] = T(0);
  }
  const T gav = valid ? ga[e] / (T)n : T(0);
  const int64_t mb = (int64_t)blockIdx.z * per_split;
  const int64_t me = min(n, mb + per_split);
  for (int64_t m0 = mb; m0 < me; m0 += kEdgeTile) {
    const int tn = (int)min((int64_t)kEdgeTile, me - m0);
    stage_h<T, RP>(hs, s, H, m0, tn, I, i, R);
    if (SUB) stage_h_opt<T, RP>(hs2, s2, H2, m0, tn, I, i, R);
    __syncthreads();
    if (valid) {
      for (int tt = 0; tt < tn; ++tt) {
        const T g = gav * sign_of(edge_phi<T, RP>(hs[tt], w, R1));
        const T* hc = SUB ? hs2[tt] : hs[tt];
#pragma unroll
        for (int c = 0; c < RP; ++c)
          if (c < R1) dw[c] = fma(g, hc[c], dw[c]);
      }
    }
    __syncthreads();
  }
  if (!valid) return;
  if (final_out) {
    if (dbw != nullptr) dbw[e] = dw[0];
    if (dW != nullptr) {
#pragma unroll
      for (int c = 1; c < RP; ++c)
        if (c < R1) dW[e * R + (c - 1)] = dw[c];
    }
  } else {
    T* dst = part + ((int64_t)blockIdx.z * ((int64_t)O * I) + e) * R1;
#pragma unroll
    for (int c = 0; c < RP; ++c)
      if (c < R1) dst[c] = dw[c];
  }
}

template <typename T>
__global__ void edge_param_finalize(const T* __restrict__ part, T* __restrict__ dbw,
                                    T* __restrict__ dW, int splits, int64_t count, int R) {
  const int R1 = R + 1;
  const int64_t total = count * R1;
  for (int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; x < total;
       x += (int64_t)gridDim.x * blockDim.x) {
    T v = part[x];
    for (int s = 1; s < splits; ++s) v += part[s * total + x];
    const int64_t e = x / R1;
    const int c = (int)(x - e * R1);
    if (c == 0) {
      if (dbw != nullptr) dbw[e] = v;
    } else if (dW != nullptr) {
      dW[e * R + (c - 1)] = v;
    }
  }
}

// Input gradients: thread (m, i), sum over outputs of g * w.
// SUB: contraction rows from (bw2, W2) (null = zero), sign from (bw, W).
template <typename T, int RP, bool SUB = false>
__global__ __launch_bounds__(kEdgeThreads) void edge_input_grad_kernel(
    const T* __restrict__ ga, const T* __restrict__ s, const T* __restrict__ H,
    const T* __restrict__ bw, const T* __restrict__ W, T* __restrict__ ds, T* __restrict__ dH,
    int64_t n, int I, int O, int R, const T* __restrict__ bw2 = nullptr,
    const T* __restrict__ W2 = nullptr) {
  __shared__ __align__(16) T ws[kEdgeTile][RP];
  __shared__ __align__(16) T ws2[SUB ? kEdgeTile : 1][RP];
  __shared__ T gs[kEdgeTile];
  const int i = blockIdx.y;
  const int64_t m = (int64_t)blockIdx.x * kEdgeThreads + threadIdx.x;
  const bool valid = m < n;
  const int R1 = R + 1;
  const int64_t f = m * I + i;
  T h[RP], dh[RP];
#pragma unroll
  for (int c = 0; c < RP; ++c) {
    T v = T(0);
    if (valid && c < R1) v = (c == 0) ? (s != nullptr ? s[f] : T(0)) : H[f * R + (c - 1)];
    h[c] = v;
    dh[c] = T(0);
  }
  const float inv = 1.0f / (float)R1;
  for (int o0 = 0; o0 < O; o0 += kEdgeTile) {
    const int to = min(kEdgeTile, O - o0);
    for (int x = threadIdx.x; x < to * R1; x += blockDim.x) {
      const int tt = small_div_e(x, inv);
      const int c = x - tt * R1;
      const int64_t e = (int64_t)(o0 + tt) * I + i;
      ws[tt][c] = (c == 0) ? (bw != nullptr ? bw[e] : T(0)) : W[e * R + (c - 1)];
      if (SUB) {
        T v = T(0);
        if (c == 0) {
          if (bw2 != nullptr) v = bw2[e];
        } else if (W2 != nullptr) {
          v = W2[e * R + (c - 1)];
        }
        ws2[tt][c] = v;
      }
    }
    for (int x = threadIdx.x; x < to; x += blockDim.x)
      gs[x] = ga[(int64_t)(o0 + x) * I + i] / (T)n;
    __syncthreads();
    if (valid) {
      for (int tt = 0; tt < to; ++tt) {
        const T* wr = ws[tt];
        T phi = T(0);
#pragma unroll
        for (int c = 0; c < RP; ++c)
          if (c < R1) phi = fma(h[c], wr[c], phi);
        const T g = gs[tt] * sign_of(phi);
        const T* wc = SUB ? ws2[tt] : wr;
#pragma unroll
        for (int c = 0; c < RP; ++c)
          if (c < R1) dh[c] = fma(g, wc[c], dh[c]);
      }
    }
    __syncthreads();
  }
  if (!valid) return;
  if (ds != nullptr) ds[f] = dh[0];
  if (dH != nullptr) {
#pragma unroll
    for (int c = 1; c < RP; ++c)
      if (c < R1) dH[f * R + (c - 1)] = dh[c];
  }
}

// d/dga of the double backward: thread (o, i),
//   out[o, i] = sum_m sign(h.w) (h1.w + h.w2)   (h1 = [s1, H1], w2 = [bw2, W2]),
// divided by n in the finalize (or here when the sum is not split).
template <typename T, int RP>
__global__ __launch_bounds__(kEdgeThreads) void edge_ga_grad_kernel(
    const T* __restrict__ s, const T* __restrict__ H, const T* __restrict__ bw,
    const T* __restrict__ W, const T* __restrict__ s1, const T* __restrict__ H1,
    const T* __restrict__ bw2, const T* __restrict__ W2, T* __restrict__ out, int64_t n, int I,
    int O, int R, int64_t per_split, bool final_out) {
  __shared__ __align__(16) T hs[kEdgeTile][RP];
  __shared__ __align__(16) T hs1[kEdgeTile][RP];
  const int i = blockIdx.y;
  const int o = blockIdx.x * kEdgeThreads + threadIdx.x;
  const bool valid = o < O;
  const int R1 = R + 1;
  const int64_t e = (int64_t)o * I + i;
  T w[RP], w2[RP];
#pragma unroll
  for (int c = 0; c < RP; ++c) {
    T v = T(0), v2 = T(0);
    if (valid && c < R1) {
      if (c == 0) {
        v = bw != nullptr ? bw[e] : T(0);
        v2 = bw2 != nullptr ? bw2[e] : T(0);
      } else {
        v = W[e * R + (c - 1)];
        v2 = W2 != nullptr ? W2[e * R + (c - 1)] : T(0);
      }
    }
    w[c] = v;
    w2[c] = v2;
  }
  const int64_t mb = (int64_t)blockIdx.z * per_split;
  const int64_t me = min(n, mb + per_split);
  T acc = T(0);
  for (int64_t m0 = mb; m0 < me; m0 += kEdgeTile) {
    const int tn = (int)min((int64_t)kEdgeTile, me - m0);
    stage_h<T, RP>(hs, s, H, m0, tn, I, i, R);
    stage_h_opt<T, RP>(hs1, s1, H1, m0, tn, I, i, R);
    __syncthreads();
    if (valid) {
      for (int tt = 0; tt < tn; ++tt) {
        const T sg = sign_of(edge_phi<T, RP>(hs[tt], w, R1));
        const T psi = edge_phi<T, RP>(hs1[tt], w, R1) + edge_phi<T, RP>(hs[tt], w2, R1);
        acc = fma(sg, psi, acc);
      }
    }
    __syncthreads();
  }
  if (!valid) return;
  if (final_out) out[e] = acc / (T)n;
  else out[(int64_t)blockIdx.z * ((int64_t)O * I) + e] = acc;
}

template <typename T>
__global__ void edge_zero_kernel(T* __restrict__ out, int64_t count) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x)
    out[e] = T(0);
}

inline int fin_blocks(int64_t total) {
  int64_t b = ceil_div(total, 256);
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

#define KAN_EDGE_DISPATCH(R1, ...)                 \
  do {                                             \
    if ((R1) <= 8) {                               \
      constexpr int RP = 8;                        \
      __VA_ARGS__;                                 \
    } else if ((R1) <= 16) {                       \
      constexpr int RP = 16;                       \
      __VA_ARGS__;                                 \
    } else if ((R1) <= 24) {                       \
      constexpr int RP = 24;                       \
      __VA_ARGS__;                                 \
    } else if ((R1) <= 32) {                       \
      constexpr int RP = 32;                       \
      __VA_ARGS__;                                 \
    } else if ((R1) <= 48) {                       \
      constexpr int RP = 48;                       \
      __VA_ARGS__;                                 \
    } else {                                       \
      constexpr int RP = 76;                       \
      __VA_ARGS__;                                 \
    }                                              \
  } while (0)

}  // namespace

int edge_pick_splits(int dtype, int64_t n, int64_t I, int64_t O, int64_t R, bool backward) {
  if (dtype == KAN_DTYPE_F32) return edge_mfma_splits(n, I, O, R, backward);
  if (edge_mfma64_applies(R)) return edge_mfma64_splits(n, I, O, backward);
  const int64_t blocks = ceil_div(O, kEdgeThreads) * I;
  const int64_t target = 4LL * device_cu_count();
  int64_t s = ceil_div(target, blocks > 0 ? blocks : 1);
  const int64_t cap = ceil_div(n, 4 * kEdgeTile);
  if (s > cap) s = cap;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return (int)s;
}

template <typename T>
int launch_edge_forward(const T* s, const T* H, const T* bw, const T* W, T* a, T* part,
                        int splits, int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st) {
  if (O == 0 || I == 0) return KAN_OK;
  if (splits > 1 && part == nullptr) return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean: missing workspace");
  if constexpr (std::is_same<T, double>::value) {
    if (edge_mfma64_applies(R)) {
      const int rc = launch_edge_forward_mfma64(s, H, bw, W, a, part, splits, n, I, O, R, st);
      if (rc != KAN_OK || splits == 1) return rc;
      hipLaunchKernelGGL((edge_forward_finalize<T>), dim3(fin_blocks(O * I)), dim3(256), 0, st,
                         part, a, splits, O * I, n);
      return check_launch("edge_abs_mean_finalize");
    }
  }
  const int64_t per_split = round_up(ceil_div(n, splits), kEdgeTile);
  dim3 grid((unsigned)ceil_div(O, kEdgeThreads), (unsigned)I, (unsigned)splits);
  const bool fin = splits == 1;
  const int R1 = (int)R + 1;
  TimedLaunch timed(kClassEdge, st, 2.0 * (double)n * (double)O * (double)I * (double)R1);
  KAN_EDGE_DISPATCH(R1, hipLaunchKernelGGL((edge_forward_kernel<T, RP>), grid,
                                           dim3(kEdgeThreads), 0, st, s, H, bw, W,
                                           fin ? a : part, n, (int)I, (int)O, (int)R, per_split,
                                           fin));
  int rc = check_launch("edge_abs_mean");
  if (rc != KAN_OK || fin) return rc;
  hipLaunchKernelGGL((edge_forward_finalize<T>), dim3(fin_blocks(O * I)), dim3(256), 0, st, part,
                     a, splits, O * I, n);
  return check_launch("edge_abs_mean_finalize");
}

template <typename T>
int launch_edge_backward(const T* ga, const T* s, const T* H, const T* bw, const T* W, T* ds,
                         T* dH, T* dbw, T* dW, T* part, int splits, int64_t n, int64_t I,
                         int64_t O, int64_t R, hipStream_t st) {
  const int R1 = (int)R + 1;
  if ((dbw != nullptr || dW != nullptr) && O > 0 && I > 0) {
    if (splits > 1 && part == nullptr)
      return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean_backward: missing workspace");
    const bool fin = splits == 1;
    int rc = KAN_OK;
    bool done = false;
    if constexpr (std::is_same<T, double>::value) {
      if (edge_mfma64_applies(R)) {
        rc = launch_edge_param_mfma64(ga, s, H, bw, W, dbw, dW, part, splits, n, I, O, R, st);
        done = true;
      }
    }
    if (!done) {
      const int64_t per_split = round_up(ceil_div(n, splits), kEdgeTile);
      dim3 grid((unsigned)ceil_div(O, kEdgeThreads), (unsigned)I, (unsigned)splits);
      TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
      KAN_EDGE_DISPATCH(R1, hipLaunchKernelGGL((edge_param_grad_kernel<T, RP>), grid,
                                               dim3(kEdgeThreads), 0, st, ga, s, H, bw, W, dbw,
                                               dW, part, n, (int)I, (int)O, (int)R, per_split,
                                               fin));
      rc = check_launch("edge_abs_mean_backward(params)");
    }
    if (rc != KAN_OK) return rc;
    if (!fin) {
      hipLaunchKernelGGL((edge_param_finalize<T>), dim3(fin_blocks(O * I * R1)), dim3(256), 0, st,
                         part, dbw, dW, splits, O * I, (int)R);
      rc = check_launch("edge_abs_mean_backward(finalize)");
      if (rc != KAN_OK) return rc;
    }
  }
  if ((ds != nullptr || dH != nullptr) && n > 0 && I > 0) {
    if constexpr (std::is_same<T, double>::value) {
      if (edge_mfma64_applies(R))
        return launch_edge_input_mfma64(ga, s, H, bw, W, ds, dH, n, I, O, R, st);
    }
    dim3 grid((unsigned)ceil_div(n, kEdgeThreads), (unsigned)I);
    TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
    KAN_EDGE_DISPATCH(R1, hipLaunchKernelGGL((edge_input_grad_kernel<T, RP>), grid,
                                             dim3(kEdgeThreads), 0, st, ga, s, H, bw, W, ds, dH,
                                             n, (int)I, (int)O, (int)R));
    int rc = check_launch("edge_abs_mean_backward(inputs)");
    if (rc != KAN_OK) return rc;
  }
  return KAN_OK;
}

// Splits over samples for the VALU edge kernels (the sample sums).
int edge_valu_splits(int64_t n, int64_t I, int64_t O) {
  const int64_t blocks = ceil_div(O, kEdgeThreads) * I;
  const int64_t target = 4LL * device_cu_count();
  int64_t s = ceil_div(target, blocks > 0 ? blocks : 1);
  const int64_t cap = ceil_div(n, 4 * kEdgeTile);
  if (s > cap) s = cap;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return (int)s;
}

size_t edge_double_backward_ws_elems(int64_t n, int64_t I, int64_t O, int64_t R) {
  const int splits = edge_valu_splits(n, I, O);
  if (splits <= 1) return 0;
  return (size_t)splits * (size_t)(O * I) * (size_t)(R + 1);  // covers the [s, O, I] slices too
}

template <typename T>
int launch_edge_double_backward(const T* ga, const T* s, const T* H, const T* bw, const T* W,
                                const T* u_ds, const T* u_dH, const T* u_dbw, const T* u_dW,
                                T* g_ga, T* g_s, T* g_H, T* g_bw, T* g_W, T* part, int64_t n,
                                int64_t I, int64_t O, int64_t R, hipStream_t st) {
  const int R1 = (int)R + 1;
  const int splits = edge_valu_splits(n, I, O);
  if (splits > 1 && part == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean_double_backward: missing workspace");
  const int64_t per_split = round_up(ceil_div(n, splits), kEdgeTile);
  const bool fin = splits == 1;
  const bool u_rows = u_ds != nullptr || u_dH != nullptr;   // sample-side incoming gradients
  const bool u_cols = u_dbw != nullptr || u_dW != nullptr;  // weight-side incoming gradients
  if (g_ga != nullptr && O > 0 && I > 0) {
    dim3 grid((unsigned)ceil_div(O, kEdgeThreads), (unsigned)I, (unsigned)splits);
    TimedLaunch timed(kClassEdgeGrad, st, 6.0 * (double)n * (double)O * (double)I * (double)R1);
    KAN_EDGE_DISPATCH(R1, hipLaunchKernelGGL((edge_ga_grad_kernel<T, RP>), grid,
                                             dim3(kEdgeThreads), 0, st, s, H, bw, W, u_ds, u_dH,
                                             u_dbw, u_dW, fin ? g_ga : part, n, (int)I, (int)O,
                                             (int)R, per_split, fin));
    int rc = check_launch("edge_abs_mean_double_backward(ga)");
    if (rc != KAN_OK) return rc;
    if (!fin) {
      hipLaunchKernelGGL((edge_forward_finalize<T>), dim3(fin_blocks(O * I)), dim3(256), 0, st,
                         part, g_ga, splits, O * I, n);
      rc = check_launch("edge_abs_mean_double_backward(ga finalize)");
      if (rc != KAN_OK) return rc;
    }
  }
  if ((g_bw != nullptr || g_W != nullptr) && O > 0 && I > 0) {
    if (!u_rows) {
      // no sample-side incoming gradient: these are zero
      if (g_bw != nullptr)
        hipLaunchKernelGGL((edge_zero_kernel<T>), dim3(fin_blocks(O * I)), dim3(256), 0, st,
                           g_bw, O * I);
      if (g_W != nullptr)
        hipLaunchKernelGGL((edge_zero_kernel<T>), dim3(fin_blocks(O * I * R)), dim3(256), 0, st,
                           g_W, O * I * R);
    } else {
      dim3 grid((unsigned)ceil_div(O, kEdgeThreads), (unsigned)I, (unsigned)splits);
      TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
      KAN_EDGE_DISPATCH(R1, hipLaunchKernelGGL((edge_param_grad_kernel<T, RP, true>), grid,
                                               dim3(kEdgeThreads), 0, st, ga, s, H, bw, W, g_bw,
                                               g_W, part, n, (int)I, (int)O, (int)R, per_split,
                                               fin, u_ds, u_dH));
      int rc = check_launch("edge_abs_mean_double_backward(params)");
      if (rc != KAN_OK) return rc;
      if (!fin) {
        hipLaunchKernelGGL((edge_param_finalize<T>), dim3(fin_blocks(O * I * R1)), dim3(256), 0,
                           st, part, g_bw, g_W, splits, O * I, (int)R);
        rc = check_launch("edge_abs_mean_double_backward(params finalize)");
        if (rc != KAN_OK) return rc;
      }
    }
  }
  if ((g_s != nullptr || g_H != nullptr) && n > 0 && I > 0) {
    if (!u_cols) {
      if (g_s != nullptr)
        hipLaunchKernelGGL((edge_zero_kernel<T>), dim3(fin_blocks(n * I)), dim3(256), 0, st, g_s,
                           n * I);
      if (g_H != nullptr)
        hipLaunchKernelGGL((edge_zero_kernel<T>), dim3(fin_blocks(n * I * R)), dim3(256), 0, st,
                           g_H, n * I * R);
    } else {
      dim3 grid((unsigned)ceil_div(n, kEdgeThreads), (unsigned)I);
      TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
      KAN_EDGE_DISPATCH(R1, hipLaunchKernelGGL((edge_input_grad_kernel<T, RP, true>), grid,
                                               dim3(kEdgeThreads), 0, st, ga, s, H, bw, W, g_s,
                                               g_H, n, (int)I, (int)O, (int)R, u_dbw, u_dW));
    }
    int rc = check_launch("edge_abs_mean_double_backward(inputs)");
    if (rc != KAN_OK) return rc;
  }
  return check_launch("edge_abs_mean_double_backward");
}

template int launch_edge_double_backward<float>(const float*, const float*, const float*,
                                                const float*, const float*, const float*,
                                                const float*, const float*, const float*, float*,
                                                float*, float*, float*, float*, float*, int64_t,
                                                int64_t, int64_t, int64_t, hipStream_t);
template int launch_edge_double_backward<double>(const double*, const double*, const double*,
                                                 const double*, const double*, const double*,
                                                 const double*, const double*, const double*,
                                                 double*, double*, double*, double*, double*,
                                                 double*, int64_t, int64_t, int64_t, int64_t,
                                                 hipStream_t);

template <>
int launch_edge_forward<float>(const float* s, const float* H, const float* bw, const float* W,
                               float* a, float* part, int splits, int64_t n, int64_t I,
                               int64_t O, int64_t R, hipStream_t st) {
  return launch_edge_forward_mfma(s, H, bw, W, a, part, splits, n, I, O, R, st);
}

template <>
int launch_edge_backward<float>(const float* ga, const float* s, const float* H, const float* bw,
                                const float* W, float* ds, float* dH, float* dbw, float* dW,
                                float* part, int splits, int64_t n, int64_t I, int64_t O,
                                int64_t R, hipStream_t st) {
  return launch_edge_backward_mfma(ga, s, H, bw, W, ds, dH, dbw, dW, part, splits, n, I, O, R,
                                   st);
}

template int launch_edge_forward<double>(const double*, const double*, const double*,
                                         const double*, double*, double*, int, int64_t, int64_t,
                                         int64_t, int64_t, hipStream_t);
template int launch_edge_backward<double>(const double*, const double*, const double*,
                                          const double*, const double*, double*, double*,
                                          double*, double*, double*, int, int64_t, int64_t,
                                          int64_t, int64_t, hipStream_t);

}  // namespace kan
