// Shared definitions for the gfx950 KAN kernels: limits, dtype codes,
// error reporting and small device helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/kan_hip.h"

namespace kan {

// Degree-0 basis count G + 2k accepted by the native path.  Mirrors
// KAN_CUDA_MAX_DEG0_BASIS (csrc/kan_ops.h:15) so that backend selection in
// the module layer is unchanged.
constexpr int64_t kMaxDeg0Basis = 71;
// in_features limit, mirroring KAN_CUDA_MAX_IN_FEATURES (csrc/kan_ops.h:17).
constexpr int64_t kMaxInFeatures = 65535;
// Knots per feature row at the limit (G + 2k + 1).
constexpr int kMaxKnots = (int)kMaxDeg0Basis + 1;
// Largest basis count R = G + k under the limit (k = 1, G = 69).
constexpr int kMaxR = 70;

// Records a formatted message as this thread's last error and returns code.
int set_error(int code, const char* fmt, ...);
// Checks hipGetLastError() after a launch; records and returns KAN_ERR_HIP.
int check_launch(const char* what);
// Number of compute units of the current device (cached per device).
int device_cu_count();
// Workgroups of `threads` threads of `kernel` that fit on one CU at once (its
// register and LDS occupancy), cached per device and kernel; 1 if unknown.
int resident_blocks_per_cu(const void* kernel, int threads);

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroups are dealt to the 8 XCDs (each with its own L2) round-robin by
// id.  This bijective remap of the dispatch order gives each XCD a
// contiguous range of logical ids, so that neighbouring work items (tiles
// sharing operand slabs, features sharing cache lines) meet in one L2.
constexpr int kNumXcd = 8;
__device__ __forceinline__ int xcd_remap(int pid, int total) {
  const int per = total / kNumXcd, rem = total % kNumXcd;
  const int xcd = pid % kNumXcd, idx = pid / kNumXcd;
  return xcd * per + min(xcd, rem) + idx;
}
__host__ __device__ inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Width of one augmented basis row [H(n, 0..I*R-1) | silu(x(n, 0..I-1))],
// padded to a multiple of 4 elements so that rows start 16-byte aligned.
inline int64_t aug_width(int64_t I, int64_t R, bool has_base) {
  return round_up(I * R + (has_base ? I : 0), 4);
}

template <typename T>
struct alignas(4 * sizeof(T)) Vec4 {
  T v[4];
};

template <typename T>
__device__ __forceinline__ T silu_of(T x) {
  return x / (T(1) + exp(-x));
}

template <typename T>
__device__ __forceinline__ T silu_grad_of(T x) {
  const T sg = T(1) / (T(1) + exp(-x));
  return sg * (T(1) + x * (T(1) - sg));
}

template <>
__device__ __forceinline__ float silu_of<float>(float x) {
  return x / (1.0f + expf(-x));
}

template <>
__device__ __forceinline__ float silu_grad_of<float>(float x) {
  const float sg = 1.0f / (1.0f + expf(-x));
  return sg * (1.0f + x * (1.0f - sg));
}

// Order-q derivative of silu(x) = x s(x), s the logistic sigmoid, q = 0..4:
//   silu^(q) = x s^(q) + q s^(q-1), with d = s (1 - s) and
//   s^(1) = d, s^(2) = d (1 - 2 s), s^(3) = d (1 - 6 d),
//   s^(4) = d (1 - 2 s) (1 - 12 d).
// q = 0 and 1 are silu_of and silu_grad_of themselves, so the first-order
// kernels and this one agree bit for bit.  Higher q returns NaN.
constexpr int kMaxSiluOrder = 4;
template <typename T>
__device__ __forceinline__ T silu_deriv_of(T x, int q) {
  if (q == 0) return silu_of<T>(x);
  if (q == 1) return silu_grad_of<T>(x);
  const T sg = T(1) / (T(1) + exp(-x));
  const T d = sg * (T(1) - sg);
  if (q == 2) return x * (d * (T(1) - T(2) * sg)) + T(2) * d;
  if (q == 3) return x * (d * (T(1) - T(6) * d)) + T(3) * (d * (T(1) - T(2) * sg));
  if (q == 4)
    return x * (d * (T(1) - T(2) * sg) * (T(1) - T(12) * d)) + T(4) * (d * (T(1) - T(6) * d));
  return T(NAN);
}

// ---- optional HIP-event timing of kernel launches ---------------------------
// When enabled (kan_hip_timing_enable), every launch below records a pair of
// events on its stream together with the launch's algorithmic work (flops
// for contractions, bytes for the memory-bound kernels), so that a caller can
// read per-class average kernel durations without a profiler.
enum KernelClass {
  kClassContraction = 0,  // MFMA contraction GEMMs (forward, params, input)
  kClassBasis = 1,        // basis evaluation (+ silu block)
  kClassBasisGrad = 2,    // input-gradient contraction of the basis
  kClassEdge = 3,         // edge statistic forward
  kClassEdgeGrad = 4,     // edge statistic backward
  kClassOther = 5,        // packing / finalize kernels
  kClassStream = 6,       // streaming probes (bytes moved)
  kNumKernelClasses = 7
};

class TimedLaunch {
 public:
  TimedLaunch(int cls, hipStream_t st, double work);
  ~TimedLaunch();

 private:
  int slot_;
  hipStream_t st_;
};

// ---- launchers implemented in the .hip translation units -----------------

// float4 streaming probe over `bytes` (a multiple of 16): mode 0 writes a,
// 1 reads a, 2 copies a to b (kan_stream.hip).
int launch_stream_probe(int mode, void* a, void* b, int64_t bytes, hipStream_t st);

// Regulariser of one layer from its edge means (kan_reg.hip).
size_t edge_reg_ws_bytes(int64_t n);
template <typename T>
int launch_edge_reg(const T* a, int64_t n, double mu1, double mu2, T* reg, double* ws,
                    hipStream_t st);
template <typename T>
int launch_edge_reg_backward(const T* g, const T* a, int64_t n, double mu1, double mu2,
                             const double* ws, T* ga, hipStream_t st);

template <typename T>
int launch_basis(const T* x, const T* grid, T* out, int64_t ld_out, T* silu_out, int64_t n,
                 int64_t I, int G, int k, int impl, hipStream_t st, int64_t ld_silu = -1);

template <typename T>
int launch_basis_grad(const T* x, const T* grid, const T* gH, int64_t ld_g, const T* gbase,
                      T* gx, int64_t n, int64_t I, int G, int k, int impl, hipStream_t st,
                      int64_t ld_base = -1);
// The same from the compact input-side product (launch_gemm_ecomp): window
// values ew [n, I, k+1] (16-byte aligned) and base columns es [n, I] or null.
int launch_basis_grad_compact(const float* x, const float* grid, const float* ew,
                              const float* es, float* gx, int64_t n, int64_t I, int G, int k,
                              hipStream_t st);

// Order-`order` derivatives of the basis, [n, I, R] (order 0 = values; order
// > k gives zeros), each item's row times scale[n, i] when scale is given;
// and their contraction gx = scale * (sum_r gH * D^order B_r
// + gbase * silu^(order)(x)), gbase and scale optional ([n, I] each).
template <typename T>
int launch_basis_deriv(const T* x, const T* grid, const T* scale, T* out, int64_t n, int64_t I,
                       int G, int k, int order, hipStream_t st);

template <typename T>
int launch_basis_deriv_contract(const T* x, const T* grid, const T* gH, const T* gbase,
                                const T* scale, T* gx, int64_t n, int64_t I, int G, int k,
                                int order, hipStream_t st);

// out[e] = silu^(order)(x[e]) * w1[e] * w2[e] (w1, w2 optional; order <= 4).
template <typename T>
int launch_silu_deriv(const T* x, const T* w1, const T* w2, T* out, int64_t count, int order,
                      hipStream_t st);

template <typename T>
int launch_pack_basis(const T* basis, const T* x, T* aug, int64_t ld_aug, int64_t n, int64_t I,
                      int64_t R, bool has_base, hipStream_t st);

template <typename T>
int launch_build_waug(const T* sw, const T* scaler, const T* bw, T* waug, int64_t ld,
                      int64_t O, int64_t I, int64_t R, hipStream_t st);

// waug_t [kaug, O] = transpose of the first kaug columns of waug.
template <typename T>
int launch_build_waug_t(const T* sw, const T* scaler, const T* bw, T* waug_t, int64_t kaug,
                        int64_t O, int64_t I, int64_t R, hipStream_t st);

template <typename T>
int launch_param_grads(const T* part, int splits, int64_t split_stride, int64_t ld,
                       const T* sw, const T* scaler, T* gsw, T* gscaler, T* gbw, int64_t O,
                       int64_t I, int64_t R, hipStream_t st);

// Refit Gram matrices per feature (kan_refit.hip): gram [I, Rn, Rn] and
// cross [I, Rn, Ro] in float64 from feature-major samples xt [I, n].
template <typename T>
int launch_refit_gram(const T* xt, const T* grid_old, const T* grid_new, double* gram,
                      double* cross, int64_t n, int64_t I, int Go, int Gn, int k,
                      hipStream_t st);

enum GemmLayout {
  kLayoutNT = 0,  // C[m,n] = sum_k A[m*lda+k] * B[n*ldb+k]
  kLayoutTN = 1,  // C[m,n] = sum_k A[k*lda+m] * B[k*ldb+n]
  kLayoutNN = 2,  // C[m,n] = sum_k A[m*lda+k] * B[k*ldb+n]
  kLayoutTT = 3,  // C[m,n] = sum_k A[k*lda+m] * B[n*ldb+k]
};

// C (+ split * split_stride) = partial product over the split's K range.
template <typename T>
int launch_gemm(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda,
                const T* B, int64_t ldb, T* C, int64_t ldc, int splits, int64_t split_stride,
                hipStream_t st);

// fp32 input-side product E = D Waug (NT against Waug^T [N, K]) contracted in
// the GEMM epilogue with dB/dx and silu'(x) into dx [M, I]; part is a
// [M, I, 3 or 2] scratch of partial sums (kan_gemm.hip).
int launch_gemm_dx(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda, const float* B,
                   int64_t ldb, const float* x, const float* grid, int64_t I, int G, int k,
                   bool has_base, float* part, float* gx, hipStream_t st);
// Whether launch_gemm_dx takes this shape (the tile configuration it would
// pick leaves room for every block's knots and samples).
bool gemm_dx_supported(int64_t M, int64_t N, int64_t K, int64_t I, int G, int k, bool has_base);

// fp32 input-side product E = D Waug in compact form: of each (sample,
// feature) only the k+1 span-window values of its spline columns, ew
// [M, I, k+1], and the base columns es [M, I] (kan_gemm.hip); the input
// gradient then takes launch_basis_grad_compact.
int launch_gemm_ecomp(int64_t M, int64_t N, int64_t K, const float* A, int64_t lda,
                      const float* B, int64_t ldb, const float* x, const float* grid, int64_t I,
                      int G, int k, bool has_base, float* ew, float* es, hipStream_t st);
bool gemm_ecomp_supported(int64_t M, int64_t N, int64_t K, int64_t I, int G, int k,
                          bool has_base);

// General product C = op(A) op(B) for any transposition pair: the split
// count from gemm_pick_splits, partial slices in ws, then a fixed-order sum
// into C (kan_gemm.hip).  ws must hold matmul_ws_elems(...) elements, with
// the same max_slice_elems: a non-negative value bounds the split slices'
// total elements (the allocation-free inference's fixed scratch), -1 leaves
// the split count to the cost model alone.
template <typename T>
int64_t matmul_ws_elems(int layout, int64_t M, int64_t N, int64_t K,
                        int64_t max_slice_elems = -1);
template <typename T>
int launch_matmul(int layout, int64_t M, int64_t N, int64_t K, const T* A, int64_t lda,
                  const T* B, int64_t ldb, T* C, int64_t ldc, T* ws, hipStream_t st,
                  int64_t max_slice_elems = -1);

// Split count the GEMM scheduler would choose for a problem (1 = no split).
template <typename T>
int gemm_pick_splits(int64_t M, int64_t N, int64_t K, int64_t max_slice_elems = -1);

// fp64 edge statistic on MFMA (kan_edge_mfma64.hip), for R + 1 <= 16; the
// VALU kernels of kan_edge.hip serve wider rows.
bool edge_mfma64_applies(int64_t R);
int edge_mfma64_splits(int64_t n, int64_t I, int64_t O, bool backward);
int launch_edge_forward_mfma64(const double* s, const double* H, const double* bw,
                               const double* W, double* a, double* part, int splits, int64_t n,
                               int64_t I, int64_t O, int64_t R, hipStream_t st);
int launch_edge_param_mfma64(const double* ga, const double* s, const double* H,
                             const double* bw, const double* W, double* dbw, double* dW,
                             double* part, int splits, int64_t n, int64_t I, int64_t O, int64_t R,
                             hipStream_t st);
int launch_edge_input_mfma64(const double* ga, const double* s, const double* H,
                             const double* bw, const double* W, double* ds, double* dH,
                             int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st);

template <typename T>
int launch_edge_forward(const T* s, const T* H, const T* bw, const T* W, T* a, T* part,
                        int splits, int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st);

template <typename T>
int launch_edge_backward(const T* ga, const T* s, const T* H, const T* bw, const T* W, T* ds,
                         T* dH, T* dbw, T* dW, T* part, int splits, int64_t n, int64_t I,
                         int64_t O, int64_t R, hipStream_t st);

// Double backward of the edge statistic (VALU kernels, fp32 and fp64): the
// gradients of <u_ds, ds> + <u_dH, dH> + <u_dbw, dbw> + <u_dW, dW> with
// respect to ga, s, H, bw and W at a fixed sign pattern (kan_edge.hip).
size_t edge_double_backward_ws_elems(int64_t n, int64_t I, int64_t O, int64_t R);
template <typename T>
int launch_edge_double_backward(const T* ga, const T* s, const T* H, const T* bw, const T* W,
                                const T* u_ds, const T* u_dH, const T* u_dbw, const T* u_dW,
                                T* g_ga, T* g_s, T* g_H, T* g_bw, T* g_W, T* part, int64_t n,
                                int64_t I, int64_t O, int64_t R, hipStream_t st);

// Sample splits of the edge statistic's forward or parameter-gradient pass
// (dtype code selects the fp32 MFMA or the fp64 VALU kernels, which partition
// differently).
int edge_pick_splits(int dtype, int64_t n, int64_t I, int64_t O, int64_t R, bool backward);

// fp32 MFMA kernels of the edge statistic (kan_edge_mfma.hip).
int edge_mfma_splits(int64_t n, int64_t I, int64_t O, int64_t R, bool backward);
int launch_edge_forward_mfma(const float* s, const float* H, const float* bw, const float* W,
                             float* a, float* part, int splits, int64_t n, int64_t I, int64_t O,
                             int64_t R, hipStream_t st);
int launch_edge_backward_mfma(const float* ga, const float* s, const float* H, const float* bw,
                              const float* W, float* ds, float* dH, float* dbw, float* dW,
                              float* part, int splits, int64_t n, int64_t I, int64_t O, int64_t R,
                              hipStream_t st);
// Backward of a layer's output y = s bw^T + <H, W> and its edge statistic
// together (D = dL/dy folded into g); see edge_linear_fold_supported.
bool edge_linear_fold_supported(int64_t n, int64_t I, int64_t O, int64_t R);
int launch_edge_linear_backward_mfma(const float* ga, const float* D, const float* s,
                                     const float* H, const float* bw, const float* W, float* ds,
                                     float* dH, float* dbw, float* dW, float* part, int splits,
                                     int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st);
// Forward of the same layer: y = s bw^T + <H, W> and a = mean_n |phi| from one
// pass over phi (edge_ylin_fwd_kernel), with part holding edge_ylin_ws_bytes.
bool edge_ylin_supported(int64_t n, int64_t I, int64_t O, int64_t R);
size_t edge_ylin_ws_bytes(int64_t n, int64_t I, int64_t O);
int launch_edge_ylin_forward(const float* s, const float* H, const float* bw, const float* W,
                             float* y, float* a, float* part, int64_t n, int64_t I, int64_t O,
                             int64_t R, hipStream_t st);

}  // namespace kan
