// fp64 edge statistic on MFMA (v_mfma_f64_16x16x4f64), for R + 1 <= 16.
// For one input feature i the edge values of a sample block are a small
// matrix product,
//     phi_i[n, o] = sum_c Hc[n, c] Wc[o, c],   c = 0..R,
// with Hc[n] = [s[n,i], H[n,i,0..R-1]] and Wc[o] = [bw[o,i], W[o,i,0..R-1]]:
//   forward   a[o,i]   = (1/n) sum_n |phi[n,o]|
//   params    dWc[o,c] = sum_n g[n,o] Hc[n,c]       g = ga[o,i] sign(phi) / n
//   inputs    dHc[n,c] = sum_o g[n,o] Wc[o,c]
// The fp64 16x16x4 MFMA takes, in lane (q = lane/16, r = lane%16), the
// operand A[row r, k = q] and B[k = q, col r] of each 4-deep step, and leaves
// C[row q + 4v, col r] in accumulator entry v.  So a product whose
// contraction runs over the rows of an accumulator takes entry v of that
// accumulator as its step-v operand (k = 4v + q is the lane's own row): the
// parameter product uses phi's accumulator as its A operand directly, and the
// input product, whose contraction runs over outputs, uses the accumulator
// of phi^T (computed from the same operands with A and B swapped, three more
// MFMAs instead of a transposition through LDS).  The weights of a block's
// outputs are staged in LDS (rows of 16 c, zero past R); sample operands come
// straight from global memory.  Sums over samples may be split across
// workgroups (partial slices added in fixed order by the finalize kernels of
// kan_edge.hip); sums inside a workgroup run in fixed wave order, so results
// are deterministic.  Replaces csrc/kan_reg_cuda.cu:34-238 for float64.

#include "kan_common.h"

namespace kan {
namespace {

typedef double f64x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f64x4 mfma64(double a, double b, f64x4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f64x4 zero4d() {
  f64x4 z;
  z[0] = z[1] = z[2] = z[3] = 0.0;
  return z;
}

// g * sign(v) with sign(0) = 0, formed by flipping g's sign bit with v's and
// a zero test (instead of two compares, a subtraction, a conversion and a
// multiply); equal to g * sign(v) up to the sign of a zero result.
__device__ __forceinline__ double g_sign_d(double g, double v) {
  const unsigned long long bits = (unsigned long long)__double_as_longlong(g) ^
                                  ((unsigned long long)__double_as_longlong(v) &
                                   0x8000000000000000ULL);
  return v != 0.0 ? __longlong_as_double((long long)bits) : 0.0;
}

// Tilings chosen by a sweep on MI355X at c4's layers (n = 16384, R + 1 = 12):
// the forward prefetches the next sample tile (it holds 4 waves per SIMD
// with it) and takes 8 output tiles per block, 4 for layers of at most 64
// outputs (8 left half the block idle there); the parameter kernel does not
// prefetch (at 1-2 waves per SIMD that cost a third of its rate) and takes
// 4 output tiles per block at 4 waves per SIMD (3 for even k-step counts,
// which would spill at 4; 8 tiles: 2 waves, 6 % slower, and half the block
// idle at O = 64); the input kernel takes 4 sample tiles per wave, at 4
// waves per SIMD where a block has more than 4 output tiles to loop over.
constexpr int kE64Threads = 256;  // 4 waves
constexpr int kE64OT = 8;         // output tiles of 16 per forward block (4 where O <= 64)
constexpr int kE64Out = kE64OT * 16;
constexpr int kE64POT = 4;        // output tiles of 16 per parameter block
constexpr int kE64NT = 4;         // sample tiles of 16 per wave (input product)
constexpr int kE64Stride = 17;    // LDS row stride (doubles) of the staged Wc rows

// Hc[n, c] of feature i (c = 0: s, else H[.., c - 1]); 0 at or past nend or c > R.
__device__ __forceinline__ double hc_at(const double* __restrict__ s,
                                        const double* __restrict__ H, int64_t n, int64_t nend,
                                        int I, int i, int R, int c) {
  if (n >= nend || c > R) return 0.0;
  if (c == 0) return s != nullptr ? s[n * I + i] : 0.0;
  return H[(n * I + i) * R + (c - 1)];
}

// Stages Wc rows of outputs o0 .. o0 + rows - 1 (zero past O and past c = R)
// and ga / n of those outputs.
__device__ __forceinline__ void stage_wc(double (*ws)[kE64Stride], double* gs,
                                         const double* __restrict__ ga,
                                         const double* __restrict__ bw,
                                         const double* __restrict__ W, int o0, int rows, int O,
                                         int I, int i, int R, double inv_n) {
  for (int e = threadIdx.x; e < rows * 16; e += blockDim.x) {
    const int ol = e >> 4, c = e & 15;
    const int o = o0 + ol;
    double v = 0.0;
    if (o < O && c <= R) {
      const int64_t ei = (int64_t)o * I + i;
      v = c == 0 ? (bw != nullptr ? bw[ei] : 0.0) : W[ei * R + (c - 1)];
    }
    ws[ol][c] = v;
  }
  if (gs != nullptr)
    for (int ol = threadIdx.x; ol < rows; ol += blockDim.x) {
      const int o = o0 + ol;
      gs[ol] = o < O ? ga[(int64_t)o * I + i] * inv_n : 0.0;
    }
}

// (feature i, output chunk, sample split) of this block
struct E64Block {
  int i, oc, split;
};
// Output chunks vary fastest, so the blocks that read one feature's sample
// rows run side by side on one XCD (xcd_remap) and share them in its L2.
__device__ __forceinline__ E64Block e64_block(int I, int ochunks) {
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  E64Block b;
  b.oc = bid % ochunks;
  const int rest = bid / ochunks;
  b.i = rest % I;
  b.split = rest / I;
  return b;
}

// Forward: a[o, i] (or the split's partial sum) for the block's 16 * OT outputs.
template <int KS, int OT>
__global__ __launch_bounds__(kE64Threads) void edge_fwd_mfma64_kernel(
    const double* __restrict__ s, const double* __restrict__ H, const double* __restrict__ bw,
    const double* __restrict__ W, double* __restrict__ out, int64_t n, int I, int O, int R,
    int64_t per_split, int ochunks, int final_out) {
  constexpr int OUT = OT * 16;
  __shared__ double ws[OUT][kE64Stride];
  __shared__ double red[4][OUT];
  const E64Block blk = e64_block(I, ochunks);
  const int o0 = blk.oc * OUT;
  stage_wc(ws, nullptr, nullptr, bw, W, o0, OUT, O, I, blk.i, R, 0.0);
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
  double b[OT][KS];
#pragma unroll
  for (int t = 0; t < OT; ++t)
#pragma unroll
    for (int k = 0; k < KS; ++k) b[t][k] = ws[16 * t + r][4 * k + q];
  double acc_abs[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) acc_abs[t] = 0.0;
  const int64_t nb = (int64_t)blk.split * per_split;
  const int64_t ne = min(n, nb + per_split);
  double a[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) a[k] = hc_at(s, H, nb + 16 * wave + r, ne, I, blk.i, R, 4 * k + q);
  for (int64_t n0 = nb + 16 * wave; n0 < ne; n0 += 64) {
    double an[KS];  // the wave's next sample tile, loaded ahead
#pragma unroll
    for (int k = 0; k < KS; ++k) an[k] = hc_at(s, H, n0 + 64 + r, ne, I, blk.i, R, 4 * k + q);
#pragma unroll
    for (int t = 0; t < OT; ++t) {
      f64x4 acc = zero4d();
#pragma unroll
      for (int k = 0; k < KS; ++k) acc = mfma64(a[k], b[t][k], acc);
      acc_abs[t] += (fabs(acc[0]) + fabs(acc[1])) + (fabs(acc[2]) + fabs(acc[3]));
    }
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = an[k];
  }
  // lanes r, r + 16, r + 32, r + 48 hold the same output column: add them,
  // then the waves' sample shares in wave order
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    double v = acc_abs[t];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (q == 0) red[wave][16 * t + r] = v;
  }
  __syncthreads();
  for (int ol = threadIdx.x; ol < OUT; ol += blockDim.x) {
    const int o = o0 + ol;
    if (o >= O) continue;
    const double v = ((red[0][ol] + red[1][ol]) + red[2][ol]) + red[3][ol];
    const int64_t e = (int64_t)o * I + blk.i;
    if (final_out) out[e] = v / (double)n;
    else out[(int64_t)blk.split * ((int64_t)O * I) + e] = v;
  }
}

// Parameters: dWc[o, c] over the block's samples for its 16 * kE64POT outputs.
template <int KS>
__global__ __launch_bounds__(kE64Threads, KS % 2 == 1 ? 4 : 3) void edge_param_mfma64_kernel(
    const double* __restrict__ ga, const double* __restrict__ s, const double* __restrict__ H,
    const double* __restrict__ bw, const double* __restrict__ W, double* __restrict__ dbw,
    double* __restrict__ dW, double* __restrict__ part, int64_t n, int I, int O, int R,
    int64_t per_split, int ochunks, int final_out) {
  constexpr int OT = kE64POT;
  constexpr int OUT = OT * 16;
  __shared__ double ws[OUT][kE64Stride];
  __shared__ double gs[OUT];
  __shared__ double red[OUT][kE64Stride];
  const E64Block blk = e64_block(I, ochunks);
  const int o0 = blk.oc * OUT;
  stage_wc(ws, gs, ga, bw, W, o0, OUT, O, I, blk.i, R, 1.0 / (double)n);
  __syncthreads();
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
  f64x4 dw[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) dw[t] = zero4d();
  const int64_t nb = (int64_t)blk.split * per_split;
  const int64_t ne = min(n, nb + per_split);
  double a[KS], hb[4];
  {
    const int64_t n0 = nb + 16 * wave;
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = hc_at(s, H, n0 + r, ne, I, blk.i, R, 4 * k + q);
#pragma unroll
    for (int v = 0; v < 4; ++v) hb[v] = hc_at(s, H, n0 + 4 * v + q, ne, I, blk.i, R, r);
  }
  for (int64_t n0 = nb + 16 * wave; n0 < ne; n0 += 64) {
#pragma unroll
    for (int t = 0; t < OT; ++t) {
      f64x4 phi = zero4d();
#pragma unroll
      for (int k = 0; k < KS; ++k) phi = mfma64(a[k], ws[16 * t + r][4 * k + q], phi);
      const double gav = gs[16 * t + r];  // column o = 16t + r of phi
#pragma unroll
      for (int v = 0; v < 4; ++v) dw[t] = mfma64(g_sign_d(gav, phi[v]), hb[v], dw[t]);
    }
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = hc_at(s, H, n0 + 64 + r, ne, I, blk.i, R, 4 * k + q);
#pragma unroll
    for (int v = 0; v < 4; ++v) hb[v] = hc_at(s, H, n0 + 64 + 4 * v + q, ne, I, blk.i, R, r);
  }
  // dw[t]: lane (q, r) holds dWc[o = 16t + q + 4v][c = r]; add the waves'
  // sample shares in wave order through LDS
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < OT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          double* cell = &red[16 * t + q + 4 * v][r];
          *cell = (w == 0 ? 0.0 : *cell) + dw[t][v];
        }
    }
    __syncthreads();
  }
  const int R1 = R + 1;
  for (int e2 = threadIdx.x; e2 < OUT * 16; e2 += blockDim.x) {
    const int ol = e2 >> 4, c = e2 & 15;
    const int o = o0 + ol;
    if (o >= O || c >= R1) continue;
    const double v = red[ol][c];
    const int64_t e = (int64_t)o * I + blk.i;
    if (final_out) {
      if (c == 0) {
        if (dbw != nullptr) dbw[e] = v;
      } else if (dW != nullptr) {
        dW[e * R + (c - 1)] = v;
      }
    } else {
      part[((int64_t)blk.split * ((int64_t)O * I) + e) * R1 + c] = v;
    }
  }
}

// Inputs: dHc[n, c] summed over every output, for the block's samples (each
// wave kE64NT tiles of 16); the outputs' weights are staged kE64Out at a time.
template <int KS, int MINB>
__global__ __launch_bounds__(kE64Threads, MINB) void edge_input_mfma64_kernel(
    const double* __restrict__ ga, const double* __restrict__ s, const double* __restrict__ H,
    const double* __restrict__ bw, const double* __restrict__ W, double* __restrict__ ds,
    double* __restrict__ dH, int64_t n, int I, int O, int R) {
  __shared__ double ws[kE64Out][kE64Stride];
  __shared__ double gs[kE64Out];
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int i = bid % I;
  const int64_t chunk = bid / I;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
  const int64_t nw = (chunk * 4 + wave) * (16 * kE64NT);  // this wave's first sample
  double hs[kE64NT][KS];
  f64x4 dh[kE64NT];
#pragma unroll
  for (int j = 0; j < kE64NT; ++j) {
#pragma unroll
    for (int k = 0; k < KS; ++k) hs[j][k] = hc_at(s, H, nw + 16 * j + r, n, I, i, R, 4 * k + q);
    dh[j] = zero4d();
  }
  const double inv_n = 1.0 / (double)n;
  for (int o0 = 0; o0 < O; o0 += kE64Out) {
    __syncthreads();  // the previous chunk's weights are no longer read
    stage_wc(ws, gs, ga, bw, W, o0, kE64Out, O, I, i, R, inv_n);
    __syncthreads();
    const int tiles = min(kE64OT, (O - o0 + 15) / 16);
    for (int t = 0; t < tiles; ++t) {
      double aw[KS], bwv[4], gq[4];
#pragma unroll
      for (int k = 0; k < KS; ++k) aw[k] = ws[16 * t + r][4 * k + q];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        bwv[v] = ws[16 * t + 4 * v + q][r];
        gq[v] = gs[16 * t + q + 4 * v];
      }
#pragma unroll
      for (int j = 0; j < kE64NT; ++j) {
        // phi^T: lane (q, r) holds phi[n = nw + 16j + r][o = o0 + 16t + q + 4v]
        f64x4 pt = zero4d();
#pragma unroll
        for (int k = 0; k < KS; ++k) pt = mfma64(aw[k], hs[j][k], pt);
#pragma unroll
        for (int v = 0; v < 4; ++v) dh[j] = mfma64(g_sign_d(gq[v], pt[v]), bwv[v], dh[j]);
      }
    }
  }
  // dh[j]: lane (q, r) holds dHc[n = nw + 16j + q + 4v][c = r]
  if (r > R) return;
#pragma unroll
  for (int j = 0; j < kE64NT; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t nn = nw + 16 * j + q + 4 * v;
      if (nn >= n) continue;
      const int64_t f = nn * I + i;
      if (r == 0) {
        if (ds != nullptr) ds[f] = dh[j][v];
      } else if (dH != nullptr) {
        dH[f * R + (r - 1)] = dh[j][v];
      }
    }
}

#define KAN_E64_KS(R1, ...)                        \
  do {                                             \
    const int ks_ = ((R1) + 3) / 4;                \
    if (ks_ <= 1) { constexpr int KS = 1; __VA_ARGS__; }        \
    else if (ks_ == 2) { constexpr int KS = 2; __VA_ARGS__; }   \
    else if (ks_ == 3) { constexpr int KS = 3; __VA_ARGS__; }   \
    else { constexpr int KS = 4; __VA_ARGS__; }                 \
  } while (0)

}  // namespace

bool edge_mfma64_applies(int64_t R) { return R + 1 <= 16; }

// Sample splits of the forward and parameter kernels: about 8 blocks per CU
// (I features x output chunks x splits), each split at least 4 sample tiles
// per wave.  The backward's count sizes the [splits, O, I, R + 1] partials
// of edge_param_finalize, the forward's the [splits, O, I] ones of
// edge_forward_finalize.
static int fwd_tiles(int64_t O) { return O <= 64 ? 4 : kE64OT; }

int edge_mfma64_splits(int64_t n, int64_t I, int64_t O, bool backward) {
  const int64_t blocks = I * ceil_div(O, 16 * (backward ? kE64POT : fwd_tiles(O)));
  const int64_t target = 8LL * device_cu_count();
  int64_t s = ceil_div(target, blocks > 0 ? blocks : 1);
  const int64_t cap = ceil_div(n, 4 * 16 * 4);
  if (s > cap) s = cap;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return (int)s;
}

int launch_edge_forward_mfma64(const double* s, const double* H, const double* bw,
                               const double* W, double* a, double* part, int splits, int64_t n,
                               int64_t I, int64_t O, int64_t R, hipStream_t st) {
  const int ot = fwd_tiles(O);
  const int64_t ochunks = ceil_div(O, 16 * ot);
  const int64_t blocks = I * ochunks * splits;
  if (blocks > 2147483647LL) return set_error(KAN_ERR_LIMIT, "edge_abs_mean: too many blocks");
  const int64_t per_split = round_up(ceil_div(n, splits), 64);
  const bool fin = splits == 1;
  const int R1 = (int)R + 1;
  TimedLaunch timed(kClassEdge, st, 2.0 * (double)n * (double)O * (double)I * (double)R1);
  if (ot == 4)
    KAN_E64_KS(R1, hipLaunchKernelGGL((edge_fwd_mfma64_kernel<KS, 4>), dim3((unsigned)blocks),
                                      dim3(kE64Threads), 0, st, s, H, bw, W, fin ? a : part, n,
                                      (int)I, (int)O, (int)R, per_split, (int)ochunks, (int)fin));
  else
    KAN_E64_KS(R1, hipLaunchKernelGGL((edge_fwd_mfma64_kernel<KS, kE64OT>), dim3((unsigned)blocks),
                                      dim3(kE64Threads), 0, st, s, H, bw, W, fin ? a : part, n,
                                      (int)I, (int)O, (int)R, per_split, (int)ochunks, (int)fin));
  return check_launch("edge_abs_mean (fp64 MFMA)");
}

int launch_edge_param_mfma64(const double* ga, const double* s, const double* H,
                             const double* bw, const double* W, double* dbw, double* dW,
                             double* part, int splits, int64_t n, int64_t I, int64_t O, int64_t R,
                             hipStream_t st) {
  const int64_t ochunks = ceil_div(O, 16 * kE64POT);
  const int64_t blocks = I * ochunks * splits;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "edge_abs_mean_backward: too many blocks");
  const int64_t per_split = round_up(ceil_div(n, splits), 64);
  const bool fin = splits == 1;
  const int R1 = (int)R + 1;
  TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
  KAN_E64_KS(R1, hipLaunchKernelGGL((edge_param_mfma64_kernel<KS>), dim3((unsigned)blocks),
                                    dim3(kE64Threads), 0, st, ga, s, H, bw, W, dbw, dW, part, n,
                                    (int)I, (int)O, (int)R, per_split, (int)ochunks, (int)fin));
  return check_launch("edge_abs_mean_backward(params, fp64 MFMA)");
}

int launch_edge_input_mfma64(const double* ga, const double* s, const double* H,
                             const double* bw, const double* W, double* ds, double* dH,
                             int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st) {
  const int64_t chunks = ceil_div(n, 4 * 16 * kE64NT);
  const int64_t blocks = I * chunks;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "edge_abs_mean_backward: too many blocks");
  const int R1 = (int)R + 1;
  TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
  if (O > 64)
    KAN_E64_KS(R1, hipLaunchKernelGGL((edge_input_mfma64_kernel<KS, 4>), dim3((unsigned)blocks),
                                      dim3(kE64Threads), 0, st, ga, s, H, bw, W, ds, dH, n,
                                      (int)I, (int)O, (int)R));
  else
    KAN_E64_KS(R1, hipLaunchKernelGGL((edge_input_mfma64_kernel<KS, 1>), dim3((unsigned)blocks),
                                      dim3(kE64Threads), 0, st, ga, s, H, bw, W, ds, dH, n,
                                      (int)I, (int)O, (int)R));
  return check_launch("edge_abs_mean_backward(inputs, fp64 MFMA)");
}

}  // namespace kan
