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
// straight from global memory, through branch-free buffer loads.  Sums over
// samples may be split across workgroups (partial slices added in fixed
// order by the finalize kernels of kan_edge.hip); sums inside a workgroup run
// in fixed wave order, so results are deterministic.  Replaces csrc/kan_reg_cuda.cu:34-238 for float64.

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
// the forward takes 8 output tiles per block, 4 for layers of at most 64
// outputs (8 left half the block idle there); the parameter kernel takes 4
// output tiles per block (8 tiles: 2 waves per SIMD, 6 % slower, and half
// the block idle at O = 64); both load the next sample tile while the
// current one runs and hold 4 waves per SIMD with it (3 for the parameter
// kernel at 4 k-steps, which would spill at 4).  The parameter kernel reads
// its staged weights from LDS for every tile: kept in registers they left
// too few for the loaded-ahead tile.  The input kernel takes 4 sample tiles
// per wave, at 4 waves per SIMD where a block has more than 4 output tiles
// to loop over.
constexpr int kE64Threads = 256;  // 4 waves
constexpr int kE64OT = 8;         // output tiles of 16 per forward block (4 where O <= 64)
constexpr int kE64Out = kE64OT * 16;
constexpr int kE64POT = 4;        // output tiles of 16 per parameter block
constexpr int kE64NT = 4;         // sample tiles of 16 per wave (input product)
constexpr int kE64Stride = 17;    // LDS row stride (doubles) of the staged Wc rows

// Branch-free loads of sample rows Hc[n, c] (one 16-row tile at a time) and
// of weight rows: a tile's buffer resource covers only its rows below the range end,
// and a lane whose column lies past R (or in the other array) uses an offset
// outside every tile, so the hardware returns 0 for both.  (Loads written as
// "cond ? load : 0" became one exec-masked branch per load, and the compiler
// waited for all loads in flight where those branches joined, so nothing
// could be loaded ahead.)  The buffer intrinsic also keeps the loads where
// they are written; plain pointer loads would be moved to their use.
constexpr uint32_t kE64Oob = 0x80000000u;  // an offset outside every tile
constexpr int kE64Word3 = 0x00020000;      // gfx9 raw buffer, 32-bit data

// rows (at most max_rows of them) of row_doubles each from base
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc64(const double* base, int64_t rows,
                                                              int64_t max_rows,
                                                              int64_t row_doubles) {
  rows = rows < 0 ? 0 : (rows > max_rows ? max_rows : rows);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<double*>(base), (short)0,
                                           (int)(rows * row_doubles * 8), kE64Word3);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc64(const double* base, int64_t rows,
                                                              int64_t row_doubles) {
  return rows_rsrc64(base, rows, 16, row_doubles);
}

__device__ __forceinline__ double buf_ld64(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 0, 0);
  return __longlong_as_double((long long)(((unsigned long long)v.y << 32) | v.x));
}

// h | sv bitwise, where at most one of the two was loaded in range (the other
// reads 0): the value of Hc at the lane's column.  Opaque, so that the OR of
// two loaded-ahead values stays at the point of use (a plain OR of two
// loop-carried values is folded back to the loads, which then wait as soon as
// they are issued); it carries the wait states an MFMA reading a VALU result
// needs, which the compiler's hazard checks do not see inside the asm.
__device__ __forceinline__ double hc_or64(double h, double sv) {
  const unsigned long long hb = (unsigned long long)__double_as_longlong(h);
  const unsigned long long sb = (unsigned long long)__double_as_longlong(sv);
  unsigned lo, hi;
  asm volatile("v_or_b32 %0, %2, %3\n\tv_or_b32 %1, %4, %5\n\ts_nop 4"
               : "=&v"(lo), "=v"(hi)
               : "v"((unsigned)hb), "v"((unsigned)sb), "v"((unsigned)(hb >> 32)),
                 "v"((unsigned)(sb >> 32)));
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

// Stages Wc rows of outputs o0 .. o0 + ROWS - 1 (zero past O and past c = R)
// and ga / n of those outputs, with branch-free buffer loads: thread x
// stages column c = x % 16 of rows x / 16 + 16 p (from bw for c = 0, else
// from W), and all its loads are in flight before the first is used.
template <int ROWS>
__device__ __forceinline__ void stage_wc(double (*ws)[kE64Stride], double* gs,
                                         const double* __restrict__ ga,
                                         const double* __restrict__ bw,
                                         const double* __restrict__ W, int o0, int O, int I,
                                         int i, int R, double inv_n) {
  static_assert(ROWS % 16 == 0 && kE64Threads == 256, "16 rows per pass of 256 threads");
  constexpr int P = ROWS / 16;
  const int c = threadIdx.x & 15, rl = threadIdx.x >> 4;
  const int64_t IR = (int64_t)I * R;
  const bool has_bw = bw != nullptr;
  const double* bwb = has_bw ? bw : W;  // (no bw: its resource covers no rows)
  const uint32_t ow = (c >= 1 && c <= R) ? (uint32_t)(((int64_t)rl * IR + (c - 1)) * 8) : kE64Oob;
  const uint32_t ob = c == 0 ? (uint32_t)((int64_t)rl * I * 8) : kE64Oob;
  double v[P], vb[P], gv = 0.0;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int orow = o0 + 16 * p;
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc64(W + ((int64_t)orow * I + i) * R, O - orow, IR);
    const __amdgpu_buffer_rsrc_t rb =
        tile_rsrc64(bwb + (int64_t)orow * I + i, has_bw ? O - orow : 0, I);
    v[p] = buf_ld64(rw, ow);
    vb[p] = buf_ld64(rb, ob);
  }
  if (gs != nullptr) {
    const __amdgpu_buffer_rsrc_t rg = rows_rsrc64(ga + (int64_t)o0 * I + i, O - o0, ROWS, I);
    gv = buf_ld64(rg, threadIdx.x < ROWS ? (uint32_t)((int64_t)threadIdx.x * I * 8) : kE64Oob);
  }
#pragma unroll
  for (int p = 0; p < P; ++p)
    ws[16 * p + rl][c] = __longlong_as_double(__double_as_longlong(v[p]) |
                                              __double_as_longlong(vb[p]));
  if (gs != nullptr && threadIdx.x < ROWS) gs[threadIdx.x] = gv * inv_n;
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
// Each wave takes every fourth sample tile of the block's range, with the
// next tile's operands loaded while the current one runs (two register
// slots, branch-free buffer loads, as in the parameter kernel below).
template <int KS, int OT>
__global__ __launch_bounds__(kE64Threads, 4) void edge_fwd_mfma64_kernel(
    const double* __restrict__ s, const double* __restrict__ H, const double* __restrict__ bw,
    const double* __restrict__ W, double* __restrict__ out, int64_t n, int I, int O, int R,
    int64_t per_split, int ochunks, int final_out) {
  constexpr int OUT = OT * 16;
  __shared__ double ws[OUT][kE64Stride];
  __shared__ double red[4][OUT];
  const E64Block blk = e64_block(I, ochunks);
  const int o0 = blk.oc * OUT;
  stage_wc<OUT>(ws, nullptr, nullptr, bw, W, o0, O, I, blk.i, R, 0.0);
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
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
  // byte offsets of Hc[row r][c = 4k + q] within a tile, from H (c >= 1) or s (c = 0)
  const int64_t IR = (int64_t)I * R;
  const bool has_s = s != nullptr;
  const double* sb = has_s ? s : H;  // (no s: its resource covers no rows)
  uint32_t oa[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int c = 4 * k + q;
    oa[k] = (c >= 1 && c <= R) ? (uint32_t)(((int64_t)r * IR + (c - 1)) * 8) : kE64Oob;
  }
  const uint32_t oas = q == 0 ? (uint32_t)((int64_t)r * I * 8) : kE64Oob;
  auto load = [&](int64_t t0, double (&a)[KS], double& as) {
    const __amdgpu_buffer_rsrc_t th = tile_rsrc64(H + (t0 * I + blk.i) * R, ne - t0, IR);
    const __amdgpu_buffer_rsrc_t ts = tile_rsrc64(sb + t0 * I + blk.i, has_s ? ne - t0 : 0, I);
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = buf_ld64(th, oa[k]);
    as = buf_ld64(ts, oas);
  };
  auto compute = [&](const double (&a)[KS], double as) {
    double av[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) av[k] = k == 0 ? hc_or64(a[0], as) : a[k];
#pragma unroll
    for (int t = 0; t < OT; ++t) {
      f64x4 acc = zero4d();
#pragma unroll
      for (int k = 0; k < KS; ++k) acc = mfma64(av[k], b[t][k], acc);
      acc_abs[t] += (fabs(acc[0]) + fabs(acc[1])) + (fabs(acc[2]) + fabs(acc[3]));
    }
  };
  // Two tiles per pass while both are in range, then the odd last one (an
  // exit between the two tiles of a pass let the compiler sink the second
  // tile's loads past the first tile's work)
  double a0[KS], as0, a1[KS], as1;
  int64_t n0 = nb + 16 * wave;
  load(n0, a0, as0);
  for (; n0 + 64 < ne; n0 += 128) {
    __builtin_amdgcn_sched_barrier(0);
    load(n0 + 64, a1, as1);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out before this tile's wait
    compute(a0, as0);
    __builtin_amdgcn_sched_barrier(0);
    load(n0 + 128, a0, as0);
    __builtin_amdgcn_sched_barrier(0);
    compute(a1, as1);
  }
  if (n0 < ne) compute(a0, as0);
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
// Each wave takes every fourth sample tile of the block's range; the operands
// of its next tile are loaded while the current one runs (two register
// slots, branch-free buffer loads).
template <int KS>
__global__ __launch_bounds__(kE64Threads, KS == 4 ? 3 : 4) void edge_param_mfma64_kernel(
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
  stage_wc<OUT>(ws, gs, ga, bw, W, o0, O, I, blk.i, R, 1.0 / (double)n);
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
  f64x4 dw[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) dw[t] = zero4d();
  const int64_t nb = (int64_t)blk.split * per_split;
  const int64_t ne = min(n, nb + per_split);
  // byte offsets within a tile: phi's A operand Hc[row r][c = 4k + q] and
  // the product's B operand Hc[row 4v + q][c = r], from H (c >= 1) or s (c = 0)
  const int64_t IR = (int64_t)I * R;
  const bool has_s = s != nullptr;
  const double* sb = has_s ? s : H;  // (no s: its resource covers no rows)
  uint32_t oa[KS], ob[4];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int c = 4 * k + q;
    oa[k] = (c >= 1 && c <= R) ? (uint32_t)(((int64_t)r * IR + (c - 1)) * 8) : kE64Oob;
  }
  const uint32_t oas = q == 0 ? (uint32_t)((int64_t)r * I * 8) : kE64Oob;  // c = 0 at k = 0
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int64_t row = 4 * v + q;
    ob[v] = (r >= 1 && r <= R) ? (uint32_t)((row * IR + (r - 1)) * 8) : kE64Oob;
  }
  auto load = [&](int64_t t0, double (&a)[KS], double& as, double (&h)[4]) {
    const __amdgpu_buffer_rsrc_t th = tile_rsrc64(H + (t0 * I + blk.i) * R, ne - t0, IR);
    const __amdgpu_buffer_rsrc_t ts = tile_rsrc64(sb + t0 * I + blk.i, has_s ? ne - t0 : 0, I);
#pragma unroll
    for (int k = 0; k < KS; ++k) a[k] = buf_ld64(th, oa[k]);
    as = buf_ld64(ts, oas);
#pragma unroll
    for (int v = 0; v < 4; ++v) h[v] = buf_ld64(th, ob[v]);
  };
  auto compute = [&](const double (&a)[KS], double as, const double (&h)[4]) {
    double av[KS], hb[4];
#pragma unroll
    for (int k = 0; k < KS; ++k) av[k] = k == 0 ? hc_or64(a[0], as) : a[k];
    // the B operand's column c = 0 (lanes r = 0, row 4v + q) is s of that
    // row, which lane 4v + q (group q = 0) holds as its A operand's s value
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const double sv = __shfl(as, 4 * v + q);
      hb[v] = hc_or64(h[v], r == 0 ? sv : 0.0);
    }
    // the staged weights are read again for every tile (an opaque zero row
    // offset keeps the reads in the loop): held in registers across the loop
    // they left too few for the loaded-ahead tile at 4 waves per SIMD
    int z;
    asm volatile("s_mov_b32 %0, 0" : "=s"(z));
    const int rz = r + z;
#pragma unroll
    for (int t = 0; t < OT; ++t) {
      f64x4 phi = zero4d();
#pragma unroll
      for (int k = 0; k < KS; ++k) phi = mfma64(av[k], ws[16 * t + rz][4 * k + q], phi);
      const double gav = gs[16 * t + rz];  // column o = 16t + r of phi
#pragma unroll
      for (int v = 0; v < 4; ++v) dw[t] = mfma64(g_sign_d(gav, phi[v]), hb[v], dw[t]);
    }
  };
  // Two tiles per pass while both are in range, then the odd last one (as
  // in the forward kernel)
  double a0[KS], as0, h0[4], a1[KS], as1, h1[4];
  int64_t n0 = nb + 16 * wave;
  load(n0, a0, as0, h0);
  for (; n0 + 64 < ne; n0 += 128) {
    __builtin_amdgcn_sched_barrier(0);
    load(n0 + 64, a1, as1, h1);
    __builtin_amdgcn_sched_barrier(0);  // the loads go out before this tile's wait
    compute(a0, as0, h0);
    __builtin_amdgcn_sched_barrier(0);
    load(n0 + 128, a0, as0, h0);
    __builtin_amdgcn_sched_barrier(0);
    compute(a1, as1, h1);
  }
  if (n0 < ne) compute(a0, as0, h0);
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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
  const int64_t nw = (chunk * 4 + wave) * (16 * kE64NT);  // this wave's first sample
  // the wave's sample operands Hc[nw + 16j + r][c = 4k + q], branch-free (as
  // in the parameter kernel); column 0 (s) is OR-ed in where it is used, so
  // that these loads and the first weight chunk's are in flight together
  const int64_t IR = (int64_t)I * R;
  const bool has_s = s != nullptr;
  const double* sb = has_s ? s : H;
  double hs[kE64NT][KS], hs0[kE64NT];
  f64x4 dh[kE64NT];
#pragma unroll
  for (int j = 0; j < kE64NT; ++j) {
    const int64_t t0 = nw + 16 * j;
    const __amdgpu_buffer_rsrc_t th = tile_rsrc64(H + (t0 * I + i) * R, n - t0, IR);
    const __amdgpu_buffer_rsrc_t ts = tile_rsrc64(sb + t0 * I + i, has_s ? n - t0 : 0, I);
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int c = 4 * k + q;
      hs[j][k] = buf_ld64(th, (c >= 1 && c <= R) ? (uint32_t)(((int64_t)r * IR + (c - 1)) * 8)
                                                 : kE64Oob);
    }
    hs0[j] = buf_ld64(ts, q == 0 ? (uint32_t)((int64_t)r * I * 8) : kE64Oob);
    dh[j] = zero4d();
  }
  const double inv_n = 1.0 / (double)n;
  for (int o0 = 0; o0 < O; o0 += kE64Out) {
    __syncthreads();  // the previous chunk's weights are no longer read
    stage_wc<kE64Out>(ws, gs, ga, bw, W, o0, O, I, i, R, inv_n);
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
        for (int k = 0; k < KS; ++k)
          pt = mfma64(aw[k], k == 0 ? hc_or64(hs[j][0], hs0[j]) : hs[j][k], pt);
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
