// fp32 edge statistic on MFMA.  For one input feature i the edge values of
// a sample block are a small matrix product,
//     phi_i[n, o] = sum_c Hc[n, c] Wc[o, c],   c = 0..R  (K = R + 1),
// with the augmented rows Hc[n] = [s[n,i], H[n,i,0..R-1]] and
// Wc[o] = [bw[o,i], W[o,i,0..R-1]], so phi never leaves registers:
//   forward   a[o,i]   = (1/n) sum_n |phi[n,o]|
//   params    dWc[o,c] = sum_n g[n,o] Hc[n,c]       g = ga[o,i] sign(phi) / n
//   inputs    dHc[n,c] = sum_o g[n,o] Wc[o,c]
// All products run v_mfma_f32_16x16x4f32 on 16x16 tiles.  Operand lane
// (q = lane/16, r = lane%16) supplies row (or column) r at k = 4s + q of
// step s; the accumulator of lane (q, r) holds column r, rows 4q + v
// (v = 0..3).  The backward kernels feed that accumulator directly as the
// operand of a second MFMA whose contraction index runs over those rows:
// step v of the second product, lane group q, uses k = 4q + v -- exactly the
// lane's own accumulator entry v -- and the other operand is loaded in the
// same k order (a permutation of the sum, not of the result).  The small
// dimension R + 1 is padded to whole k-steps of 4 and column tiles of 16.
// Replaces csrc/kan_reg_cuda.cu:34-238 for float32 (float64 keeps the VALU
// kernels of kan_edge.hip).  Sums over samples may be split across
// workgroups; each split writes its own partial slice, added in a fixed order
// by the finalize kernels, so results are deterministic.

#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "kan_common.h"

namespace kan {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kEdgeMfThreads = 256;  // 4 waves
// Sample ranges of splits and waves are whole groups of 4 tiles of 16, so
// that the forward kernel's prefetch loop has no early exit (an exit would
// make the compiler wait for every load in flight at the loop head); tiles
// past the last sample are read as zeros.
constexpr int64_t kEdgeRowQuant = 64;
// Output layout of the forward and parameter kernels: each wave owns OT
// 16-wide output tiles; WS waves split a block's samples between them (their
// partial sums meet in LDS, in wave order), and WO = 4 / WS waves cover
// different outputs, so a block covers WO * OT * 16 outputs.  Narrow layers
// (small O) use WS > 1 instead of leaving waves idle.
template <int OT, int WS>
struct EdgeTiling {
  static constexpr int kWO = 4 / WS;
  static constexpr int kBlockOut = kWO * OT * 16;
  static_assert(kWO * WS == 4, "4 waves per block");
};

__device__ __forceinline__ f32x4 mfma16(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// c / d for 0 <= c < 2^16 and inv_d = 1/d (d >= 1): exact, since (c + 0.5)/d
// lies at least 0.5/d from an integer and the float product errs far less
__device__ __forceinline__ int small_div_f(int c, float inv_d) {
  return (int)(((float)c + 0.5f) * inv_d);
}

__device__ __forceinline__ f32x4 zero4() {
  f32x4 z;
  z[0] = z[1] = z[2] = z[3] = 0.0f;
  return z;
}

// g * sign(v) with sign(0) = 0, formed by flipping g's sign bit with v's
// (a copysign and a zero test instead of two compares, a subtraction, a
// conversion and a multiply); bit-identical to g * sign(v).
__device__ __forceinline__ float g_sign(float g, float v) {
  const unsigned bits = __float_as_uint(g) ^ (__float_as_uint(v) & 0x80000000u);
  return v != 0.0f ? __uint_as_float(bits) : 0.0f;
}

// Buffer-resource loads of the augmented sample values Hc[n, c] of feature
// i, one tile of 16 rows at a time (n0 wave-uniform): H rows lie I*R floats
// apart, s rows I floats apart.  A tile's resource covers only its rows below
// ne, and a lane whose column lies past R (or in the other array) uses an
// offset past every tile's range, so the hardware returns 0 for both: no
// branch, select or clamp around a load.  The loads go through the buffer
// intrinsic rather than plain pointer loads, which the compiler would move
// from the prefetch point to the point of use (a phi of loads becomes a load
// of a phi), leaving nothing in flight.
constexpr uint32_t kBufOob = 0x80000000u;      // an offset outside every tile
constexpr int kBufWord3 = 0x00020000;          // gfx9 raw buffer, 32-bit data

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const float* base, int64_t rows,
                                                            int64_t row_floats) {
  rows = rows < 0 ? 0 : (rows > 16 ? 16 : rows);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0,
                                           (int)(rows * row_floats * 4), kBufWord3);
}

// (the builtin returns the 32 bits as an integer: reinterpret, not convert)
__device__ __forceinline__ float buf_ld(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0));
}

// KS consecutive floats at byte offset off (16-byte loads, then the rest in
// one 12-, 8- or 4-byte load)
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x3v __attribute__((ext_vector_type(3)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
template <int KS>
__device__ __forceinline__ void buf_ld_run(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                           float (&d)[KS]) {
#pragma unroll
  for (int j = 0; j + 4 <= KS; j += 4) {
    const u32x4v v = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(off + 4 * j), 0, 0);
    d[j] = __uint_as_float(v.x);
    d[j + 1] = __uint_as_float(v.y);
    d[j + 2] = __uint_as_float(v.z);
    d[j + 3] = __uint_as_float(v.w);
  }
  constexpr int j = KS / 4 * 4;
  if constexpr (KS - j == 3) {
    const u32x3v v = __builtin_amdgcn_raw_buffer_load_b96(rs, (int)(off + 4 * j), 0, 0);
    d[j] = __uint_as_float(v.x);
    d[j + 1] = __uint_as_float(v.y);
    d[j + 2] = __uint_as_float(v.z);
  } else if constexpr (KS - j == 2) {
    const u32x2v v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(off + 4 * j), 0, 0);
    d[j] = __uint_as_float(v.x);
    d[j + 1] = __uint_as_float(v.y);
  } else if constexpr (KS - j == 1) {
    d[j] = buf_ld(rs, off + 4 * j);
  }
}

// The two resources of the tile at n0 (s's covers nothing without s).
struct HcTile {
  __amdgpu_buffer_rsrc_t h, s;
};

struct HcRows {
  const float* s;  // (H in place of a missing s, whose rows then count as 0)
  const float* H;
  int64_t I, R;
  int i;
  bool has_s;
  __device__ HcRows(const float* s_, const float* H_, int64_t I_, int64_t R_, int i_)
      : s(s_ != nullptr ? s_ : H_), H(H_), I(I_), R(R_), i(i_), has_s(s_ != nullptr) {}
  __device__ __forceinline__ HcTile tile(int64_t n0, int64_t ne) const {
    HcTile t;
    t.h = tile_rsrc(H + (n0 * I + i) * R, ne - n0, I * R);
    t.s = tile_rsrc(s + n0 * I + i, has_s ? ne - n0 : 0, I);
    return t;
  }
  // byte offsets of row rr, column c within a tile, into H and into s
  __device__ __forceinline__ uint32_t off_h(int rr, int c) const {
    return (c >= 1 && c <= R) ? (uint32_t)(((int64_t)rr * I * R + (c - 1)) * 4) : kBufOob;
  }
  __device__ __forceinline__ uint32_t off_s(int rr, int c) const {
    return c == 0 ? (uint32_t)((int64_t)rr * I * 4) : kBufOob;
  }
  // byte offset of H column col of row rr within a tile
  __device__ __forceinline__ uint32_t off_col(int rr, int col) const {
    return (uint32_t)(((int64_t)rr * I * R + col) * 4);
  }
};

// Contraction slots of phi = Hc Wc^T.  Slot (k-step k, lane group q) of a
// sample row holds one augmented column c, the same in the A operand (the
// row) and the B operand (the weights), so any assignment of columns to
// slots gives phi.  Lane group q takes a contiguous run of KS H columns of
// its row, loaded with one multi-dword load: its nominal run is
// [st, st + KS), st = R - KS (q + 1), so the four runs tile the row from its
// end.  A group whose nominal start is negative loads [0, KS) instead and
// owns only columns [0, st + KS) of it (the rest are other groups' columns,
// given weight 0); the group whose nominal run holds column -1 carries the
// base column c = 0 (from s) in its last slot.  KS <= R for every k-step
// class, so a run never leaves its feature's R columns: a tile's resource
// holds a run wholly or not at all.  (One load per row and tile instead of
// one per k-step: the scattered single-column loads kept the texture units
// busy at 16 rows per quarter-wave and instruction.)
template <int KS>
struct PhiSlots {
  int st;      // nominal run start R - KS (q + 1)
  int col0;    // first H column loaded
  bool owner;  // the last slot carries s (c = 0)
  __device__ PhiSlots(int q, int R) : st(R - KS * (q + 1)) {
    col0 = st > 0 ? st : 0;
    owner = st <= -1 && st + KS > -1;
  }
  // augmented column of slot k (-1: none; weight 0)
  __device__ __forceinline__ int c(int k) const {
    if (st >= 0) return st + k + 1;
    if (k < st + KS) return k + 1;
    return (owner && k == KS - 1) ? 0 : -1;
  }
  // AND mask of the loaded value in the last slot (0 where s replaces it)
  __device__ __forceinline__ uint32_t keep() const { return owner ? 0u : 0xffffffffu; }
};

// Where column 0 can occur a lane loads from both arrays; at most one of the
// two is in range, so OR-ing their bits gives the value exactly.  The OR is
// taken where the tile is used, as an opaque instruction: a plain OR of two
// loop-carried values is folded back to the loads (an OR of phis becomes a
// phi of ORs), which would then wait for them as soon as they are issued.
// The compiler's hazard checks do not see inside the asm, so it carries the
// wait states an MFMA reading a VALU result needs (2 on this ISA; 5 given).
__device__ __forceinline__ float hc_or(float h, float sv) {
  float v;
  asm volatile("v_or_b32 %0, %1, %2\n\ts_nop 4" : "=v"(v) : "v"(h), "v"(sv));
  return v;
}

// The last slot of a phi run: the loaded H value, or s in the group that
// carries the base column (keep = 0 there; sv reads 0 in every other group),
// as one opaque instruction for the reasons given at hc_or.
__device__ __forceinline__ float hc_sel(float h, uint32_t keep, float sv) {
  float v;
  asm volatile("v_and_or_b32 %0, %1, %2, %3\n\ts_nop 4" : "=v"(v) : "v"(h), "v"(keep), "v"(sv));
  return v;
}

// augmented weight value Wc[o, c]
__device__ __forceinline__ float wc_val(const float* __restrict__ bw, const float* __restrict__ W,
                                        int64_t o, int I, int i, int R, int c) {
  const int64_t e = o * I + i;
  if (c == 0) return bw != nullptr ? bw[e] : 0.0f;
  return W[e * R + (c - 1)];
}

struct EdgeGeom {
  int64_t n;
  int I, O, R;
  int64_t per_split;  // samples per split (multiple of kEdgeRowQuant)
  int ochunks;        // output chunks of kBlockOut
  int splits;
};

// Forward: block (i, output chunk, split); wave w owns kOT output tiles.
// KS = ceil((R+1)/4) k-steps.  The A fragments of the next P sample tiles are
// in flight while the current tile runs (P = 4 for KS <= 4, fewer for wider
// K to bound registers).
template <int KS, int OT, int WS>
__global__ __launch_bounds__(kEdgeMfThreads) void edge_fwd_mfma_kernel(
    const float* __restrict__ s, const float* __restrict__ H, const float* __restrict__ bw,
    const float* __restrict__ W, float* __restrict__ out, EdgeGeom g, int final_out) {
  typedef EdgeTiling<OT, WS> Tl;
  constexpr int kOT = OT;
  constexpr int P = KS <= 4 ? 4 : (KS <= 8 ? 2 : 1);
  __shared__ float red[WS > 1 ? WS * Tl::kBlockOut : 1];
  // (features in XCD-contiguous ranges: the H rows of neighbouring features
  // share cache lines)
  const int64_t bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int i = (int)(bid % g.I);
  const int oc = (int)((bid / g.I) % g.ochunks);
  const int split = (int)(bid / ((int64_t)g.I * g.ochunks));
  // (wave index through readfirstlane: the compiler then keeps the sample
  // range, and the buffer resources built from it, in scalar registers)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wo = wave % Tl::kWO, wsi = wave / Tl::kWO;
  const int q = lane >> 4, r = lane & 15;
  const int obase = oc * Tl::kBlockOut + wo * kOT * 16;
  if (WS == 1 && obase >= g.O) return;  // (with WS > 1 every wave reaches the barrier)

  const PhiSlots<KS> ps(q, g.R);
  float w[kOT][KS];
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
    const int o = obase + t * 16 + r;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int c = ps.c(k);
      w[t][k] = (o < g.O && c >= 0) ? wc_val(bw, W, o, g.I, i, g.R, c) : 0.0f;
    }
  }
  float tot[kOT];
#pragma unroll
  for (int t = 0; t < kOT; ++t) tot[t] = 0.0f;

  int64_t nb = (int64_t)split * g.per_split;
  int64_t ne = min(g.n, nb + g.per_split);
  if (WS > 1) {  // this wave's share of the split's samples
    const int64_t per_wave = round_up(ceil_div(g.per_split, (int64_t)WS), kEdgeRowQuant);
    nb += wsi * per_wave;
    ne = min(ne, nb + per_wave);
  }
  // S register slots of sample tiles, S - 1 tiles ahead: sub-tile p uses slot
  // p and first refills the slot sub-tile p - 1 has just finished with, so
  // no old and new value of a slot are live together (which would cost
  // register copies that wait for the loads at the loop end).
  constexpr int S = P < 2 ? 2 : P;
  float an[S][KS], asn[S];  // asn: s (the group that carries c = 0)
  const HcRows hr(s, H, g.I, g.R, i);
  const uint32_t oh = hr.off_col(r, ps.col0);
  const uint32_t os = ps.owner ? hr.off_s(r, 0) : kBufOob;
  const uint32_t keep = ps.keep();
  auto load_a = [&](int64_t n0, float (&dst)[KS], float& dsts) {
    const HcTile t = hr.tile(n0, ne);
    buf_ld_run<KS>(t.h, oh, dst);
    dsts = buf_ld(t.s, os);
  };
  // (slots issued in order, so that the wait for slot 0 at the loop head
  // leaves the later slots in flight on the first pass as on the others)
#pragma unroll
  for (int p = 0; p < S - 1; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    load_a(nb + 16 * p, an[p], asn[p]);
  }
  for (int64_t n0 = nb; n0 < ne; n0 += 16 * S) {
#pragma unroll
    for (int p = 0; p < S; ++p) {
      const int64_t nt = n0 + 16 * p;
      constexpr int kLag = S - 1;
      const int fill = (p + kLag) % S;
      // keep each sub-tile's instructions in place: the scheduler would
      // otherwise take the column-0 ORs (and their waits) up to the loads
      __builtin_amdgcn_sched_barrier(0);
      load_a(nt + 16 * kLag, an[fill], asn[fill]);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before this tile's wait
      float a[KS];
#pragma unroll
      for (int k = 0; k < KS; ++k) a[k] = k == KS - 1 ? hc_sel(an[p][k], keep, asn[p]) : an[p][k];
      // k outermost: the kOT accumulation chains are independent, so a wave
      // issues MFMAs back to back instead of waiting on one chain at a time
      f32x4 acc[kOT];
#pragma unroll
      for (int t = 0; t < kOT; ++t) acc[t] = zero4();
#pragma unroll
      for (int k = 0; k < KS; ++k)
#pragma unroll
        for (int t = 0; t < kOT; ++t) acc[t] = mfma16(a[k], w[t][k], acc[t]);
#pragma unroll
      for (int t = 0; t < kOT; ++t)
        tot[t] += (fabsf(acc[t][0]) + fabsf(acc[t][1])) + (fabsf(acc[t][2]) + fabsf(acc[t][3]));
    }
  }
  // combine the four row groups of each column in a fixed order
  float colsum[kOT];
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
    const float s1 = tot[t] + __shfl_xor(tot[t], 16);
    colsum[t] = s1 + __shfl_xor(s1, 32);
  }
  if (WS > 1) {  // then the sample shares of the WS waves, in wave order
#pragma unroll
    for (int t = 0; t < kOT; ++t)
      if (q == 0) red[wsi * Tl::kBlockOut + wo * kOT * 16 + t * 16 + r] = colsum[t];
    __syncthreads();
    if (wsi != 0 || obase >= g.O) return;
#pragma unroll
    for (int t = 0; t < kOT; ++t) {
      const int c = wo * kOT * 16 + t * 16 + r;
      float v = red[c];
      for (int w = 1; w < WS; ++w) v += red[w * Tl::kBlockOut + c];
      colsum[t] = v;
    }
  }
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
    const int o = obase + t * 16 + r;
    if (q == 0 && o < g.O) {
      const int64_t e = (int64_t)o * g.I + i;
      if (final_out) out[e] = colsum[t] / (float)g.n;
      else out[(int64_t)split * g.O * g.I + e] = colsum[t];
    }
  }
}

// Forward of a narrow layer (at most 4 output tiles, K = R + 1 <= 16) with
// its sample rows staged through LDS.  Loading a 16-row MFMA operand tile
// straight from [n, I, R] (rows I*R floats apart, R floats used per row)
// makes every quarter-wave of a load touch 16 rows, and for a narrow layer,
// whose rows feed only O/16 output tiles, the texture units then bound the
// kernel.  Here a block takes kStF consecutive features, whose rows are
// contiguous (kStF*R floats), and a chunk of kStRows samples: the block
// loads the chunk with consecutive lanes on consecutive addresses (16-byte
// vectors where I % 4 == 0 and the arrays are aligned) and stores it to LDS
// rows [H(i0..i0+3, 0..R-1) | s(i0..i0+3) | 0 ...]; wave w then runs feature
// i0 + w over the chunk's 16-row tiles, lane (q, r) reading its operand
// column c = 4 k + q of row r at a fixed offset (s, an H column, or the zero
// slot).  The next chunk's loads are in flight (registers) while the current
// one is computed; two LDS buffers and one barrier per chunk.
constexpr int kStF = 4;       // features per block (one per wave)
constexpr int kStRows = 64;   // samples per staged chunk (= kEdgeRowQuant)

template <int KS>
struct StageGeom {
  // row: 4R <= 4(4KS - 1) H floats, 4 s values, zero slot; the stride is
  // 4 * odd, so the 16 rows x 4 columns a wave reads fall in distinct banks
  static constexpr int kS = 4 * (4 * KS + 1 + ((4 * KS + 1) % 2 == 0 ? 1 : 0));
  static constexpr int kBuf = kStRows * kS;       // floats per chunk buffer
  static constexpr int kEPT = 4 * KS;             // scalar path: floats per thread (R <= 4KS-1)
  static_assert(kS >= 4 * (4 * KS - 1) + 5 && (kS / 4) % 2 == 1, "row layout");
};

// The chunk at n0 (rows below ne), through resources based at the chunk
// (rows past ne read as 0).  VEC: element v = thread + 256 j (j < KS) of the
// chunk's 64 R H vectors then 64 s vectors (I % 4 == 0: every group is
// whole, rows and s rows 16-byte aligned).  Scalar: H floats e = thread +
// 256 j of the [kStRows, nf*R] block and s value thread of [kStRows, nf].
template <int KS, bool VEC>
struct StageLoader {
  typedef StageGeom<KS> SG;
  static constexpr int kN = VEC ? KS : SG::kEPT;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  u32x4 hv4[VEC ? KS : 1];
  float hv[VEC ? 1 : SG::kEPT], sv;
  __device__ __forceinline__ void load(const float* __restrict__ s, const float* __restrict__ H,
                                       int64_t n0, int64_t ne, int I, int R, int i0, int nf,
                                       float inv_fr, float inv_nf) {
    const int64_t IR = (int64_t)I * R;
    const int rows = (int)min((int64_t)kStRows, ne - n0);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(H + n0 * IR + (int64_t)i0 * R), (short)0, (int)(rows * IR * 4),
        kBufWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(s != nullptr ? s + n0 * I + i0 : H), (short)0,
        s != nullptr ? (int)(rows * (int64_t)I * 4) : 0, kBufWord3);
    const int t = (int)threadIdx.x;
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const int v = t + kEdgeMfThreads * j;
        if (v < kStRows * R) {
          const int row = small_div_f(v, inv_fr);  // inv_fr = 1 / R here
          hv4[j] = __builtin_amdgcn_raw_buffer_load_b128(
              rh, (int)(((int64_t)row * IR + 4 * (v - row * R)) * 4), 0, 0);
        } else {
          const int row = v - kStRows * R;
          hv4[j] = __builtin_amdgcn_raw_buffer_load_b128(
              rs, row < kStRows ? (int)((int64_t)row * I * 4) : (int)kBufOob, 0, 0);
        }
      }
    } else {
      const int FR = nf * R, elems = kStRows * FR;
#pragma unroll
      for (int j = 0; j < SG::kEPT; ++j) {
        const int e = t + kEdgeMfThreads * j;
        const int row = small_div_f(e, inv_fr);
        hv[j] = buf_ld(rh, e < elems ? (uint32_t)(((int64_t)row * IR + (e - row * FR)) * 4)
                                     : kBufOob);
      }
      const int row = small_div_f(t, inv_nf);
      sv = buf_ld(rs, t < kStRows * nf ? (uint32_t)(((int64_t)row * I + (t - row * nf)) * 4)
                                       : kBufOob);
    }
  }
  // the registers of a chunk that lies wholly past the range (read as zeros)
  __device__ __forceinline__ void clear() {
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < KS; ++j) hv4[j] = u32x4{0u, 0u, 0u, 0u};
    } else {
#pragma unroll
      for (int j = 0; j < SG::kEPT; ++j) hv[j] = 0.0f;
      sv = 0.0f;
    }
  }
  // SKEW: row j of the chunk starts at j kS + 4 (j / 16) instead of j kS
  template <bool SKEW = false>
  __device__ __forceinline__ void store(float* __restrict__ buf, int R, int nf, float inv_fr,
                                        float inv_nf) const {
    const int t = (int)threadIdx.x;
    auto row_at = [](int row) { return row * SG::kS + (SKEW ? 4 * (row >> 4) : 0); };
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const int v = t + kEdgeMfThreads * j;
        int off;
        if (v < kStRows * R) {
          const int row = small_div_f(v, inv_fr);
          off = row_at(row) + 4 * (v - row * R);
        } else {
          off = row_at(v - kStRows * R) + 4 * R;
        }
        if (v < kStRows * (R + 1)) *reinterpret_cast<u32x4*>(buf + off) = hv4[j];
      }
    } else {
      const int FR = nf * R, elems = kStRows * FR;
#pragma unroll
      for (int j = 0; j < SG::kEPT; ++j) {
        const int e = t + kEdgeMfThreads * j;
        if (e < elems) {
          const int row = small_div_f(e, inv_fr);
          buf[row_at(row) + (e - row * FR)] = hv[j];
        }
      }
      if (t < kStRows * nf) {
        const int row = small_div_f(t, inv_nf);
        buf[row_at(row) + 4 * R + (t - row * nf)] = sv;
      }
    }
  }
};

template <int KS, int OT, bool VEC>
__global__ __launch_bounds__(kEdgeMfThreads) void edge_fwd_stage_kernel(
    const float* __restrict__ s, const float* __restrict__ H, const float* __restrict__ bw,
    const float* __restrict__ W, float* __restrict__ out, EdgeGeom g, int final_out) {
  typedef StageGeom<KS> SG;
  __shared__ float lds[2][SG::kBuf];
  const int groups = (g.I + kStF - 1) / kStF;
  const int64_t bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int i0 = (int)(bid % groups) * kStF;
  const int split = (int)(bid / groups);
  const int nf = min(kStF, g.I - i0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int q = lane >> 4, r = lane & 15;
  const int i = i0 + wave;
  const bool active = wave < nf;
  const int R = g.R;
  const float inv_fr = 1.0f / (float)(VEC ? R : nf * R), inv_nf = 1.0f / (float)nf;

  // the zero slot (and features past nf) stay zero
  for (int e = threadIdx.x; e < 2 * SG::kBuf; e += kEdgeMfThreads) (&lds[0][0])[e] = 0.0f;

  float w[OT][KS];
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    const int o = t * 16 + r;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int c = 4 * k + q;
      w[t][k] = (active && o < g.O && c <= R) ? wc_val(bw, W, o, g.I, i, R, c) : 0.0f;
    }
  }
  // LDS column of operand column c = 4 k + q: s, H(i, c - 1) or the zero slot
  int col[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int c = 4 * k + q;
    col[k] = c == 0 ? 4 * R + wave : (c <= R ? wave * R + c - 1 : 4 * R + 4);
  }
  float tot[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) tot[t] = 0.0f;

  const int64_t nb = (int64_t)split * g.per_split;
  const int64_t ne = min(g.n, nb + g.per_split);
  StageLoader<KS, VEC> ld;
  if (nb < ne) ld.load(s, H, nb, ne, g.I, R, i0, nf, inv_fr, inv_nf);
  __syncthreads();  // (the zero fill)
  int buf = 0;
  for (int64_t n0 = nb; n0 < ne; n0 += kStRows, buf ^= 1) {
    ld.store(lds[buf], R, nf, inv_fr, inv_nf);
    if (n0 + kStRows < ne) ld.load(s, H, n0 + kStRows, ne, g.I, R, i0, nf, inv_fr, inv_nf);
    __syncthreads();
    if (active) {
      const float* rowp = lds[buf] + r * SG::kS;
#pragma unroll
      for (int tt = 0; tt < kStRows / 16; ++tt) {
        float a[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) a[k] = rowp[tt * 16 * SG::kS + col[k]];
        f32x4 acc[OT];
#pragma unroll
        for (int t = 0; t < OT; ++t) acc[t] = zero4();
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
          for (int t = 0; t < OT; ++t) acc[t] = mfma16(a[k], w[t][k], acc[t]);
#pragma unroll
        for (int t = 0; t < OT; ++t)
          tot[t] += (fabsf(acc[t][0]) + fabsf(acc[t][1])) + (fabsf(acc[t][2]) + fabsf(acc[t][3]));
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    const float s1 = tot[t] + __shfl_xor(tot[t], 16);
    const float cs = s1 + __shfl_xor(s1, 32);
    const int o = t * 16 + r;
    if (q == 0 && o < g.O) {
      const int64_t e = (int64_t)o * g.I + i;
      if (final_out) out[e] = cs / (float)g.n;
      else out[(int64_t)split * g.O * g.I + e] = cs;
    }
  }
}

// Staging of 64-row chunks for edge_ylin_fwd_kernel with 16-byte loads
// (I % kStF == 0, aligned operands): the chunk holds 64 R H vectors (each
// row's 4 features x R floats are contiguous) and 64 s vectors; vector
// v = thread + 256 jj.  Since 64 R is a multiple of 64, each
// wave's vectors of one jj are all H, all s or all past the end, so the
// choice is a scalar branch.  Per-lane offsets are the same for every
// feature group, for both halves and for both operands (H rows and W rows
// are both I R floats apart, s and bw rows I), so they are computed once.
template <int KS>
struct YlinVecLoader {
  typedef StageGeom<KS> SG;
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  uint32_t goff[KS];  // byte offset in the chunk's H (or s) resource
  int loff[KS];       // float offset in the staged half
  u32x4 hv4[KS];
  __device__ __forceinline__ static int kind(int jj, int wave, int R) {
    const int vw = kEdgeMfThreads * jj + 64 * wave;  // the wave's first vector
    return vw < kStRows * R ? 0 : (vw < kStRows * (R + 1) ? 1 : 2);
  }
  __device__ __forceinline__ void init(int I, int R, int wave) {
    const int t = (int)threadIdx.x;
    const float inv_r = 1.0f / (float)R;
#pragma unroll
    for (int jj = 0; jj < KS; ++jj) {
      const int v = t + kEdgeMfThreads * jj;
      const int kd = kind(jj, wave, R);
      int row = 0, l = 0;
      uint32_t g = 0;
      if (kd == 0) {
        row = small_div_f(v, inv_r);
        const int piece = v - row * R;
        g = (uint32_t)(((int64_t)row * I * R + 4 * piece) * 4);
        l = 4 * piece;
      } else if (kd == 1) {
        row = v - kStRows * R;
        g = (uint32_t)((int64_t)row * I * 4);
        l = 4 * R;
      }
      goff[jj] = g;
      loff[jj] = row * SG::kS + 4 * (row >> 4) + l;
    }
  }
  // rows [c0, c0 + 64) of X [rows, I, R] / xs [rows, I] at features i0.., rows
  // at or past ne read as zero
  __device__ __forceinline__ void load(const float* __restrict__ xs, const float* __restrict__ X,
                                       int64_t c0, int64_t ne, int I, int R, int i0, int wave) {
    const int64_t IR = (int64_t)I * R;
    const int64_t rows = ne - c0 < kStRows ? (ne - c0 > 0 ? ne - c0 : 0) : kStRows;
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X + c0 * IR + (int64_t)i0 * R), (short)0, (int)(rows * IR * 4),
        kBufWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(xs != nullptr ? xs + c0 * I + i0 : X), (short)0,
        xs != nullptr ? (int)(rows * (int64_t)I * 4) : 0, kBufWord3);
#pragma unroll
    for (int jj = 0; jj < KS; ++jj) {
      const int kd = kind(jj, wave, R);
      if (kd == 0) hv4[jj] = __builtin_amdgcn_raw_buffer_load_b128(rh, (int)goff[jj], 0, 0);
      else if (kd == 1) hv4[jj] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)goff[jj], 0, 0);
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ buf, int R, int wave) const {
#pragma unroll
    for (int jj = 0; jj < KS; ++jj)
      if (kind(jj, wave, R) != 2) *reinterpret_cast<u32x4*>(buf + loff[jj]) = hv4[jj];
  }
};

// Layer output and edge statistic of a regularised layer in one pass.  The
// output y[n, o] = s bw^T + H W^T (flattened over I and R) is the sum over
// features of the very edge values whose absolute means the statistic
// takes, y = sum_i phi_i, so phi is formed once: a block owns 128 samples x
// 128 outputs (4 waves as 2 sample halves x 2 output halves, 4 x 4 tiles of
// 16 each) and walks the features in groups of kStF, staging the H rows of
// its samples and the W rows of its outputs through LDS in the row layout of
// the staged kernels ([H | s | zero slot]; the W side is the same layout
// with bw for s).  Per feature a wave forms phi on its 16 tiles, adds it to
// the output accumulators and |phi| to the feature's column sums; after each
// group the two sample halves add their column sums in LDS, in wave order,
// and write one partial row per feature, apart[block row][i][o], which
// edge_ylin_finalize adds in order.  Features are summed into y in index
// order, so both results are deterministic.
template <int KS, bool VEC>
__global__ __launch_bounds__(kEdgeMfThreads, 2) void edge_ylin_fwd_kernel(
    const float* __restrict__ s, const float* __restrict__ H, const float* __restrict__ bw,
    const float* __restrict__ W, float* __restrict__ y, float* __restrict__ apart, int64_t n,
    int I, int O, int R, int oblocks) {
  typedef StageGeom<KS> SG;
  constexpr int kRows = 2 * kStRows;  // samples (and outputs) of a block
  // row j of a staged half starts at j kS + 4 (j / 16): within a 16-row
  // tile the rows fall in distinct banks (kS = 4 x odd), and the skew keeps a
  // lane's reads of two tiles (16 kS apart, a multiple of the 64 banks) off
  // one bank when the compiler pairs them into one instruction
  constexpr int kHalf = kStRows * SG::kS + 4 * (kStRows / 16);
  __shared__ float lh[2 * kHalf];
  __shared__ float lw[2 * kHalf];
  __shared__ float red[2][kStF][64];
  const int bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int ob = bid % oblocks;
  const int64_t nblk = bid / oblocks;
  const int64_t n0 = nblk * kRows;
  const int o0 = ob * kRows;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int q = lane >> 4, r = lane & 15;
  const int wn = wave >> 1, wo = wave & 1;
  const int groups = (I + kStF - 1) / kStF;

  // zero slots (never written by the stores) read as zero
  for (int e = threadIdx.x; e < 2 * kHalf; e += kEdgeMfThreads) {
    lh[e] = 0.0f;
    lw[e] = 0.0f;
  }
  // 16-byte staging (YlinVecLoader) or the staged kernels' scalar loader
  typedef typename std::conditional<VEC, YlinVecLoader<KS>, StageLoader<KS, false>>::type Loader;
  Loader ldh[2], ldw[2];
  if constexpr (VEC) {
    ldh[0].init(I, R, wave);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int jj = 0; jj < KS; ++jj) {
        ldh[h].goff[jj] = ldw[h].goff[jj] = ldh[0].goff[jj];
        ldh[h].loff[jj] = ldw[h].loff[jj] = ldh[0].loff[jj];
      }
    }
  }
  auto load_group = [&](int g) {
    const int i0 = g * kStF, nf = min(kStF, I - i0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (VEC) {
        ldh[h].load(s, H, n0 + h * kStRows, n, I, R, i0, wave);
        ldw[h].load(bw, W, o0 + h * kStRows, O, I, R, i0, wave);
      } else {
        const float inv_fr = 1.0f / (float)(nf * R), inv_nf = 1.0f / (float)nf;
        if (n0 + h * kStRows < n) ldh[h].load(s, H, n0 + h * kStRows, n, I, R, i0, nf, inv_fr, inv_nf);
        else ldh[h].clear();
        if (o0 + h * kStRows < O) ldw[h].load(bw, W, o0 + h * kStRows, O, I, R, i0, nf, inv_fr, inv_nf);
        else ldw[h].clear();
      }
    }
  };
  f32x4 yacc[4][4];
#pragma unroll
  for (int tn = 0; tn < 4; ++tn)
#pragma unroll
    for (int to = 0; to < 4; ++to) yacc[tn][to] = zero4();
  load_group(0);
  // operand columns: c = 4 k + q reads column colk[k] + f inck[k] of feature
  // f's group row (s: 4R + f; H(f, c - 1): f R + c - 1; past R: the zero slot)
  int colk[KS], inck[KS];
#pragma unroll
  for (int k = 0; k < KS; ++k) {
    const int c = 4 * k + q;
    colk[k] = c == 0 ? 4 * R : (c <= R ? c - 1 : 4 * R + 4);
    inck[k] = c == 0 ? 1 : (c <= R ? R : 0);
  }
  const float* pa = lh + wn * kHalf + r * SG::kS;
  const float* pw = lw + wo * kHalf + r * SG::kS;
  for (int g = 0; g < groups; ++g) {
    const int i0 = g * kStF, nf = min(kStF, I - i0);
    __syncthreads();  // the previous group's rows are no longer read
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if constexpr (VEC) {
        ldh[h].store(lh + h * kHalf, R, wave);
        ldw[h].store(lw + h * kHalf, R, wave);
      } else {
        const float inv_fr = 1.0f / (float)(nf * R), inv_nf = 1.0f / (float)nf;
        ldh[h].template store<true>(lh + h * kHalf, R, nf, inv_fr, inv_nf);
        ldw[h].template store<true>(lw + h * kHalf, R, nf, inv_fr, inv_nf);
      }
    }
    if (g + 1 < groups) load_group(g + 1);
    __syncthreads();
    float asum[kStF][4];
#pragma unroll
    for (int f = 0; f < kStF; ++f) {
#pragma unroll
      for (int to = 0; to < 4; ++to) asum[f][to] = 0.0f;
      if (f < nf) {
        float a[4][KS], w[4][KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          const int col = colk[k] + f * inck[k];
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            a[t][k] = pa[t * (16 * SG::kS + 4) + col];
            w[t][k] = pw[t * (16 * SG::kS + 4) + col];
          }
        }
        // per sample tile, the four output tiles' MFMA chains interleaved
#pragma unroll
        for (int tn = 0; tn < 4; ++tn) {
          f32x4 phi[4];
#pragma unroll
          for (int to = 0; to < 4; ++to) phi[to] = zero4();
#pragma unroll
          for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int to = 0; to < 4; ++to) phi[to] = mfma16(a[tn][k], w[to][k], phi[to]);
#pragma unroll
          for (int to = 0; to < 4; ++to) {
            yacc[tn][to] += phi[to];
            asum[f][to] += (fabsf(phi[to][0]) + fabsf(phi[to][1])) +
                           (fabsf(phi[to][2]) + fabsf(phi[to][3]));
          }
        }
      }
    }
    // column sums over the wave's 64 samples (lanes q hold rows 4q..4q+3 of
    // each tile), then the two sample halves in wave order
#pragma unroll
    for (int f = 0; f < kStF; ++f)
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        const float s1 = asum[f][to] + __shfl_xor(asum[f][to], 16);
        asum[f][to] = s1 + __shfl_xor(s1, 32);
      }
    if (wn == 0 && q == 0) {
#pragma unroll
      for (int f = 0; f < kStF; ++f)
#pragma unroll
        for (int to = 0; to < 4; ++to) red[wo][f][to * 16 + r] = asum[f][to];
    }
    __syncthreads();
    if (wn == 1 && q == 0) {
#pragma unroll
      for (int f = 0; f < kStF; ++f) {
        if (f >= nf) continue;
        float* dst = apart + ((int64_t)nblk * I + i0 + f) * O;
#pragma unroll
        for (int to = 0; to < 4; ++to) {
          const int o = o0 + wo * 64 + to * 16 + r;
          if (o < O) dst[o] = red[wo][f][to * 16 + r] + asum[f][to];
        }
      }
    }
  }
  // y: lane (q, r) of tile (tn, to) holds rows 4q + v, column r
#pragma unroll
  for (int tn = 0; tn < 4; ++tn)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t nn = n0 + wn * 64 + tn * 16 + 4 * q + v;
      if (nn >= n) continue;
#pragma unroll
      for (int to = 0; to < 4; ++to) {
        const int o = o0 + wo * 64 + to * 16 + r;
        if (o < O) y[nn * O + o] = yacc[tn][to][v];
      }
    }
}

// a[o, i] = (sum over block rows b of apart[b][i][o]) / n, as four
// interleaved partial sums (b mod 4, each in order) added in a fixed order,
// so that four loads are in flight per thread
__global__ void edge_ylin_finalize(const float* __restrict__ apart, float* __restrict__ a,
                                   int nblk, int I, int O, int64_t n) {
  const int64_t count = (int64_t)I * O;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int b = 0;
    for (; b + 4 <= nblk; b += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u) p[u] += apart[(int64_t)(b + u) * count + e];
    }
    for (int u = 0; b < nblk; ++b, ++u) p[u] += apart[(int64_t)b * count + e];
    const int64_t i = e / O, o = e - i * O;
    a[o * I + i] = ((p[0] + p[1]) + (p[2] + p[3])) / (float)n;
  }
}

// Parameter gradients: block (i, output chunk, split).  Per 16-sample tile:
// phi (rows n, columns o) -> g in registers -> dWc[o, c] += sum_n g Hc with
// the accumulator entries as the A operand.  CT column tiles of 16 cover c.
// With HASD the layer output's gradient D [n, O] is added to g (the weight
// gradients of y = s bw^T + H W^T and of the statistic together).
template <int KS, int CT, int OT, int WS, bool HASD>
__global__ __launch_bounds__(kEdgeMfThreads) void edge_param_mfma_kernel(
    const float* __restrict__ ga, const float* __restrict__ D, const float* __restrict__ s,
    const float* __restrict__ H, const float* __restrict__ bw, const float* __restrict__ W,
    float* __restrict__ dbw, float* __restrict__ dW, float* __restrict__ part, EdgeGeom g,
    int final_out) {
  typedef EdgeTiling<OT, WS> Tl;
  constexpr int kOT = OT;
  // partial dWc of the WS sample shares: [WS][block outputs][CT * 16]
  __shared__ float red[WS > 1 ? WS * Tl::kBlockOut * CT * 16 : 1];
  // (features in XCD-contiguous ranges: the H rows of neighbouring features
  // share cache lines)
  const int64_t bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int i = (int)(bid % g.I);
  const int oc = (int)((bid / g.I) % g.ochunks);
  const int split = (int)(bid / ((int64_t)g.I * g.ochunks));
  // (wave index through readfirstlane: the compiler then keeps the sample
  // range, and the buffer resources built from it, in scalar registers)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wo = wave % Tl::kWO, wsi = wave / Tl::kWO;
  const int q = lane >> 4, r = lane & 15;
  const int obase = oc * Tl::kBlockOut + wo * kOT * 16;
  if (WS == 1 && obase >= g.O) return;
  const int R1 = g.R + 1;
  const float inv_n = 1.0f / (float)g.n;

  const PhiSlots<KS> ps(q, g.R);
  float w[kOT][KS], gav[kOT];
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
    const int o = obase + t * 16 + r;
    gav[t] = o < g.O ? ga[(int64_t)o * g.I + i] * inv_n : 0.0f;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int c = ps.c(k);
      w[t][k] = (o < g.O && c >= 0) ? wc_val(bw, W, o, g.I, i, g.R, c) : 0.0f;
    }
  }
  f32x4 dacc[kOT][CT];
#pragma unroll
  for (int t = 0; t < kOT; ++t)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) dacc[t][ct] = zero4();

  int64_t nb = (int64_t)split * g.per_split;
  int64_t ne = min(g.n, nb + g.per_split);
  if (WS > 1) {
    const int64_t per_wave = round_up(ceil_div(g.per_split, (int64_t)WS), kEdgeRowQuant);
    nb += wsi * per_wave;
    ne = min(ne, nb + per_wave);
  }
  // Operands of the next sample tile are loaded while the current one runs:
  // A of phi (row n0 + r, the run of PhiSlots) and B of the second product
  // (Hc[n0 + 4q + v, 16ct + r]), in two register slots used alternately
  // (the slot rotation of the forward kernel with S = 2).
  float an[2][KS], asn[2], hn[2][CT][4], hsn[2][4];  // asn, hsn: s parts
  const HcRows hr(s, H, g.I, g.R, i);
  uint32_t ob[CT][4], obs[4];
  const uint32_t oa = hr.off_col(r, ps.col0);
  const uint32_t oas = ps.owner ? hr.off_s(r, 0) : kBufOob;
  const uint32_t keep = ps.keep();
#pragma unroll
  for (int v = 0; v < 4; ++v) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) ob[ct][v] = hr.off_h(4 * q + v, ct * 16 + r);
    obs[v] = hr.off_s(4 * q + v, r);  // column 0 only at ct = 0
  }
  auto load_tile = [&](int64_t n0, float (&da)[KS], float& das, float (&dh)[CT][4],
                       float (&dhs)[4]) {
    const HcTile t = hr.tile(n0, ne);
    buf_ld_run<KS>(t.h, oa, da);
    das = buf_ld(t.s, oas);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) dh[ct][v] = buf_ld(t.h, ob[ct][v]);
      dhs[v] = buf_ld(t.s, obs[v]);
    }
  };
  load_tile(nb, an[0], asn[0], hn[0], hsn[0]);
  for (int64_t n0 = nb; n0 < ne; n0 += 32) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // (instructions kept per sub-tile, as in the forward kernel)
      __builtin_amdgcn_sched_barrier(0);
      load_tile(n0 + 16 * p + 16, an[p ^ 1], asn[p ^ 1], hn[p ^ 1], hsn[p ^ 1]);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before this tile's wait
      float a[KS], hb[CT][4];
#pragma unroll
      for (int k = 0; k < KS; ++k) a[k] = k == KS - 1 ? hc_sel(an[p][k], keep, asn[p]) : an[p][k];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          hb[ct][v] = ct == 0 ? hc_or(hn[p][0][v], hsn[p][v]) : hn[p][ct][v];
      // D[n0 + 4q + v, obase + 16t + r] in the accumulator layout of g (rows
      // past the range and columns past O read as zeros)
      float dq[HASD ? kOT : 1][4];
      if constexpr (HASD) {
        const int64_t nt = n0 + 16 * p;
        const __amdgpu_buffer_rsrc_t rd = tile_rsrc(D + nt * g.O, ne - nt, g.O);
#pragma unroll
        for (int t = 0; t < kOT; ++t) {
          const int oc = obase + t * 16 + r;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t off = oc < g.O ? (uint32_t)(((4 * q + v) * g.O + oc) * 4) : kBufOob;
            dq[t][v] = buf_ld(rd, off);
          }
        }
      }
      // both products with the output tiles innermost (independent chains)
      f32x4 acc[kOT];
#pragma unroll
      for (int t = 0; t < kOT; ++t) acc[t] = zero4();
#pragma unroll
      for (int k = 0; k < KS; ++k)
#pragma unroll
        for (int t = 0; t < kOT; ++t) acc[t] = mfma16(a[k], w[t][k], acc[t]);
      float gv[kOT][4];
#pragma unroll
      for (int t = 0; t < kOT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) gv[t][v] = g_sign(gav[t], acc[t][v]);
      if constexpr (HASD) {
#pragma unroll
        for (int t = 0; t < kOT; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) gv[t][v] += dq[t][v];
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int t = 0; t < kOT; ++t) dacc[t][ct] = mfma16(gv[t][v], hb[ct][v], dacc[t][ct]);
    }
  }
  if (WS > 1) {  // add the WS sample shares in wave order
    constexpr int kCols = CT * 16;
#pragma unroll
    for (int t = 0; t < kOT; ++t)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          red[(wsi * Tl::kBlockOut + wo * kOT * 16 + t * 16 + 4 * q + v) * kCols + ct * 16 + r] =
              dacc[t][ct][v];
    __syncthreads();
    if (wsi != 0 || obase >= g.O) return;
#pragma unroll
    for (int t = 0; t < kOT; ++t)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = wo * kOT * 16 + t * 16 + 4 * q + v;
          float acc = red[row * kCols + ct * 16 + r];
          for (int w = 1; w < WS; ++w) acc += red[(w * Tl::kBlockOut + row) * kCols + ct * 16 + r];
          dacc[t][ct][v] = acc;
        }
  }
  // dacc[t][ct]: lane (q, r) holds column c = 16ct + r, rows o = obase + 16t + 4q + v
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c = ct * 16 + r;
      if (c >= R1) continue;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int o = obase + t * 16 + 4 * q + v;
        if (o >= g.O) continue;
        const int64_t e = (int64_t)o * g.I + i;
        const float val = dacc[t][ct][v];
        if (final_out) {
          if (c == 0) {
            if (dbw != nullptr) dbw[e] = val;
          } else if (dW != nullptr) {
            dW[e * g.R + (c - 1)] = val;
          }
        } else {
          part[((int64_t)split * g.O * g.I + e) * R1 + c] = val;
        }
      }
    }
  }
}

// Input gradients.  The work items are (i, sample block of 4 waves x NTW
// tiles of 16) in feature-major order; workgroup b of the grid takes the
// contiguous items [b W / G, (b + 1) W / G), so the items are spread evenly
// over a grid that the device holds at once, and a workgroup restages
// weights only where its feature changes.  The feature's weights and ga/n
// are staged in LDS one output chunk at a time; each wave computes phi^T
// tiles (rows o, columns n) for its samples, g in registers, and
// dHc^T[c, n] += sum_o Wc[o, c] g[n, o] with the accumulator entries as the
// B operand.
constexpr int kInChunkFloats = 8192;  // LDS floats for one staged weight chunk
constexpr int kInMaxRows = 1024;

template <int KS, int CT, int NTW, bool PF>
__global__ __launch_bounds__(kEdgeMfThreads) void edge_input_mfma_kernel(
    const float* __restrict__ ga, const float* __restrict__ s, const float* __restrict__ H,
    const float* __restrict__ bw, const float* __restrict__ W, float* __restrict__ ds,
    float* __restrict__ dH, EdgeGeom g, int oc_rows) {
  __shared__ float wl[kInChunkFloats];
  __shared__ float gl[kInMaxRows];
  const int64_t nblk = ceil_div(g.n, (int64_t)(64 * NTW));
  const int64_t items = nblk * g.I;
  const int64_t item_lo = (int64_t)blockIdx.x * items / gridDim.x;
  const int64_t item_hi = ((int64_t)blockIdx.x + 1) * items / gridDim.x;
  int i = -1;  // feature of the current item (and of the staged weights)
  // (wave index through readfirstlane: the compiler then keeps the sample
  // range, and the buffer resources built from it, in scalar registers)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int q = lane >> 4, r = lane & 15;
  const int R1 = g.R + 1;
  const int stride = R1 | 1;  // odd row stride of the staged weights
  const float inv_n = 1.0f / (float)g.n;
  const bool one_chunk = g.O <= oc_rows;  // weights staged once per feature

  auto stage = [&](int o0, int orows) {
    __syncthreads();
    for (int e = threadIdx.x; e < oc_rows * R1; e += kEdgeMfThreads) {
      const int oo = e / R1, c = e - oo * R1;
      wl[oo * stride + c] = oo < orows ? wc_val(bw, W, o0 + oo, g.I, i, g.R, c) : 0.0f;
    }
    for (int e = threadIdx.x; e < oc_rows; e += kEdgeMfThreads)
      gl[e] = e < orows ? ga[(int64_t)(o0 + e) * g.I + i] * inv_n : 0.0f;
    __syncthreads();
  };
  // Sample rows through buffer resources of the item's feature (see HcRows);
  // rows past n and items past item_hi read as zeros.  With PF the next
  // item's rows are loaded while the current item runs, in two register
  // slots used alternately (narrow layers, where an item's few output tiles
  // cannot hide the loads; wide layers keep one slot and a wave more per
  // SIMD instead).
  const PhiSlots<KS> ps(q, g.R);
  uint32_t oh;
  {
    const HcRows hr0(s, H, g.I, g.R, 0);
    oh = hr0.off_col(r, ps.col0);
  }
  const uint32_t os = ps.owner ? (uint32_t)((int64_t)r * g.I * 4) : kBufOob;
  const uint32_t keep = ps.keep();
  auto load_item = [&](int64_t item, float (&dh)[NTW][KS], float (&dsv)[NTW]) {
    const bool live = item < item_hi;
    const int fi = live ? (int)(item / nblk) : 0;
    const int64_t nbase = (item - (int64_t)fi * nblk) * (int64_t)(64 * NTW);
    const HcRows hr(s, H, g.I, g.R, fi);
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const HcTile t = hr.tile(nbase + (int64_t)(j * 4 + wave) * 16, live ? g.n : 0);
      buf_ld_run<KS>(t.h, oh, dh[j]);
      dsv[j] = buf_ld(t.s, os);
    }
  };
  float h0[NTW][KS], s0[NTW], h1[NTW][KS], s1[NTW];
  auto process = [&](int64_t item, const float (&dh)[NTW][KS], const float (&dsv)[NTW]) {
    const int fi = (int)(item / nblk);
    const int64_t sb = item - (int64_t)fi * nblk;
    if (fi != i) {
      i = fi;
      if (one_chunk) stage(0, g.O);
    }
    // this wave's sample tiles: n0 = nbase + (j*4 + wave)*16
    const int64_t nbase = sb * (int64_t)(64 * NTW);
    float a[NTW][KS];
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int k = 0; k < KS; ++k)
        a[j][k] = k == KS - 1 ? hc_sel(dh[j][k], keep, dsv[j]) : dh[j][k];
    f32x4 dacc[NTW][CT];
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) dacc[j][ct] = zero4();

    for (int o0 = 0; o0 < g.O; o0 += oc_rows) {
      const int orows = min(oc_rows, g.O - o0);
      if (!one_chunk) stage(o0, orows);
      for (int ot = 0; ot < orows; ot += 16) {
        // A operand of phi^T: Wc[o = ot + r, c = slot (k, q)]
        float wa[KS];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          const int c = ps.c(k);
          wa[k] = c >= 0 ? wl[(ot + r) * stride + c] : 0.0f;
        }
        // g scale of the accumulator rows o = ot + 4q + v
        float gs[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) gs[v] = gl[ot + 4 * q + v];
        // A operand of the second product: Wc[o = ot + 4q + v, c = 16ct + r]
        float wb[CT][4];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int c = ct * 16 + r;
#pragma unroll
          for (int v = 0; v < 4; ++v)
            wb[ct][v] = c < R1 ? wl[(ot + 4 * q + v) * stride + c] : 0.0f;
        }
        // both products with the sample tiles innermost (independent chains)
        f32x4 acc[NTW];
#pragma unroll
        for (int j = 0; j < NTW; ++j) acc[j] = zero4();
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
          for (int j = 0; j < NTW; ++j) acc[j] = mfma16(wa[k], a[j][k], acc[j]);
        float gv[NTW][4];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) gv[j][v] = g_sign(gs[v], acc[j][v]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < NTW; ++j) dacc[j][ct] = mfma16(wb[ct][v], gv[j][v], dacc[j][ct]);
      }
    }
    // dacc[j][ct]: lane (q, r) holds column n = tile + r, rows c = 16ct + 4q + v
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      const int64_t nn = nbase + (int64_t)(j * 4 + wave) * 16 + r;
      if (nn >= g.n) continue;
      const int64_t f = nn * g.I + i;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int c = ct * 16 + 4 * q + v;
          if (c >= R1) continue;
          const float val = dacc[j][ct][v];
          if (c == 0) {
            if (ds != nullptr) ds[f] = val;
          } else if (dH != nullptr) {
            dH[f * g.R + (c - 1)] = val;
          }
        }
      }
    }
  };
  if constexpr (!PF) {
    (void)h1;
    (void)s1;
    for (int64_t item = item_lo; item < item_hi; ++item) {
      load_item(item, h0, s0);
      process(item, h0, s0);
    }
  } else {
    load_item(item_lo, h0, s0);
    for (int64_t item = item_lo; item < item_hi; item += 2) {
      __builtin_amdgcn_sched_barrier(0);
      load_item(item + 1, h1, s1);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before this item's wait
      process(item, h0, s0);
      if (item + 1 < item_hi) {
        __builtin_amdgcn_sched_barrier(0);
        load_item(item + 2, h0, s0);
        __builtin_amdgcn_sched_barrier(0);
        process(item + 1, h1, s1);
      }
    }
  }
}

// Fused backward (both gradient sides of one layer): block (i, split), with
// a tiling whose one output chunk covers every output (O <= 512), so that a
// block owns whole samples.  Per 16-sample tile each wave computes phi (rows n, columns o) for
// its kOT output tiles once and uses g = ga sign(phi) / n twice:
//   params  dWc[o, c] += sum_n g[n, o] Hc[n, c]   (accumulator entries as the
//           A operand, as in edge_param_mfma_kernel);
//   inputs  dHc^T[c, n] += sum_o Wc[o, c] g[n, o] (g transposed through a
//           per-wave LDS tile, then the B operand, as in
//           edge_input_mfma_kernel).
// 11 MFMAs per 16 x 16 (n, o) tile instead of the 14 of the two kernels (phi
// is not recomputed), and the sample rows are read once.  Waves that split
// the outputs (WO > 1) add their dHc partials through LDS in wave order once
// per group of GP sample tiles; waves that split the samples (WS > 1) add
// their dWc partials at the end, as in the parameter kernel.  Every wave runs
// the same number of groups (tiles past a wave's range read as zeros and
// contribute nothing), so the group barriers are reached by all.
template <int OT, int WS>
struct EdgeBwdLds {
  typedef EdgeTiling<OT, WS> Tl;
  static constexpr int kWO = Tl::kWO;
  static constexpr int kGP = kWO > 1 ? 4 / WS : 4;  // sample tiles per group
  static constexpr int kTS = 20;                    // transposed tile row stride
  static constexpr int kTrans = 4 * OT * 16 * kTS;  // one tile per (wave, t)
  static constexpr int kRedIn = kWO > 1 ? WS * kWO * kGP * 256 : 0;
};

__device__ __forceinline__ void edge_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int KS, int OT, int WS, bool HASD>
__global__ __launch_bounds__(kEdgeMfThreads) void edge_bwd_mfma_kernel(
    const float* __restrict__ ga, const float* __restrict__ D, const float* __restrict__ s,
    const float* __restrict__ H, const float* __restrict__ bw, const float* __restrict__ W,
    float* __restrict__ ds, float* __restrict__ dH, float* __restrict__ dbw,
    float* __restrict__ dW, float* __restrict__ part, EdgeGeom g, int final_out) {
  static_assert(KS <= 4, "one column tile of 16 covers c");
  typedef EdgeTiling<OT, WS> Tl;
  typedef EdgeBwdLds<OT, WS> L;
  constexpr int kOT = OT, kWO = Tl::kWO, GP = L::kGP, TS = L::kTS;
  __shared__ __align__(16) float trans[L::kTrans];
  __shared__ __align__(16) float red_in[L::kRedIn > 0 ? L::kRedIn : 4];
  __shared__ float red[WS > 1 ? WS * Tl::kBlockOut * 16 : 1];
  const int64_t bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int i = (int)(bid % g.I);
  const int split = (int)(bid / g.I);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wo = wave % kWO, wsi = wave / kWO;
  const int q = lane >> 4, r = lane & 15;
  const int obase = wo * kOT * 16;  // (waves past O keep zero weights and g)
  const int R1 = g.R + 1;
  const float inv_n = 1.0f / (float)g.n;

  // phi's B operand Wc[o = obase + 16t + r, c = slot (k, q)]; the input
  // product's A operand Wc[o = obase + 16t + 4q + v, c = r]; ga / n of
  // columns o.
  const PhiSlots<KS> ps(q, g.R);
  float w[kOT][KS], wb[kOT][4], gav[kOT];
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
    const int o = obase + t * 16 + r;
    gav[t] = o < g.O ? ga[(int64_t)o * g.I + i] * inv_n : 0.0f;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int c = ps.c(k);
      w[t][k] = (o < g.O && c >= 0) ? wc_val(bw, W, o, g.I, i, g.R, c) : 0.0f;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int ov = obase + t * 16 + 4 * q + v;
      wb[t][v] = (ov < g.O && r < R1) ? wc_val(bw, W, ov, g.I, i, g.R, r) : 0.0f;
    }
  }
  f32x4 dacc[kOT];
#pragma unroll
  for (int t = 0; t < kOT; ++t) dacc[t] = zero4();

  const int64_t bnb = (int64_t)split * g.per_split;
  const int64_t bne = min(g.n, bnb + g.per_split);
  const int64_t per_wave =
      WS > 1 ? round_up(ceil_div(g.per_split, (int64_t)WS), kEdgeRowQuant) : g.per_split;
  const int64_t nb = bnb + (WS > 1 ? wsi * per_wave : 0);
  const int64_t ne = min(bne, nb + per_wave);
  // groups of GP tiles: the same count for every wave (that of wave 0)
  const int64_t span0 = min(per_wave, bne - bnb);
  const int64_t groups = span0 > 0 ? ceil_div(span0, (int64_t)(16 * GP)) : 0;

  // S register slots of sample-tile operands, S - 1 tiles ahead (the slot
  // rotation of the forward kernel): tile j of a group uses slot j % S and
  // first refills the slot tile j - 1 has just finished with.  With the
  // layer-output gradient (HASD) two slots, to leave registers for its rows.
  constexpr int S = HASD ? 2 : GP;
  static_assert(GP % S == 0, "slots divide the group");
  float an[S][KS], asn[S], hn[S][4], hsn[S][4];
  const HcRows hr(s, H, g.I, g.R, i);
  uint32_t ob[4], obs[4];
  const uint32_t oa = hr.off_col(r, ps.col0);
  const uint32_t oas = ps.owner ? hr.off_s(r, 0) : kBufOob;
  const uint32_t keep = ps.keep();
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    ob[v] = hr.off_h(4 * q + v, r);
    obs[v] = hr.off_s(4 * q + v, r);
  }
  auto load_tile = [&](int64_t n0, float (&da)[KS], float& das, float (&dh)[4], float (&dhs)[4]) {
    const HcTile t = hr.tile(n0, ne);
    buf_ld_run<KS>(t.h, oa, da);
    das = buf_ld(t.s, oas);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      dh[v] = buf_ld(t.h, ob[v]);
      dhs[v] = buf_ld(t.s, obs[v]);
    }
  };
  // dHc^T of one sample tile: lane (q, r) holds c = 4q + v, n = n0 + r;
  // rows at or past lim (the end of the tile owner's sample range) are not
  // written (they belong to another wave's range or lie past n)
  auto write_din = [&](const f32x4& d, int64_t n0, int64_t lim) {
    const int64_t nn = n0 + r;
    if (nn >= lim) return;
    const int64_t f = nn * g.I + i;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = 4 * q + v;
      if (c >= R1) continue;
      if (c == 0) {
        if (ds != nullptr) ds[f] = d[v];
      } else if (dH != nullptr) {
        dH[f * g.R + (c - 1)] = d[v];
      }
    }
  };
  float* tb = trans + wave * (kOT * 16 * TS);

#pragma unroll
  for (int p = 0; p < S - 1; ++p) {
    __builtin_amdgcn_sched_barrier(0);
    load_tile(nb + 16 * p, an[p], asn[p], hn[p], hsn[p]);
  }
  for (int64_t gi = 0; gi < groups; ++gi) {
    const int64_t g0 = nb + gi * (16 * GP);
    f32x4 din[GP];
#pragma unroll
    for (int j = 0; j < GP; ++j) {
      const int p = j % S, fill = (j + S - 1) % S;
      __builtin_amdgcn_sched_barrier(0);
      load_tile(g0 + 16 * (j + S - 1), an[fill], asn[fill], hn[fill], hsn[fill]);
      __builtin_amdgcn_sched_barrier(0);  // the loads go out before this tile's wait
      float a[KS], hb[4];
#pragma unroll
      for (int k = 0; k < KS; ++k) a[k] = k == KS - 1 ? hc_sel(an[p][k], keep, asn[p]) : an[p][k];
#pragma unroll
      for (int v = 0; v < 4; ++v) hb[v] = hc_or(hn[p][v], hsn[p][v]);
      // layer-output gradient in the accumulator layout of g,
      // D[n0 + 4q + v, obase + 16t + r] (16 consecutive columns of 4 rows per
      // load; rows past the range and columns past O read as zeros), issued
      // before phi so that its MFMAs cover the loads
      float dq[HASD ? kOT : 1][4];
      if constexpr (HASD) {
        const int64_t nt = g0 + 16 * j;
        const __amdgpu_buffer_rsrc_t rd = tile_rsrc(D + nt * g.O, ne - nt, g.O);
#pragma unroll
        for (int t = 0; t < kOT; ++t) {
          const int oc = obase + t * 16 + r;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const uint32_t off = oc < g.O ? (uint32_t)(((4 * q + v) * g.O + oc) * 4) : kBufOob;
            dq[t][v] = buf_ld(rd, off);
          }
        }
      }
      f32x4 acc[kOT];
#pragma unroll
      for (int t = 0; t < kOT; ++t) acc[t] = zero4();
#pragma unroll
      for (int k = 0; k < KS; ++k)
#pragma unroll
        for (int t = 0; t < kOT; ++t) acc[t] = mfma16(a[k], w[t][k], acc[t]);
      float gv[kOT][4];
#pragma unroll
      for (int t = 0; t < kOT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) gv[t][v] = g_sign(gav[t], acc[t][v]);
      if constexpr (HASD) {
        // both products then carry the layer output's gradient as well
#pragma unroll
        for (int t = 0; t < kOT; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) gv[t][v] += dq[t][v];
      }
      // g[n = 4q + v, o = 16t + r] -> tile t at [n][o] (four scalar stores
      // per lane and tile, bank-conflict free; the reads below then take
      // one 16-byte load per tile, all in flight before the first wait)
#pragma unroll
      for (int t = 0; t < kOT; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) tb[t * 16 * TS + (4 * q + v) * TS + r] = gv[t][v];
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int t = 0; t < kOT; ++t) dacc[t] = mfma16(gv[t][v], hb[v], dacc[t]);
      edge_wave_sync();
      // g[n = r, o = 16t + 4q + v]
      float gt[kOT][4];
#pragma unroll
      for (int t = 0; t < kOT; ++t) {
        const f32x4 gq = *reinterpret_cast<const f32x4*>(tb + t * 16 * TS + r * TS + 4 * q);
#pragma unroll
        for (int v = 0; v < 4; ++v) gt[t][v] = gq[v];
      }
      edge_wave_sync();  // (the next tile's stores come after these reads)
      f32x4 d0 = zero4(), d1 = zero4();
#pragma unroll
      for (int v = 0; v < 4; ++v)
#pragma unroll
        for (int t = 0; t < kOT; t += 2) {
          d0 = mfma16(wb[t][v], gt[t][v], d0);
          if (t + 1 < kOT) d1 = mfma16(wb[t + 1][v], gt[t + 1][v], d1);
        }
#pragma unroll
      for (int v = 0; v < 4; ++v) din[j][v] = d0[v] + d1[v];
    }
    if constexpr (kWO == 1) {
#pragma unroll
      for (int j = 0; j < GP; ++j) write_din(din[j], g0 + 16 * j, ne);
    } else {
      // partials of the kWO output ranges, added in wave order: task
      // wave -> (sample share ws2, tile j2); WS * GP = 4 tasks
#pragma unroll
      for (int j = 0; j < GP; ++j)
        *reinterpret_cast<f32x4*>(red_in + (((wsi * kWO + wo) * GP + j) * 64 + lane) * 4) = din[j];
      __syncthreads();
      const int ws2 = wave / GP, j2 = wave % GP;
      f32x4 d = *reinterpret_cast<const f32x4*>(red_in + (((ws2 * kWO) * GP + j2) * 64 + lane) * 4);
#pragma unroll
      for (int w2 = 1; w2 < kWO; ++w2) {
        const f32x4 e =
            *reinterpret_cast<const f32x4*>(red_in + (((ws2 * kWO + w2) * GP + j2) * 64 + lane) * 4);
#pragma unroll
        for (int v = 0; v < 4; ++v) d[v] += e[v];
      }
      const int64_t nb2 = bnb + (WS > 1 ? ws2 * per_wave : 0);
      const int64_t ne2 = min(bne, nb2 + per_wave);
      const int64_t n2 = nb2 + gi * (16 * GP) + 16 * j2;
      write_din(d, n2, ne2);
      __syncthreads();
    }
  }
  if (WS > 1) {  // add the WS sample shares of dWc in wave order
#pragma unroll
    for (int t = 0; t < kOT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        red[(wsi * Tl::kBlockOut + wo * kOT * 16 + t * 16 + 4 * q + v) * 16 + r] = dacc[t][v];
    __syncthreads();
    if (wsi != 0) return;
#pragma unroll
    for (int t = 0; t < kOT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = wo * kOT * 16 + t * 16 + 4 * q + v;
        float acc = red[row * 16 + r];
        for (int w2 = 1; w2 < WS; ++w2) acc += red[(w2 * Tl::kBlockOut + row) * 16 + r];
        dacc[t][v] = acc;
      }
  }
  // dacc[t]: lane (q, r) holds column c = r, rows o = obase + 16t + 4q + v
  if (r >= R1) return;
#pragma unroll
  for (int t = 0; t < kOT; ++t) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = obase + t * 16 + 4 * q + v;
      if (o >= g.O) continue;
      const int64_t e = (int64_t)o * g.I + i;
      const float val = dacc[t][v];
      if (final_out) {
        if (r == 0) {
          if (dbw != nullptr) dbw[e] = val;
        } else if (dW != nullptr) {
          dW[e * g.R + (r - 1)] = val;
        }
      } else {
        part[((int64_t)split * g.O * g.I + e) * R1 + r] = val;
      }
    }
  }
}

// Fused backward of a narrow layer (O <= 64, R + 1 <= 16) on staged rows:
// the products of edge_bwd_mfma_kernel (phi, then g = ga sign(phi) / n (+ D)
// into dWc[o, c] += sum_n g Hc and dHc^T[c, n] += sum_o Wc g), with the
// block layout of edge_fwd_stage_kernel: kStF features (wave w: feature
// i0 + w, every output) and chunks of kStRows samples.  Per chunk the block
// stages the Hc rows in LDS, the waves compute, and each writes its dHc
// values into an LDS copy of the chunk's row layout, which the block then
// stores to ds and dH with consecutive lanes on consecutive addresses.  Two
// barriers per chunk.  The layer-output gradient D is read per sample tile
// straight from global memory in the accumulator layout of g (4 rows of 16
// consecutive columns per load), so the block needs no LDS for it: with
// 16-byte staging (VEC) and R + 1 <= 12 three blocks fit a CU (46 KB of LDS,
// at most 168 VGPRs per lane).

template <int KS, int OT, bool HASD, bool VEC>
__global__ __launch_bounds__(kEdgeMfThreads, VEC && KS <= 3 ? 3 : 1) void edge_bwd_stage_kernel(
    const float* __restrict__ ga, const float* __restrict__ D, const float* __restrict__ s,
    const float* __restrict__ H, const float* __restrict__ bw, const float* __restrict__ W,
    float* __restrict__ ds, float* __restrict__ dH, float* __restrict__ dbw,
    float* __restrict__ dW, float* __restrict__ part, EdgeGeom g, int final_out) {
  typedef StageGeom<KS> SG;
  constexpr int TS = 20;  // transposed g tile row stride
  __shared__ __align__(16) float hs[SG::kBuf];
  __shared__ __align__(16) float os[SG::kBuf];
  __shared__ __align__(16) float trans[4 * OT * 16 * TS];
  const int groups = (g.I + kStF - 1) / kStF;
  const int64_t bid = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int i0 = (int)(bid % groups) * kStF;
  const int split = (int)(bid / groups);
  const int nf = min(kStF, g.I - i0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int t_ = (int)threadIdx.x;
  const int q = lane >> 4, r = lane & 15;
  const int i = i0 + wave;
  const bool active = wave < nf;
  const int R = g.R, R1 = R + 1, O = g.O, I = g.I;
  const int64_t IR = (int64_t)I * R;
  const float inv_n = 1.0f / (float)g.n;
  const float inv_fr = 1.0f / (float)(VEC ? R : nf * R), inv_nf = 1.0f / (float)nf;

  // the zero slot and features past nf stay zero
  for (int e = t_; e < SG::kBuf; e += kEdgeMfThreads) hs[e] = 0.0f;

  // LDS column of augmented column c of this wave's feature
  auto colof = [&](int c) { return c == 0 ? 4 * R + wave : (c <= R ? wave * R + c - 1 : 4 * R + 4); };
  // phi's B operand Wc[o = 16t + r, c = 4k + q]; the input product's A
  // operand Wc[o = 16t + 4q + v, c = r]; ga / n of columns o
  float w[OT][KS], wb[OT][4], gav[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) {
    const int o = t * 16 + r;
    gav[t] = (active && o < O) ? ga[(int64_t)o * I + i] * inv_n : 0.0f;
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      const int c = 4 * k + q;
      w[t][k] = (active && o < O && c <= R) ? wc_val(bw, W, o, I, i, R, c) : 0.0f;
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int ov = t * 16 + 4 * q + v;
      wb[t][v] = (active && ov < O && r < R1) ? wc_val(bw, W, ov, I, i, R, r) : 0.0f;
    }
  }
  int colk[KS], colo[4];
#pragma unroll
  for (int k = 0; k < KS; ++k) colk[k] = colof(4 * k + q);
#pragma unroll
  for (int v = 0; v < 4; ++v) colo[v] = colof(4 * q + v);
  const int colr = colof(r);
  f32x4 dacc[OT];
#pragma unroll
  for (int t = 0; t < OT; ++t) dacc[t] = zero4();

  const int64_t nb = (int64_t)split * g.per_split;
  const int64_t ne = min(g.n, nb + g.per_split);
  StageLoader<KS, VEC> ld;
  // dL/dy offsets in the accumulator layout of g: D[n0 + 16 tt + 4q + v, 16t + r]
  uint32_t doff[HASD ? OT : 1][4];
  if constexpr (HASD) {
#pragma unroll
    for (int t = 0; t < OT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        doff[t][v] = 16 * t + r < O ? (uint32_t)(((4 * q + v) * O + 16 * t + r) * 4) : kBufOob;
  }
  if (nb < ne) ld.load(s, H, nb, ne, I, R, i0, nf, inv_fr, inv_nf);
  float* tb = trans + wave * (OT * 16 * TS);
  __syncthreads();  // (the zero fills)
  for (int64_t n0 = nb; n0 < ne; n0 += kStRows) {
    ld.store(hs, R, nf, inv_fr, inv_nf);
    if (n0 + kStRows < ne) ld.load(s, H, n0 + kStRows, ne, I, R, i0, nf, inv_fr, inv_nf);
    __syncthreads();
    if (active) {
#pragma unroll 1
      for (int tt = 0; tt < kStRows / 16; ++tt) {
        const float* ra = hs + (16 * tt + r) * SG::kS;
        float a[KS], hb[4];
#pragma unroll
        for (int k = 0; k < KS; ++k) a[k] = ra[colk[k]];
#pragma unroll
        for (int v = 0; v < 4; ++v) hb[v] = hs[(16 * tt + 4 * q + v) * SG::kS + colr];
        float dq[HASD ? OT : 1][4];
        if constexpr (HASD) {
          const int64_t nt = n0 + 16 * tt;
          const __amdgpu_buffer_rsrc_t rd = tile_rsrc(D + nt * O, ne - nt, O);
#pragma unroll
          for (int t = 0; t < OT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) dq[t][v] = buf_ld(rd, doff[t][v]);
        }
        f32x4 acc[OT];
#pragma unroll
        for (int t = 0; t < OT; ++t) acc[t] = zero4();
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
          for (int t = 0; t < OT; ++t) acc[t] = mfma16(a[k], w[t][k], acc[t]);
        float gv[OT][4];
#pragma unroll
        for (int t = 0; t < OT; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            gv[t][v] = g_sign(gav[t], acc[t][v]);
            if constexpr (HASD) gv[t][v] += dq[t][v];
          }
        // g[n = 4q + v, o = 16t + r] -> tile t at [n][o] (as in
        // edge_bwd_mfma_kernel)
#pragma unroll
        for (int t = 0; t < OT; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) tb[t * 16 * TS + (4 * q + v) * TS + r] = gv[t][v];
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int t = 0; t < OT; ++t) dacc[t] = mfma16(gv[t][v], hb[v], dacc[t]);
        edge_wave_sync();
        // g[n = r, o = 16t + 4q + v]
        float gt[OT][4];
#pragma unroll
        for (int t = 0; t < OT; ++t) {
          const f32x4 gq = *reinterpret_cast<const f32x4*>(tb + t * 16 * TS + r * TS + 4 * q);
#pragma unroll
          for (int v = 0; v < 4; ++v) gt[t][v] = gq[v];
        }
        edge_wave_sync();  // (the next tile's stores come after these reads)
        f32x4 d0 = zero4(), d1 = zero4();
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int t = 0; t < OT; t += 2) {
            d0 = mfma16(wb[t][v], gt[t][v], d0);
            if (t + 1 < OT) d1 = mfma16(wb[t + 1][v], gt[t + 1][v], d1);
          }
        // dHc[n = 16 tt + r, c = 4q + v]
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (4 * q + v <= R) os[(16 * tt + r) * SG::kS + colo[v]] = d0[v] + d1[v];
      }
    }
    __syncthreads();
    // the chunk's dHc rows below ne to ds and dH
    const int rows = (int)min((int64_t)kStRows, ne - n0);
    if constexpr (VEC) {
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const int v = t_ + kEdgeMfThreads * j;
        if (v < kStRows * R) {
          const int row = small_div_f(v, inv_fr);
          const int c4 = v - row * R;
          if (row < rows && dH != nullptr)
            *reinterpret_cast<f32x4*>(dH + (n0 + row) * IR + (int64_t)i0 * R + 4 * c4) =
                *reinterpret_cast<const f32x4*>(os + row * SG::kS + 4 * c4);
        } else if (v < kStRows * (R + 1)) {
          const int row = v - kStRows * R;
          if (row < rows && ds != nullptr)
            *reinterpret_cast<f32x4*>(ds + (n0 + row) * I + i0) =
                *reinterpret_cast<const f32x4*>(os + row * SG::kS + 4 * R);
        }
      }
    } else {
      const int FR = nf * R;
#pragma unroll
      for (int j = 0; j < SG::kEPT; ++j) {
        const int e = t_ + kEdgeMfThreads * j;
        if (e < kStRows * FR) {
          const int row = small_div_f(e, inv_fr);
          if (row < rows && dH != nullptr)
            dH[(n0 + row) * IR + (int64_t)i0 * R + (e - row * FR)] = os[row * SG::kS + (e - row * FR)];
        }
      }
      if (t_ < kStRows * nf) {
        const int row = small_div_f(t_, inv_nf);
        if (row < rows && ds != nullptr)
          ds[(n0 + row) * I + i0 + (t_ - row * nf)] = os[row * SG::kS + 4 * R + (t_ - row * nf)];
      }
    }
  }
  // dacc[t]: lane (q, r) holds column c = r, rows o = 16t + 4q + v
  if (!active || r >= R1) return;
#pragma unroll
  for (int t = 0; t < OT; ++t) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = t * 16 + 4 * q + v;
      if (o >= O) continue;
      const int64_t e = (int64_t)o * I + i;
      const float val = dacc[t][v];
      if (final_out) {
        if (r == 0) {
          if (dbw != nullptr) dbw[e] = val;
        } else if (dW != nullptr) {
          dW[e * R + (r - 1)] = val;
        }
      } else {
        part[((int64_t)split * O * I + e) * R1 + r] = val;
      }
    }
  }
}

__global__ void edge_fwd_finalize_f32(const float* __restrict__ part, float* __restrict__ a,
                                      int splits, int64_t count, int64_t n) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < count;
       e += (int64_t)gridDim.x * blockDim.x) {
    float v = part[e];
    for (int s = 1; s < splits; ++s) v += part[s * count + e];
    a[e] = v / (float)n;
  }
}

__global__ void edge_param_finalize_f32(const float* __restrict__ part, float* __restrict__ dbw,
                                        float* __restrict__ dW, int splits, int64_t count, int R) {
  const int R1 = R + 1;
  const int64_t total = count * R1;
  for (int64_t x = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; x < total;
       x += (int64_t)gridDim.x * blockDim.x) {
    float v = part[x];
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

inline int fin_blocks_f32(int64_t total) {
  int64_t b = ceil_div(total, 256);
  if (b > 65536) b = 65536;
  return (int)(b < 1 ? 1 : b);
}

// k-steps KS = ceil((R+1)/4) (exact up to 4, then by class) and column tiles
// CT = ceil(4 KS / 16) of the backward products.
#define KAN_EDGE_MF_DISPATCH(R1, ...)                           \
  do {                                                          \
    const int ks_ = ((R1) + 3) / 4;                             \
    if (ks_ <= 1) { constexpr int KS = 1, CT = 1; __VA_ARGS__; }   \
    else if (ks_ == 2) { constexpr int KS = 2, CT = 1; __VA_ARGS__; } \
    else if (ks_ == 3) { constexpr int KS = 3, CT = 1; __VA_ARGS__; } \
    else if (ks_ == 4) { constexpr int KS = 4, CT = 1; __VA_ARGS__; } \
    else if (ks_ <= 6) { constexpr int KS = 6, CT = 2; __VA_ARGS__; } \
    else if (ks_ <= 8) { constexpr int KS = 8, CT = 2; __VA_ARGS__; } \
    else if (ks_ <= 12) { constexpr int KS = 12, CT = 3; __VA_ARGS__; } \
    else { constexpr int KS = 19, CT = 5; __VA_ARGS__; }        \
  } while (0)

// k-steps KS = ceil((R+1)/4) for R + 1 <= 16 (one column tile of 16).
#define KAN_EDGE_MF_DISPATCH4(R1, ...)                                  \
  do {                                                                  \
    const int ks_ = ((R1) + 3) / 4;                                     \
    if (ks_ <= 1) { constexpr int KS = 1; __VA_ARGS__; }                \
    else if (ks_ == 2) { constexpr int KS = 2; __VA_ARGS__; }           \
    else if (ks_ == 3) { constexpr int KS = 3; __VA_ARGS__; }           \
    else { constexpr int KS = 4; __VA_ARGS__; }                         \
  } while (0)

}  // namespace

// Both gradient sides of a layer in one fused kernel where it applies
// (route KAN_ROUTE_EDGE_FUSED; 0 takes the separate parameter and input
// kernels).
bool edge_fused_enabled() { return kan_hip_get_route(KAN_ROUTE_EDGE_FUSED) != 0; }

// (OT, WS) of the forward and parameter kernels for a layer width O; see
// EdgeTiling.  Returns the block's output coverage.
int edge_tiling(int64_t O, int* ot, int* ws) {
  const int64_t tiles = ceil_div(O, 16);
  if (tiles >= 32) { *ot = 8; *ws = 1; }
  else if (tiles >= 16) { *ot = 4; *ws = 1; }
  else if (tiles >= 8) { *ot = 4; *ws = 2; }
  else if (tiles >= 4) { *ot = 4; *ws = 4; }
  else { *ot = 2; *ws = 4; }
  return (4 / *ws) * *ot * 16;
}

// The forward and the fused backward of a narrow layer stage their rows
// through LDS (edge_fwd_stage_kernel, edge_bwd_stage_kernel): at most 4
// output tiles, R + 1 <= 16.
static bool edge_fwd_staged(int64_t O, int64_t R) { return O <= 64 && R + 1 <= 16; }
static bool edge_bwd_staged(int64_t O, int64_t R) {
  return edge_fused_enabled() && O <= 64 && R + 1 <= 16;
}

// Sample splits: about 8 workgroups per CU (measured at c4's layers, where
// longer workgroups in fewer whole rounds ran slower than many short ones the
// hardware balances by itself).  The forward pass of a narrow layer, whose
// waves already split each workgroup's samples (WS > 1), takes 4 times as
// many: its partial sums are only O x I per split.  At least 256 samples per
// split, at most 64 splits.
int edge_mfma_splits(int64_t n, int64_t I, int64_t O, int64_t R, bool backward) {
  int ot, ws;
  const int64_t ochunks = ceil_div(O, (int64_t)edge_tiling(O, &ot, &ws));
  int64_t blocks = I * ochunks;
  int64_t target = (!backward && ws > 1 ? 32LL : 8LL) * device_cu_count();
  if (backward ? edge_bwd_staged(O, R) : edge_fwd_staged(O, R)) {  // blocks of kStF features
    blocks = ceil_div(I, (int64_t)kStF);
    target = 8LL * device_cu_count();
  }
  int64_t s = ceil_div(target, blocks > 0 ? blocks : 1);
  const int64_t cap = ceil_div(n, 256);
  if (s > cap) s = cap;
  if (s > 64) s = 64;
  if (s < 1) s = 1;
  return (int)s;
}

int launch_edge_forward_mfma(const float* s, const float* H, const float* bw, const float* W,
                             float* a, float* part, int splits, int64_t n, int64_t I, int64_t O,
                             int64_t R, hipStream_t st) {
  if (O == 0 || I == 0) return KAN_OK;
  if (splits > 1 && part == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean: missing workspace");
  const int R1 = (int)R + 1;
  EdgeGeom g;
  g.n = n;
  g.I = (int)I;
  g.O = (int)O;
  g.R = (int)R;
  g.splits = splits;
  g.per_split = round_up(ceil_div(n, splits), kEdgeRowQuant);
  int ot, ws;
  g.ochunks = (int)ceil_div(O, (int64_t)edge_tiling(O, &ot, &ws));
  const bool staged = edge_fwd_staged(O, R);
  const int64_t blocks =
      (staged ? ceil_div(I, (int64_t)kStF) : I * g.ochunks) * (int64_t)splits;
  if (blocks > 2147483647LL) return set_error(KAN_ERR_LIMIT, "edge_abs_mean: too many blocks");
  const bool fin = splits == 1;
  TimedLaunch timed(kClassEdge, st, 2.0 * (double)n * (double)O * (double)I * (double)R1);
  if (staged) {
    auto al = [](const float* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool vec = I % kStF == 0 && al(H) && (s == nullptr || al(s));
#define KAN_EDGE_FWD_ST(OTV, VV)                                                                \
  KAN_EDGE_MF_DISPATCH4(R1, hipLaunchKernelGGL((edge_fwd_stage_kernel<KS, OTV, VV>),            \
                                               dim3((unsigned)blocks), dim3(kEdgeMfThreads), 0, \
                                               st, s, H, bw, W, fin ? a : part, g, fin ? 1 : 0))
    if (vec) {
      if (O > 32) KAN_EDGE_FWD_ST(4, true);
      else if (O > 16) KAN_EDGE_FWD_ST(2, true);
      else KAN_EDGE_FWD_ST(1, true);
    } else {
      if (O > 32) KAN_EDGE_FWD_ST(4, false);
      else if (O > 16) KAN_EDGE_FWD_ST(2, false);
      else KAN_EDGE_FWD_ST(1, false);
    }
#undef KAN_EDGE_FWD_ST
  } else {
#define KAN_EDGE_FWD(OTV, WSV)                                                                  \
  KAN_EDGE_MF_DISPATCH(R1, (void)CT; hipLaunchKernelGGL((edge_fwd_mfma_kernel<KS, OTV, WSV>),   \
                                                          dim3((unsigned)blocks),                \
                                                          dim3(kEdgeMfThreads), 0, st, s, H, bw, \
                                                          W, fin ? a : part, g, fin ? 1 : 0))
  if (ot == 8) KAN_EDGE_FWD(8, 1);
  else if (ws == 1) KAN_EDGE_FWD(4, 1);
  else if (ws == 2) KAN_EDGE_FWD(4, 2);
  else if (ot == 4) KAN_EDGE_FWD(4, 4);
  else KAN_EDGE_FWD(2, 4);
#undef KAN_EDGE_FWD
  }
  int rc = check_launch("edge_abs_mean");
  if (rc != KAN_OK || fin) return rc;
  hipLaunchKernelGGL(edge_fwd_finalize_f32, dim3(fin_blocks_f32(O * I)), dim3(256), 0, st, part,
                     a, splits, O * I, n);
  return check_launch("edge_abs_mean_finalize");
}

// Weight gradients of the statistic (with D also those of the layer output).
int launch_edge_params(const float* ga, const float* D, const float* s, const float* H,
                       const float* bw, const float* W, float* dbw, float* dW, float* part,
                       int splits, int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st) {
  const int R1 = (int)R + 1;
  EdgeGeom g;
  g.n = n;
  g.I = (int)I;
  g.O = (int)O;
  g.R = (int)R;
  g.splits = splits;
  g.per_split = round_up(ceil_div(n, splits), kEdgeRowQuant);
  int ot, ws;
  g.ochunks = (int)ceil_div(O, (int64_t)edge_tiling(O, &ot, &ws));
  if (splits > 1 && part == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean_backward: missing workspace");
  const int64_t blocks = I * g.ochunks * (int64_t)splits;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "edge_abs_mean_backward: too many blocks");
  const bool fin = splits == 1;
  {
    TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
#define KAN_EDGE_PAR(OTV, WSV, HD)                                                              \
  KAN_EDGE_MF_DISPATCH(R1, hipLaunchKernelGGL((edge_param_mfma_kernel<KS, CT, OTV, WSV, HD>),   \
                                              dim3((unsigned)blocks), dim3(kEdgeMfThreads),     \
                                              0, st, ga, D, s, H, bw, W, dbw, dW, part, g,      \
                                              fin ? 1 : 0))
#define KAN_EDGE_PAR_T(HD)                   \
  if (ot == 8) KAN_EDGE_PAR(8, 1, HD);       \
  else if (ws == 1) KAN_EDGE_PAR(4, 1, HD);  \
  else if (ws == 2) KAN_EDGE_PAR(4, 2, HD);  \
  else if (ot == 4) KAN_EDGE_PAR(4, 4, HD);  \
  else KAN_EDGE_PAR(2, 4, HD)
    if (D != nullptr) {
      KAN_EDGE_PAR_T(true);
    } else {
      KAN_EDGE_PAR_T(false);
    }
#undef KAN_EDGE_PAR_T
#undef KAN_EDGE_PAR
    const int rc = check_launch("edge_abs_mean_backward(params)");
    if (rc != KAN_OK || fin) return rc;
  }
  hipLaunchKernelGGL(edge_param_finalize_f32, dim3(fin_blocks_f32(O * I * R1)), dim3(256), 0, st,
                     part, dbw, dW, splits, O * I, (int)R);
  return check_launch("edge_abs_mean_backward(finalize)");
}

// The fused backward (both gradient sides; with D also the layer output's
// gradient) for O <= 512 and R + 1 <= 16.
int launch_edge_fused(const float* ga, const float* D, const float* s, const float* H,
                      const float* bw, const float* W, float* ds, float* dH, float* dbw,
                      float* dW, float* part, int splits, int64_t n, int64_t I, int64_t O,
                      int64_t R, hipStream_t st) {
  const int R1 = (int)R + 1;
  EdgeGeom g;
  g.n = n;
  g.I = (int)I;
  g.O = (int)O;
  g.R = (int)R;
  g.splits = splits;
  g.per_split = round_up(ceil_div(n, splits), kEdgeRowQuant);
  g.ochunks = 1;
  // the narrowest block tiling that covers every output (one chunk)
  int ot, ws;
  if (O <= 32) { ot = 2; ws = 4; }
  else if (O <= 64) { ot = 4; ws = 4; }
  else if (O <= 128) { ot = 4; ws = 2; }
  else if (O <= 256) { ot = 4; ws = 1; }
  else { ot = 8; ws = 1; }
  if (splits > 1 && part == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean_backward: missing workspace");
  const bool staged = edge_bwd_staged(O, R);
  const int64_t blocks = (staged ? ceil_div(I, (int64_t)kStF) : I) * (int64_t)splits;
  if (blocks > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "edge_abs_mean_backward: too many blocks");
  const bool fin = splits == 1;
  if (staged) {
    TimedLaunch timed(kClassEdgeGrad, st, 6.0 * (double)n * (double)O * (double)I * (double)R1);
    auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    const bool vec = I % kStF == 0 && al(H) && (s == nullptr || al(s)) && al(dH) && al(ds);
#define KAN_EDGE_BWD_ST(OTV, HD, VV)                                                            \
  KAN_EDGE_MF_DISPATCH4(R1, hipLaunchKernelGGL((edge_bwd_stage_kernel<KS, OTV, HD, VV>),        \
                                               dim3((unsigned)blocks), dim3(kEdgeMfThreads), 0, \
                                               st, ga, D, s, H, bw, W, ds, dH, dbw, dW, part, g, \
                                               fin ? 1 : 0))
#define KAN_EDGE_BWD_ST_O(HD, VV)                \
  if (O > 32) KAN_EDGE_BWD_ST(4, HD, VV);        \
  else if (O > 16) KAN_EDGE_BWD_ST(2, HD, VV);   \
  else KAN_EDGE_BWD_ST(1, HD, VV)
    if (D != nullptr) {
      if (vec) { KAN_EDGE_BWD_ST_O(true, true); } else { KAN_EDGE_BWD_ST_O(true, false); }
    } else {
      if (vec) { KAN_EDGE_BWD_ST_O(false, true); } else { KAN_EDGE_BWD_ST_O(false, false); }
    }
#undef KAN_EDGE_BWD_ST_O
#undef KAN_EDGE_BWD_ST
    const int rc = check_launch("edge_abs_mean_backward(fused, staged)");
    if (rc != KAN_OK || fin) return rc;
  } else {
    TimedLaunch timed(kClassEdgeGrad, st, 6.0 * (double)n * (double)O * (double)I * (double)R1);
#define KAN_EDGE_BWD(OTV, WSV, HD)                                                             \
  KAN_EDGE_MF_DISPATCH4(R1, hipLaunchKernelGGL((edge_bwd_mfma_kernel<KS, OTV, WSV, HD>),       \
                                               dim3((unsigned)blocks), dim3(kEdgeMfThreads), 0, \
                                               st, ga, D, s, H, bw, W, ds, dH, dbw, dW, part, g, \
                                               fin ? 1 : 0))
#define KAN_EDGE_BWD_T(HD)                    \
  if (ot == 8) KAN_EDGE_BWD(8, 1, HD);        \
  else if (ws == 1) KAN_EDGE_BWD(4, 1, HD);   \
  else if (ws == 2) KAN_EDGE_BWD(4, 2, HD);   \
  else if (ot == 4) KAN_EDGE_BWD(4, 4, HD);   \
  else KAN_EDGE_BWD(2, 4, HD)
    if (D != nullptr) {
      KAN_EDGE_BWD_T(true);
    } else {
      KAN_EDGE_BWD_T(false);
    }
#undef KAN_EDGE_BWD_T
#undef KAN_EDGE_BWD
    const int rc = check_launch("edge_abs_mean_backward(fused)");
    if (rc != KAN_OK || fin) return rc;
  }
  hipLaunchKernelGGL(edge_param_finalize_f32, dim3(fin_blocks_f32(O * I * R1)), dim3(256), 0, st,
                     part, dbw, dW, splits, O * I, (int)R);
  return check_launch("edge_abs_mean_backward(finalize)");
}

bool edge_linear_fold_supported(int64_t n, int64_t I, int64_t O, int64_t R) {
  return n > 0 && I > 0 && O > 0 && O <= 512 && R + 1 <= 16;
}

int launch_edge_linear_backward_mfma(const float* ga, const float* D, const float* s,
                                     const float* H, const float* bw, const float* W, float* ds,
                                     float* dH, float* dbw, float* dW, float* part, int splits,
                                     int64_t n, int64_t I, int64_t O, int64_t R, hipStream_t st) {
  if (!edge_linear_fold_supported(n, I, O, R))
    return set_error(KAN_ERR_LIMIT,
                     "edge_linear_backward: needs 0 < out_features <= 512, num_basis + 1 <= 16 "
                     "and n > 0");
  if (ds == nullptr && dH == nullptr)  // weight gradients only: the parameter kernel
    return dbw == nullptr && dW == nullptr
               ? KAN_OK
               : launch_edge_params(ga, D, s, H, bw, W, dbw, dW, part, splits, n, I, O, R, st);
  return launch_edge_fused(ga, D, s, H, bw, W, ds, dH, dbw, dW, part, splits, n, I, O, R, st);
}

bool edge_ylin_supported(int64_t n, int64_t I, int64_t O, int64_t R) {
  return n > 0 && I > 0 && O > 0 && R >= 1 && R + 1 <= 16;
}

size_t edge_ylin_ws_bytes(int64_t n, int64_t I, int64_t O) {
  return sizeof(float) * (size_t)ceil_div(n, (int64_t)(2 * kStRows)) * (size_t)I * (size_t)O;
}

int launch_edge_ylin_forward(const float* s, const float* H, const float* bw, const float* W,
                             float* y, float* a, float* part, int64_t n, int64_t I, int64_t O,
                             int64_t R, hipStream_t st) {
  if (!edge_ylin_supported(n, I, O, R))
    return set_error(KAN_ERR_LIMIT,
                     "edge_linear_forward: needs n, in_features, out_features > 0 and "
                     "num_basis + 1 <= 16");
  if ((s == nullptr) != (bw == nullptr))
    return set_error(KAN_ERR_INVALID, "edge_linear_forward: s and base_weight must both be given or both be empty");
  const int64_t nblk = ceil_div(n, (int64_t)(2 * kStRows));
  const int64_t oblocks = ceil_div(O, (int64_t)(2 * kStRows));
  const int64_t blocks = nblk * oblocks;
  if (blocks > 2147483647LL || nblk > 2147483647LL)
    return set_error(KAN_ERR_LIMIT, "edge_linear_forward: too many blocks");
  auto al = [](const float* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const bool vec = I % kStF == 0 && al(H) && al(W) && (s == nullptr || (al(s) && al(bw)));
  const int R1 = (int)R + 1;
  {
    TimedLaunch timed(kClassEdge, st, 2.0 * (double)n * (double)O * (double)I * (double)R1);
#define KAN_YLIN(VV)                                                                           \
  KAN_EDGE_MF_DISPATCH4(R1, hipLaunchKernelGGL((edge_ylin_fwd_kernel<KS, VV>),                 \
                                               dim3((unsigned)blocks), dim3(kEdgeMfThreads), 0, \
                                               st, s, H, bw, W, y, part, n, (int)I, (int)O,    \
                                               (int)R, (int)oblocks))
    if (vec) KAN_YLIN(true);
    else KAN_YLIN(false);
#undef KAN_YLIN
    const int rc = check_launch("edge_linear_forward");
    if (rc != KAN_OK) return rc;
  }
  hipLaunchKernelGGL(edge_ylin_finalize, dim3(fin_blocks_f32(O * I)), dim3(256), 0, st, part, a,
                     (int)nblk, (int)I, (int)O, n);
  return check_launch("edge_linear_forward(finalize)");
}

int launch_edge_backward_mfma(const float* ga, const float* s, const float* H, const float* bw,
                              const float* W, float* ds, float* dH, float* dbw, float* dW,
                              float* part, int splits, int64_t n, int64_t I, int64_t O, int64_t R,
                              hipStream_t st) {
  const int R1 = (int)R + 1;
  EdgeGeom g;
  g.n = n;
  g.I = (int)I;
  g.O = (int)O;
  g.R = (int)R;
  g.splits = splits;
  g.per_split = round_up(ceil_div(n, splits), kEdgeRowQuant);
  int ot, ws;
  g.ochunks = (int)ceil_div(O, (int64_t)edge_tiling(O, &ot, &ws));
  const bool need_p = (dbw != nullptr || dW != nullptr) && O > 0 && I > 0;
  const bool need_x = (ds != nullptr || dH != nullptr) && n > 0 && I > 0 && O > 0;
  if (need_p && need_x && O <= 512 && R1 <= 16 && edge_fused_enabled())
    return launch_edge_fused(ga, nullptr, s, H, bw, W, ds, dH, dbw, dW, part, splits, n, I, O, R,
                             st);
  if (need_p) {
    const int rc = launch_edge_params(ga, nullptr, s, H, bw, W, dbw, dW, part, splits, n, I, O, R,
                                      st);
    if (rc != KAN_OK) return rc;
  }
  if (need_x) {
    constexpr int NTW = 4;
    const int64_t nblk = ceil_div(n, 64 * NTW);
    // staged output rows per chunk: a multiple of 16 that fits the LDS stage
    int oc_rows = (int)(kInChunkFloats / (R1 | 1)) / 16 * 16;
    if (oc_rows > kInMaxRows) oc_rows = kInMaxRows;
    if ((int64_t)oc_rows > round_up(O, 16)) oc_rows = (int)round_up(O, 16);
    // the items are shared by 4 rounds of resident workgroups (measured best
    // at c4's layers between one round and one item per workgroup)
    const int64_t items = I * nblk;
    // next-item prefetch for layers of at most 256 outputs (measured: 590 ->
    // 553 us at c4's 64-wide layer, 2 % slower at its 512-wide one)
    const bool pf = O <= 256;
    const void* fn = nullptr;
    KAN_EDGE_MF_DISPATCH(R1, fn = pf ? reinterpret_cast<const void*>(
                                           &edge_input_mfma_kernel<KS, CT, NTW, true>)
                                     : reinterpret_cast<const void*>(
                                           &edge_input_mfma_kernel<KS, CT, NTW, false>));
    int64_t blocks = 4LL * device_cu_count() * resident_blocks_per_cu(fn, kEdgeMfThreads);
    if (blocks > items) blocks = items;
    TimedLaunch timed(kClassEdgeGrad, st, 4.0 * (double)n * (double)O * (double)I * (double)R1);
#define KAN_EDGE_INP(PFV)                                                                   \
  KAN_EDGE_MF_DISPATCH(R1, hipLaunchKernelGGL((edge_input_mfma_kernel<KS, CT, NTW, PFV>),   \
                                              dim3((unsigned)blocks), dim3(kEdgeMfThreads), \
                                              0, st, ga, s, H, bw, W, ds, dH, g, oc_rows))
    if (pf) KAN_EDGE_INP(true);
    else KAN_EDGE_INP(false);
#undef KAN_EDGE_INP
    int rc = check_launch("edge_abs_mean_backward(inputs)");
    if (rc != KAN_OK) return rc;
  }
  return KAN_OK;
}

}  // namespace kan
