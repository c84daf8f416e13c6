// Streaming probes: the HBM ceilings the memory-bound kernels of the path are
// judged against (kan_hip_stream_probe).  Measurement support only; nothing
// on the KANLinear path calls them.
//
// Modes 0-2 are the fastest plain forms found by a sweep on MI355X (chunk
// per workgroup from 1 to 64 KiB, 64 to 1024 threads, one to sixteen float4
// per lane, persistent grid-stride loops, non-temporal loads and stores,
// XCD-aware workgroup order): every workgroup moves one float4 per lane and
// exits, and workgroup ids are remapped (xcd_remap) so that each XCD streams
// one contiguous stretch of the buffer.  More float4 per lane, longer
// workgroups and persistent loops all measured slower (16 KiB per workgroup:
// 6.0 TB/s written; a 16 KiB grid-stride loop: 5.0-5.4 TB/s), as did
// non-temporal stores; non-temporal loads gain about 5 % for reads.
//   0 write: 256 threads, 4 KiB per workgroup        (about 7.0 TB/s)
//   1 read:  512 threads, 8 KiB, non-temporal loads   (about 7.2 TB/s)
//   2 copy:  256 threads, 4 KiB, non-temporal loads
// Mode 3 is the write pattern of basis_kernel at c3's layout: rows of 14336
// floats (13 * 1024 basis values, then 1024 SiLU values), each wave writing
// per row one 64-feature segment of 13 * 64 floats and its 64 SiLU values,
// four rows per workgroup step, four steps, workgroup order as the basis
// kernels' (xcd_remap, feature block fastest).  It is the ceiling of that
// access pattern alone, without the kernel's loads and arithmetic.
// Modes 4-6 are candidate patterns for the basis kernels on the same layout:
//   4 one row segment per workgroup: 13 * 64 floats as one float4 per lane
//     (208 lanes) and the segment's 64 SiLU values (16 lanes), then exit;
//   5 its read counterpart (basis_grad): the segment and its base column
//     read with non-temporal loads, 64 floats written per workgroup to b
//     ([rows, 1024], the input gradient's shape);
//   6 mode 3 with one step per workgroup (4 rows of one feature block);
//   7, 8 mode 4's workgroup-wide segments for 4 and 16 consecutive rows of
//     one feature block, one row after the other;
//   9 mode 4 with one-wave workgroups (4 float4 per lane, the last partial);
//   10 mode 5 with two adjacent segments per 512-thread workgroup.

#include "kan_common.h"

namespace kan {

namespace {

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int T, bool NT_LOAD>
__global__ void __launch_bounds__(T) stream_kernel(int mode, const f32x4v* __restrict__ src,
                                                   f32x4v* __restrict__ dst,
                                                   float* __restrict__ sink, int64_t n4) {
  const int64_t chunk = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int64_t i = chunk * T + threadIdx.x;
  if (i >= n4) return;
  if (mode == 0) {
    const f32x4v v = {1.0f, 2.0f, 3.0f, 4.0f};
    dst[i] = v;
    return;
  }
  const f32x4v v = NT_LOAD ? __builtin_nontemporal_load(src + i) : src[i];
  if (mode == 2) {
    dst[i] = v;
  } else if (v.x + v.y + v.z + v.w == -1234567.0f) {
    sink[0] = v.x;  // a value the inputs never produce: the loads stay, nothing is written
  }
}

// c3's basis layout (see the header comment)
constexpr int kSegLd = 14336, kSegR = 13, kSegFb = 64, kSegBlocks = 16, kSegIters = 4;

template <int ITERS>
__global__ void __launch_bounds__(256) segment_write_kernel(float* __restrict__ dst,
                                                            int64_t rows) {
  const int id = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int fb = id % kSegBlocks;
  const int64_t rg = id / kSegBlocks;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int seg4 = kSegFb * kSegR / 4;  // float4 per segment
  const f32x4v v = {1.0f, 2.0f, 3.0f, 4.0f};
  for (int it = 0; it < ITERS; ++it) {
    const int64_t r = (rg * ITERS + it) * 4 + wave;
    if (r >= rows) return;
    float* row = dst + r * kSegLd;
    f32x4v* seg = reinterpret_cast<f32x4v*>(row + (int64_t)fb * kSegFb * kSegR);
    for (int c = lane; c < seg4; c += 64) seg[c] = v;
    row[kSegBlocks * kSegFb * kSegR + fb * kSegFb + lane] = 5.0f;
  }
}

// ROWS consecutive rows of one feature block per workgroup, one row at a
// time: the workgroup's lanes cover the row's segment (208 float4) and its
// SiLU piece (16 float4) with one float4 each (modes 4 and 5: ROWS = 1;
// 7 and 8: 4 and 16 rows).  READ: the segment read with non-temporal loads,
// 64 floats written per row to b.
template <bool READ, int ROWS>
__global__ void __launch_bounds__(256) segment_coop_kernel(float* __restrict__ a,
                                                           float* __restrict__ b, int64_t rows) {
  const int id = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int fb = id % kSegBlocks;
  const int64_t r0 = (int64_t)(id / kSegBlocks) * ROWS;
  const int t = threadIdx.x;
  constexpr int seg4 = kSegFb * kSegR / 4;  // 208 float4
  if (t >= seg4 + kSegFb / 4) return;
  const int64_t off = t < seg4 ? (int64_t)fb * kSegFb * kSegR + 4 * t
                               : kSegBlocks * kSegFb * kSegR + fb * kSegFb + 4 * (t - seg4);
  for (int j = 0; j < ROWS; ++j) {
    const int64_t r = r0 + j;
    if (r >= rows) return;
    f32x4v* p = reinterpret_cast<f32x4v*>(a + r * kSegLd + off);
    if (!READ) {
      const f32x4v v = {1.0f, 2.0f, 3.0f, 4.0f};
      *p = v;
      continue;
    }
    const f32x4v v = __builtin_nontemporal_load(p);
    const float sum = (v.x + v.y) + (v.z + v.w);
    float* dst = b + r * (kSegBlocks * kSegFb) + fb * kSegFb + t;
    if (t < kSegFb) *dst = sum;
    else if (sum == -1234567.0f) *dst = sum;  // a value the inputs never produce: the load stays
  }
}

// One row segment per one-wave workgroup (mode 9: 224 float4 over 64 lanes)
// and, for reads, NSEG adjacent segments of one row with their base pieces
// per 256 * NSEG-thread workgroup (mode 10: NSEG = 2).
__global__ void __launch_bounds__(64) segment_wave_kernel(float* __restrict__ a, int64_t rows) {
  const int id = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int fb = id % kSegBlocks;
  const int64_t r = id / kSegBlocks;
  if (r >= rows) return;
  constexpr int seg4 = kSegFb * kSegR / 4;
  float* row = a + r * kSegLd;
  const f32x4v v = {1.0f, 2.0f, 3.0f, 4.0f};
  for (int t = threadIdx.x; t < seg4 + kSegFb / 4; t += 64) {
    const int64_t off = t < seg4 ? (int64_t)fb * kSegFb * kSegR + 4 * t
                                 : kSegBlocks * kSegFb * kSegR + fb * kSegFb + 4 * (t - seg4);
    *reinterpret_cast<f32x4v*>(row + off) = v;
  }
}

template <int NSEG>
__global__ void __launch_bounds__(256 * NSEG) segment_read_kernel(const float* __restrict__ a,
                                                                  float* __restrict__ b,
                                                                  int64_t rows) {
  constexpr int nfb = kSegBlocks / NSEG;
  const int id = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int fb = id % nfb;
  const int64_t r = id / nfb;
  if (r >= rows) return;
  constexpr int seg4 = NSEG * kSegFb * kSegR / 4;
  const int t = threadIdx.x;
  if (t >= seg4 + NSEG * kSegFb / 4) return;
  const int64_t off = t < seg4 ? (int64_t)fb * NSEG * kSegFb * kSegR + 4 * t
                               : kSegBlocks * kSegFb * kSegR + fb * NSEG * kSegFb + 4 * (t - seg4);
  const f32x4v v = __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(a + r * kSegLd + off));
  const float sum = (v.x + v.y) + (v.z + v.w);
  float* dst = b + r * (kSegBlocks * kSegFb) + fb * NSEG * kSegFb + t;
  if (t < NSEG * kSegFb) *dst = sum;
  else if (sum == -1234567.0f) *dst = sum;  // a value the inputs never produce: the load stays
}

}  // namespace

int launch_stream_probe(int mode, void* a, void* b, int64_t bytes, hipStream_t st) {
  const int64_t n4 = bytes / 16;
  if (n4 <= 0) return KAN_OK;
  if (mode >= 3) {
    const int64_t rows = bytes / ((int64_t)kSegLd * 4);
    if (rows <= 0) return KAN_OK;
    const int iters = mode == 3 ? kSegIters : 1;
    const int64_t groups = mode == 4 || mode == 5 || mode == 9 || mode == 10 ? rows
                           : mode == 7                          ? ceil_div(rows, 4)
                           : mode == 8                          ? ceil_div(rows, 16)
                                                                : ceil_div(rows, 4 * iters);
    if (groups * kSegBlocks > 2147483647LL)
      return set_error(KAN_ERR_LIMIT, "stream_probe: buffer too large");
    const double moved = (double)rows * kSegLd * 4.0 +
                         (mode == 5 || mode == 10 ? (double)rows * kSegBlocks * kSegFb * 4.0 : 0.0);
    TimedLaunch t(kClassStream, st, moved);
    const unsigned grid = (unsigned)(groups * kSegBlocks);
    if (mode == 3)
      segment_write_kernel<kSegIters><<<grid, 256, 0, st>>>((float*)a, rows);
    else if (mode == 6)
      segment_write_kernel<1><<<grid, 256, 0, st>>>((float*)a, rows);
    else if (mode == 4)
      segment_coop_kernel<false, 1><<<grid, 256, 0, st>>>((float*)a, nullptr, rows);
    else if (mode == 5)
      segment_coop_kernel<true, 1><<<grid, 256, 0, st>>>((float*)a, (float*)b, rows);
    else if (mode == 7)
      segment_coop_kernel<false, 4><<<grid, 256, 0, st>>>((float*)a, nullptr, rows);
    else if (mode == 8)
      segment_coop_kernel<false, 16><<<grid, 256, 0, st>>>((float*)a, nullptr, rows);
    else if (mode == 9)
      segment_wave_kernel<<<grid, 64, 0, st>>>((float*)a, rows);
    else
      segment_read_kernel<2><<<(unsigned)(rows * (kSegBlocks / 2)), 512, 0, st>>>(
          (const float*)a, (float*)b, rows);
    return check_launch("stream_probe");
  }
  const int threads = mode == 1 ? 512 : 256;
  const int64_t blocks = ceil_div(n4, threads);
  if (blocks > 2147483647LL) return set_error(KAN_ERR_LIMIT, "stream_probe: buffer too large");
  const double moved = (double)(n4 * 16) * (mode == 2 ? 2.0 : 1.0);
  TimedLaunch t(kClassStream, st, moved);
  if (mode == 1) {
    stream_kernel<512, true><<<(unsigned)blocks, 512, 0, st>>>(
        mode, (const f32x4v*)a, nullptr, (float*)b, n4);
  } else {
    stream_kernel<256, true><<<(unsigned)blocks, 256, 0, st>>>(
        mode, (const f32x4v*)a, (f32x4v*)(mode == 2 ? b : a), nullptr, n4);
  }
  return check_launch("stream_probe");
}

}  // namespace kan
