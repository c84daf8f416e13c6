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

__global__ void __launch_bounds__(256) segment_write_kernel(float* __restrict__ dst,
                                                            int64_t rows) {
  const int id = xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int fb = id % kSegBlocks;
  const int64_t rg = id / kSegBlocks;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int seg4 = kSegFb * kSegR / 4;  // float4 per segment
  const f32x4v v = {1.0f, 2.0f, 3.0f, 4.0f};
  for (int it = 0; it < kSegIters; ++it) {
    const int64_t r = (rg * kSegIters + it) * 4 + wave;
    if (r >= rows) return;
    float* row = dst + r * kSegLd;
    f32x4v* seg = reinterpret_cast<f32x4v*>(row + (int64_t)fb * kSegFb * kSegR);
    for (int c = lane; c < seg4; c += 64) seg[c] = v;
    row[kSegBlocks * kSegFb * kSegR + fb * kSegFb + lane] = 5.0f;
  }
}

}  // namespace

int launch_stream_probe(int mode, void* a, void* b, int64_t bytes, hipStream_t st) {
  const int64_t n4 = bytes / 16;
  if (n4 <= 0) return KAN_OK;
  if (mode == 3) {
    const int64_t rows = bytes / ((int64_t)kSegLd * 4);
    if (rows <= 0) return KAN_OK;
    const int64_t groups = ceil_div(rows, 4 * kSegIters);
    if (groups * kSegBlocks > 2147483647LL)
      return set_error(KAN_ERR_LIMIT, "stream_probe: buffer too large");
    TimedLaunch t(kClassStream, st, (double)rows * kSegLd * 4.0);
    segment_write_kernel<<<(unsigned)(groups * kSegBlocks), 256, 0, st>>>((float*)a, rows);
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
