// Streaming probes: float4 write, read and copy kernels over one buffer,
// the HBM ceiling the memory-bound kernels of the path are judged against
// (kan_hip_stream_probe).  Measurement support only; nothing on the KANLinear
// path calls them.

#include "kan_common.h"

namespace kan {

namespace {

constexpr int kStreamThreads = 256;
constexpr int kStreamUnroll = 4;  // float4 per thread, loads issued together
// Each workgroup covers one contiguous chunk of 256 x 4 float4 = 16 KiB:
// pass u moves 256 consecutive float4 (4 KiB, one per lane).
constexpr int64_t kChunk4 = (int64_t)kStreamThreads * kStreamUnroll;

__global__ void __launch_bounds__(kStreamThreads)
stream_write_kernel(float4* __restrict__ dst, int64_t n4) {
  const int64_t base = (int64_t)blockIdx.x * kChunk4 + threadIdx.x;
  const float4 v = make_float4(1.0f, 2.0f, 3.0f, 4.0f);
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) {
    const int64_t i = base + u * kStreamThreads;
    if (i < n4) dst[i] = v;
  }
}

// The sum is written only when it equals a value the inputs never produce,
// so the loads stay and the kernel writes nothing in practice.
__global__ void __launch_bounds__(kStreamThreads)
stream_read_kernel(const float4* __restrict__ src, float* __restrict__ sink, int64_t n4) {
  const int64_t base = (int64_t)blockIdx.x * kChunk4 + threadIdx.x;
  float4 v[kStreamUnroll];
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) {
    const int64_t i = base + u * kStreamThreads;
    v[u] = i < n4 ? src[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  if (acc == -1234567.0f) sink[0] = acc;
}

__global__ void __launch_bounds__(kStreamThreads)
stream_copy_kernel(const float4* __restrict__ src, float4* __restrict__ dst, int64_t n4) {
  const int64_t base = (int64_t)blockIdx.x * kChunk4 + threadIdx.x;
  float4 v[kStreamUnroll];
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) {
    const int64_t i = base + u * kStreamThreads;
    if (i < n4) v[u] = src[i];
  }
#pragma unroll
  for (int u = 0; u < kStreamUnroll; ++u) {
    const int64_t i = base + u * kStreamThreads;
    if (i < n4) dst[i] = v[u];
  }
}

}  // namespace

int launch_stream_probe(int mode, void* a, void* b, int64_t bytes, hipStream_t st) {
  const int64_t n4 = bytes / 16;
  if (n4 <= 0) return KAN_OK;
  const int64_t blocks = ceil_div(n4, kChunk4);
  if (blocks > 2147483647LL) return set_error(KAN_ERR_LIMIT, "stream_probe: buffer too large");
  const double moved = (double)(n4 * 16) * (mode == 2 ? 2.0 : 1.0);
  TimedLaunch t(kClassStream, st, moved);
  if (mode == 0) {
    stream_write_kernel<<<(unsigned)blocks, kStreamThreads, 0, st>>>((float4*)a, n4);
  } else if (mode == 1) {
    stream_read_kernel<<<(unsigned)blocks, kStreamThreads, 0, st>>>((const float4*)a, (float*)b, n4);
  } else {
    stream_copy_kernel<<<(unsigned)blocks, kStreamThreads, 0, st>>>((const float4*)a, (float4*)b, n4);
  }
  return check_launch("stream_probe");
}

}  // namespace kan
