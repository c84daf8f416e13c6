// extern "C" entry points of libkan_hip.so (declared in include/kan_hip.h).
// Every entry point validates its sizes and limits before any launch, so a
// rejected call leaves nothing running on the device.  Launch errors are
// reported through the status code and kan_hip_last_error().

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <type_traits>
#include <vector>

#include "kan_common.h"

namespace kan {

namespace {
thread_local std::string g_last_error;
std::atomic<int> g_basis_impl{1};
std::mutex g_cu_mutex;
int g_cu_count[64] = {0};
std::map<std::pair<int, const void*>, int> g_resident;  // (device, kernel) -> blocks per CU

// Routing switches (KAN_ROUTE_* in kan_hip.h).  Each starts from its
// environment variable, read once when the library is loaded, and changes
// only through kan_hip_set_route, so a workspace query and the launch it
// sizes see the same route unless the caller switches it in between.
//  * FUSED_DX (KAN_HIP_FUSED_DX=1): contract dx inside the input-side GEMM
//    (no E buffer: the workspace shrinks by n * (ld - 3 I) floats, at about
//    10% more time for that GEMM).  Default off.
//  * COMPACT_E (KAN_HIP_COMPACT_E=1 always, =0 never, else automatic): the
//    input-side product of the fp32 backward with the local basis stores only
//    each item's k+1 span-window values of E (and the base columns), which the
//    input gradient then reads.  It pays where rows are long: at R = 68 (c5)
//    the product took 0.16 ms more and the input gradient 0.80 ms less than
//    through the full E [n, ld]; at R = 13 (c3) the epilogue's span searches
//    cost 0.54 ms against 0.39 ms saved.  Automatic means R >= kCompactMinR.
//  * EDGE_FUSED (KAN_HIP_EDGE_FUSED=0 turns it off): both gradient sides of
//    an edge-statistic layer in one kernel where it applies.
//  * GEMM_TILE (KAN_HIP_GEMM_TILE=256, 128, 256x64 or 256w4): forces the fp32
//    tile configuration (values 0-3; float64 products take 0 as 256x128,
//    1 as 128x128, 2 as the pipelined 128x128 tile and 3 as the pipelined
//    64x64 tile); otherwise the cost model picks it.
constexpr int64_t kCompactMinR = 25;

int route_from_env(int route) {
  switch (route) {
    case KAN_ROUTE_FUSED_DX: {
      const char* v = std::getenv("KAN_HIP_FUSED_DX");
      return v != nullptr && v[0] == '1' ? 1 : 0;
    }
    case KAN_ROUTE_COMPACT_E: {
      const char* v = std::getenv("KAN_HIP_COMPACT_E");
      if (v != nullptr && v[0] == '0') return 0;
      if (v != nullptr && v[0] == '1') return 1;
      return -1;
    }
    case KAN_ROUTE_EDGE_FUSED: {
      const char* v = std::getenv("KAN_HIP_EDGE_FUSED");
      return v != nullptr && std::strcmp(v, "0") == 0 ? 0 : 1;
    }
    case KAN_ROUTE_GEMM_TILE: {
      const char* v = std::getenv("KAN_HIP_GEMM_TILE");
      if (v == nullptr) return -1;
      if (std::strcmp(v, "256") == 0) return 0;
      if (std::strcmp(v, "128") == 0) return 1;
      if (std::strcmp(v, "256x64") == 0) return 2;
      if (std::strcmp(v, "256w4") == 0) return 3;
      return -1;
    }
    default:
      return 0;
  }
}

std::atomic<int> g_route[KAN_ROUTE_COUNT] = {
    {route_from_env(KAN_ROUTE_FUSED_DX)}, {route_from_env(KAN_ROUTE_COMPACT_E)},
    {route_from_env(KAN_ROUTE_EDGE_FUSED)}, {route_from_env(KAN_ROUTE_GEMM_TILE)}};

bool fused_dx_enabled() { return g_route[KAN_ROUTE_FUSED_DX].load() == 1; }

bool compact_e_wanted(int64_t R) {
  const int v = g_route[KAN_ROUTE_COMPACT_E].load();
  return v < 0 ? R >= kCompactMinR : v == 1;
}
}  // namespace

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(KAN_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return KAN_OK;
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  if (g_cu_count[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    g_cu_count[dev] = cus;
  }
  return g_cu_count[dev];
}

int resident_blocks_per_cu(const void* kernel, int threads) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 1;
  }
  std::lock_guard<std::mutex> lock(g_cu_mutex);
  const auto key = std::make_pair(dev, kernel);
  auto it = g_resident.find(key);
  if (it != g_resident.end()) return it->second;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, threads, 0) != hipSuccess ||
      blocks < 1) {
    (void)hipGetLastError();
    blocks = 1;
  }
  g_resident[key] = blocks;
  return blocks;
}

// ---- HIP-event timing -------------------------------------------------------

namespace {
struct TimingRecord {
  int cls;
  hipEvent_t start, stop;
  double work;
};
std::mutex g_timing_mutex;
std::atomic<bool> g_timing_on{false};
std::vector<TimingRecord> g_timing;
constexpr size_t kMaxTimingRecords = 1 << 16;

void timing_clear_locked() {
  for (TimingRecord& r : g_timing) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  g_timing.clear();
}
}  // namespace

TimedLaunch::TimedLaunch(int cls, hipStream_t st, double work) : slot_(-1), st_(st) {
  if (!g_timing_on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  if (g_timing.size() >= kMaxTimingRecords) return;
  TimingRecord r;
  r.cls = cls;
  r.work = work;
  if (hipEventCreate(&r.start) != hipSuccess) {
    (void)hipGetLastError();
    return;
  }
  if (hipEventCreate(&r.stop) != hipSuccess) {
    (void)hipEventDestroy(r.start);
    (void)hipGetLastError();
    return;
  }
  (void)hipEventRecord(r.start, st);
  slot_ = (int)g_timing.size();
  g_timing.push_back(r);
}

TimedLaunch::~TimedLaunch() {
  if (slot_ < 0) return;
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  if ((size_t)slot_ < g_timing.size()) (void)hipEventRecord(g_timing[slot_].stop, st_);
}

namespace {

int check_dtype(int dtype, const char* who) {
  if (dtype != KAN_DTYPE_F32 && dtype != KAN_DTYPE_F64)
    return set_error(KAN_ERR_INVALID, "%s: only FP32 and FP64 inputs are supported (dtype code %d)", who, dtype);
  return KAN_OK;
}

// Layer limits, mirroring kan_check_inputs (csrc/kan_ops.h:39-76) except the
// 32-bit index guard: every kernel here indexes with 64-bit offsets.
int check_layer(const char* who, int64_t n, int64_t I, int64_t O, int64_t G, int64_t k) {
  if (k < 1 || k > 3) return set_error(KAN_ERR_INVALID, "spline_order must be 1, 2 or 3; got %lld", (long long)k);
  if (G < 1) return set_error(KAN_ERR_INVALID, "%s: grid too short for spline_order %lld (G=%lld)", who, (long long)k, (long long)G);
  if (n < 0 || I < 0 || O < 0) return set_error(KAN_ERR_INVALID, "%s: negative size", who);
  if (G + 2 * k > kMaxDeg0Basis)
    return set_error(KAN_ERR_LIMIT,
                     "CUDA kernel supports G + 2k <= %lld (got G=%lld, k=%lld); use backend='reference' for larger grids",
                     (long long)kMaxDeg0Basis, (long long)G, (long long)k);
  if (I > kMaxInFeatures)
    return set_error(KAN_ERR_LIMIT, "CUDA kernel supports in_features <= %lld, got %lld",
                     (long long)kMaxInFeatures, (long long)I);
  return KAN_OK;
}

int need_ptr(const void* p, const char* who, const char* name) {
  if (p == nullptr) return set_error(KAN_ERR_INVALID, "%s: %s must not be NULL", who, name);
  return KAN_OK;
}

#define KAN_TRY(expr)              \
  do {                             \
    const int kan_rc_ = (expr);    \
    if (kan_rc_ != KAN_OK) return kan_rc_; \
  } while (0)

struct BackwardPlan {
  int64_t R, ld, kaug;
  bool need_x, need_params, fused_dx, compact_dx;
  int splits;
  size_t waug_elems, e_elems, part_elems;
  size_t ew_elems;  // compact route: window values [n, I, k+1], then the base columns
};

// Inference workspace: the augmented basis [n, ld], then the split-K
// partial slices of the product (elements).
// A non-negative scratch_elems (the allocation-free call's fixed scratch)
// bounds the product's split slices to what the scratch holds after the
// basis; the cost model then picks among the split counts that fit.  The
// launch must pass the same bound (infer_slice_cap).
inline int64_t infer_slice_cap(int64_t scratch_elems, int64_t aug_elems) {
  return scratch_elems < 0 ? -1 : std::max<int64_t>(0, scratch_elems - aug_elems);
}

template <typename T>
void infer_plan(int64_t n, int64_t I, int64_t O, int64_t R, bool has_base, int64_t* ld,
                int64_t* kaug, int64_t* aug_elems, int64_t* part_elems,
                int64_t scratch_elems = -1) {
  *ld = aug_width(I, R, has_base);
  *kaug = I * R + (has_base ? I : 0);
  *aug_elems = round_up(n * *ld, 64);
  *part_elems = matmul_ws_elems<T>(kLayoutNT, n, O, *kaug,
                                   infer_slice_cap(scratch_elems, *aug_elems));
}

template <typename T>
BackwardPlan plan_backward(int64_t n, int64_t I, int64_t O, int64_t G, int64_t k, bool has_base,
                           bool need_x, bool need_params) {
  BackwardPlan p;
  p.R = G + k;
  p.ld = aug_width(I, p.R, has_base);
  p.kaug = I * p.R + (has_base ? I : 0);
  p.need_x = need_x;
  p.need_params = need_params;
  p.splits = need_params ? gemm_pick_splits<T>(O, p.kaug, n) : 1;
  // transposed weight [kaug, O] (rounded to 256 bytes: E follows it)
  p.waug_elems = need_x ? (size_t)round_up(p.kaug * O, 64) : 0;
  // fp32 with the local basis: dx is contracted inside the input-side GEMM,
  // which leaves [n, I, 3 or 2] partial sums instead of E [n, ld]
  const bool local_f32 = std::is_same<T, float>::value && g_basis_impl.load() == 1;
  p.fused_dx = need_x && local_f32 && fused_dx_enabled() &&
               gemm_dx_supported(n, p.kaug, O, I, (int)G, (int)k, has_base);
  p.compact_dx = need_x && local_f32 && !p.fused_dx && compact_e_wanted(p.R) &&
                 gemm_ecomp_supported(n, p.kaug, O, I, (int)G, (int)k, has_base);
  p.ew_elems = p.compact_dx ? (size_t)round_up(n * I * (k + 1), 64) : 0;
  p.e_elems = !need_x         ? 0
              : p.fused_dx   ? (size_t)(n * I * (has_base ? 3 : 2))
              : p.compact_dx ? p.ew_elems + (size_t)(has_base ? round_up(n * I, 64) : 0)
                             : (size_t)(n * p.ld);
  p.part_elems = need_params ? (size_t)p.splits * (size_t)(O * p.ld) : 0;
  return p;
}

// Forward workspace: the augmented weight [O, ld], then the split-K partial
// slices of the output product (elements).  Products with few output tiles
// (few samples or outputs, long K: c5's layer, small networks) are split over
// K and summed in a fixed order; large ones (c3) are not split.
template <typename T>
void forward_plan(int64_t n, int64_t I, int64_t O, int64_t R, bool has_base, int64_t* ld,
                  int64_t* kaug, int64_t* waug_elems, int64_t* part_elems) {
  *ld = aug_width(I, R, has_base);
  *kaug = I * R + (has_base ? I : 0);
  *waug_elems = round_up(O * *ld, 64);
  *part_elems = matmul_ws_elems<T>(kLayoutNT, n, O, *kaug);
}

template <typename T>
int forward_impl(const void* x, const void* grid, const void* bw, const void* sw,
                 const void* scaler, void* out, void* aug, void* ws, size_t ws_bytes, int64_t n,
                 int64_t I, int64_t O, int64_t G, int64_t k, hipStream_t st) {
  const int64_t R = G + k;
  const bool has_base = bw != nullptr;
  int64_t ld, kaug, waug_elems, part_elems;
  forward_plan<T>(n, I, O, R, has_base, &ld, &kaug, &waug_elems, &part_elems);
  const size_t need = sizeof(T) * (size_t)(waug_elems + part_elems);
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "kan_forward: workspace of %zu bytes is smaller than the %zu required",
                     ws_bytes, need);
  const T* tx = static_cast<const T*>(x);
  T* taug = static_cast<T*>(aug);
  T* twaug = static_cast<T*>(ws);
  KAN_TRY(launch_build_waug<T>(static_cast<const T*>(sw), static_cast<const T*>(scaler),
                               static_cast<const T*>(bw), twaug, ld, O, I, R, st));
  KAN_TRY(launch_basis<T>(tx, static_cast<const T*>(grid), taug, ld,
                          has_base ? taug + I * R : nullptr, n, I, (int)G, (int)k,
                          g_basis_impl.load(), st));
  return launch_matmul<T>(kLayoutNT, n, O, kaug, taug, ld, twaug, ld, static_cast<T*>(out), O,
                          twaug + waug_elems, st);
}

template <typename T>
int backward_impl(const void* D, const void* x, const void* grid, const void* bw,
                  const void* sw, const void* scaler, const void* aug, void* gx, void* gbw,
                  void* gsw, void* gscaler, void* ws, size_t ws_bytes, int64_t n, int64_t I,
                  int64_t O, int64_t G, int64_t k, hipStream_t st) {
  const bool has_base = bw != nullptr;
  const bool need_x = gx != nullptr;
  const bool need_params = gsw != nullptr || gscaler != nullptr || gbw != nullptr;
  const BackwardPlan p = plan_backward<T>(n, I, O, G, k, has_base, need_x, need_params);
  const size_t need_bytes = sizeof(T) * (p.waug_elems + p.e_elems + p.part_elems);
  if (ws_bytes < need_bytes || (need_bytes > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "kan_backward: workspace of %zu bytes is smaller than the %zu required",
                     ws_bytes, need_bytes);
  T* base = static_cast<T*>(ws);
  T* waug = base;
  T* E = waug + p.waug_elems;
  T* part = E + p.e_elems;
  const T* tD = static_cast<const T*>(D);
  const T* taug = static_cast<const T*>(aug);
  const int impl = g_basis_impl.load();
  if (need_x) {
    KAN_TRY(launch_build_waug_t<T>(static_cast<const T*>(sw), static_cast<const T*>(scaler),
                                   static_cast<const T*>(bw), waug, p.kaug, O, I, p.R, st));
    if constexpr (std::is_same<T, float>::value) {
      if (p.fused_dx) {
        KAN_TRY(launch_gemm_dx(n, p.kaug, O, tD, O, waug, O, static_cast<const float*>(x),
                               static_cast<const float*>(grid), I, (int)G, (int)k, has_base, E,
                               static_cast<float*>(gx), st));
      }
    }
  }
  if constexpr (std::is_same<T, float>::value) {
    if (need_x && p.compact_dx) {
      // E's span-window values and base columns only, then dx from them
      float* ew = E;
      float* es = has_base ? E + p.ew_elems : nullptr;
      KAN_TRY(launch_gemm_ecomp(n, p.kaug, O, tD, O, waug, O, static_cast<const float*>(x),
                                static_cast<const float*>(grid), I, (int)G, (int)k, has_base, ew,
                                es, st));
      KAN_TRY(launch_basis_grad_compact(static_cast<const float*>(x),
                                        static_cast<const float*>(grid), ew, es,
                                        static_cast<float*>(gx), n, I, (int)G, (int)k, st));
    }
  }
  if (need_x && !p.fused_dx && !p.compact_dx) {
    // E[n, k'] = sum_o D[n, o] Waug[o, k'] = sum_o D[n, o] WaugT[k', o]  (both K-contiguous)
    KAN_TRY(launch_gemm<T>(kLayoutNT, n, p.kaug, O, tD, O, waug, O, E, p.ld, 1, 0, st));
    KAN_TRY(launch_basis_grad<T>(static_cast<const T*>(x), static_cast<const T*>(grid), E, p.ld,
                                 has_base ? E + I * p.R : nullptr, static_cast<T*>(gx), n, I,
                                 (int)G, (int)k, impl, st));
  }
  if (need_params) {
    // G[o, k'] = sum_n D[n, o] Aug[n, k']  (split over n when the tile count is low)
    KAN_TRY(launch_gemm<T>(kLayoutTN, O, p.kaug, n, tD, O, taug, p.ld, part, p.ld, p.splits,
                           O * p.ld, st));
    KAN_TRY(launch_param_grads<T>(part, p.splits, O * p.ld, p.ld, static_cast<const T*>(sw),
                                  static_cast<const T*>(scaler), static_cast<T*>(gsw),
                                  static_cast<T*>(gscaler), static_cast<T*>(gbw), O, I, p.R, st));
  }
  return KAN_OK;
}

int check_edge(const char* who, int dtype, const void* s, const void* H, const void* bw,
               const void* W, int64_t n, int64_t I, int64_t O, int64_t R) {
  KAN_TRY(check_dtype(dtype, who));
  KAN_TRY(need_ptr(H, who, "H"));
  KAN_TRY(need_ptr(W, who, "W"));
  if ((s == nullptr) != (bw == nullptr))
    return set_error(KAN_ERR_INVALID, "%s: s and base_weight must both be given or both be empty", who);
  if (R < 1 || R > 72) return set_error(KAN_ERR_LIMIT, "edge_abs_mean: R must be <= 72, got %lld", (long long)R);
  if (I > kMaxInFeatures) return set_error(KAN_ERR_LIMIT, "edge_abs_mean: too many input features");
  if (n < 1) return set_error(KAN_ERR_INVALID, "edge_abs_mean: need at least one sample");
  if (I < 0 || O < 0) return set_error(KAN_ERR_INVALID, "%s: negative size", who);
  return KAN_OK;
}

size_t edge_ws_bytes(int dtype, int64_t n, int64_t I, int64_t O, int64_t R, bool backward) {
  const int splits = edge_pick_splits(dtype, n, I, O, R, backward);
  if (splits <= 1) return 0;
  const size_t elem = dtype == KAN_DTYPE_F64 ? 8 : 4;
  return elem * (size_t)splits * (size_t)(O * I) * (size_t)(backward ? R + 1 : 1);
}

}  // namespace
}  // namespace kan

using namespace kan;

// ---- allocation-free inference (kan_hip_infer_noalloc) ----------------------
// Fixed device scratch that replaces the caller workspace of kan_hip_infer.
// Each GPU the library runs on holds its own copy until the process ends.
// Host code never uses the array's name as an address: the per-device
// address comes from hipGetSymbolAddress on the first call on that device.
static __device__ __align__(256) unsigned char scratch[KAN_NOALLOC_SCRATCH_BYTES];

namespace kan {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// Address of this device's scratch (looked up once per device, with the
// device current).
int scratch_of_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(KAN_ERR_HIP, "kan_infer_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(KAN_ERR_INVALID, "kan_infer_noalloc: device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return set_error(KAN_ERR_HIP, "kan_infer_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KAN_OK;
}
}  // namespace
}  // namespace kan

// Digest of the sources and flags this library was built from, passed by
// the build script; the Python loader compares it with the sources beside
// the library and refuses a library built from other sources.
#ifndef KAN_SOURCE_HASH
#define KAN_SOURCE_HASH "unset"
#endif

extern "C" {

const char* kan_hip_last_error(void) { return g_last_error.c_str(); }

const char* kan_hip_source_hash(void) { return KAN_SOURCE_HASH; }

int kan_hip_limits(int64_t* max_deg0_basis, int64_t* max_in_features) {
  if (max_deg0_basis != nullptr) *max_deg0_basis = kMaxDeg0Basis;
  if (max_in_features != nullptr) *max_in_features = kMaxInFeatures;
  return KAN_OK;
}

int kan_hip_set_basis_impl(int64_t impl) {
  if (impl != 0 && impl != 1)
    return set_error(KAN_ERR_INVALID, "basis impl must be 0 (recurrence) or 1 (local)");
  g_basis_impl.store((int)impl);
  return KAN_OK;
}

int64_t kan_hip_get_basis_impl(void) { return g_basis_impl.load(); }

int kan_hip_set_route(int route, int value) {
  static const int lo[KAN_ROUTE_COUNT] = {0, -1, 0, -1};
  static const int hi[KAN_ROUTE_COUNT] = {1, 1, 1, 3};
  if (route < 0 || route >= KAN_ROUTE_COUNT)
    return set_error(KAN_ERR_INVALID, "unknown route %d", route);
  if (value < lo[route] || value > hi[route])
    return set_error(KAN_ERR_INVALID, "route %d takes values %d..%d, got %d", route, lo[route],
                     hi[route], value);
  g_route[route].store(value);
  return KAN_OK;
}

int kan_hip_get_route(int route) {
  return route >= 0 && route < KAN_ROUTE_COUNT ? g_route[route].load() : -2;
}

int kan_hip_timing_enable(int on) {
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  timing_clear_locked();
  g_timing_on.store(on != 0);
  return KAN_OK;
}

int kan_hip_timing_read(int kernel_class, double* total_ms, int64_t* launches, double* work) {
  if (kernel_class < 0 || kernel_class >= kNumKernelClasses)
    return set_error(KAN_ERR_INVALID, "timing_read: unknown kernel class %d", kernel_class);
  std::lock_guard<std::mutex> lock(g_timing_mutex);
  double ms = 0.0, w = 0.0;
  int64_t cnt = 0;
  for (const TimingRecord& r : g_timing) {
    if (r.cls != kernel_class) continue;
    if (hipEventSynchronize(r.stop) != hipSuccess)
      return set_error(KAN_ERR_HIP, "timing_read: %s", hipGetErrorString(hipGetLastError()));
    float e = 0.0f;
    if (hipEventElapsedTime(&e, r.start, r.stop) != hipSuccess)
      return set_error(KAN_ERR_HIP, "timing_read: %s", hipGetErrorString(hipGetLastError()));
    ms += e;
    w += r.work;
    ++cnt;
  }
  if (total_ms != nullptr) *total_ms = ms;
  if (launches != nullptr) *launches = cnt;
  if (work != nullptr) *work = w;
  return KAN_OK;
}

int kan_hip_stream_probe(int mode, void* a, void* b, int64_t bytes, void* stream) {
  if (mode < 0 || mode > 10)
    return set_error(KAN_ERR_INVALID,
                     "stream_probe: mode must be 0 (write), 1 (read), 2 (copy) or 3-10 (row segments)");
  if (bytes < 0 || bytes % 16 != 0)
    return set_error(KAN_ERR_INVALID, "stream_probe: bytes must be a non-negative multiple of 16");
  if (bytes > 0 && (a == nullptr || ((mode == 1 || mode == 2 || mode == 5 || mode == 10) && b == nullptr) ||
                    ((uintptr_t)a % 16) != 0 || (mode == 2 && ((uintptr_t)b % 16) != 0)))
    return set_error(KAN_ERR_INVALID, "stream_probe: buffers must be non-null and 16-byte aligned");
  return launch_stream_probe(mode, a, b, bytes, (hipStream_t)stream);
}

int kan_hip_basis(int dtype, const void* x, const void* grid, void* basis, int64_t n, int64_t I,
                  int64_t G, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_basis"));
  KAN_TRY(check_layer("kan_basis", n, I, 0, G, k));
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_basis", "x"));
  KAN_TRY(need_ptr(grid, "kan_basis", "grid"));
  KAN_TRY(need_ptr(basis, "kan_basis", "basis"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t R = G + k;
  if (dtype == KAN_DTYPE_F32)
    return launch_basis<float>(static_cast<const float*>(x), static_cast<const float*>(grid),
                               static_cast<float*>(basis), I * R, nullptr, n, I, (int)G, (int)k,
                               g_basis_impl.load(), st);
  return launch_basis<double>(static_cast<const double*>(x), static_cast<const double*>(grid),
                              static_cast<double*>(basis), I * R, nullptr, n, I, (int)G, (int)k,
                              g_basis_impl.load(), st);
}

namespace {
int matmul_layout(int trans_a, int trans_b) {
  if (trans_a == 0 && trans_b == 0) return kLayoutNN;
  if (trans_a == 0 && trans_b == 1) return kLayoutNT;
  if (trans_a == 1 && trans_b == 0) return kLayoutTN;
  if (trans_a == 1 && trans_b == 1) return kLayoutTT;
  return -1;
}

int check_matmul(int dtype, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                 int64_t lda, int64_t ldb, int64_t ldc) {
  KAN_TRY(check_dtype(dtype, "kan_matmul"));
  if (matmul_layout(trans_a, trans_b) < 0)
    return set_error(KAN_ERR_INVALID, "kan_matmul: trans_a and trans_b must be 0 or 1");
  if (M < 0 || N < 0 || K < 0) return set_error(KAN_ERR_INVALID, "kan_matmul: negative size");
  // leading dimensions cover the rows they index
  const int64_t a_row = trans_a ? M : K, b_row = trans_b ? K : N;
  if ((M * K > 0 && lda < a_row) || (K * N > 0 && ldb < b_row) || (M * N > 0 && ldc < N))
    return set_error(KAN_ERR_INVALID, "kan_matmul: leading dimension smaller than the row");
  return KAN_OK;
}
}  // namespace

int kan_hip_matmul_workspace(int dtype, int trans_a, int trans_b, int64_t M, int64_t N,
                             int64_t K, size_t* bytes) {
  KAN_TRY(need_ptr(bytes, "kan_matmul_workspace", "bytes"));
  KAN_TRY(check_matmul(dtype, trans_a, trans_b, M, N, K, trans_a ? M : K, trans_b ? K : N, N));
  const int layout = matmul_layout(trans_a, trans_b);
  *bytes = dtype == KAN_DTYPE_F32 ? 4 * (size_t)matmul_ws_elems<float>(layout, M, N, K)
                                  : 8 * (size_t)matmul_ws_elems<double>(layout, M, N, K);
  return KAN_OK;
}

int kan_hip_matmul(int dtype, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                   const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                   void* ws, size_t ws_bytes, void* stream) {
  KAN_TRY(check_matmul(dtype, trans_a, trans_b, M, N, K, lda, ldb, ldc));
  if (M * N == 0) return KAN_OK;
  KAN_TRY(need_ptr(C, "kan_matmul", "C"));
  if (K > 0) {
    KAN_TRY(need_ptr(A, "kan_matmul", "A"));
    KAN_TRY(need_ptr(B, "kan_matmul", "B"));
  }
  const int layout = matmul_layout(trans_a, trans_b);
  const size_t elem = dtype == KAN_DTYPE_F32 ? 4 : 8;
  const size_t need = elem * (size_t)(dtype == KAN_DTYPE_F32
                                          ? matmul_ws_elems<float>(layout, M, N, K)
                                          : matmul_ws_elems<double>(layout, M, N, K));
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "kan_matmul: workspace of %zu bytes is smaller than the %zu required",
                     ws_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_matmul<float>(layout, M, N, K, static_cast<const float*>(A), lda,
                                static_cast<const float*>(B), ldb, static_cast<float*>(C), ldc,
                                static_cast<float*>(ws), st);
  return launch_matmul<double>(layout, M, N, K, static_cast<const double*>(A), lda,
                               static_cast<const double*>(B), ldb, static_cast<double*>(C), ldc,
                               static_cast<double*>(ws), st);
}

int kan_hip_basis_deriv(int dtype, const void* x, const void* grid, const void* scale, void* out,
                        int64_t n, int64_t I, int64_t G, int64_t k, int64_t order,
                        void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_basis_deriv"));
  KAN_TRY(check_layer("kan_basis_deriv", n, I, 0, G, k));
  if (order < 0 || order > 64)
    return set_error(KAN_ERR_INVALID, "kan_basis_deriv: order must lie in 0..64, got %lld",
                     (long long)order);
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_basis_deriv", "x"));
  KAN_TRY(need_ptr(grid, "kan_basis_deriv", "grid"));
  KAN_TRY(need_ptr(out, "kan_basis_deriv", "out"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_basis_deriv<float>(static_cast<const float*>(x), static_cast<const float*>(grid),
                                     static_cast<const float*>(scale), static_cast<float*>(out),
                                     n, I, (int)G, (int)k, (int)order, st);
  return launch_basis_deriv<double>(static_cast<const double*>(x),
                                    static_cast<const double*>(grid),
                                    static_cast<const double*>(scale), static_cast<double*>(out),
                                    n, I, (int)G, (int)k, (int)order, st);
}

int kan_hip_basis_deriv_contract(int dtype, const void* x, const void* grid, const void* gH,
                                 const void* gbase, const void* scale, void* gx, int64_t n,
                                 int64_t I, int64_t G, int64_t k, int64_t order, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_basis_deriv_contract"));
  KAN_TRY(check_layer("kan_basis_deriv_contract", n, I, 0, G, k));
  if (order < 0 || order > 64)
    return set_error(KAN_ERR_INVALID,
                     "kan_basis_deriv_contract: order must lie in 0..64, got %lld",
                     (long long)order);
  if (gbase != nullptr && order > kMaxSiluOrder)
    return set_error(KAN_ERR_INVALID,
                     "kan_basis_deriv_contract: the base term supports orders 0..%d, got %lld",
                     kMaxSiluOrder, (long long)order);
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_basis_deriv_contract", "x"));
  KAN_TRY(need_ptr(grid, "kan_basis_deriv_contract", "grid"));
  KAN_TRY(need_ptr(gH, "kan_basis_deriv_contract", "grad_basis"));
  KAN_TRY(need_ptr(gx, "kan_basis_deriv_contract", "grad_x"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_basis_deriv_contract<float>(
        static_cast<const float*>(x), static_cast<const float*>(grid),
        static_cast<const float*>(gH), static_cast<const float*>(gbase),
        static_cast<const float*>(scale), static_cast<float*>(gx), n, I, (int)G, (int)k,
        (int)order, st);
  return launch_basis_deriv_contract<double>(
      static_cast<const double*>(x), static_cast<const double*>(grid),
      static_cast<const double*>(gH), static_cast<const double*>(gbase),
      static_cast<const double*>(scale), static_cast<double*>(gx), n, I, (int)G, (int)k,
      (int)order, st);
}

int kan_hip_silu_deriv(int dtype, const void* x, const void* scale, void* out, int64_t count,
                       int64_t order, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_silu_deriv"));
  if (count < 0) return set_error(KAN_ERR_INVALID, "kan_silu_deriv: negative count");
  if (order < 0 || order > kMaxSiluOrder)
    return set_error(KAN_ERR_INVALID, "kan_silu_deriv: order must lie in 0..%d, got %lld",
                     kMaxSiluOrder, (long long)order);
  if (count == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_silu_deriv", "x"));
  KAN_TRY(need_ptr(out, "kan_silu_deriv", "out"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_silu_deriv<float>(static_cast<const float*>(x), static_cast<const float*>(scale),
                                     nullptr, static_cast<float*>(out), count, (int)order, st);
  return launch_silu_deriv<double>(static_cast<const double*>(x),
                                   static_cast<const double*>(scale), nullptr,
                                   static_cast<double*>(out), count, (int)order, st);
}

int kan_hip_basis_grad(int dtype, const void* x, const void* grid, const void* gH, void* gx,
                       int64_t n, int64_t I, int64_t G, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_basis_grad"));
  KAN_TRY(check_layer("kan_basis_grad", n, I, 0, G, k));
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_basis_grad", "x"));
  KAN_TRY(need_ptr(grid, "kan_basis_grad", "grid"));
  KAN_TRY(need_ptr(gH, "kan_basis_grad", "grad_basis"));
  KAN_TRY(need_ptr(gx, "kan_basis_grad", "grad_x"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t R = G + k;
  // The derivative contraction always uses the local kernel, as the
  // reference's basis_grad does (csrc/kan_cuda.cu:459-464).
  if (dtype == KAN_DTYPE_F32)
    return launch_basis_grad<float>(static_cast<const float*>(x), static_cast<const float*>(grid),
                                    static_cast<const float*>(gH), I * R, nullptr,
                                    static_cast<float*>(gx), n, I, (int)G, (int)k, 1, st);
  return launch_basis_grad<double>(static_cast<const double*>(x), static_cast<const double*>(grid),
                                   static_cast<const double*>(gH), I * R, nullptr,
                                   static_cast<double*>(gx), n, I, (int)G, (int)k, 1, st);
}

int kan_hip_basis_silu(int dtype, const void* x, const void* grid, void* basis, void* silu,
                       int64_t n, int64_t I, int64_t G, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_basis_silu"));
  KAN_TRY(check_layer("kan_basis_silu", n, I, 0, G, k));
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_basis_silu", "x"));
  KAN_TRY(need_ptr(grid, "kan_basis_silu", "grid"));
  KAN_TRY(need_ptr(basis, "kan_basis_silu", "basis"));
  KAN_TRY(need_ptr(silu, "kan_basis_silu", "silu"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t R = G + k;
  if (dtype == KAN_DTYPE_F32)
    return launch_basis<float>(static_cast<const float*>(x), static_cast<const float*>(grid),
                               static_cast<float*>(basis), I * R, static_cast<float*>(silu), n, I,
                               (int)G, (int)k, g_basis_impl.load(), st, I);
  return launch_basis<double>(static_cast<const double*>(x), static_cast<const double*>(grid),
                              static_cast<double*>(basis), I * R, static_cast<double*>(silu), n, I,
                              (int)G, (int)k, g_basis_impl.load(), st, I);
}

int kan_hip_basis_silu_grad(int dtype, const void* x, const void* grid, const void* gH,
                            const void* gs, void* gx, int64_t n, int64_t I, int64_t G, int64_t k,
                            void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_basis_silu_grad"));
  KAN_TRY(check_layer("kan_basis_silu_grad", n, I, 0, G, k));
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(x, "kan_basis_silu_grad", "x"));
  KAN_TRY(need_ptr(grid, "kan_basis_silu_grad", "grid"));
  KAN_TRY(need_ptr(gH, "kan_basis_silu_grad", "grad_basis"));
  KAN_TRY(need_ptr(gs, "kan_basis_silu_grad", "grad_silu"));
  KAN_TRY(need_ptr(gx, "kan_basis_silu_grad", "grad_x"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t R = G + k;
  if (dtype == KAN_DTYPE_F32)
    return launch_basis_grad<float>(static_cast<const float*>(x), static_cast<const float*>(grid),
                                    static_cast<const float*>(gH), I * R,
                                    static_cast<const float*>(gs), static_cast<float*>(gx), n, I,
                                    (int)G, (int)k, 1, st, I);
  return launch_basis_grad<double>(static_cast<const double*>(x), static_cast<const double*>(grid),
                                   static_cast<const double*>(gH), I * R,
                                   static_cast<const double*>(gs), static_cast<double*>(gx), n, I,
                                   (int)G, (int)k, 1, st, I);
}

int64_t kan_hip_aug_width(int64_t I, int64_t G, int64_t k, int has_base) {
  if (I < 0 || G < 1 || k < 1 || k > 3) return -1;
  return aug_width(I, G + k, has_base != 0);
}

int kan_hip_forward_workspace(int dtype, int64_t n, int64_t I, int64_t O, int64_t G, int64_t k,
                              int has_base, size_t* bytes) {
  KAN_TRY(check_dtype(dtype, "kan_forward_workspace"));
  KAN_TRY(check_layer("kan_forward_workspace", n, I, O, G, k));
  KAN_TRY(need_ptr(bytes, "kan_forward_workspace", "bytes"));
  int64_t ld, kaug, we, pe;
  if (dtype == KAN_DTYPE_F32) forward_plan<float>(n, I, O, G + k, has_base != 0, &ld, &kaug, &we, &pe);
  else forward_plan<double>(n, I, O, G + k, has_base != 0, &ld, &kaug, &we, &pe);
  *bytes = (dtype == KAN_DTYPE_F32 ? 4 : 8) * (size_t)(we + pe);
  return KAN_OK;
}

int kan_hip_forward(int dtype, const void* x, const void* grid, const void* bw, const void* sw,
                    const void* scaler, void* out, void* aug, void* ws, size_t ws_bytes,
                    int64_t n, int64_t I, int64_t O, int64_t G, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_forward"));
  KAN_TRY(check_layer("kan_forward", n, I, O, G, k));
  // Pointers are only required for buffers of non-zero size.
  const int64_t R = G + k;
  const int64_t ld = aug_width(I, R, bw != nullptr);
  if (O * I > 0) KAN_TRY(need_ptr(sw, "kan_forward", "spline_weight"));
  if (O * ld > 0) KAN_TRY(need_ptr(ws, "kan_forward", "workspace"));
  if (n * I > 0) {
    KAN_TRY(need_ptr(x, "kan_forward", "x"));
    KAN_TRY(need_ptr(grid, "kan_forward", "grid"));
  }
  if (n * ld > 0) KAN_TRY(need_ptr(aug, "kan_forward", "basis_aug"));
  if (n * O > 0) KAN_TRY(need_ptr(out, "kan_forward", "output"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return forward_impl<float>(x, grid, bw, sw, scaler, out, aug, ws, ws_bytes, n, I, O, G, k, st);
  return forward_impl<double>(x, grid, bw, sw, scaler, out, aug, ws, ws_bytes, n, I, O, G, k, st);
}

int kan_hip_pack_weight(int dtype, const void* bw, const void* sw, const void* scaler, void* waug,
                        int64_t I, int64_t O, int64_t G, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_pack_weight"));
  KAN_TRY(check_layer("kan_pack_weight", 0, I, O, G, k));
  const int64_t R = G + k;
  const int64_t ld = aug_width(I, R, bw != nullptr);
  if (O * ld == 0) return KAN_OK;
  KAN_TRY(need_ptr(sw, "kan_pack_weight", "spline_weight"));
  KAN_TRY(need_ptr(waug, "kan_pack_weight", "weight_aug"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_build_waug<float>(static_cast<const float*>(sw), static_cast<const float*>(scaler),
                                    static_cast<const float*>(bw), static_cast<float*>(waug), ld, O,
                                    I, R, st);
  return launch_build_waug<double>(static_cast<const double*>(sw),
                                   static_cast<const double*>(scaler),
                                   static_cast<const double*>(bw), static_cast<double*>(waug), ld,
                                   O, I, R, st);
}


int kan_hip_infer_workspace(int dtype, int64_t n, int64_t I, int64_t O, int64_t G, int64_t k,
                            int has_base, size_t* bytes) {
  KAN_TRY(check_dtype(dtype, "kan_infer_workspace"));
  KAN_TRY(check_layer("kan_infer_workspace", n, I, O, G, k));
  KAN_TRY(need_ptr(bytes, "kan_infer_workspace", "bytes"));
  int64_t ld, kaug, a, pe;
  if (dtype == KAN_DTYPE_F32) infer_plan<float>(n, I, O, G + k, has_base != 0, &ld, &kaug, &a, &pe);
  else infer_plan<double>(n, I, O, G + k, has_base != 0, &ld, &kaug, &a, &pe);
  *bytes = (dtype == KAN_DTYPE_F32 ? 4 : 8) * (size_t)(a + pe);
  return KAN_OK;
}

namespace {
// kan_hip_infer with the split slices bounded by scratch_elems (-1: none).
int infer_run(int dtype, const void* x, const void* grid, const void* waug, void* out, void* ws,
              size_t ws_bytes, int64_t n, int64_t I, int64_t O, int64_t G, int64_t k,
              int has_base, void* stream, int64_t scratch_elems) {
  KAN_TRY(need_ptr(out, "kan_infer", "output"));
  KAN_TRY(need_ptr(waug, "kan_infer", "weight_aug"));
  if (n * I > 0) {
    KAN_TRY(need_ptr(x, "kan_infer", "x"));
    KAN_TRY(need_ptr(grid, "kan_infer", "grid"));
  }
  const int64_t R = G + k;
  int64_t ld, kaug, aug_elems, part_elems;
  const size_t elem = dtype == KAN_DTYPE_F32 ? 4 : 8;
  if (dtype == KAN_DTYPE_F32)
    infer_plan<float>(n, I, O, R, has_base != 0, &ld, &kaug, &aug_elems, &part_elems,
                      scratch_elems);
  else
    infer_plan<double>(n, I, O, R, has_base != 0, &ld, &kaug, &aug_elems, &part_elems,
                       scratch_elems);
  const int64_t cap = infer_slice_cap(scratch_elems, aug_elems);
  const size_t need = elem * (size_t)(aug_elems + part_elems);
  if (ws_bytes < need || ws == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "kan_infer: workspace of %zu bytes is smaller than the %zu required",
                     ws_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define KAN_INFER_CALL(T)                                                                        \
  do {                                                                                           \
    T* aug = static_cast<T*>(ws);                                                                \
    KAN_TRY(launch_basis<T>(static_cast<const T*>(x), static_cast<const T*>(grid), aug, ld,      \
                            has_base ? aug + I * R : nullptr, n, I, (int)G, (int)k,              \
                            g_basis_impl.load(), st));                                           \
    return launch_matmul<T>(kLayoutNT, n, O, kaug, aug, ld, static_cast<const T*>(waug), ld,     \
                            static_cast<T*>(out), O, aug + aug_elems, st, cap);                  \
  } while (0)
  if (dtype == KAN_DTYPE_F32) KAN_INFER_CALL(float);
  KAN_INFER_CALL(double);
#undef KAN_INFER_CALL
}
}  // namespace

int kan_hip_infer(int dtype, const void* x, const void* grid, const void* waug, void* out,
                  void* ws, size_t ws_bytes, int64_t n, int64_t I, int64_t O, int64_t G, int64_t k,
                  int has_base, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_infer"));
  KAN_TRY(check_layer("kan_infer", n, I, O, G, k));
  if (n * O == 0) return KAN_OK;
  return infer_run(dtype, x, grid, waug, out, ws, ws_bytes, n, I, O, G, k, has_base, stream, -1);
}

int kan_hip_infer_noalloc(int dtype, const void* x, const void* grid, const void* waug, void* out,
                          int64_t n, int64_t I, int64_t O, int64_t G, int64_t k, int has_base,
                          void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_infer_noalloc"));
  KAN_TRY(check_layer("kan_infer_noalloc", n, I, O, G, k));
  if (n * O == 0) return KAN_OK;
  const int64_t R = G + k;
  int64_t ld, kaug, aug_elems, part_elems;
  const size_t elem = dtype == KAN_DTYPE_F32 ? 4 : 8;
  const int64_t scratch_elems = (int64_t)(KAN_NOALLOC_SCRATCH_BYTES / elem);
  if (dtype == KAN_DTYPE_F32)
    infer_plan<float>(n, I, O, R, has_base != 0, &ld, &kaug, &aug_elems, &part_elems,
                      scratch_elems);
  else
    infer_plan<double>(n, I, O, R, has_base != 0, &ld, &kaug, &aug_elems, &part_elems,
                       scratch_elems);
  const size_t need = elem * (size_t)(aug_elems + part_elems);
  if (need > (size_t)KAN_NOALLOC_SCRATCH_BYTES)
    return set_error(KAN_ERR_WORKSPACE,
                     "kan_infer_noalloc: %lld samples of this layer need %zu bytes of scratch, more "
                     "than the library's fixed %zu bytes; call kan_hip_infer with a workspace "
                     "(or split the batch)",
                     (long long)n, need, (size_t)KAN_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  KAN_TRY(scratch_of_current_device(&ws));
  // Every element of the workspace that the kernels read is written first in
  // the same call (basis columns below kaug, whole split slices), so the
  // previous call's contents need no clearing.
  return infer_run(dtype, x, grid, waug, out, ws, (size_t)KAN_NOALLOC_SCRATCH_BYTES, n, I, O, G, k,
                   has_base, stream, scratch_elems);
}

int kan_hip_pack_basis(int dtype, const void* basis, const void* x, void* aug, int64_t n,
                       int64_t I, int64_t G, int64_t k, int has_base, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_pack_basis"));
  KAN_TRY(check_layer("kan_pack_basis", n, I, 0, G, k));
  if (n == 0 || I == 0) return KAN_OK;
  KAN_TRY(need_ptr(basis, "kan_pack_basis", "basis"));
  KAN_TRY(need_ptr(aug, "kan_pack_basis", "basis_aug"));
  if (has_base) KAN_TRY(need_ptr(x, "kan_pack_basis", "x"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t R = G + k;
  const int64_t ld = aug_width(I, R, has_base != 0);
  if (dtype == KAN_DTYPE_F32)
    return launch_pack_basis<float>(static_cast<const float*>(basis), static_cast<const float*>(x),
                                    static_cast<float*>(aug), ld, n, I, R, has_base != 0, st);
  return launch_pack_basis<double>(static_cast<const double*>(basis), static_cast<const double*>(x),
                                   static_cast<double*>(aug), ld, n, I, R, has_base != 0, st);
}

int kan_hip_backward_workspace(int dtype, int64_t n, int64_t I, int64_t O, int64_t G, int64_t k,
                               int has_base, int need_x, int need_params, size_t* bytes) {
  KAN_TRY(check_dtype(dtype, "kan_backward_workspace"));
  KAN_TRY(check_layer("kan_backward_workspace", n, I, O, G, k));
  KAN_TRY(need_ptr(bytes, "kan_backward_workspace", "bytes"));
  BackwardPlan p;
  size_t elem;
  if (dtype == KAN_DTYPE_F32) {
    p = plan_backward<float>(n, I, O, G, k, has_base != 0, need_x != 0, need_params != 0);
    elem = 4;
  } else {
    p = plan_backward<double>(n, I, O, G, k, has_base != 0, need_x != 0, need_params != 0);
    elem = 8;
  }
  *bytes = elem * (p.waug_elems + p.e_elems + p.part_elems);
  return KAN_OK;
}

int kan_hip_backward(int dtype, const void* D, const void* x, const void* grid, const void* bw,
                     const void* sw, const void* scaler, const void* aug, void* gx, void* gbw,
                     void* gsw, void* gscaler, void* ws, size_t ws_bytes, int64_t n, int64_t I,
                     int64_t O, int64_t G, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "kan_backward"));
  KAN_TRY(check_layer("kan_backward", n, I, O, G, k));
  if (gbw != nullptr && bw == nullptr)
    return set_error(KAN_ERR_INVALID, "kan_backward: grad_base_weight requested without base_weight");
  if (gscaler != nullptr && scaler == nullptr)
    return set_error(KAN_ERR_INVALID, "kan_backward: grad_spline_scaler requested without spline_scaler");
  const bool need_params = gsw != nullptr || gscaler != nullptr || gbw != nullptr;
  if (O * I > 0) KAN_TRY(need_ptr(sw, "kan_backward", "spline_weight"));
  if (n * O > 0) KAN_TRY(need_ptr(D, "kan_backward", "grad_output"));
  if (n * I > 0 && gx != nullptr) {
    KAN_TRY(need_ptr(x, "kan_backward", "x"));
    KAN_TRY(need_ptr(grid, "kan_backward", "grid"));
  }
  if (n > 0 && I > 0 && need_params) KAN_TRY(need_ptr(aug, "kan_backward", "basis_aug"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return backward_impl<float>(D, x, grid, bw, sw, scaler, aug, gx, gbw, gsw, gscaler, ws,
                                ws_bytes, n, I, O, G, k, st);
  return backward_impl<double>(D, x, grid, bw, sw, scaler, aug, gx, gbw, gsw, gscaler, ws,
                               ws_bytes, n, I, O, G, k, st);
}

int kan_hip_edge_workspace(int dtype, int64_t n, int64_t I, int64_t O, int64_t R, int backward,
                           size_t* bytes) {
  KAN_TRY(check_dtype(dtype, "edge_workspace"));
  KAN_TRY(need_ptr(bytes, "edge_workspace", "bytes"));
  if (n < 0 || I < 0 || O < 0 || R < 0) return set_error(KAN_ERR_INVALID, "edge_workspace: negative size");
  *bytes = edge_ws_bytes(dtype, n, I, O, R, backward != 0);
  return KAN_OK;
}

int kan_hip_edge_abs_mean(int dtype, const void* s, const void* H, const void* bw, const void* W,
                          void* a, void* ws, size_t ws_bytes, int64_t n, int64_t I, int64_t O,
                          int64_t R, void* stream) {
  KAN_TRY(check_edge("edge_abs_mean", dtype, s, H, bw, W, n, I, O, R));
  KAN_TRY(need_ptr(a, "edge_abs_mean", "a"));
  const size_t need = edge_ws_bytes(dtype, n, I, O, R, false);
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  const int splits = need > 0 ? edge_pick_splits(dtype, n, I, O, R, false) : 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_edge_forward<float>(static_cast<const float*>(s), static_cast<const float*>(H),
                                      static_cast<const float*>(bw), static_cast<const float*>(W),
                                      static_cast<float*>(a), static_cast<float*>(ws), splits, n,
                                      I, O, R, st);
  return launch_edge_forward<double>(static_cast<const double*>(s), static_cast<const double*>(H),
                                     static_cast<const double*>(bw), static_cast<const double*>(W),
                                     static_cast<double*>(a), static_cast<double*>(ws), splits, n,
                                     I, O, R, st);
}

int kan_hip_edge_abs_mean_backward(int dtype, const void* ga, const void* s, const void* H,
                                   const void* bw, const void* W, void* gs, void* gH, void* gbw,
                                   void* gW, void* ws, size_t ws_bytes, int64_t n, int64_t I,
                                   int64_t O, int64_t R, void* stream) {
  KAN_TRY(check_edge("edge_abs_mean_backward", dtype, s, H, bw, W, n, I, O, R));
  KAN_TRY(need_ptr(ga, "edge_abs_mean_backward", "grad_a"));
  if ((gs != nullptr || gbw != nullptr) && bw == nullptr)
    return set_error(KAN_ERR_INVALID, "edge_abs_mean_backward: base gradients requested without a base branch");
  const bool want_params = gbw != nullptr || gW != nullptr;
  const size_t need = want_params ? edge_ws_bytes(dtype, n, I, O, R, true) : 0;
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean_backward: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  const int splits = need > 0 ? edge_pick_splits(dtype, n, I, O, R, true) : 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_edge_backward<float>(
        static_cast<const float*>(ga), static_cast<const float*>(s), static_cast<const float*>(H),
        static_cast<const float*>(bw), static_cast<const float*>(W), static_cast<float*>(gs),
        static_cast<float*>(gH), static_cast<float*>(gbw), static_cast<float*>(gW),
        static_cast<float*>(ws), splits, n, I, O, R, st);
  return launch_edge_backward<double>(
      static_cast<const double*>(ga), static_cast<const double*>(s), static_cast<const double*>(H),
      static_cast<const double*>(bw), static_cast<const double*>(W), static_cast<double*>(gs),
      static_cast<double*>(gH), static_cast<double*>(gbw), static_cast<double*>(gW),
      static_cast<double*>(ws), splits, n, I, O, R, st);
}

int kan_hip_edge_linear_supported(int dtype, int64_t n, int64_t I, int64_t O, int64_t R) {
  return dtype == KAN_DTYPE_F32 && edge_linear_fold_supported(n, I, O, R) ? 1 : 0;
}

int kan_hip_edge_linear_backward(int dtype, const void* ga, const void* gy, const void* s,
                                 const void* H, const void* bw, const void* W, void* gs, void* gH,
                                 void* gbw, void* gW, void* ws, size_t ws_bytes, int64_t n,
                                 int64_t I, int64_t O, int64_t R, void* stream) {
  KAN_TRY(check_edge("edge_linear_backward", dtype, s, H, bw, W, n, I, O, R));
  KAN_TRY(need_ptr(ga, "edge_linear_backward", "grad_a"));
  KAN_TRY(need_ptr(gy, "edge_linear_backward", "grad_y"));
  if ((gs != nullptr || gbw != nullptr) && bw == nullptr)
    return set_error(KAN_ERR_INVALID, "edge_linear_backward: base gradients requested without a base branch");
  if (!kan_hip_edge_linear_supported(dtype, n, I, O, R))
    return set_error(KAN_ERR_LIMIT, "edge_linear_backward: needs float32, n > 0, out_features <= 512, num_basis + 1 <= 16");
  const size_t need = edge_ws_bytes(dtype, n, I, O, R, true);
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "edge_linear_backward: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  const int splits = edge_pick_splits(dtype, n, I, O, R, true);
  return launch_edge_linear_backward_mfma(
      static_cast<const float*>(ga), static_cast<const float*>(gy), static_cast<const float*>(s),
      static_cast<const float*>(H), static_cast<const float*>(bw), static_cast<const float*>(W),
      static_cast<float*>(gs), static_cast<float*>(gH), static_cast<float*>(gbw),
      static_cast<float*>(gW), static_cast<float*>(ws), splits, n, I, O, R,
      static_cast<hipStream_t>(stream));
}

int kan_hip_edge_linear_forward_supported(int dtype, int64_t n, int64_t I, int64_t O, int64_t R) {
  return dtype == KAN_DTYPE_F32 && edge_ylin_supported(n, I, O, R) ? 1 : 0;
}

int kan_hip_edge_linear_forward_workspace(int dtype, int64_t n, int64_t I, int64_t O, int64_t R,
                                          size_t* bytes) {
  KAN_TRY(need_ptr(bytes, "edge_linear_forward_workspace", "bytes"));
  if (!kan_hip_edge_linear_forward_supported(dtype, n, I, O, R))
    return set_error(KAN_ERR_LIMIT, "edge_linear_forward: needs float32, n, in_features, out_features > 0 and num_basis + 1 <= 16");
  *bytes = edge_ylin_ws_bytes(n, I, O);
  return KAN_OK;
}

int kan_hip_edge_linear_forward(int dtype, const void* s, const void* H, const void* bw,
                                const void* W, void* y, void* a, void* ws, size_t ws_bytes,
                                int64_t n, int64_t I, int64_t O, int64_t R, void* stream) {
  KAN_TRY(check_edge("edge_linear_forward", dtype, s, H, bw, W, n, I, O, R));
  KAN_TRY(need_ptr(y, "edge_linear_forward", "y"));
  KAN_TRY(need_ptr(a, "edge_linear_forward", "a"));
  if (!kan_hip_edge_linear_forward_supported(dtype, n, I, O, R))
    return set_error(KAN_ERR_LIMIT, "edge_linear_forward: needs float32, n, in_features, out_features > 0 and num_basis + 1 <= 16");
  const size_t need = edge_ylin_ws_bytes(n, I, O);
  if (ws_bytes < need || ws == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_linear_forward: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  return launch_edge_ylin_forward(static_cast<const float*>(s), static_cast<const float*>(H),
                                  static_cast<const float*>(bw), static_cast<const float*>(W),
                                  static_cast<float*>(y), static_cast<float*>(a),
                                  static_cast<float*>(ws), n, I, O, R,
                                  static_cast<hipStream_t>(stream));
}

int kan_hip_edge_reg_workspace(int dtype, int64_t count, size_t* bytes) {
  KAN_TRY(check_dtype(dtype, "edge_reg_workspace"));
  KAN_TRY(need_ptr(bytes, "edge_reg_workspace", "bytes"));
  if (count < 0) return set_error(KAN_ERR_INVALID, "edge_reg_workspace: negative count");
  *bytes = edge_reg_ws_bytes(count);
  return KAN_OK;
}

int kan_hip_edge_reg(int dtype, const void* a, int64_t count, double mu1, double mu2, void* reg,
                     void* ws, size_t ws_bytes, void* stream) {
  KAN_TRY(check_dtype(dtype, "edge_reg"));
  if (count < 0) return set_error(KAN_ERR_INVALID, "edge_reg: negative count");
  if (count > 0) KAN_TRY(need_ptr(a, "edge_reg", "a"));
  KAN_TRY(need_ptr(reg, "edge_reg", "reg"));
  const size_t need = edge_reg_ws_bytes(count);
  if (ws_bytes < need || ws == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_reg: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  double* w = static_cast<double*>(ws);
  if (dtype == KAN_DTYPE_F32)
    return launch_edge_reg<float>(static_cast<const float*>(a), count, mu1, mu2,
                                  static_cast<float*>(reg), w, st);
  return launch_edge_reg<double>(static_cast<const double*>(a), count, mu1, mu2,
                                 static_cast<double*>(reg), w, st);
}

int kan_hip_edge_reg_backward(int dtype, const void* grad_reg, const void* a, int64_t count,
                              double mu1, double mu2, const void* ws, size_t ws_bytes,
                              void* grad_a, void* stream) {
  KAN_TRY(check_dtype(dtype, "edge_reg_backward"));
  if (count < 0) return set_error(KAN_ERR_INVALID, "edge_reg_backward: negative count");
  if (count == 0) return KAN_OK;
  KAN_TRY(need_ptr(grad_reg, "edge_reg_backward", "grad_reg"));
  KAN_TRY(need_ptr(a, "edge_reg_backward", "a"));
  KAN_TRY(need_ptr(grad_a, "edge_reg_backward", "grad_a"));
  const size_t need = edge_reg_ws_bytes(count);
  if (ws_bytes < need || ws == nullptr)
    return set_error(KAN_ERR_WORKSPACE, "edge_reg_backward: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const double* w = static_cast<const double*>(ws);
  if (dtype == KAN_DTYPE_F32)
    return launch_edge_reg_backward<float>(static_cast<const float*>(grad_reg),
                                           static_cast<const float*>(a), count, mu1, mu2, w,
                                           static_cast<float*>(grad_a), st);
  return launch_edge_reg_backward<double>(static_cast<const double*>(grad_reg),
                                          static_cast<const double*>(a), count, mu1, mu2, w,
                                          static_cast<double*>(grad_a), st);
}

int kan_hip_edge_abs_mean_double_backward_workspace(int dtype, int64_t n, int64_t I, int64_t O,
                                                    int64_t R, size_t* bytes) {
  KAN_TRY(check_dtype(dtype, "edge_abs_mean_double_backward_workspace"));
  KAN_TRY(need_ptr(bytes, "edge_abs_mean_double_backward_workspace", "bytes"));
  if (n < 0 || I < 0 || O < 0 || R < 1)
    return set_error(KAN_ERR_INVALID, "edge_abs_mean_double_backward_workspace: bad sizes");
  *bytes = (dtype == KAN_DTYPE_F32 ? 4 : 8) * edge_double_backward_ws_elems(n, I, O, R);
  return KAN_OK;
}

int kan_hip_edge_abs_mean_double_backward(int dtype, const void* ga, const void* s,
                                          const void* H, const void* bw, const void* W,
                                          const void* u_ds, const void* u_dH, const void* u_dbw,
                                          const void* u_dW, void* g_ga, void* g_s, void* g_H,
                                          void* g_bw, void* g_W, void* ws, size_t ws_bytes,
                                          int64_t n, int64_t I, int64_t O, int64_t R,
                                          void* stream) {
  KAN_TRY(check_edge("edge_abs_mean_double_backward", dtype, s, H, bw, W, n, I, O, R));
  KAN_TRY(need_ptr(ga, "edge_abs_mean_double_backward", "grad_a"));
  if (bw == nullptr && (u_ds != nullptr || u_dbw != nullptr || g_s != nullptr || g_bw != nullptr))
    return set_error(KAN_ERR_INVALID,
                     "edge_abs_mean_double_backward: base-branch operands without a base branch");
  const size_t need = (dtype == KAN_DTYPE_F32 ? 4 : 8) * edge_double_backward_ws_elems(n, I, O, R);
  if (ws_bytes < need || (need > 0 && ws == nullptr))
    return set_error(KAN_ERR_WORKSPACE, "edge_abs_mean_double_backward: workspace of %zu bytes is smaller than the %zu required", ws_bytes, need);
  hipStream_t st = static_cast<hipStream_t>(stream);
#define KAN_EDB_CALL(T)                                                                         \
  launch_edge_double_backward<T>(                                                               \
      static_cast<const T*>(ga), static_cast<const T*>(s), static_cast<const T*>(H),            \
      static_cast<const T*>(bw), static_cast<const T*>(W), static_cast<const T*>(u_ds),         \
      static_cast<const T*>(u_dH), static_cast<const T*>(u_dbw), static_cast<const T*>(u_dW),   \
      static_cast<T*>(g_ga), static_cast<T*>(g_s), static_cast<T*>(g_H), static_cast<T*>(g_bw), \
      static_cast<T*>(g_W), static_cast<T*>(ws), n, I, O, R, st)
  if (dtype == KAN_DTYPE_F32) return KAN_EDB_CALL(float);
  return KAN_EDB_CALL(double);
#undef KAN_EDB_CALL
}

int kan_hip_refit_gram(int dtype, const void* x_t, const void* grid_old, const void* grid_new,
                       double* gram, double* cross, int64_t n, int64_t I, int64_t G_old,
                       int64_t G_new, int64_t k, void* stream) {
  KAN_TRY(check_dtype(dtype, "refit_gram"));
  KAN_TRY(check_layer("refit_gram", n, I, 0, G_old, k));
  KAN_TRY(check_layer("refit_gram", n, I, 0, G_new, k));
  if (I == 0) return KAN_OK;
  KAN_TRY(need_ptr(grid_old, "refit_gram", "grid_old"));
  KAN_TRY(need_ptr(grid_new, "refit_gram", "grid_new"));
  KAN_TRY(need_ptr(gram, "refit_gram", "gram"));
  KAN_TRY(need_ptr(cross, "refit_gram", "cross"));
  if (n > 0) KAN_TRY(need_ptr(x_t, "refit_gram", "x_t"));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == KAN_DTYPE_F32)
    return launch_refit_gram<float>(static_cast<const float*>(x_t),
                                    static_cast<const float*>(grid_old),
                                    static_cast<const float*>(grid_new), gram, cross, n, I,
                                    (int)G_old, (int)G_new, (int)k, st);
  return launch_refit_gram<double>(static_cast<const double*>(x_t),
                                   static_cast<const double*>(grid_old),
                                   static_cast<const double*>(grid_new), gram, cross, n, I,
                                   (int)G_old, (int)G_new, (int)k, st);
}

}  // extern "C"
