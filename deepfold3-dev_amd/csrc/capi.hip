// Library-wide C-ABI entry points: errors, version, dtype casts and the
// elementwise residual add (the eval-mode dropout-add).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "capi.h"
#include "common.h"

namespace pf {

static thread_local char g_err[512] = "";
static thread_local int g_err_code = 0;

void set_error(int code, const char* fmt, ...) {
  g_err_code = code;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int ok() {
  g_err_code = 0;
  g_err[0] = '\0';
  return PF_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(PF_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return PF_ERR_LAUNCH;
  }
  return ok();
}

int cu_count() {
  static std::mutex mu;
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

// ---- kernel timer: events recorded around one selected launch site
namespace {
std::mutex g_timer_mu;
std::string g_timer_name;  // empty: timing off
std::vector<hipEvent_t> g_free_events;
std::vector<std::pair<hipEvent_t, hipEvent_t>> g_pending;
hipEvent_t g_ref = nullptr;  // recorded when timing starts; intervals are end(stop) - end(start)
double g_timer_total_ms = 0.0;
long g_timer_count = 0;

hipEvent_t take_event() {
  if (!g_free_events.empty()) {
    hipEvent_t e = g_free_events.back();
    g_free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

void recycle_locked() {
  for (auto& pr : g_pending) {
    g_free_events.push_back(pr.first);
    g_free_events.push_back(pr.second);
  }
  g_pending.clear();
}
}  // namespace

KernelTimer::KernelTimer(const char* name, hipStream_t stream) : stream_(stream) {
  std::lock_guard<std::mutex> lk(g_timer_mu);
  if (g_timer_name.empty() || g_timer_name != name || !g_ref) return;
  hipEvent_t e = take_event();
  if (e && hipEventRecord(e, stream_) == hipSuccess) start_ = e;
}

void KernelTimer::stop() {
  if (!start_) return;
  std::lock_guard<std::mutex> lk(g_timer_mu);
  hipEvent_t e = take_event();
  if (e && hipEventRecord(e, stream_) == hipSuccess) g_pending.emplace_back((hipEvent_t)start_, e);
  start_ = nullptr;
}

}  // namespace pf

template <class TS, class TD>
__global__ void cast_kernel(const TS* __restrict__ src, TD* __restrict__ dst, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = from_f32<TD>(to_f32(src[i]));
}

// out[i] = res[i] + x[i], in the dtype of res (x may be another dtype).
template <class TR, class TX>
__global__ void add_kernel(const TR* __restrict__ res, const TX* __restrict__ x, TR* __restrict__ out, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = from_f32<TR>(to_f32(res[i]) + to_f32(x[i]));
}

static unsigned grid_for(size_t n) {
  size_t g = (n + 255) / 256;
  return (unsigned)(g > 65536 ? 65536 : (g == 0 ? 1 : g));
}

extern "C" {

const char* pf_last_error(void) { return pf::g_err; }

int pf_kernel_timer_start(const char* kernel) {
  PF_REQUIRE(kernel != nullptr, PF_ERR_INVALID_ARG, "pf_kernel_timer_start: null name");
  PF_REQUIRE(hipDeviceSynchronize() == hipSuccess, PF_ERR_LAUNCH, "pf_kernel_timer_start: device error");
  std::lock_guard<std::mutex> lk(pf::g_timer_mu);
  pf::g_timer_name = kernel;
  pf::g_timer_total_ms = 0.0;
  pf::g_timer_count = 0;
  pf::recycle_locked();
  if (!pf::g_ref) {
    PF_REQUIRE(hipEventCreate(&pf::g_ref) == hipSuccess, PF_ERR_LAUNCH, "pf_kernel_timer_start: event");
  }
  hipError_t e = hipEventRecord(pf::g_ref, nullptr);
  if (e == hipSuccess) e = hipEventSynchronize(pf::g_ref);
  PF_REQUIRE(e == hipSuccess, PF_ERR_LAUNCH, "pf_kernel_timer_start: %s", hipGetErrorString(e));
  return pf::ok();
}

int pf_kernel_timer_read(double* total_ms, long* count) {
  PF_REQUIRE(total_ms && count, PF_ERR_INVALID_ARG, "pf_kernel_timer_read: null pointer");
  std::lock_guard<std::mutex> lk(pf::g_timer_mu);
  for (auto& pr : pf::g_pending) {
    // elapsed(ref, x) = end(x) - start(ref): the difference is end(stop) - end(start).
    float t0 = 0.f, t1 = 0.f;
    hipError_t e = hipEventSynchronize(pr.second);
    if (e == hipSuccess) e = hipEventElapsedTime(&t0, pf::g_ref, pr.first);
    if (e == hipSuccess) e = hipEventElapsedTime(&t1, pf::g_ref, pr.second);
    PF_REQUIRE(e == hipSuccess, PF_ERR_LAUNCH, "pf_kernel_timer_read: %s", hipGetErrorString(e));
    pf::g_timer_total_ms += (double)t1 - (double)t0;
    pf::g_timer_count += 1;
  }
  pf::recycle_locked();
  *total_ms = pf::g_timer_total_ms;
  *count = pf::g_timer_count;
  return pf::ok();
}

int pf_kernel_timer_stop(void) {
  std::lock_guard<std::mutex> lk(pf::g_timer_mu);
  pf::g_timer_name.clear();
  return pf::ok();
}
int pf_last_error_code(void) { return pf::g_err_code; }
int pf_version(void) { return PF_ABI_VERSION; }

int pf_cast(const void* src, int src_dtype, void* dst, int dst_dtype, size_t n, void* stream) {
  PF_REQUIRE(src && dst, PF_ERR_INVALID_ARG, "pf_cast: null pointer");
  PF_REQUIRE((src_dtype == PF_F32 || src_dtype == PF_BF16) && (dst_dtype == PF_F32 || dst_dtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "pf_cast: dtype codes must be PF_F32 or PF_BF16");
  if (n == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  unsigned g = grid_for(n);
  if (src_dtype == PF_F32 && dst_dtype == PF_F32)
    cast_kernel<float, float><<<g, 256, 0, s>>>((const float*)src, (float*)dst, n);
  else if (src_dtype == PF_F32)
    cast_kernel<float, bf16><<<g, 256, 0, s>>>((const float*)src, (bf16*)dst, n);
  else if (dst_dtype == PF_F32)
    cast_kernel<bf16, float><<<g, 256, 0, s>>>((const bf16*)src, (float*)dst, n);
  else
    cast_kernel<bf16, bf16><<<g, 256, 0, s>>>((const bf16*)src, (bf16*)dst, n);
  return pf::check_launch("pf_cast");
}

int pf_add(const void* res, int res_dtype, const void* x, int x_dtype, void* out, size_t n, void* stream) {
  PF_REQUIRE(res && x && out, PF_ERR_INVALID_ARG, "pf_add: null pointer");
  PF_REQUIRE((res_dtype == PF_F32 || res_dtype == PF_BF16) && (x_dtype == PF_F32 || x_dtype == PF_BF16),
             PF_ERR_UNSUPPORTED, "pf_add: dtype codes must be PF_F32 or PF_BF16");
  if (n == 0) return pf::ok();
  hipStream_t s = pf::as_stream(stream);
  unsigned g = grid_for(n);
  if (res_dtype == PF_F32 && x_dtype == PF_F32)
    add_kernel<float, float><<<g, 256, 0, s>>>((const float*)res, (const float*)x, (float*)out, n);
  else if (res_dtype == PF_F32)
    add_kernel<float, bf16><<<g, 256, 0, s>>>((const float*)res, (const bf16*)x, (float*)out, n);
  else if (x_dtype == PF_F32)
    add_kernel<bf16, float><<<g, 256, 0, s>>>((const bf16*)res, (const float*)x, (bf16*)out, n);
  else
    add_kernel<bf16, bf16><<<g, 256, 0, s>>>((const bf16*)res, (const bf16*)x, (bf16*)out, n);
  return pf::check_launch("pf_add");
}

}  // extern "C"
