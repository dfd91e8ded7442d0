// Host runtime of the library: the C ABI's per-thread error state, per-device facts and workspaces.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "lq_common.hpp"
#include "lq_workspace.hpp"

namespace lq {

namespace {
thread_local std::string g_error;
std::mutex g_mutex;
constexpr int kMaxDevices = 64;
Workspace g_ws[kMaxDevices];
int g_cus[kMaxDevices] = {};
}  // namespace

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LQ_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return LQ_OK;
}

int device_cus(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return 256;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

Workspace* workspace_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(LQ_ERR_DEVICE, "workspace: no current device");
    return nullptr;
  }
  return &g_ws[dev];
}

int Workspace::reserve_stream(size_t bytes, size_t counters_needed) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (bytes > partial_bytes) {
    const size_t cap = std::max(bytes, size_t(64) << 20);
    if (partials) (void)hipFree(partials);
    partials = nullptr;
    partial_bytes = 0;
    if (hipMalloc(&partials, cap) != hipSuccess) return fail(LQ_ERR_DEVICE, "workspace: partial buffer allocation failed");
    partial_bytes = cap;
  }
  if (counters_needed > counter_count) {
    const size_t cap = std::max(counters_needed, size_t(1) << 16);
    if (counters) (void)hipFree(counters);
    counters = nullptr;
    counter_count = 0;
    if (hipMalloc(&counters, cap * sizeof(int)) != hipSuccess ||
        hipMemset(counters, 0, cap * sizeof(int)) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "workspace: counter allocation failed");
    counter_count = cap;
  }
  if (!sync) {
    if (hipMalloc(&sync, 16 * sizeof(int)) != hipSuccess || hipMemset(sync, 0, 16 * sizeof(int)) != hipSuccess) {
      sync = nullptr;
      return fail(LQ_ERR_DEVICE, "workspace: counter allocation failed");
    }
  }
  return LQ_OK;
}

int Workspace::reserve_prefill(size_t bytes, size_t counters_needed) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (bytes > pf_partial_bytes) {
    if (pf_partials) (void)hipFree(pf_partials);
    pf_partials = nullptr;
    pf_partial_bytes = 0;
    if (hipMalloc(&pf_partials, bytes) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "workspace: prefill partial buffer allocation failed");
    pf_partial_bytes = bytes;
  }
  if (counters_needed > pf_counter_count) {
    const size_t cap = std::max(counters_needed, size_t(4096));
    if (pf_counters) (void)hipFree(pf_counters);
    pf_counters = nullptr;
    pf_counter_count = 0;
    if (hipMalloc(&pf_counters, cap * sizeof(int)) != hipSuccess ||
        hipMemset(pf_counters, 0, cap * sizeof(int)) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "workspace: prefill counter allocation failed");
    pf_counter_count = cap;
  }
  return LQ_OK;
}

}  // namespace lq

extern "C" {

const char* lq_last_error(void) { return lq::g_error.c_str(); }

const char* lq_version(void) { return "ling-gemm-mi355x 0.1 (gfx950)"; }

int lq_init(void) {
  lq::Workspace* ws = lq::workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  int rc = ws->reserve_stream(size_t(64) << 20, size_t(1) << 16);
  if (rc) return rc;
  return hipDeviceSynchronize() == hipSuccess ? LQ_OK : lq::fail(LQ_ERR_DEVICE, "lq_init: device synchronize failed");
}

}  // extern "C"
