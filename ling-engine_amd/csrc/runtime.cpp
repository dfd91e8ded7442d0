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
  if (external) {
    if (bytes > partial_bytes || counters_needed > counter_count)
      return fail(LQ_ERR_ARG, "workspace: the caller's workspace is too small for this launch (" +
                                  std::to_string(bytes) + " bytes of partial sums and " +
                                  std::to_string(counters_needed) + " counters needed; see lq_stream_workspace_bytes)");
    return LQ_OK;
  }
  if (bytes > partial_bytes) {
    const size_t cap = std::max(bytes, size_t(64) << 20);
    if (partials) (void)hipFree(partials);
    partials = nullptr;
    partial_bytes = 0;
    if (hipMalloc(&partials, cap) != hipSuccess) return fail(LQ_ERR_DEVICE, "workspace: partial buffer allocation failed");
    partial_bytes = cap;
  }
  if (counters_needed > counter_count) {
    const size_t cap = std::max(counters_needed, size_t(1) << 20);
    if (counters) (void)hipFree(counters);
    counters = nullptr;
    counter_count = 0;
    if (hipMalloc(&counters, cap * sizeof(int)) != hipSuccess ||
        hipMemset(counters, 0, cap * sizeof(int)) != hipSuccess)
      return fail(LQ_ERR_DEVICE, "workspace: counter allocation failed");
    counter_count = cap;
  }
  if (!sync) {
    if (hipMalloc(&sync, 64 * sizeof(int)) != hipSuccess || hipMemset(sync, 0, 64 * sizeof(int)) != hipSuccess) {
      sync = nullptr;
      return fail(LQ_ERR_DEVICE, "workspace: counter allocation failed");
    }
  }
  return LQ_OK;
}

// Allocated once, at the bound the caller passes (reserve_prefill_scratch), and never reallocated: a graph captured
// with these pointers must stay valid.
int Workspace::reserve_prefill(size_t bytes, size_t counters_needed) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (pf_partials) {
    if (bytes > pf_partial_bytes || counters_needed > pf_counter_count)
      return fail(LQ_ERR_DEVICE, "workspace: prefill split scratch is smaller than its bound");
    return LQ_OK;
  }
  if (hipMalloc(&pf_partials, bytes) != hipSuccess) {
    pf_partials = nullptr;
    return fail(LQ_ERR_DEVICE, "workspace: prefill partial buffer allocation failed");
  }
  if (hipMalloc(&pf_counters, counters_needed * sizeof(int)) != hipSuccess ||
      hipMemset(pf_counters, 0, counters_needed * sizeof(int)) != hipSuccess) {
    (void)hipFree(pf_partials);
    pf_partials = nullptr;
    pf_counters = nullptr;
    return fail(LQ_ERR_DEVICE, "workspace: prefill counter allocation failed");
  }
  pf_partial_bytes = bytes;
  pf_counter_count = counters_needed;
  return LQ_OK;
}

// Caller-owned layout: [0, 256) sync words, [256, 256 + 4 kExtCounters) counters, then the partial sums.
constexpr size_t kExtCounters = size_t(1) << 16;
constexpr size_t kExtHead = 256 + 4 * kExtCounters;

int Workspace::set_external(void* buf, size_t bytes) {
  std::lock_guard<std::mutex> lock(g_mutex);
  if (buf && (reinterpret_cast<uintptr_t>(buf) % 256 != 0 || bytes < kExtHead + 256 * 1024))
    return fail(LQ_ERR_ARG, "set_workspace: the buffer must be 256-byte aligned and at least " +
                                std::to_string(kExtHead + 256 * 1024) + " bytes");
  if (buf && hipMemset(buf, 0, kExtHead) != hipSuccess)
    return fail(LQ_ERR_DEVICE, "set_workspace: clearing the counters failed");
  if (!external) {  // release the library's own buffers (hipFree waits for work that uses them)
    if (partials) (void)hipFree(partials);
    if (counters) (void)hipFree(counters);
    if (sync) (void)hipFree(sync);
  }
  partials = nullptr;
  counters = nullptr;
  sync = nullptr;
  partial_bytes = 0;
  counter_count = 0;
  external = buf != nullptr;
  if (external) {
    uint8_t* b = static_cast<uint8_t*>(buf);
    sync = reinterpret_cast<int*>(b);
    counters = reinterpret_cast<int*>(b + 256);
    counter_count = kExtCounters;
    partials = reinterpret_cast<float*>(b + kExtHead);
    partial_bytes = bytes - kExtHead;
  }
  return LQ_OK;
}

}  // namespace lq

extern "C" {

const char* lq_last_error(void) { return lq::g_error.c_str(); }

const char* lq_version(void) { return "ling-gemm-mi355x 0.1 (gfx950)"; }

size_t lq_stream_workspace_bytes(int max_rows) {
  if (max_rows < 1 || max_rows > LQ_MAX_STREAM_ROWS) return 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  return lq::kExtHead + lq::stream_partial_bound(static_cast<size_t>(lq::device_cus(dev)), max_rows);
}

int lq_set_workspace(void* buffer, size_t bytes) {
  lq::Workspace* ws = lq::workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  return ws->set_external(buffer, bytes);
}

int lq_init(void) {
  lq::Workspace* ws = lq::workspace_for_current_device();
  if (!ws) return LQ_ERR_DEVICE;
  // the bound of any skinny launch, so that no later call allocates (graph capture)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return lq::fail(LQ_ERR_DEVICE, "lq_init: no current device");
  const size_t bound = lq::stream_partial_bound(static_cast<size_t>(lq::device_cus(dev)), LQ_MAX_STREAM_ROWS);
  int rc = ws->external ? LQ_OK : ws->reserve_stream(std::max(bound, size_t(64) << 20), size_t(1) << 20);
  if (rc) return rc;
  rc = lq::reserve_prefill_scratch(ws);
  if (rc) return rc;
  rc = lq::noalloc_init_current_device();
  if (rc) return rc;
  return hipDeviceSynchronize() == hipSuccess ? LQ_OK : lq::fail(LQ_ERR_DEVICE, "lq_init: device synchronize failed");
}

}  // extern "C"
