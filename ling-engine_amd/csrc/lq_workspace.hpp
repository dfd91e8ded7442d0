// Per-device workspace of the skinny GEMMs: split-K partial sums, per-tile-group arrival counters (kept
// zero between launches: the last workgroup of a group resets its counter), the one-launch FFN's counters and
// the prefill GEMM's split-tile partials.
// Grow-only; allocated on first use or by lq_init().
#pragma once

#include <cstddef>
#include <cstdint>

namespace lq {

struct Workspace {
  float* partials = nullptr;
  size_t partial_bytes = 0;
  int* counters = nullptr;
  size_t counter_count = 0;
  int* sync = nullptr;
  bool external = false;  // partials, counters and sync live in a caller-owned buffer (lq_set_workspace)
  // sync[64]: the one-launch FFN's phase-A arrivals, exits, deadline flag, ready flag at [32] (zeroed once, self-resetting)
  // prefill tail split: FP32 partial tiles and per-tile arrival counters (zeroed once, self-resetting)
  float* pf_partials = nullptr;
  size_t pf_partial_bytes = 0;
  int* pf_counters = nullptr;
  size_t pf_counter_count = 0;
  // Ensure capacity; returns LQ_OK or LQ_ERR_DEVICE (message set).
  int reserve_stream(size_t partial_bytes_needed, size_t counters_needed);
  int reserve_prefill(size_t partial_bytes_needed, size_t counters_needed);
  // Use [buf, buf + bytes) for partials, counters and sync (null: back to the library's own); see lq_set_workspace.
  int set_external(void* buf, size_t bytes);
};

// Bytes of split-K partial sums a skinny launch with up to `rows` activation rows can need on a device with `cus`
// CUs: two slots per workgroup of at most 4 tiles x G groups x 4 floats x 256 threads, and up to 4 x cus
// workgroups (a multi launch splits each of its up to 4 matrices over its own workgroups; the one-launch FFN's
// two phases at 2 tiles each take less).
inline size_t stream_partial_bound(size_t cus, int rows) {
  const size_t G = static_cast<size_t>((rows + 15) / 16);
  return 2 * 4 * cus * 4 * G * 4 * 256 * sizeof(float);
}

// The calling thread's current device's workspace (created on first call), or null (error set).
Workspace* workspace_for_current_device();
// Reserves the prefill's tail-split scratch at its bound (one FP32 tile per CU, one counter per CU), once.
int reserve_prefill_scratch(Workspace* ws);
// Looks up the no-allocation entry point's scratch on the current device and clears its counters (synchronously).
int noalloc_init_current_device();

}  // namespace lq
