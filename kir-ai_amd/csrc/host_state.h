// Host-side state shared by the C-ABI translation units (api.cpp, block_pool.cpp):
// the context, the device KV pool, and small helpers.  Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "llh_internal.h"
#include "llm_hip.h"

namespace llh {

constexpr size_t kCounterSlots = 65536;  // (sequence, kv head) arrival counters
constexpr size_t kCounterBytes = kCounterSlots * sizeof(int32_t);
constexpr size_t kAlign = 256;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Process-wide BlockId source: 1, 2, 3, ... (0 is BlockId::INVALID,
// crates/llm-kv-cache/src/block_id.rs:11-41).
uint64_t next_block_id();

}  // namespace llh

struct llh_ctx {
  int device = 0;
  int cus = 256;  // compute units of the device (sizes the persistent decode grid)
  std::mutex mu;
  std::string last_error;
  void *ws = nullptr;
  size_t ws_bytes = 0;
  int32_t *d_err = nullptr;
  std::atomic<uint64_t> decode_calls{0}, prefill_calls{0}, append_calls{0}, not_handled{0}, device_errors{0},
      shape_errors{0}, stream_decode_calls{0};
  // kernel timing (measurement only)
  std::atomic<int> timing{0};
  std::mutex timing_mu;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[2];
  std::vector<hipEvent_t> event_pool;
  double timed_ms[2] = {0.0, 0.0};
  int64_t timed_n[2] = {0, 0};

  hipEvent_t take_event() {
    if (!event_pool.empty()) {
      hipEvent_t e = event_pool.back();
      event_pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
  // records the start event of `kind` on stream s; returns the pair index or -1
  std::pair<hipEvent_t, hipEvent_t> timing_begin(hipStream_t s) {
    if (!timing.load()) return {nullptr, nullptr};
    std::lock_guard<std::mutex> g(timing_mu);
    hipEvent_t a = take_event(), b = take_event();
    if (!a || !b || hipEventRecord(a, s) != hipSuccess) return {nullptr, nullptr};
    return {a, b};
  }
  void timing_end(int kind, std::pair<hipEvent_t, hipEvent_t> ev, hipStream_t s) {
    if (!ev.first) return;
    std::lock_guard<std::mutex> g(timing_mu);
    if (hipEventRecord(ev.second, s) == hipSuccess) pending[kind].push_back(ev);
  }

  int fail(int status, const std::string &msg) {
    {
      std::lock_guard<std::mutex> g(err_mu);
      last_error = msg;
    }
    if (status == LLH_ERR_DEVICE) device_errors++;
    if (status == LLH_ERR_INVALID_SHAPE) shape_errors++;
    return status;
  }
  int hip_fail(hipError_t e, const char *what) {
    return fail(LLH_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
  }
  // Ensures the workspace holds `bytes`; the counter region is zeroed on growth.
  int ensure_ws(size_t bytes) {
    std::lock_guard<std::mutex> g(mu);
    if (bytes <= ws_bytes) return LLH_OK;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    if (ws) {
      e = hipDeviceSynchronize();
      if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
      (void)hipFree(ws);
      ws = nullptr;
      ws_bytes = 0;
    }
    size_t nb = llh::align_up(std::max(bytes, llh::kCounterBytes + llh::kAlign));
    e = hipMalloc(&ws, nb);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(workspace)");
    e = hipMemset(ws, 0, nb);
    if (e != hipSuccess) return hip_fail(e, "hipMemset(workspace)");
    ws_bytes = nb;
    return LLH_OK;
  }
  std::mutex err_mu;
};

struct llh_kv_pool {
  llh_ctx *ctx = nullptr;
  llh::PoolView view{};
  void *k = nullptr, *v = nullptr, *ks = nullptr, *vs = nullptr;
  size_t k_bytes = 0, s_bytes = 0;
};

inline size_t elem_bytes(int32_t format) { return format == LLH_KV_BF16 ? 2 : 1; }

inline size_t scale_bytes_per_block(int32_t format, int32_t kv_heads, int32_t block_tokens) {
  if (format == LLH_KV_INT8) return (size_t)kv_heads * block_tokens * 2;
  if (format == LLH_KV_FP8_E4M3) return (size_t)kv_heads * 4;
  return 0;
}

