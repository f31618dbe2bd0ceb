// Host-side state shared by the C-ABI translation units (api.cpp, block_pool.cpp):
// the context, its per-stream device workspaces, the device KV pool, and small
// helpers.  Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "llh_internal.h"
#include "llm_hip.h"

namespace llh {

constexpr size_t kAlign = 256;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Process-wide BlockId source: 1, 2, 3, ... (0 is BlockId::INVALID,
// crates/llm-kv-cache/src/block_id.rs:11-41).
uint64_t next_block_id();

// Device scratch of one stream: split partials, merge descriptors and the
// fused projection's staging, plus the stream's own device error word (the
// sticky flags the kernels of this stream's calls raise).  A call holds `mu`
// from planning through its last launch, so two threads on one stream never
// interleave their use of the scratch, and a growth (which frees the old
// buffer) never happens under another call.  `err` is allocated with the slot
// and lives as long as it: calls that need no scratch (writes, appends,
// gathers) take it without the lock.
struct StreamWorkspace {
  hipStream_t stream = nullptr;
  void *ptr = nullptr;
  size_t bytes = 0;
  int32_t *err = nullptr;
  std::mutex mu;
};

}  // namespace llh

struct llh_ctx {
  int device = 0;
  int cus = 256;  // compute units of the device (sizes the persistent decode grid)
  int32_t *d_err = nullptr;
  std::atomic<uint64_t> decode_calls{0}, prefill_calls{0}, append_calls{0}, not_handled{0}, device_errors{0},
      shape_errors{0}, stream_decode_calls{0}, trait_tuned_calls{0}, generic_prefill_calls{0}, fused_append_calls{0},
      d256_decode_calls{0}, generic_decode_calls{0};
  std::atomic<int32_t> options[LLH_OPT_COUNT] = {};

  // per-stream workspaces; ws_mu guards the list, ws_min_bytes and retired_flags
  std::mutex ws_mu;
  std::vector<std::shared_ptr<llh::StreamWorkspace>> workspaces;
  size_t ws_min_bytes = 0;
  int32_t retired_flags = 0;  // flags the error words of released slots held

  std::mutex err_mu;
  std::string last_error;

  // kernel timing (measurement only)
  std::atomic<int> timing{0};
  std::mutex timing_mu;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[2];
  std::vector<hipEvent_t> event_pool;
  double timed_ms[2] = {0.0, 0.0};
  int64_t timed_n[2] = {0, 0};

  int32_t opt(int o) const { return options[o].load(std::memory_order_relaxed); }

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
  // records the start event on stream s; returns the pair (or nulls when timing is off)
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

  // The workspace slot of stream s, created (with its zeroed error word) on
  // first use; nullptr when the error word cannot be allocated.
  std::shared_ptr<llh::StreamWorkspace> slot(hipStream_t s) {
    std::lock_guard<std::mutex> g(ws_mu);
    for (auto &w : workspaces)
      if (w->stream == s) return w;
    auto w = std::make_shared<llh::StreamWorkspace>();
    w->stream = s;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = hipMalloc(&w->err, sizeof(int32_t));
    // zeroed on the slot's own stream, so it lands before the stream's first kernel
    if (e == hipSuccess) e = hipMemsetAsync(w->err, 0, sizeof(int32_t), s);
    if (e != hipSuccess) {
      if (w->err) (void)hipFree(w->err);
      return nullptr;
    }
    workspaces.push_back(w);
    return w;
  }
  // The error word the kernels of a call on stream s raise their flags in: the
  // stream's own, or the context's when it cannot be had -- also while s is
  // being captured into a graph and has no slot yet (creating one allocates).
  int32_t *err_word(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
      std::lock_guard<std::mutex> g(ws_mu);
      for (auto &w : workspaces)
        if (w->stream == s) return w->err;
      return d_err;
    }
    auto w = slot(s);
    return w ? w->err : d_err;
  }
  size_t min_ws() {
    std::lock_guard<std::mutex> g(ws_mu);
    return ws_min_bytes;
  }
  // Grows a locked slot to at least `bytes` (zeroed on every allocation).  The
  // old buffer is freed once the slot's stream has drained, so no kernel still
  // reads it.
  int grow_locked(llh::StreamWorkspace &w, size_t bytes) {
    bytes = std::max(bytes, min_ws());
    if (w.ptr && bytes <= w.bytes) return LLH_OK;
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    if (w.ptr) {
      e = hipStreamSynchronize(w.stream);
      if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize(workspace)");
      (void)hipFree(w.ptr);
      w.ptr = nullptr;
      w.bytes = 0;
    }
    const size_t nb = llh::align_up(std::max(bytes, llh::kAlign));
    e = hipMalloc(&w.ptr, nb);
    if (e != hipSuccess) {
      w.ptr = nullptr;
      return hip_fail(e, "hipMalloc(workspace)");
    }
    // zeroed on the slot's own stream: a null-stream memset is asynchronous to the
    // host and unordered with non-blocking streams, so it could land after this
    // stream's next kernel
    e = hipMemsetAsync(w.ptr, 0, nb, w.stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemsetAsync(workspace)");
    w.bytes = nb;
    return LLH_OK;
  }
};

// A batched call's hold on its stream's workspace: locks the slot for the
// lifetime of the lease (through the call's last launch).
struct WsLease {
  std::shared_ptr<llh::StreamWorkspace> w;
  std::unique_lock<std::mutex> lock;
  int acquire(llh_ctx *ctx, hipStream_t s, size_t bytes) {
    w = ctx->slot(s);
    if (!w) return ctx->fail(LLH_ERR_DEVICE, "stream error word allocation failed");
    lock = std::unique_lock<std::mutex>(w->mu);
    return ctx->grow_locked(*w, bytes);
  }
  int32_t *err() const { return w->err; }
  char *base() const { return static_cast<char *>(w->ptr); }
};

namespace llh {

// A decode step planned on the host: the kernel choice and the byte layout of
// its workspace (offsets from the workspace base, `bytes` in all).  Shared by
// llh_paged_decode (per-stream workspace) and llh_paged_decode_noalloc (the
// library's static scratch).
struct DecodePlan {
  bool empty = false;  // nothing to launch (no sequences)
  bool fast = false;   // tuned kernels (else the reference-order kernel)
  bool d256 = false;   // tuned: the head_dim-256 (G = 8, bf16 / fp16) kernels (split-K, or stream when stream_wgs > 0)
  int group = 0;
  int split_blocks = 0, max_splits = 0, stream_wgs = 0;
  size_t ml_off = 0, o_off = 0, desc_off = 0;  // tuned: partial (max, sum), partial outputs, segment descriptors
  int score_stride = 0;
  size_t scores_off = 0;  // reference order: score rows
  size_t bytes = 0;
};
// max_bytes: the most workspace the caller can give; a layout choice that would
// need more falls back to one that fits (llh_paged_decode_noalloc's scratch)
int plan_decode(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_q,
                const void *d_out, float score_scale, DecodePlan *plan, size_t max_bytes = SIZE_MAX);
// err: the device error word the kernels raise flags in; timed = false leaves out
// the kernel-timing events (no event is created or recorded); k_new / v_new
// (tuned kernels): fused append of each sequence's new token
int launch_planned_decode(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const DecodePlan &plan,
                          const void *d_q, void *d_out, float score_scale, hipStream_t s, char *ws, int32_t *err,
                          bool timed = true, const uint16_t *k_new = nullptr, const uint16_t *v_new = nullptr);
// Resolves this device's address of the no-allocation scratch (device current).
int noalloc_init(int device);

}  // namespace llh

struct llh_kv_pool {
  llh_ctx *ctx = nullptr;
  llh::PoolView view{};
  void *k = nullptr, *v = nullptr, *ks = nullptr, *vs = nullptr;
  size_t k_bytes = 0, s_bytes = 0;
};

inline size_t elem_bytes(int32_t format) { return format == LLH_KV_BF16 || format == LLH_KV_F16 ? 2 : 1; }

// int8 and fp8 pools keep the K and V scales in one allocation as (K, V) pairs
// (int8_scale_index, fp8_scale_index): the V scale pointer is inside the K
// scales' allocation, one element further.
inline bool scales_interleaved(int32_t format) { return format == LLH_KV_INT8 || format == LLH_KV_FP8_E4M3; }
inline size_t v_scale_offset_bytes(int32_t format) {
  return format == LLH_KV_INT8 ? llh::kInt8VScaleOffsetBytes : llh::kFp8VScaleOffsetBytes;
}

inline size_t scale_bytes_per_block(int32_t format, int32_t kv_heads, int32_t block_tokens) {
  if (format == LLH_KV_INT8) return (size_t)kv_heads * block_tokens * 2;
  if (format == LLH_KV_INT8_ROW) return (size_t)block_tokens * 4;  // f32 per token row, shared by the heads
  if (format == LLH_KV_FP8_E4M3) return (size_t)kv_heads * 4;
  return 0;
}
