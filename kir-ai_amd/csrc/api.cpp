// Host side of libllm_hip: the C ABI declared in include/llm_hip.h.
//
// Batched entry points validate shapes, size the split-K grid, and launch the
// kernels asynchronously on the caller's stream.  The trait-mirror entry
// points re-state kir-ai's LayerKvCache ring (crates/llm-kv-cache/src/layer.rs)
// over device-resident 16-token blocks and answer the NativeMatvecBackend
// attention hooks (crates/llm-backend/src/core/native_matvec.rs:619-668)
// synchronously, as the Metal backend does after awaiting its command buffer.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "host_state.h"

using namespace llh;

namespace {

std::atomic<uint64_t> g_next_block_id{1};
std::atomic<uint64_t> g_next_cache_id{1};

}  // namespace

uint64_t llh::next_block_id() { return g_next_block_id.fetch_add(1); }

namespace {

int env_int(const char *name, int dflt) {
  const char *v = std::getenv(name);
  if (!v || !*v) return dflt;
  return std::atoi(v);
}

// Initial option values, read once when a context is created.
void read_env_options(llh_ctx *ctx) {
  const char *k = std::getenv("LLH_DECODE_KERNEL");
  int kernel = 0;
  if (k && std::strcmp(k, "split") == 0) kernel = 1;
  if (k && std::strcmp(k, "stream") == 0) kernel = 2;
  ctx->options[LLH_OPT_DECODE_KERNEL] = kernel;
  ctx->options[LLH_OPT_DECODE_SPLIT_BLOCKS] = env_int("LLH_DECODE_SPLIT_BLOCKS", 0);
  ctx->options[LLH_OPT_DECODE_STREAM_WGS] = env_int("LLH_DECODE_STREAM_WGS", 0);
  ctx->options[LLH_OPT_FORCE_GENERIC] = env_int("LLH_FORCE_GENERIC", 0);
  ctx->options[LLH_OPT_PREFILL_HEADS_PER_WG] = env_int("LLH_PREFILL_HEADS_PER_WG", 0);
  ctx->options[LLH_OPT_TRAIT_REFERENCE_ORDER] = env_int("LLH_TRAIT_REFERENCE_ORDER", 0);
}

// Split-K sizing for the tuned decode kernel.  `est_blocks` bounds the blocks
// any one sequence attends (it sizes the grid and the partial buffer).  The
// split size is a power of two in [4, 256], measured on MI355X:
//  * bf16 pools are memory-bound: 8 blocks (two per wavefront, so each
//    wavefront has a block in flight behind the one it computes) beat larger
//    splits on ragged and on long contexts (C2 52 us at 8 against 59-65 at
//    16-64, C4 decode 15.9 us against 18.6 at 4); steps too small to give 512
//    workgroups that way use 4;
//  * int8 / fp8 pools are bound by their per-block arithmetic: the split that
//    brings the workgroup count closest to 2048 (C5: 128 blocks, 278 us
//    against 292 at 64 and 290 at 256).
// The total work comes from the caller's hint when given, else from the
// max_seq_len bound.
constexpr int kMaxDecodeSplits = 1024;  // partials one merge workgroup combines
constexpr int kD256MaxSplits = 64;      // partials the head_dim-256 merge combines

struct SplitPlan {
  int split_blocks;
  int max_splits;
  int est_blocks;
};

SplitPlan plan_splits(const llh_ctx *ctx, int num_seqs, int kv_heads, int max_seq_len, int window,
                      int total_tokens_hint, int format) {
  int span = max_seq_len;
  if (window > 0) span = std::min(span, window);
  const int est_blocks = (span + kFastBlockTokens - 1) / kFastBlockTokens + 1;
  int split = ctx->opt(LLH_OPT_DECODE_SPLIT_BLOCKS);
  if (split <= 0) {
    long long blocks = (long long)num_seqs * est_blocks;
    if (total_tokens_hint > 0) blocks = (long long)total_tokens_hint / kFastBlockTokens + num_seqs;
    auto wgs = [&](int s) { return (double)kv_heads * (double)(blocks + (long long)num_seqs * (s / 2)) / s; };
    if (format == LLH_KV_BF16 || format == LLH_KV_F16) {
      split = wgs(8) >= 512.0 ? 8 : 4;
    } else {
      const double target = 2048.0;
      double best = 1e30;
      split = 4;
      for (int s = 4; s <= 256; s *= 2) {
        const double w = wgs(s);
        const double cost = w > target ? w / target : target / w;
        if (cost < best) {
          best = cost;
          split = s;
        }
      }
    }
  }
  split = std::min(std::max(split, 4), 256);
  while ((est_blocks + split - 1) / split > kMaxDecodeSplits && split < 256) split *= 2;
  SplitPlan p;
  p.split_blocks = split;
  p.est_blocks = est_blocks;
  p.max_splits = (est_blocks + split - 1) / split;
  return p;
}

// Persistent stream decode: two workgroups of four wavefronts per compute unit,
// all resident at once, the best grid measured on MI355X for C2 (one and three
// per CU run 2-8% slower) and for C5 int8 / fp8 (three and four per CU, which
// run in rounds, 2-4% slower).  It is chosen when the step has at least
// kStreamMinUnitsPerWave units (block x kv head) per wavefront (and fewer than
// 2^31 units); smaller steps (C1, C4 decode) use split-K.
// LLH_OPT_DECODE_KERNEL overrides the choice, LLH_OPT_DECODE_STREAM_WGS the grid.
constexpr int kStreamWgsPerCu = 2;
constexpr int kStreamMaxWgs = 1024;
constexpr int kStreamMinUnitsPerWave = 8;

int stream_grid(const llh_ctx *ctx) {
  const int wgs = ctx->opt(LLH_OPT_DECODE_STREAM_WGS);
  return std::min(kStreamMaxWgs, std::max(1, wgs > 0 ? wgs : kStreamWgsPerCu * ctx->cus));
}

// The head_dim-256 kernels: the persistent stream grid when the step gives every
// wavefront at least kD256StreamMinUnitsPerWave units (block x kv head), else 0
// (split-K).  One workgroup per compute unit, measured on MI355X for the Qwen3.6
// step (32 x U[256, 4096], Hq16 / Hkv2): 256 workgroups 32.8 us, 192 33.8, 320
// (some CUs running two) 42.3, 512 37.4, split-K 38.3.  Fewer, longer ranges
// leave fewer partials (8 KiB per wavefront) for the merge.
// LLH_OPT_DECODE_KERNEL forces either, LLH_OPT_DECODE_STREAM_WGS sets the grid.
constexpr int kD256StreamMinUnitsPerWave = 2;

int plan_stream_d256(const llh_ctx *ctx, int num_seqs, int kv_heads, int est_blocks, int total_tokens_hint) {
  const int force = ctx->opt(LLH_OPT_DECODE_KERNEL);
  if (force == 1) return 0;
  const int opt_wgs = ctx->opt(LLH_OPT_DECODE_STREAM_WGS);
  const int wgs = std::min(kStreamMaxWgs, std::max(1, opt_wgs > 0 ? opt_wgs : ctx->cus));
  const long long max_units = (long long)kv_heads * est_blocks * num_seqs;
  if (max_units >= (1LL << 31)) return 0;
  if (force == 2) return wgs;
  const long long units = total_tokens_hint > 0
                              ? (long long)kv_heads * ((long long)total_tokens_hint / kFastBlockTokens + num_seqs)
                              : max_units;
  return units >= (long long)kD256StreamMinUnitsPerWave * 4 * wgs ? wgs : 0;
}

// Returns the stream grid (workgroups) for this step, or 0 for split-K.
int plan_stream(const llh_ctx *ctx, int format, int num_seqs, int kv_heads, int est_blocks, int total_tokens_hint) {
  const int force = ctx->opt(LLH_OPT_DECODE_KERNEL);
  const bool want_split = force == 1;
  const bool want_stream = force == 2;
  if (want_split) return 0;
  const int wgs = stream_grid(ctx);
  const long long waves = 4LL * wgs;
  const long long max_units = (long long)kv_heads * est_blocks * num_seqs;
  if (max_units >= (1LL << 31)) return 0;
  if (want_stream) return wgs;
  const long long units = total_tokens_hint > 0
                              ? (long long)kv_heads * ((long long)total_tokens_hint / kFastBlockTokens + num_seqs)
                              : max_units;
  return units >= kStreamMinUnitsPerWave * waves ? wgs : 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
extern "C" {

int llh_ctx_create(int device, llh_ctx **out) {
  if (!out) return LLH_ERR_NULL;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return LLH_ERR_DEVICE;
  auto *ctx = new llh_ctx();
  ctx->device = device;
  // (hipMemset is asynchronous to the host: wait for it before any stream can use the flags)
  if (hipSetDevice(device) != hipSuccess || hipMalloc(&ctx->d_err, sizeof(int32_t)) != hipSuccess ||
      hipMemset(ctx->d_err, 0, sizeof(int32_t)) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
      hipDeviceGetAttribute(&ctx->cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
    delete ctx;
    return LLH_ERR_DEVICE;
  }
  ctx->cus = std::max(1, ctx->cus);
  if (noalloc_init(device) != LLH_OK) {  // this device's copy of the no-allocation scratch
    (void)hipFree(ctx->d_err);
    delete ctx;
    return LLH_ERR_DEVICE;
  }
  read_env_options(ctx);
  *out = ctx;
  return LLH_OK;
}

int llh_ctx_destroy(llh_ctx *ctx) {
  if (!ctx) return LLH_ERR_NULL;
  (void)hipSetDevice(ctx->device);
  (void)hipDeviceSynchronize();
  for (auto &list : ctx->pending)
    for (auto &ev : list) {
      (void)hipEventDestroy(ev.first);
      (void)hipEventDestroy(ev.second);
    }
  for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
  for (auto &w : ctx->workspaces) {
    if (w->ptr) (void)hipFree(w->ptr);
    if (w->err) (void)hipFree(w->err);
  }
  if (ctx->d_err) (void)hipFree(ctx->d_err);
  delete ctx;
  return LLH_OK;
}

const char *llh_ctx_last_error(const llh_ctx *ctx) {
  if (!ctx) return "null context";
  // a copy per thread: another thread's failure may replace ctx->last_error at any time
  static thread_local std::string copy;
  auto *c = const_cast<llh_ctx *>(ctx);
  std::lock_guard<std::mutex> g(c->err_mu);
  copy = c->last_error;
  return copy.c_str();
}

int llh_ctx_reserve_workspace(llh_ctx *ctx, size_t bytes) {
  if (!ctx) return LLH_ERR_NULL;
  std::vector<std::shared_ptr<StreamWorkspace>> slots;
  {
    std::lock_guard<std::mutex> g(ctx->ws_mu);
    ctx->ws_min_bytes = std::max(ctx->ws_min_bytes, bytes);
    slots = ctx->workspaces;
  }
  for (auto &w : slots) {
    std::lock_guard<std::mutex> g(w->mu);
    const int st = ctx->grow_locked(*w, 0);
    if (st != LLH_OK) return st;
  }
  return LLH_OK;
}

int llh_ctx_reserve_stream_workspace(llh_ctx *ctx, void *stream, size_t bytes) {
  if (!ctx) return LLH_ERR_NULL;
  WsLease lease;
  return lease.acquire(ctx, static_cast<hipStream_t>(stream), bytes);
}

}  // extern "C"

// Drops the workspace slot of `stream` (scratch and error word).  A stream the
// caller may already have destroyed is waited for with the whole device; a live
// one (a layer cache's own) with its own synchronisation.  Flags still set in
// the slot's word are folded into the context's word, so llh_ctx_device_errors
// keeps seeing them.
static int release_slot(llh_ctx *ctx, hipStream_t stream, bool stream_alive) {
  std::shared_ptr<StreamWorkspace> w;
  {
    std::lock_guard<std::mutex> g(ctx->ws_mu);
    auto it = std::find_if(ctx->workspaces.begin(), ctx->workspaces.end(),
                           [&](const std::shared_ptr<StreamWorkspace> &x) { return x->stream == stream; });
    if (it == ctx->workspaces.end()) return LLH_OK;
    w = *it;
    ctx->workspaces.erase(it);
  }
  std::lock_guard<std::mutex> g(w->mu);  // waits for a call still holding it
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = stream_alive ? hipStreamSynchronize(stream) : hipDeviceSynchronize();
  int32_t flags = 0;
  if (e == hipSuccess && w->err) e = hipMemcpy(&flags, w->err, sizeof(int32_t), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return ctx->hip_fail(e, "release stream workspace");
  if (flags) {
    std::lock_guard<std::mutex> g2(ctx->ws_mu);
    ctx->retired_flags |= flags;
  }
  if (w->ptr) (void)hipFree(w->ptr);
  if (w->err) (void)hipFree(w->err);
  w->ptr = nullptr;
  w->err = nullptr;
  w->bytes = 0;
  return LLH_OK;
}

extern "C" {

int llh_ctx_release_stream(llh_ctx *ctx, void *stream) {
  if (!ctx) return LLH_ERR_NULL;
  // the stream may already be gone: the whole device is waited for
  return release_slot(ctx, static_cast<hipStream_t>(stream), false);
}

int llh_ctx_set_option(llh_ctx *ctx, int32_t option, int32_t value) {
  if (!ctx) return LLH_ERR_NULL;
  if (option < 0 || option >= LLH_OPT_COUNT) return ctx->fail(LLH_ERR_INVALID_SHAPE, "unknown option");
  ctx->options[option].store(value);
  return LLH_OK;
}

int llh_ctx_get_option(const llh_ctx *ctx, int32_t option, int32_t *value) {
  if (!ctx || !value) return LLH_ERR_NULL;
  if (option < 0 || option >= LLH_OPT_COUNT) return LLH_ERR_INVALID_SHAPE;
  *value = ctx->opt(option);
  return LLH_OK;
}

size_t llh_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len) {
  if (num_seqs <= 0 || num_q_heads <= 0 || max_seq_len < 0) return 0;
  // the smallest split size gives the largest partial count
  const int est_blocks = (max_seq_len + kFastBlockTokens - 1) / kFastBlockTokens + 1;
  const size_t max_splits = (size_t)(est_blocks + 3) / 4;
  const size_t rows = (size_t)num_seqs * num_q_heads * max_splits;
  const size_t generic = (size_t)num_seqs * num_q_heads * std::max(1, max_seq_len) * sizeof(float);
  // stream kernel: two partial slots per wavefront of the largest grid, G <= 8 rows each
  const size_t srows = (size_t)2 * 4 * kStreamMaxWgs * std::min(num_q_heads, 8);
  const size_t stream = align_up(srows * sizeof(float2)) + align_up(srows * kFastHeadDim * sizeof(float)) +
                        align_up((size_t)num_seqs * num_q_heads * 2 * sizeof(int32_t));
  // head_dim-256 split-K kernel: at most kD256MaxSplits partial rows per (sequence, head), 256 floats each
  const size_t rows256 = (size_t)num_seqs * num_q_heads * std::min<size_t>(max_splits, kD256MaxSplits);
  const size_t d256 = align_up(rows256 * sizeof(float2)) + rows256 * kD256HeadDim * sizeof(float);
  // head_dim-256 stream kernel (groups of 8 query heads): two slots per wavefront, 8 rows of 256 floats each
  const size_t srows256 = num_q_heads >= kD256Group ? (size_t)2 * 4 * kStreamMaxWgs * kD256Group : 0;
  const size_t stream256 = srows256 ? align_up(srows256 * sizeof(float2)) +
                                          align_up(srows256 * kD256HeadDim * sizeof(float)) +
                                          align_up((size_t)num_seqs * num_q_heads * 2 * sizeof(int32_t))
                                    : 0;
  return std::max({align_up(rows * sizeof(float2)) + rows * kFastHeadDim * sizeof(float), generic, stream, d256,
                   stream256});
}

int llh_ctx_metrics(const llh_ctx *ctx, llh_metrics *out) {
  if (!ctx || !out) return LLH_ERR_NULL;
  out->decode_calls = ctx->decode_calls.load();
  out->prefill_calls = ctx->prefill_calls.load();
  out->append_calls = ctx->append_calls.load();
  out->not_handled = ctx->not_handled.load();
  out->device_errors = ctx->device_errors.load();
  out->shape_errors = ctx->shape_errors.load();
  out->stream_decode_calls = ctx->stream_decode_calls.load();
  out->trait_tuned_calls = ctx->trait_tuned_calls.load();
  out->generic_prefill_calls = ctx->generic_prefill_calls.load();
  out->fused_append_calls = ctx->fused_append_calls.load();
  out->d256_decode_calls = ctx->d256_decode_calls.load();
  out->generic_decode_calls = ctx->generic_decode_calls.load();
  std::lock_guard<std::mutex> g(const_cast<llh_ctx *>(ctx)->ws_mu);
  out->stream_slots = ctx->workspaces.size();
  out->workspace_bytes = 0;
  for (auto &w : ctx->workspaces) out->workspace_bytes += w->bytes;
  return LLH_OK;
}

int llh_ctx_device_errors(llh_ctx *ctx, int32_t *flags, int32_t reset) {
  if (!ctx || !flags) return LLH_ERR_NULL;
  *flags = 0;
  std::lock_guard<std::mutex> g(ctx->ws_mu);  // no slot comes or goes meanwhile
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  std::vector<int32_t *> words{ctx->d_err};
  for (auto &w : ctx->workspaces)
    if (w->err) words.push_back(w->err);
  for (int32_t *word : words) {
    int32_t f = 0;
    if (e == hipSuccess) e = hipMemcpy(&f, word, sizeof(int32_t), hipMemcpyDeviceToHost);
    if (e == hipSuccess && reset && f) e = hipMemset(word, 0, sizeof(int32_t));
    *flags |= f;
  }
  *flags |= ctx->retired_flags;
  if (reset) ctx->retired_flags = 0;
  if (e == hipSuccess && reset) e = hipDeviceSynchronize();  // the resets land before any later kernel
  if (e != hipSuccess) return ctx->hip_fail(e, "device error flags");
  return LLH_OK;
}

int llh_ctx_stream_device_errors(llh_ctx *ctx, void *stream, int32_t *flags, int32_t reset) {
  if (!ctx || !flags) return LLH_ERR_NULL;
  *flags = 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int32_t *word = nullptr;
  {
    std::lock_guard<std::mutex> g(ctx->ws_mu);
    for (auto &w : ctx->workspaces)
      if (w->stream == s) word = w->err;
  }
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e == hipSuccess && word) e = hipMemcpyAsync(flags, word, sizeof(int32_t), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess && word) e = hipStreamSynchronize(s);
  if (e == hipSuccess && word && reset && *flags) e = hipMemsetAsync(word, 0, sizeof(int32_t), s);
  if (e == hipSuccess && word && reset && *flags) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return ctx->hip_fail(e, "stream device error flags");
  return LLH_OK;
}

int llh_ctx_set_kernel_timing(llh_ctx *ctx, int32_t enable) {
  if (!ctx) return LLH_ERR_NULL;
  ctx->timing.store(enable ? 1 : 0);
  return LLH_OK;
}

int llh_ctx_kernel_time(llh_ctx *ctx, int32_t kind, double *total_ms, int64_t *count, int32_t reset) {
  if (!ctx || !total_ms || !count) return LLH_ERR_NULL;
  if (kind != 0 && kind != 1) return ctx->fail(LLH_ERR_INVALID_SHAPE, "timing kind must be 0 (decode) or 1 (prefill)");
  std::lock_guard<std::mutex> g(ctx->timing_mu);
  for (auto &ev : ctx->pending[kind]) {
    float ms = 0.0f;
    hipError_t e = hipEventSynchronize(ev.second);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.first, ev.second);
    if (e != hipSuccess) return ctx->hip_fail(e, "kernel timing");
    ctx->timed_ms[kind] += ms;
    ctx->timed_n[kind] += 1;
    ctx->event_pool.push_back(ev.first);
    ctx->event_pool.push_back(ev.second);
  }
  ctx->pending[kind].clear();
  *total_ms = ctx->timed_ms[kind];
  *count = ctx->timed_n[kind];
  if (reset) {
    ctx->timed_ms[kind] = 0.0;
    ctx->timed_n[kind] = 0;
  }
  return LLH_OK;
}

// ---------------------------------------------------------------------------
// pool
// ---------------------------------------------------------------------------

int llh_kv_pool_create(llh_ctx *ctx, int32_t format, int32_t block_tokens, int32_t kv_heads, int32_t head_dim,
                       int64_t n_blocks, llh_kv_pool **out) {
  if (!ctx || !out) return LLH_ERR_NULL;
  *out = nullptr;
  if (format < LLH_KV_BF16 || format > LLH_KV_F16)
    return ctx->fail(LLH_ERR_UNSUPPORTED, "unsupported KV format");
  if (block_tokens <= 0 || kv_heads <= 0 || head_dim <= 0 || n_blocks <= 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "kv pool sizes must be positive");
  if (elem_bytes(format) == 1 && (block_tokens % 4 != 0 || head_dim % 4 != 0))
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "quantised pools need block_tokens and head_dim divisible by 4");
  if (n_blocks > INT32_MAX) return ctx->fail(LLH_ERR_INVALID_SHAPE, "block indices are int32");
  auto *pool = new llh_kv_pool();
  pool->view.format = format;  // destroy() reads it on the error path below
  pool->ctx = ctx;
  pool->k_bytes = (size_t)n_blocks * kv_heads * block_tokens * head_dim * elem_bytes(format);
  pool->s_bytes = (size_t)n_blocks * scale_bytes_per_block(format, kv_heads, block_tokens);
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc(&pool->k, pool->k_bytes);
  if (e == hipSuccess) e = hipMalloc(&pool->v, pool->k_bytes);
  if (scales_interleaved(format)) {
    if (e == hipSuccess) e = hipMalloc(&pool->ks, 2 * pool->s_bytes);
    if (e == hipSuccess) e = hipMemset(pool->ks, 0, 2 * pool->s_bytes);
    if (e == hipSuccess) pool->vs = static_cast<char *>(pool->ks) + v_scale_offset_bytes(format);
  } else {
    if (e == hipSuccess && pool->s_bytes) e = hipMalloc(&pool->ks, pool->s_bytes);
    if (e == hipSuccess && pool->s_bytes) e = hipMalloc(&pool->vs, pool->s_bytes);
    if (e == hipSuccess && pool->s_bytes) e = hipMemset(pool->ks, 0, pool->s_bytes);
    if (e == hipSuccess && pool->s_bytes) e = hipMemset(pool->vs, 0, pool->s_bytes);
  }
  // null-stream memsets are asynchronous to the host and unordered with non-blocking
  // streams: the pool is ready for any stream only once they have completed
  if (e == hipSuccess && pool->s_bytes) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    llh_kv_pool_destroy(pool);
    return ctx->hip_fail(e, "hipMalloc(kv pool)");
  }
  pool->view = PoolView{format, block_tokens, kv_heads, head_dim, n_blocks, pool->k, pool->v, pool->ks, pool->vs};
  *out = pool;
  return LLH_OK;
}

int llh_kv_pool_destroy(llh_kv_pool *pool) {
  if (!pool) return LLH_ERR_NULL;
  if (pool->ctx) (void)hipSetDevice(pool->ctx->device);
  if (pool->k) (void)hipFree(pool->k);
  if (pool->v) (void)hipFree(pool->v);
  if (pool->ks) (void)hipFree(pool->ks);
  if (pool->vs && !scales_interleaved(pool->view.format)) (void)hipFree(pool->vs);
  delete pool;
  return LLH_OK;
}

int llh_kv_pool_get_info(const llh_kv_pool *pool, llh_kv_pool_info *out) {
  if (!pool || !out) return LLH_ERR_NULL;
  out->format = pool->view.format;
  out->block_tokens = pool->view.block_tokens;
  out->kv_heads = pool->view.kv_heads;
  out->head_dim = pool->view.head_dim;
  out->n_blocks = pool->view.n_blocks;
  out->d_k = pool->k;
  out->d_v = pool->v;
  out->d_k_scales = pool->ks;
  out->d_v_scales = pool->vs;
  out->k_bytes = pool->k_bytes;
  out->scale_bytes = pool->s_bytes;
  return LLH_OK;
}

int llh_kv_write_blocks(llh_ctx *ctx, llh_kv_pool *pool, const int32_t *d_blocks, const void *d_k, const void *d_v,
                        int32_t n, void *stream) {
  if (!ctx || !pool) return LLH_ERR_NULL;
  if (n < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "negative block count");
  if (n == 0) return LLH_OK;
  if (!d_blocks || !d_k || !d_v) return ctx->fail(LLH_ERR_NULL, "null device pointer");
  WriteBlocksArgs a{};
  a.pool = pool->view;
  a.k_dst = pool->k;
  a.v_dst = pool->v;
  a.ks_dst = pool->ks;
  a.vs_dst = pool->vs;
  a.blocks = d_blocks;
  a.k = static_cast<const uint16_t *>(d_k);
  a.v = static_cast<const uint16_t *>(d_v);
  a.n = n;
  a.err = ctx->err_word(static_cast<hipStream_t>(stream));
  hipError_t e = launch_write_blocks(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "write_blocks launch");
  return LLH_OK;
}

// d_slots null: row i is sequence i's new token, appended at position
// seq_lens[i] - 1 through block-table row i (the decode step's append).
static int kv_append(llh_ctx *ctx, llh_kv_pool *pool, const int64_t *d_slots, const void *d_k, const void *d_v,
                     int32_t n, int32_t src_f32, void *stream, const int32_t *d_seq_lens = nullptr,
                     const int32_t *d_tables = nullptr, int32_t max_blocks = 0) {
  if (!ctx || !pool) return LLH_ERR_NULL;
  if (n < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "negative token count");
  if (n == 0) return LLH_OK;
  if ((!d_slots && (!d_seq_lens || !d_tables)) || !d_k || !d_v)
    return ctx->fail(LLH_ERR_NULL, "null device pointer");
  AppendArgs a{};
  a.pool = pool->view;
  a.k_dst = pool->k;
  a.v_dst = pool->v;
  a.ks_dst = pool->ks;
  a.vs_dst = pool->vs;
  a.slots = d_slots;
  a.k = d_k;
  a.v = d_v;
  a.n = n;
  a.src_f32 = src_f32;
  a.err = ctx->err_word(static_cast<hipStream_t>(stream));
  a.seq_lens = d_seq_lens;
  a.tables = d_tables;
  a.max_blocks = max_blocks;
  ctx->append_calls++;
  hipError_t e = launch_append(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "append launch");
  return LLH_OK;
}

int llh_kv_append(llh_ctx *ctx, llh_kv_pool *pool, const int64_t *d_slots, const void *d_k, const void *d_v,
                  int32_t n, void *stream) {
  return kv_append(ctx, pool, d_slots, d_k, d_v, n, 0, stream);
}

int llh_kv_append_f32(llh_ctx *ctx, llh_kv_pool *pool, const int64_t *d_slots, const float *d_k, const float *d_v,
                      int32_t n, void *stream) {
  return kv_append(ctx, pool, d_slots, d_k, d_v, n, 1, stream);
}

int llh_kv_export_rows_f32(llh_ctx *ctx, const llh_kv_pool *pool, const int64_t *d_slots, int64_t n, float *d_k,
                           float *d_v, void *stream) {
  if (!ctx || !pool) return LLH_ERR_NULL;
  if (n < 0 || n > INT32_MAX) return ctx->fail(LLH_ERR_INVALID_SHAPE, "row count out of range");
  if (n == 0) return LLH_OK;
  if (!d_slots || !d_k || !d_v) return ctx->fail(LLH_ERR_NULL, "null device pointer");
  ExportArgs a{};
  a.pool = pool->view;
  a.slots = d_slots;
  a.k = d_k;
  a.v = d_v;
  a.n = (int32_t)n;
  a.err = ctx->err_word(static_cast<hipStream_t>(stream));
  hipError_t e = launch_export_rows(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "export launch");
  return LLH_OK;
}

// ---------------------------------------------------------------------------
// batched attention
// ---------------------------------------------------------------------------

static int check_desc_common(llh_ctx *ctx, const llh_kv_pool *pool, int32_t num_seqs, int32_t q_heads,
                             int32_t max_blocks, int32_t window) {
  if (num_seqs < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "num_seqs must be >= 0");
  if (q_heads <= 0 || q_heads % pool->view.kv_heads != 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "num_q_heads must be a positive multiple of kv_heads");
  if (max_blocks <= 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "max_blocks_per_seq must be positive");
  if (window < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "window must be >= 0");
  return LLH_OK;
}

}  // extern "C"

// The kernels read block-table rows modulo their length (a ring of blocks serves
// a sliding window), so two attended positions alias one slot when a sequence
// attends more tokens than its row holds.  Rejects a call whose bound allows it.
static int check_span(llh_ctx *ctx, const llh_kv_pool *pool, int32_t max_seq_len, int32_t window,
                      int32_t max_blocks) {
  const int64_t span = window > 0 ? std::min<int64_t>(window, max_seq_len) : max_seq_len;
  if (span > (int64_t)max_blocks * pool->view.block_tokens)
    return ctx->fail(LLH_ERR_INVALID_SHAPE,
                     "attended span exceeds the block-table row (max_blocks_per_seq * block_tokens)");
  return LLH_OK;
}

// Plans one decode step: validates the call, chooses the kernel and lays out
// its workspace (offsets from the workspace base; plan->bytes in all).
int llh::plan_decode(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_q,
                     const void *d_out, float score_scale, DecodePlan *plan, size_t max_bytes) {
  if (!ctx || !pool || !desc || !plan) return LLH_ERR_NULL;
  *plan = DecodePlan{};
  int st = check_desc_common(ctx, pool, desc->num_seqs, desc->num_q_heads, desc->max_blocks_per_seq, desc->window);
  if (st != LLH_OK) return st;
  if (desc->num_seqs == 0) {
    plan->empty = true;
    return LLH_OK;
  }
  if (desc->max_seq_len < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "max_seq_len must be >= 0");
  st = check_span(ctx, pool, desc->max_seq_len, desc->window, desc->max_blocks_per_seq);
  if (st != LLH_OK) return st;
  if (!d_q || !desc->d_seq_lens || !desc->d_block_tables)
    return ctx->fail(LLH_ERR_NULL, "null device pointer in decode call");
  if (!std::isfinite(score_scale)) return ctx->fail(LLH_ERR_NON_FINITE, "score scale must be finite");
  const PoolView &pv = pool->view;
  const int group = desc->num_q_heads / pv.kv_heads;
  // The fast kernels move q and output rows in 16-byte vectors; rows that are
  // not 16-byte aligned go through the element-wise generic kernel.
  const bool rows_aligned = (reinterpret_cast<uintptr_t>(d_q) & 15) == 0 &&
                            (reinterpret_cast<uintptr_t>(d_out) & 15) == 0;
  plan->group = group;
  plan->fast = pv.format != LLH_KV_INT8_ROW && pv.head_dim == kFastHeadDim && pv.block_tokens == kFastBlockTokens &&
               rows_aligned &&
               (group == 1 || group == 2 || group == 4 || group == 8) && !ctx->opt(LLH_OPT_FORCE_GENERIC);
  // head_dim 256 (Qwen3.5 / 3.6 full attention: Hq16 / Hkv2): bf16 or fp16 pools, G = 8
  plan->d256 = (pv.format == LLH_KV_BF16 || pv.format == LLH_KV_F16) && pv.head_dim == kD256HeadDim &&
               pv.block_tokens == kFastBlockTokens &&
               rows_aligned && group == kD256Group && !ctx->opt(LLH_OPT_FORCE_GENERIC);
  if (plan->d256) {
    plan->fast = true;
    SplitPlan sp = plan_splits(ctx, desc->num_seqs, pv.kv_heads, desc->max_seq_len, desc->window,
                               desc->total_tokens_hint, pv.format);
    // persistent stream: partials (max, sum) and outputs of two slots per wavefront, segment descriptors
    const int wgs = plan_stream_d256(ctx, desc->num_seqs, pv.kv_heads, sp.est_blocks, desc->total_tokens_hint);
    if (wgs > 0) {
      const size_t rows = (size_t)2 * 4 * wgs * kD256Group;
      const size_t o_off = align_up(rows * sizeof(float2));
      const size_t desc_off = align_up(o_off + rows * kD256HeadDim * sizeof(float));
      const size_t bytes = align_up(desc_off + (size_t)desc->num_seqs * pv.kv_heads * 2 * sizeof(int32_t));
      if (bytes <= max_bytes) {
        plan->stream_wgs = wgs;
        plan->ml_off = 0;
        plan->o_off = o_off;
        plan->desc_off = desc_off;
        plan->bytes = bytes;
        return LLH_OK;
      }
    }
    if (ctx->opt(LLH_OPT_DECODE_SPLIT_BLOCKS) <= 0) {
      // Long splits: each wavefront keeps one block in flight, so a workgroup's
      // start (q, first loads) and its merge are paid once per split.  The longest
      // split of at most 64 blocks that still gives >= 160 workgroups (measured on
      // MI355X for the Qwen3.6 step, 32 x U[256, 4096]: 64 blocks 38.2 us, 32 41.7,
      // 16 43.1, 8 41.0; 128 61.2).
      long long blocks = (long long)desc->num_seqs * sp.est_blocks;
      if (desc->total_tokens_hint > 0) blocks = (long long)desc->total_tokens_hint / kFastBlockTokens + desc->num_seqs;
      auto wgs = [&](int s) { return (double)pv.kv_heads * (double)(blocks + (long long)desc->num_seqs * (s / 2)) / s; };
      int split = 64;
      while (split > 4 && wgs(split) < 160.0) split /= 2;
      sp.split_blocks = split;
      sp.max_splits = (sp.est_blocks + split - 1) / split;
    }
    // the merge takes at most kD256MaxSplits partials: longer spans get longer splits
    while (sp.max_splits > kD256MaxSplits) {
      sp.split_blocks *= 2;
      sp.max_splits = (sp.est_blocks + sp.split_blocks - 1) / sp.split_blocks;
    }
    plan->split_blocks = sp.split_blocks;
    plan->max_splits = sp.max_splits;
    const size_t rows = (size_t)desc->num_seqs * desc->num_q_heads * sp.max_splits;
    plan->ml_off = 0;
    plan->o_off = align_up(rows * sizeof(float2));
    plan->bytes = align_up(plan->o_off + rows * kD256HeadDim * sizeof(float));
    return LLH_OK;
  }
  if (plan->fast) {
    const SplitPlan sp = plan_splits(ctx, desc->num_seqs, pv.kv_heads, desc->max_seq_len, desc->window,
                                     desc->total_tokens_hint, pv.format);
    plan->stream_wgs =
        plan_stream(ctx, pv.format, desc->num_seqs, pv.kv_heads, sp.est_blocks, desc->total_tokens_hint);
    if (!plan->stream_wgs && sp.max_splits > kMaxDecodeSplits)
      return ctx->fail(LLH_ERR_INVALID_SHAPE, "context too long for one decode call (over 4M attended tokens)");
    plan->split_blocks = sp.split_blocks;
    plan->max_splits = sp.max_splits;
    // partial rows: split-K [B][Hq][max_splits]; stream [2 * waves][G]
    const size_t rows = plan->stream_wgs ? (size_t)2 * 4 * plan->stream_wgs * group
                                         : (size_t)desc->num_seqs * desc->num_q_heads * sp.max_splits;
    plan->ml_off = 0;
    plan->o_off = plan->ml_off + align_up(rows * sizeof(float2));
    plan->desc_off = align_up(plan->o_off + rows * kFastHeadDim * sizeof(float));
    plan->bytes = align_up(plan->desc_off +
                           (plan->stream_wgs ? (size_t)desc->num_seqs * pv.kv_heads * 2 * sizeof(int32_t) : 0));
    return LLH_OK;
  }
  // any other shape: the reference-order kernel, with a score row per (sequence, head)
  const int span = desc->window > 0 ? std::min(desc->window, desc->max_seq_len) : desc->max_seq_len;
  plan->score_stride = std::max(1, span);
  plan->scores_off = 0;
  plan->bytes = align_up(plan->scores_off + (size_t)desc->num_seqs * desc->num_q_heads * plan->score_stride *
                                                 sizeof(float));
  return LLH_OK;
}

// Launches a planned decode step with its workspace at `ws` (plan.bytes long).
int llh::launch_planned_decode(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc,
                               const DecodePlan &plan, const void *d_q, void *d_out, float score_scale,
                               hipStream_t s, char *ws, int32_t *err, bool timed, const uint16_t *k_new,
                               const uint16_t *v_new) {
  const PoolView &pv = pool->view;
  ctx->decode_calls++;
  if (plan.fast) {
    DecodeArgs a{};
    a.pool = pv;
    a.q = static_cast<const uint16_t *>(d_q);
    a.out = static_cast<uint16_t *>(d_out);
    a.seq_lens = desc->d_seq_lens;
    a.tables = desc->d_block_tables;
    a.ws_o = reinterpret_cast<float *>(ws + plan.o_off);
    a.ws_ml = reinterpret_cast<float2 *>(ws + plan.ml_off);
    a.err = err;
    a.num_seqs = desc->num_seqs;
    a.q_heads = desc->num_q_heads;
    a.max_blocks = desc->max_blocks_per_seq;
    a.window = desc->window;
    a.split_blocks = plan.split_blocks;
    a.max_splits = plan.max_splits;
    a.stream_wgs = plan.stream_wgs;
    a.max_seq_len = desc->max_seq_len;
    a.seg_desc = plan.stream_wgs ? reinterpret_cast<int32_t *>(ws + plan.desc_off) : nullptr;
    if (plan.stream_wgs) ctx->stream_decode_calls++;
    if (plan.d256) ctx->d256_decode_calls++;
    a.scale_log2e = score_scale * 1.4426950408889634f;
    a.k_new = k_new;
    a.v_new = v_new;
    a.gate = static_cast<const uint16_t *>(desc->d_gate);
    struct TimingHook {
      llh_ctx *ctx;
      std::pair<hipEvent_t, hipEvent_t> ev;
    } th{ctx, {nullptr, nullptr}};
    const LaunchHook hook = [](void *u, int phase, hipStream_t st) {
      auto *t = static_cast<TimingHook *>(u);
      if (phase == 0)
        t->ev = t->ctx->timing_begin(st);
      else
        t->ctx->timing_end(0, t->ev, st);
    };
    hipError_t e = plan.d256 ? launch_decode_d256(a, desc->max_seq_len, s, timed ? &th : nullptr, timed ? hook : nullptr)
                             : launch_decode(a, plan.group, desc->max_seq_len, s, timed ? &th : nullptr,
                                             timed ? hook : nullptr);
    if (e != hipSuccess) return ctx->hip_fail(e, "decode launch");
    return LLH_OK;
  }
  GenericDecodeArgs g{};
  g.pool = pv;
  g.q = d_q;
  g.out = d_out;
  g.seq_lens = desc->d_seq_lens;
  g.starts = nullptr;
  g.tables = desc->d_block_tables;
  g.scores = reinterpret_cast<float *>(ws + plan.scores_off);
  g.err = err;
  g.num_seqs = desc->num_seqs;
  g.q_heads = desc->num_q_heads;
  g.max_blocks = desc->max_blocks_per_seq;
  g.window = desc->window;
  g.ring_tokens = 0;
  g.score_stride = plan.score_stride;
  g.scale = score_scale;
  g.gate = static_cast<const uint16_t *>(desc->d_gate);
  ctx->generic_decode_calls++;
  hipError_t e = launch_decode_generic(g, 0, 0, s);
  if (e != hipSuccess) return ctx->hip_fail(e, "generic decode launch");
  return LLH_OK;
}

// One decode step on the stream's workspace.  With d_out == nullptr the bf16
// output goes to a buffer of `extra_bytes` placed after the step's own regions
// (returned in *extra_ptr), so a following kernel on the stream can consume it
// without any allocation; the caller keeps `lease` through that launch.
static int paged_decode_impl(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_q,
                             void *d_out, float score_scale, void *stream, size_t extra_bytes, void **extra_ptr,
                             WsLease &lease) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  if (!d_out && !extra_ptr && desc->num_seqs > 0) return ctx->fail(LLH_ERR_NULL, "null device pointer in decode call");
  DecodePlan plan;
  int st = plan_decode(ctx, pool, desc, d_q, d_out, score_scale, &plan);
  if (st != LLH_OK || plan.empty) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  st = lease.acquire(ctx, s, plan.bytes + extra_bytes);
  if (st != LLH_OK) return st;
  char *ws = lease.base();
  if (extra_ptr) *extra_ptr = ws + plan.bytes;
  if (!d_out) d_out = ws + plan.bytes;
  return launch_planned_decode(ctx, pool, desc, plan, d_q, d_out, score_scale, s, ws, lease.err());
}

static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int check_projection(llh_ctx *ctx, const void *d_w, int32_t rows, int32_t cols, float *d_out) {
  if (!d_w || !d_out) return ctx->fail(LLH_ERR_NULL, "null device pointer in projection call");
  if (rows <= 0 || cols <= 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "projection rows and columns must be > 0");
  if (cols % kMatvecColsMultiple != 0 || !aligned16(d_w)) {
    ctx->not_handled++;
    return ctx->fail(LLH_ERR_UNSUPPORTED, "projection takes 16-byte aligned weights with columns a multiple of 128");
  }
  return LLH_OK;
}

// One decode step whose bf16 attention output stays in the stream's workspace,
// then out[b] = W_o attn[b] on the same stream (both launches under one lease).
static int decode_projection_impl(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc,
                                  const void *d_q, const void *d_w_o, int32_t rows, float *d_out, float score_scale,
                                  void *stream) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  if (desc->num_seqs <= 0) return desc->num_seqs == 0 ? LLH_OK : ctx->fail(LLH_ERR_INVALID_SHAPE, "num_seqs < 0");
  const int32_t cols = desc->num_q_heads * pool->view.head_dim;
  int st = check_projection(ctx, d_w_o, rows, cols, d_out);
  if (st != LLH_OK) return st;
  const size_t attn_bytes = align_up((size_t)desc->num_seqs * cols * sizeof(uint16_t));
  const int ksplit = matvec_ksplit(rows, cols, desc->num_seqs, ctx->cus);
  const size_t partial_bytes = ksplit > 1 ? (size_t)ksplit * desc->num_seqs * rows * sizeof(float) : 0;
  void *attn = nullptr;  // the attention output, then the projection's partial tiles
  WsLease lease;         // held through the projection launch
  st = paged_decode_impl(ctx, pool, desc, d_q, nullptr, score_scale, stream, attn_bytes + partial_bytes, &attn,
                         lease);
  if (st != LLH_OK) return st;
  MatvecArgs a{};
  a.w = static_cast<const uint16_t *>(d_w_o);
  a.x = attn;
  a.out = d_out;
  a.rows = rows;
  a.cols = cols;
  a.n = desc->num_seqs;
  a.ldx = cols;
  a.ldo = rows;
  a.x_f32 = 0;
  a.ksplit = ksplit;
  a.partial = ksplit > 1 ? reinterpret_cast<float *>(static_cast<char *>(attn) + attn_bytes) : nullptr;
  hipError_t e = launch_matvec_bf16(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "projection launch");
  return LLH_OK;
}

extern "C" {

int llh_paged_decode(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_q, void *d_out,
                     float score_scale, void *stream) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  if (!d_out && desc->num_seqs > 0) return ctx->fail(LLH_ERR_NULL, "null device pointer in decode call");
  WsLease lease;
  return paged_decode_impl(ctx, pool, desc, d_q, d_out, score_scale, stream, 0, nullptr, lease);
}

int llh_paged_decode_append(llh_ctx *ctx, llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_k_new,
                            const void *d_v_new, const void *d_q, void *d_out, float score_scale, void *stream) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  if (desc->num_seqs > 0 && (!d_out || !d_k_new || !d_v_new))
    return ctx->fail(LLH_ERR_NULL, "null device pointer in decode call");
  DecodePlan plan;
  int st = plan_decode(ctx, pool, desc, d_q, d_out, score_scale, &plan);
  if (st != LLH_OK || plan.empty) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const PoolView &pv = pool->view;
  // fp8 blocks keep one scale per (block, head) that a token at offset 0 restarts
  // and a later token may grow, re-encoding only the tokens before it: a block
  // that still holds live (in-window) tokens of an older pass round the ring
  // must never receive the new token.  That holds when the row outlasts the
  // window by a block's worth of slots (window + block_tokens - 1 <= row) or the
  // ring never wraps (max_seq_len <= row).
  const int64_t row_tokens = (int64_t)desc->max_blocks_per_seq * pv.block_tokens;
  if (pv.format == LLH_KV_FP8_E4M3 && desc->max_seq_len > row_tokens &&
      (int64_t)desc->window + pv.block_tokens - 1 > row_tokens)
    return ctx->fail(LLH_ERR_INVALID_SHAPE,
                     "fp8 append over a window ring needs window + block_tokens - 1 <= max_blocks_per_seq * "
                     "block_tokens (one block more than the window)");
  // one launch on the tuned kernels (new-token rows 16-byte aligned): bf16 pools attend
  // the new token from its rows, int8 / fp8 pools quantise it into the block that
  // receives it; at head_dim 256 the stream kernel (bf16 and fp16 pools) writes the
  // token's rows and attends them from the registers of the block it loads.  fp8 pools
  // on the persistent stream kernel are the exception: the scale-growth re-encode
  // doubles that kernel's code and costs more than the separate append launch it
  // saves; fp16 pools at head_dim 128 and the head_dim-256 split-K kernel have no fused
  // form.  Every other case appends through the append kernel first, then decodes.
  const bool fused = plan.fast && (pv.format != LLH_KV_F16 || plan.d256) && aligned16(d_k_new) &&
                     aligned16(d_v_new) &&
                     !(pv.format == LLH_KV_FP8_E4M3 && plan.stream_wgs > 0) && (!plan.d256 || plan.stream_wgs > 0);
  WsLease lease;
  st = lease.acquire(ctx, s, plan.bytes);
  if (st != LLH_OK) return st;
  char *ws = lease.base();
  if (fused) {
    ctx->fused_append_calls++;
    return launch_planned_decode(ctx, pool, desc, plan, d_q, d_out, score_scale, s, ws, lease.err(), true,
                                 static_cast<const uint16_t *>(d_k_new), static_cast<const uint16_t *>(d_v_new));
  }
  // the append kernel finds each new token's slot through the descriptor's table rows
  st = kv_append(ctx, pool, nullptr, d_k_new, d_v_new, desc->num_seqs, 0, stream, desc->d_seq_lens,
                 desc->d_block_tables, desc->max_blocks_per_seq);
  if (st != LLH_OK) return st;
  return launch_planned_decode(ctx, pool, desc, plan, d_q, d_out, score_scale, s, ws, lease.err());
}

int llh_matvec_bf16_f32(llh_ctx *ctx, const void *d_w, int32_t rows, int32_t cols, const void *d_x, int32_t x_f32,
                        int32_t n, float *d_out, void *stream) {
  if (!ctx) return LLH_ERR_NULL;
  if (n < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "input count must be >= 0");
  if (n == 0) return LLH_OK;
  int st = check_projection(ctx, d_w, rows, cols, d_out);
  if (st != LLH_OK) return st;
  if (!d_x) return ctx->fail(LLH_ERR_NULL, "null device pointer in projection call");
  if (!aligned16(d_x)) return ctx->fail(LLH_ERR_UNSUPPORTED, "projection inputs must be 16-byte aligned");
  MatvecArgs a{};
  a.w = static_cast<const uint16_t *>(d_w);
  a.x = d_x;
  a.out = d_out;
  a.rows = rows;
  a.cols = cols;
  a.n = n;
  a.ldx = cols;
  a.ldo = rows;
  a.x_f32 = x_f32 ? 1 : 0;
  a.ksplit = matvec_ksplit(rows, cols, n, ctx->cus);
  WsLease lease;
  if (a.ksplit > 1) {  // partial tiles in the stream's workspace
    st = lease.acquire(ctx, static_cast<hipStream_t>(stream), (size_t)a.ksplit * n * rows * sizeof(float));
    if (st != LLH_OK) return st;
    a.partial = reinterpret_cast<float *>(lease.base());
  }
  hipError_t e = launch_matvec_bf16(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "projection launch");
  return LLH_OK;
}

int llh_paged_decode_output_projection(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc,
                                       const void *d_q, const void *d_w_o, int32_t rows, float *d_out,
                                       float score_scale, void *stream) {
  return decode_projection_impl(ctx, pool, desc, d_q, d_w_o, rows, d_out, score_scale, stream);
}

int llh_paged_prefill(llh_ctx *ctx, const llh_kv_pool *pool, const llh_prefill_desc *desc, const void *d_q,
                      void *d_out, float score_scale, void *stream) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  int st = check_desc_common(ctx, pool, desc->num_seqs, desc->num_q_heads, desc->max_blocks_per_seq, desc->window);
  if (st != LLH_OK) return st;
  if (desc->num_seqs == 0 || desc->total_q_rows == 0) return LLH_OK;
  if (desc->total_q_rows < 0 || desc->max_chunk_len < 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "row counts must be >= 0");
  const PoolView &pv = pool->view;
  if (pv.head_dim > kGenericPrefillMaxDim) {
    ctx->not_handled++;
    return ctx->fail(LLH_ERR_UNSUPPORTED, "prefill takes head_dim <= " + std::to_string(kGenericPrefillMaxDim));
  }
  if (!d_q || !d_out || !desc->d_chunk_starts || !desc->d_context_lens || !desc->d_block_tables)
    return ctx->fail(LLH_ERR_NULL, "null device pointer in prefill call");
  if (((reinterpret_cast<uintptr_t>(d_q) | reinterpret_cast<uintptr_t>(d_out)) & 1) != 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "prefill q and output must be bf16-aligned (2 bytes)");
  if (!std::isfinite(score_scale)) return ctx->fail(LLH_ERR_NON_FINITE, "score scale must be finite");
  // the tuned MFMA kernels take 16-token blocks and 16-byte aligned rows at head_dim
  // 128 (bf16, int8, fp8, fp16 pools) and 256 (bf16, fp16); every other call runs the
  // element-wise kernel
  const bool tuned_shape = pv.block_tokens == kFastBlockTokens &&
                           ((reinterpret_cast<uintptr_t>(d_q) | reinterpret_cast<uintptr_t>(d_out)) & 15) == 0 &&
                           ctx->opt(LLH_OPT_FORCE_GENERIC) == 0;
  const bool fast = tuned_shape && pv.format != LLH_KV_INT8_ROW && pv.head_dim == kFastHeadDim;
  const bool fast256 =
      tuned_shape && (pv.format == LLH_KV_BF16 || pv.format == LLH_KV_F16) && pv.head_dim == kD256HeadDim;
  PrefillArgs a{};
  a.pool = pv;
  a.q = static_cast<const uint16_t *>(d_q);
  a.out = static_cast<uint16_t *>(d_out);
  a.chunk_starts = desc->d_chunk_starts;
  a.context_lens = desc->d_context_lens;
  a.tables = desc->d_block_tables;
  a.err = ctx->err_word(static_cast<hipStream_t>(stream));
  a.num_seqs = desc->num_seqs;
  a.q_heads = desc->num_q_heads;
  a.max_blocks = desc->max_blocks_per_seq;
  a.window = desc->window;
  a.q_tiles = std::max(1, (desc->max_chunk_len + 127) / 128);
  a.scale_log2e = score_scale * 1.4426950408889634f;
  a.scale = score_scale;
  a.gate = static_cast<const uint16_t *>(desc->d_gate);
  ctx->prefill_calls++;
  auto ev = ctx->timing_begin(static_cast<hipStream_t>(stream));
  hipError_t e;
  if (fast) {
    // two query heads of a kv head per workgroup share its K/V tile stream when the group is even
    const int group = desc->num_q_heads / pv.kv_heads;
    const int hpw_env = ctx->opt(LLH_OPT_PREFILL_HEADS_PER_WG);
    const int variant = (hpw_env == 1 || group % 2 != 0) ? kPrefillOneHead : kPrefillTwoHeads;
    e = launch_prefill(a, variant, static_cast<hipStream_t>(stream));
  } else if (fast256) {
    e = launch_prefill_d256(a, static_cast<hipStream_t>(stream));
  } else {
    ctx->generic_prefill_calls++;
    e = launch_prefill_generic(a, desc->total_q_rows, static_cast<hipStream_t>(stream));
  }
  ctx->timing_end(1, ev, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "prefill launch");
  return LLH_OK;
}

int llh_debug_gather(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, int32_t seq, int32_t lo,
                     int32_t hi, int32_t tensor, void *d_out, void *stream) {
  if (!ctx || !pool || !desc) return LLH_ERR_NULL;
  if (seq < 0 || seq >= desc->num_seqs || lo < 0 || hi < lo || (tensor != 0 && tensor != 1) ||
      desc->max_blocks_per_seq <= 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "gather arguments out of range");
  if (hi == lo) return LLH_OK;
  if (!d_out || !desc->d_block_tables) return ctx->fail(LLH_ERR_NULL, "null device pointer");
  GatherArgs a{};
  a.pool = pool->view;
  a.table = desc->d_block_tables + (size_t)seq * desc->max_blocks_per_seq;
  a.max_blocks = desc->max_blocks_per_seq;
  a.lo = lo;
  a.hi = hi;
  a.tensor = tensor;
  a.ring_tokens = 0;
  a.out = d_out;
  a.err = ctx->err_word(static_cast<hipStream_t>(stream));
  hipError_t e = launch_gather(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "gather launch");
  return LLH_OK;
}

int llh_debug_decode_fp8(llh_ctx *ctx, const uint8_t *d_codes, float *d_out, int32_t n, void *stream) {
  if (!ctx) return LLH_ERR_NULL;
  if (n < 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "negative count");
  if (n > 0 && (!d_codes || !d_out)) return ctx->fail(LLH_ERR_NULL, "null device pointer");
  hipError_t e = launch_decode_fp8(d_codes, d_out, n, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return ctx->hip_fail(e, "fp8 decode launch");
  return LLH_OK;
}

int llh_debug_fp8_encode_check(llh_ctx *ctx, uint64_t *h_mismatches) {
  if (!ctx || !h_mismatches) return LLH_ERR_NULL;
  unsigned long long *d = nullptr;
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc(&d, sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMemset(d, 0, sizeof(unsigned long long));
  if (e == hipSuccess) e = launch_fp8_encode_check(d, nullptr);
  unsigned long long h = 0;
  if (e == hipSuccess) e = hipMemcpy(&h, d, sizeof(h), hipMemcpyDeviceToHost);
  if (d) (void)hipFree(d);
  if (e != hipSuccess) return ctx->hip_fail(e, "fp8 encode check");
  *h_mismatches = h;
  return LLH_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// LayerKvCache mirror
// ---------------------------------------------------------------------------
namespace {

constexpr int kRingBlockTokens = 16;

// Device blocks shared by a cache and its clones, with reference counts
// (the Arc<CacheBlockStorage> sharing of crates/llm-kv-cache/src/block.rs:124-160).
// `mu` is held by every trait call on any cache of the store from its first
// read of the store through its final stream wait, so a growth (which frees
// the old buffers) or a copy never overlaps another cache's kernels.
struct BlockStore {
  llh_ctx *ctx = nullptr;
  int32_t format = 0;
  int32_t kv_heads = 0;
  int32_t head_dim = 0;
  int64_t capacity = 0;
  void *k = nullptr, *v = nullptr, *ks = nullptr, *vs = nullptr;
  size_t kblock = 0, sblock = 0;
  std::vector<int32_t> refs;
  std::vector<int32_t> free_list;
  std::mutex mu;

  ~BlockStore() {
    if (ctx) (void)hipSetDevice(ctx->device);
    for (void *p : {k, v, ks, vs_alloc()})
      if (p) (void)hipFree(p);
  }
  // the V scales' own allocation (none for int8: they sit inside the K scales' one)
  void *vs_alloc() const { return scales_interleaved(format) ? nullptr : vs; }
  PoolView view() const {
    return PoolView{format, kRingBlockTokens, kv_heads, head_dim, capacity, k, v, ks, vs};
  }
  // Grows the store with its copies on stream s (waited for before the old
  // buffers go); callers hold `mu`, so no kernel of any cache of the store is
  // in flight (every trait call waits for its own stream before releasing it).
  hipError_t allocate(int64_t cap, hipStream_t s) {
    kblock = (size_t)kv_heads * kRingBlockTokens * head_dim * elem_bytes(format);
    sblock = scale_bytes_per_block(format, kv_heads, kRingBlockTokens);
    // scale bytes per block in the K scales' allocation (int8, fp8: K and V scale pairs)
    const bool il = scales_interleaved(format);
    const size_t kscale = il ? 2 * sblock : sblock;
    void *nk = nullptr, *nv = nullptr, *nks = nullptr, *nvs = nullptr;
    hipError_t e = hipMalloc(&nk, kblock * cap);
    if (e == hipSuccess) e = hipMalloc(&nv, kblock * cap);
    if (e == hipSuccess && sblock) e = hipMalloc(&nks, kscale * cap);
    if (e == hipSuccess && sblock && !il) e = hipMalloc(&nvs, sblock * cap);
    if (e == hipSuccess) e = hipMemsetAsync(nk, 0, kblock * cap, s);
    if (e == hipSuccess) e = hipMemsetAsync(nv, 0, kblock * cap, s);
    if (e == hipSuccess && sblock) e = hipMemsetAsync(nks, 0, kscale * cap, s);
    if (e == hipSuccess && sblock && !il) e = hipMemsetAsync(nvs, 0, sblock * cap, s);
    if (e == hipSuccess && capacity > 0) {
      e = hipMemcpyAsync(nk, k, kblock * capacity, hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess) e = hipMemcpyAsync(nv, v, kblock * capacity, hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess && sblock) e = hipMemcpyAsync(nks, ks, kscale * capacity, hipMemcpyDeviceToDevice, s);
      if (e == hipSuccess && sblock && !il)
        e = hipMemcpyAsync(nvs, vs, sblock * capacity, hipMemcpyDeviceToDevice, s);
    }
    if (il && nks) nvs = static_cast<char *>(nks) + v_scale_offset_bytes(format);
    // the copies must land before any cache's stream touches the new buffers
    // (the next trait call, on whichever stream, starts after this wait) and
    // before the old buffers are freed
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      for (void *p : {nk, nv, nks, il ? nullptr : nvs})
        if (p) (void)hipFree(p);
      return e;
    }
    for (void *p : {k, v, ks, vs_alloc()})
      if (p) (void)hipFree(p);
    k = nk;
    v = nv;
    ks = nks;
    vs = nvs;
    for (int64_t i = cap - 1; i >= capacity; i--) free_list.push_back((int32_t)i);
    refs.resize(cap, 0);
    capacity = cap;
    return hipSuccess;
  }
  // returns a pool index with refcount 1, growing the store (on stream s) when full
  hipError_t take(int32_t &out, hipStream_t s) {
    if (free_list.empty()) {
      hipError_t e = allocate(capacity * 2, s);
      if (e != hipSuccess) return e;
    }
    out = free_list.back();
    free_list.pop_back();
    refs[out] = 1;
    return hipSuccess;
  }
  void release(int32_t idx) {
    if (--refs[idx] == 0) free_list.push_back(idx);
  }
  hipError_t copy_block(int32_t src, int32_t dst, hipStream_t s) {
    hipError_t e = hipMemcpyAsync((char *)k + kblock * dst, (char *)k + kblock * src, kblock,
                                  hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess)
      e = hipMemcpyAsync((char *)v + kblock * dst, (char *)v + kblock * src, kblock, hipMemcpyDeviceToDevice, s);
    const size_t kscale = scales_interleaved(format) ? 2 * sblock : sblock;
    if (e == hipSuccess && sblock)
      e = hipMemcpyAsync((char *)ks + kscale * dst, (char *)ks + kscale * src, kscale, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess && sblock && !scales_interleaved(format))
      e = hipMemcpyAsync((char *)vs + sblock * dst, (char *)vs + sblock * src, sblock, hipMemcpyDeviceToDevice, s);
    return e;
  }
};

// Scratch of the synchronous trait calls: a device buffer and a pinned host
// staging buffer, reused per call (a call waits for its stream before returning).
struct TraitScratch {
  void *dev = nullptr;
  size_t dev_bytes = 0;
  void *host = nullptr;
  size_t host_bytes = 0;
  hipError_t ensure(size_t dev_n, size_t host_n) {
    if (dev_n > dev_bytes) {
      if (dev) (void)hipFree(dev);
      dev = nullptr;
      dev_bytes = 0;
      const size_t nb = align_up(std::max(dev_n, (size_t)4096));
      hipError_t e = hipMalloc(&dev, nb);
      if (e != hipSuccess) return e;
      dev_bytes = nb;
    }
    if (host_n > host_bytes) {
      if (host) (void)hipHostFree(host);
      host = nullptr;
      host_bytes = 0;
      const size_t nb = align_up(std::max(host_n, (size_t)4096));
      hipError_t e = hipHostMalloc(&host, nb, hipHostMallocDefault);
      if (e != hipSuccess) return e;
      host_bytes = nb;
    }
    return hipSuccess;
  }
  ~TraitScratch() {
    if (dev) (void)hipFree(dev);
    if (host) (void)hipHostFree(host);
  }
};

uint16_t host_f32_to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float host_bf16_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

}  // namespace

struct llh_layer_cache {
  llh_ctx *ctx = nullptr;
  std::shared_ptr<BlockStore> store;
  uint64_t id = 0;
  uint64_t revision = 0;
  size_t max_tokens = 0, kv_heads = 0, head_dim = 0;
  int32_t format = 0;
  size_t token_count = 0, tokens_seen = 0, window_start = 0;
  bool non_finite_rows = false;  // a row with a non-finite value was appended (bf16 caches)
  std::vector<int32_t> table;    // pool index per ring block
  std::vector<uint64_t> ids;     // BlockId per ring block
  hipStream_t stream = nullptr;  // this cache's own stream (default priority)
  TraitScratch scratch;
  std::mutex mu;

  size_t vector_len() const { return kv_heads * head_dim; }
  ~llh_layer_cache() {
    if (stream) (void)hipStreamDestroy(stream);
  }
};


extern "C" {

int llh_layer_cache_create(llh_ctx *ctx, size_t max_tokens, size_t kv_heads, size_t head_dim, int32_t format,
                           llh_layer_cache **out) {
  if (!ctx || !out) return LLH_ERR_NULL;
  *out = nullptr;
  if (max_tokens == 0 || kv_heads == 0 || head_dim == 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "invalid KV cache shape");
  if (format != LLH_KV_BF16 && format != LLH_KV_INT8 && format != LLH_KV_INT8_ROW)
    return ctx->fail(LLH_ERR_UNSUPPORTED, "unsupported KV cache format for the layer cache");
  if (max_tokens > (size_t)INT32_MAX / 2 || kv_heads * head_dim > (1u << 20))
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "KV cache shape too large");
  auto *c = new llh_layer_cache();
  c->ctx = ctx;
  c->max_tokens = max_tokens;
  c->kv_heads = kv_heads;
  c->head_dim = head_dim;
  c->format = format;
  c->id = g_next_cache_id.fetch_add(1);
  const size_t nb = (max_tokens + kRingBlockTokens - 1) / kRingBlockTokens;
  c->store = std::make_shared<BlockStore>();
  c->store->ctx = ctx;
  c->store->format = format;
  c->store->kv_heads = (int32_t)kv_heads;
  c->store->head_dim = (int32_t)head_dim;
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = c->store->allocate((int64_t)nb * 2 + 2, c->stream);
  for (size_t i = 0; e == hipSuccess && i < nb; i++) {
    int32_t idx;
    e = c->store->take(idx, c->stream);
    c->table.push_back(idx);
    c->ids.push_back(next_block_id());
  }
  if (e != hipSuccess) {
    delete c;
    return ctx->hip_fail(e, "layer cache allocation");
  }
  *out = c;
  return LLH_OK;
}

// LayerKvCache::from_snapshot (layer.rs:467-507) and from_prefix_cache_state
// (layer.rs:544-581) on the device: a fresh cache (new id) whose ring holds the
// given logical rows, logical row i in ring slot (window_start + i) % max_tokens,
// with the given revision, token count, tokens seen and window start.  The rows
// go through the append kernel (bf16 rounding, int8 quantisation), in chunks, so
// the ring holds exactly what appending them one by one would write.
int llh_layer_cache_create_from_rows(llh_ctx *ctx, const llh_layer_cache_rows *r, llh_layer_cache **out) {
  if (!ctx || !r || !out) return LLH_ERR_NULL;
  *out = nullptr;
  // from_prefix_cache_state's checks, in its order (layer.rs:545-553)
  if (r->max_tokens == 0 || r->kv_heads == 0 || r->head_dim == 0 || r->token_count > r->max_tokens ||
      r->tokens_seen < r->token_count || r->window_start >= r->max_tokens)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "invalid KV cache state");
  llh_layer_cache *c = nullptr;
  int st = llh_layer_cache_create(ctx, r->max_tokens, r->kv_heads, r->head_dim, r->format, &c);
  if (st != LLH_OK) return st;
  const size_t vl = c->vector_len();
  const size_t n = r->token_count;
  // from_snapshot's length check (layer.rs:482-496): KvCacheError::ShapeMismatch
  if (r->keys_len != n * vl) {
    llh_layer_cache_destroy(c);
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "KV rows do not match token_count * key_value_heads * head_dim");
  }
  if (n > 0 && (!r->h_keys || !r->h_values)) {
    llh_layer_cache_destroy(c);
    return ctx->fail(LLH_ERR_NULL, "null row pointer");
  }
  bool finite = true;
  for (size_t i = 0; i < n * vl && finite; i++) finite = std::isfinite(r->h_keys[i]) && std::isfinite(r->h_values[i]);
  if (!finite && (r->format == LLH_KV_INT8 || r->format == LLH_KV_INT8_ROW)) {
    llh_layer_cache_destroy(c);
    return ctx->fail(LLH_ERR_NON_FINITE, "int8 KV cache rows must be finite");
  }
  hipError_t e = hipSuccess;
  if (n > 0) {
    BlockStore &bs = *c->store;
    std::lock_guard<std::mutex> gs(bs.mu);  // through the stream waits
    const size_t chunk = std::max<size_t>(1, std::min<size_t>(n, ((size_t)16 << 20) / (vl * sizeof(float))));
    const size_t k_off = align_up(chunk * sizeof(int64_t));
    const size_t v_off = k_off + align_up(chunk * vl * sizeof(float));
    void *tmp = nullptr;
    e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc(&tmp, v_off + chunk * vl * sizeof(float));
    std::vector<int64_t> slots(chunk);
    int32_t *err = ctx->err_word(c->stream);
    for (size_t i0 = 0; e == hipSuccess && i0 < n; i0 += chunk) {
      const size_t m = std::min(chunk, n - i0);
      for (size_t i = 0; i < m; i++) {
        const size_t phys = (r->window_start + i0 + i) % r->max_tokens;
        slots[i] = (int64_t)c->table[phys / kRingBlockTokens] * kRingBlockTokens + (int64_t)(phys % kRingBlockTokens);
      }
      char *d = static_cast<char *>(tmp);
      e = hipMemcpyAsync(d, slots.data(), m * sizeof(int64_t), hipMemcpyHostToDevice, c->stream);
      if (e == hipSuccess)
        e = hipMemcpyAsync(d + k_off, r->h_keys + i0 * vl, m * vl * sizeof(float), hipMemcpyHostToDevice, c->stream);
      if (e == hipSuccess)
        e = hipMemcpyAsync(d + v_off, r->h_values + i0 * vl, m * vl * sizeof(float), hipMemcpyHostToDevice,
                           c->stream);
      AppendArgs a{};
      a.pool = bs.view();
      a.k_dst = bs.k;
      a.v_dst = bs.v;
      a.ks_dst = bs.ks;
      a.vs_dst = bs.vs;
      a.slots = reinterpret_cast<const int64_t *>(d);
      a.k = d + k_off;
      a.v = d + v_off;
      a.n = (int32_t)m;
      a.src_f32 = 1;
      a.err = err;
      if (e == hipSuccess) e = launch_append(a, c->stream);
      // the host slot list is refilled for the next chunk only after this one's copies
      if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    }
    if (tmp) (void)hipFree(tmp);
  }
  if (e != hipSuccess) {
    llh_layer_cache_destroy(c);
    return ctx->hip_fail(e, "layer cache rows");
  }
  ctx->append_calls += n;
  c->token_count = n;
  c->tokens_seen = r->tokens_seen;
  c->window_start = r->window_start;
  c->revision = r->revision;
  c->non_finite_rows = !finite;
  *out = c;
  return LLH_OK;
}

int llh_layer_cache_destroy(llh_layer_cache *cache) {
  if (!cache) return LLH_ERR_NULL;
  {
    std::lock_guard<std::mutex> g(cache->store->mu);
    for (int32_t idx : cache->table) cache->store->release(idx);
  }
  (void)hipSetDevice(cache->ctx->device);
  // the workspace slot of the cache's stream (its tuned trait calls' scratch and
  // error word) goes before the stream does
  const int st = release_slot(cache->ctx, cache->stream, true);
  delete cache;
  return st;
}

int llh_layer_cache_clone(const llh_layer_cache *cache, llh_layer_cache **out) {
  if (!cache || !out) return LLH_ERR_NULL;
  *out = nullptr;
  auto *src = const_cast<llh_layer_cache *>(cache);
  std::lock_guard<std::mutex> g0(src->mu);
  auto *c = new llh_layer_cache();
  c->ctx = src->ctx;
  c->store = src->store;
  c->id = g_next_cache_id.fetch_add(1);
  c->revision = src->revision;
  c->max_tokens = src->max_tokens;
  c->kv_heads = src->kv_heads;
  c->head_dim = src->head_dim;
  c->format = src->format;
  c->token_count = src->token_count;
  c->tokens_seen = src->tokens_seen;
  c->window_start = src->window_start;
  c->non_finite_rows = src->non_finite_rows;
  c->table = src->table;
  c->ids = src->ids;
  hipError_t e = hipSetDevice(c->ctx->device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    c->table.clear();
    delete c;
    return src->ctx->hip_fail(e, "layer cache stream");
  }
  {
    std::lock_guard<std::mutex> g(c->store->mu);
    for (int32_t idx : c->table) c->store->refs[idx]++;
  }
  *out = c;
  return LLH_OK;
}

int llh_layer_cache_clear(llh_layer_cache *cache) {
  if (!cache) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(cache->mu);
  cache->token_count = 0;
  cache->tokens_seen = 0;
  cache->window_start = 0;
  cache->non_finite_rows = false;
  cache->revision += 1;
  return LLH_OK;
}

int llh_layer_cache_get_state(const llh_layer_cache *cache_c, llh_layer_cache_state *out) {
  if (!cache_c || !out) return LLH_ERR_NULL;
  auto *cache = const_cast<llh_layer_cache *>(cache_c);
  std::lock_guard<std::mutex> g(cache->mu);
  out->id = cache->id;
  out->revision = cache->revision;
  out->max_tokens = cache->max_tokens;
  out->kv_heads = cache->kv_heads;
  out->head_dim = cache->head_dim;
  out->token_count = cache->token_count;
  out->tokens_seen = cache->tokens_seen;
  out->window_start = cache->window_start;
  out->block_count = cache->table.size();
  out->format = cache->format;
  out->block_tokens = kRingBlockTokens;
  return LLH_OK;
}

int llh_layer_cache_block_ids(const llh_layer_cache *cache_c, uint64_t *h_out, size_t capacity, size_t *count) {
  if (!cache_c || !count) return LLH_ERR_NULL;
  auto *cache = const_cast<llh_layer_cache *>(cache_c);
  std::lock_guard<std::mutex> g(cache->mu);
  *count = cache->ids.size();
  if (h_out) std::memcpy(h_out, cache->ids.data(), std::min(capacity, cache->ids.size()) * sizeof(uint64_t));
  return capacity >= cache->ids.size() || !h_out ? LLH_OK : LLH_ERR_CAPACITY;
}

// Runs of logical tokens contiguous in one device block, in logical order:
// the closed form of append_active_block_run / remove_oldest_active_block_token
// (layer.rs:1097-1162) for 16-token blocks.
int llh_layer_cache_active_blocks(const llh_layer_cache *cache_c, llh_block_run *h_out, size_t capacity,
                                  size_t *count) {
  if (!cache_c || !count) return LLH_ERR_NULL;
  auto *cache = const_cast<llh_layer_cache *>(cache_c);
  std::lock_guard<std::mutex> g(cache->mu);
  std::vector<llh_block_run> runs;
  for (size_t i = 0; i < cache->token_count; i++) {
    const size_t phys = (cache->window_start + i) % cache->max_tokens;
    const size_t bi = phys / kRingBlockTokens;
    const size_t off = phys % kRingBlockTokens;
    if (!runs.empty()) {
      llh_block_run &r = runs.back();
      if (r.block_index == bi && r.logical_token_start + r.token_count == i &&
          r.physical_token_start + r.token_count == phys && r.block_token_start + r.token_count == off) {
        r.token_count++;
        continue;
      }
    }
    runs.push_back(llh_block_run{cache->ids[bi], bi, i, phys, off, 1});
  }
  *count = runs.size();
  if (h_out) std::memcpy(h_out, runs.data(), std::min(capacity, runs.size()) * sizeof(llh_block_run));
  return capacity >= runs.size() || !h_out ? LLH_OK : LLH_ERR_CAPACITY;
}

static int layer_append(llh_ctx *ctx, llh_layer_cache *cache, const float *h_key, const float *h_value, size_t len,
                        bool sliding) {
  if (!ctx || !cache || !h_key || !h_value) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(cache->mu);
  if (len != cache->vector_len()) return ctx->fail(LLH_ERR_INVALID_SHAPE, "KV row length does not match the cache");
  bool finite = true;
  for (size_t i = 0; i < len && finite; i++) finite = std::isfinite(h_key[i]) && std::isfinite(h_value[i]);
  if (!finite && (cache->format == LLH_KV_INT8 || cache->format == LLH_KV_INT8_ROW))
    return ctx->fail(LLH_ERR_NON_FINITE, "int8 KV cache rows must be finite");
  const bool full = cache->token_count == cache->max_tokens;
  if (full && !sliding) return ctx->fail(LLH_ERR_CAPACITY, "KV cache capacity exceeded");
  const size_t phys = full ? cache->window_start : cache->token_count;
  const size_t bi = phys / kRingBlockTokens;
  const size_t off = phys % kRingBlockTokens;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return ctx->hip_fail(e, "hipSetDevice");
  BlockStore &bs = *cache->store;
  std::lock_guard<std::mutex> gs(bs.mu);  // through the stream wait below
  const size_t row_bytes = len * sizeof(float);
  const size_t k_off = kAlign, v_off = kAlign + align_up(row_bytes);
  const size_t bytes = v_off + row_bytes;
  e = cache->scratch.ensure(bytes, bytes);
  if (e != hipSuccess) return ctx->hip_fail(e, "scratch allocation");
  // copy-on-write: a block shared with a clone gets a fresh device block and id
  const int32_t idx = cache->table[bi];
  if (bs.refs[idx] > 1) {
    int32_t fresh;
    e = bs.take(fresh, cache->stream);
    if (e == hipSuccess) e = bs.copy_block(idx, fresh, cache->stream);
    if (e != hipSuccess) return ctx->hip_fail(e, "copy-on-write block");
    bs.release(idx);
    cache->table[bi] = fresh;
    cache->ids[bi] = next_block_id();
  }
  char *hb = static_cast<char *>(cache->scratch.host);
  char *sb = static_cast<char *>(cache->scratch.dev);
  const int64_t slot = (int64_t)cache->table[bi] * kRingBlockTokens + (int64_t)off;
  std::memcpy(hb, &slot, sizeof(slot));
  std::memcpy(hb + k_off, h_key, row_bytes);
  std::memcpy(hb + v_off, h_value, row_bytes);
  e = hipMemcpyAsync(sb, hb, bytes, hipMemcpyHostToDevice, cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "row upload");
  AppendArgs a{};
  a.pool = bs.view();
  a.k_dst = bs.k;
  a.v_dst = bs.v;
  a.ks_dst = bs.ks;
  a.vs_dst = bs.vs;
  a.slots = reinterpret_cast<const int64_t *>(sb);
  a.k = sb + k_off;
  a.v = sb + v_off;
  a.n = 1;
  a.src_f32 = 1;
  a.err = ctx->err_word(cache->stream);
  e = launch_append(a, cache->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "append");
  ctx->append_calls++;
  if (!finite) cache->non_finite_rows = true;
  if (full) {
    cache->window_start = (cache->window_start + 1) % cache->max_tokens;
  } else {
    cache->token_count += 1;
  }
  cache->tokens_seen += 1;
  cache->revision += 1;
  return LLH_OK;
}

int llh_append_kv_cache_sliding_f32(llh_ctx *ctx, llh_layer_cache *cache, const float *h_key, const float *h_value,
                                    size_t len) {
  return layer_append(ctx, cache, h_key, h_value, len, true);
}

int llh_append_kv_cache_f32(llh_ctx *ctx, llh_layer_cache *cache, const float *h_key, const float *h_value,
                            size_t len) {
  return layer_append(ctx, cache, h_key, h_value, len, false);
}

}  // extern "C"

// The tuned decode kernels serve a trait call when the cache has the tuned
// shape (head_dim 128, a GQA group of 1, 2, 4 or 8) and its ring is whole
// blocks (then ring slot p % max_tokens is table[(p / 16) % blocks] at offset
// p % 16, the batched kernels' own mapping), and nothing non-finite can reach
// the scores: the reference's softmax_f32 errors on non-finite scores
// (math.rs:485-489), which only the reference-order kernel reports, so finite
// q and rows are checked here and a non-finite result is recomputed there.
static bool trait_tuned_ok(const llh_ctx *ctx, const llh_layer_cache *cache, const float *h_query, size_t qdim,
                           size_t heads, size_t kv_heads) {
  if (ctx->opt(LLH_OPT_TRAIT_REFERENCE_ORDER) || cache->format == LLH_KV_INT8_ROW) return false;
  const size_t group = heads / kv_heads;
  if (cache->head_dim != (size_t)kFastHeadDim || cache->max_tokens % kRingBlockTokens != 0 || cache->non_finite_rows)
    return false;
  if (group != 1 && group != 2 && group != 4 && group != 8) return false;
  for (size_t i = 0; i < qdim; i++)
    if (!std::isfinite(h_query[i])) return false;
  return true;
}

// Attention over the first row_count logical rows on the tuned kernels: one
// decode step of a batch of one (q rounded to bf16, bf16 output widened to f32),
// through the cache's stream and its stream workspace.  With d_w the attention
// output is projected on the device (llh_paged_decode_output_projection).
// Sets *finite = false when the output holds a non-finite value.
static int cache_mix_tuned(llh_ctx *ctx, llh_layer_cache *cache, const float *h_query, size_t qdim, size_t row_count,
                           size_t heads, float score_scale, const void *d_w, int32_t w_rows, float *h_output,
                           size_t out_len, bool *finite) {
  BlockStore &bs = *cache->store;
  const size_t nb = cache->table.size();
  const size_t off_table = kAlign;  // int32 [nb]; header: seq_len
  const size_t off_q = off_table + align_up(nb * sizeof(int32_t));
  const size_t off_out = off_q + align_up(qdim * sizeof(uint16_t));
  const size_t out_bytes = d_w ? out_len * sizeof(float) : qdim * sizeof(uint16_t);
  const size_t bytes = off_out + out_bytes;
  hipError_t e = cache->scratch.ensure(bytes, bytes);
  if (e != hipSuccess) return ctx->hip_fail(e, "scratch allocation");
  char *hb = static_cast<char *>(cache->scratch.host);
  char *sb = static_cast<char *>(cache->scratch.dev);
  // logical row i lives in ring slot (window_start + i) % max_tokens
  // (layer.rs:1080-1095): the kernels address it as position window_start + i,
  // whose block is table[(p / 16) % blocks] at offset p % 16 (whole-block ring)
  const int32_t len = (int32_t)(cache->window_start + row_count);
  std::memcpy(hb, &len, sizeof(len));
  std::memcpy(hb + off_table, cache->table.data(), nb * sizeof(int32_t));
  auto *qh = reinterpret_cast<uint16_t *>(hb + off_q);
  for (size_t i = 0; i < qdim; i++) qh[i] = host_f32_to_bf16(h_query[i]);
  e = hipMemcpyAsync(sb, hb, off_out, hipMemcpyHostToDevice, cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "attention upload");
  llh_kv_pool pool{};
  pool.ctx = ctx;
  pool.view = bs.view();
  llh_decode_desc desc{};
  desc.num_seqs = 1;
  desc.num_q_heads = (int32_t)heads;
  desc.max_blocks_per_seq = (int32_t)nb;
  desc.max_seq_len = len;
  desc.window = (int32_t)row_count;  // attends [len - row_count, len): the first row_count logical rows
  desc.total_tokens_hint = (int32_t)row_count;
  desc.d_seq_lens = reinterpret_cast<const int32_t *>(sb);
  desc.d_block_tables = reinterpret_cast<const int32_t *>(sb + off_table);
  int st;
  if (d_w) {
    st = decode_projection_impl(ctx, &pool, &desc, sb + off_q, d_w, w_rows, reinterpret_cast<float *>(sb + off_out),
                                score_scale, cache->stream);
  } else {
    WsLease lease;
    st = paged_decode_impl(ctx, &pool, &desc, sb + off_q, sb + off_out, score_scale, cache->stream, 0, nullptr, lease);
  }
  if (st != LLH_OK) return st;
  e = hipMemcpyAsync(hb + off_out, sb + off_out, out_bytes, hipMemcpyDeviceToHost, cache->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "attention");
  *finite = true;
  if (d_w) {
    std::memcpy(h_output, hb + off_out, out_len * sizeof(float));
  } else {
    const auto *oh = reinterpret_cast<const uint16_t *>(hb + off_out);
    for (size_t i = 0; i < qdim; i++) h_output[i] = host_bf16_to_f32(oh[i]);
  }
  for (size_t i = 0; i < out_len; i++) *finite = *finite && std::isfinite(h_output[i]);
  return LLH_OK;
}

// Attention over the first row_count logical rows of a layer cache, f32 in and
// out.  With d_w != nullptr the f32 attention output is projected on the
// device by W [w_rows][heads * head_dim] bf16 and h_output receives the w_rows
// projected values instead.
static int cache_mix_impl(llh_ctx *ctx, const llh_layer_cache *cache_c, const float *h_query, size_t query_len,
                          size_t row_count, size_t num_attention_heads, size_t num_key_value_heads, size_t head_dim,
                          float score_scale, const void *d_w, int32_t w_rows, float *h_output, size_t output_len) {
  if (!ctx || !cache_c || !h_query || !h_output) return LLH_ERR_NULL;
  auto *cache = const_cast<llh_layer_cache *>(cache_c);
  std::lock_guard<std::mutex> g(cache->mu);
  if (num_attention_heads == 0 || num_key_value_heads == 0 || head_dim == 0 ||
      num_attention_heads % num_key_value_heads != 0)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "invalid attention head shape");
  if (num_key_value_heads != cache->kv_heads || head_dim != cache->head_dim)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "attention shape does not match the KV cache");
  const size_t qdim = num_attention_heads * head_dim;
  if (query_len != qdim) return ctx->fail(LLH_ERR_INVALID_SHAPE, "query length does not match heads * head_dim");
  if (!d_w && output_len < qdim) return ctx->fail(LLH_ERR_INVALID_SHAPE, "attention output buffer too small");
  const size_t out_len = d_w ? (size_t)w_rows : qdim;
  if (row_count > cache->token_count)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "row count exceeds cache token count");
  if (!std::isfinite(score_scale)) return ctx->fail(LLH_ERR_NON_FINITE, "softmax scores must be finite");
  if (row_count == 0) {  // weighted sum of nothing (primitives.rs:1125-1128), projected: still zero
    std::fill(h_output, h_output + out_len, 0.0f);
    return LLH_OK;
  }
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return ctx->hip_fail(e, "hipSetDevice");
  BlockStore &bs = *cache->store;
  std::lock_guard<std::mutex> gs(bs.mu);  // through the stream wait
  if (trait_tuned_ok(ctx, cache, h_query, qdim, num_attention_heads, num_key_value_heads)) {
    bool finite = false;
    const int st = cache_mix_tuned(ctx, cache, h_query, qdim, row_count, num_attention_heads, score_scale, d_w, w_rows,
                                   h_output, out_len, &finite);
    if (st != LLH_OK || finite) {
      if (st == LLH_OK) ctx->trait_tuned_calls++;
      return st;
    }
    // a non-finite output: the reference-order kernel reports the reference's error
  }
  const size_t nb = cache->table.size();
  const size_t off_table = kAlign;                               // int32 [nb]
  const size_t off_q = off_table + align_up(nb * sizeof(int32_t));
  const size_t off_out = off_q + align_up(qdim * sizeof(float));
  const size_t off_scores = off_out + align_up(qdim * sizeof(float));
  const size_t off_proj = off_scores + align_up(num_attention_heads * row_count * sizeof(float));
  const size_t need = off_proj + (d_w ? (size_t)w_rows * sizeof(float) : 0);
  e = cache->scratch.ensure(need, need);
  if (e != hipSuccess) return ctx->hip_fail(e, "scratch allocation");
  char *hb = static_cast<char *>(cache->scratch.host);
  char *sb = static_cast<char *>(cache->scratch.dev);
  // header: err flag, start, end; logical row i is ring slot (window_start + i) % max_tokens
  // (layer.rs:1080-1095), addressed as position window_start + i modulo the ring
  const int32_t hdr[4] = {0, (int32_t)cache->window_start, (int32_t)(cache->window_start + row_count), 0};
  std::memcpy(hb, hdr, sizeof(hdr));
  std::memcpy(hb + off_table, cache->table.data(), nb * sizeof(int32_t));
  std::memcpy(hb + off_q, h_query, qdim * sizeof(float));
  e = hipMemcpyAsync(sb, hb, off_out, hipMemcpyHostToDevice, cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "attention upload");
  GenericDecodeArgs a{};
  a.pool = bs.view();
  a.q = sb + off_q;
  a.out = sb + off_out;
  a.err = reinterpret_cast<int32_t *>(sb);
  a.starts = reinterpret_cast<const int32_t *>(sb) + 1;
  a.seq_lens = reinterpret_cast<const int32_t *>(sb) + 2;
  a.tables = reinterpret_cast<const int32_t *>(sb + off_table);
  a.scores = reinterpret_cast<float *>(sb + off_scores);
  a.num_seqs = 1;
  a.q_heads = (int32_t)num_attention_heads;
  a.max_blocks = (int32_t)nb;
  a.window = 0;
  a.ring_tokens = (int32_t)cache->max_tokens;
  a.score_stride = (int32_t)row_count;
  a.scale = score_scale;
  e = launch_decode_generic(a, 1, 1, cache->stream);
  if (e == hipSuccess && d_w) {
    MatvecArgs m{};
    m.w = static_cast<const uint16_t *>(d_w);
    m.x = sb + off_out;
    m.out = reinterpret_cast<float *>(sb + off_proj);
    m.rows = w_rows;
    m.cols = (int32_t)qdim;
    m.n = 1;
    m.ldx = (int32_t)qdim;
    m.ldo = w_rows;
    m.x_f32 = 1;
    e = launch_matvec_bf16(m, cache->stream);
  }
  const size_t res_off = d_w ? off_proj : off_out;
  if (e == hipSuccess) e = hipMemcpyAsync(hb, sb, sizeof(int32_t), hipMemcpyDeviceToHost, cache->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(hb + res_off, sb + res_off, out_len * sizeof(float), hipMemcpyDeviceToHost, cache->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "attention");
  int32_t flags = 0;
  std::memcpy(&flags, hb, sizeof(flags));
  std::memcpy(h_output, hb + res_off, out_len * sizeof(float));
  ctx->decode_calls++;
  if (flags & kErrNonFinite) return ctx->fail(LLH_ERR_NON_FINITE, "softmax scores must be finite");
  if (flags & kErrBadBlock) return ctx->fail(LLH_ERR_STALE, "KV cache block table is stale");
  return LLH_OK;
}


extern "C" {

int llh_full_attention_cache_mix_f32_in_place(llh_ctx *ctx, const llh_layer_cache *cache_c, const float *h_query,
                                              size_t query_len, size_t row_count, size_t num_attention_heads,
                                              size_t num_key_value_heads, size_t head_dim, float score_scale,
                                              float *h_output, size_t output_len) {
  return cache_mix_impl(ctx, cache_c, h_query, query_len, row_count, num_attention_heads, num_key_value_heads,
                        head_dim, score_scale, nullptr, 0, h_output, output_len);
}

// full_attention_cache_mix_bf16_output_projection_f32_in_place
// (crates/llm-backend/src/core/native_matvec.rs:671-685; Metal form
// crates/llm-native-runtime/src/native_matvec.rs:4418-4492): shapes the fused
// path does not take return LLH_NOT_HANDLED (the trait's Ok(false)).
int llh_full_attention_cache_mix_bf16_output_projection_f32_in_place(
    llh_ctx *ctx, const llh_layer_cache *cache_c, const float *h_query, size_t query_len, size_t row_count,
    size_t num_attention_heads, size_t num_key_value_heads, size_t head_dim, float score_scale, const void *d_w_o,
    int32_t w_rows, int32_t w_cols, float *h_output, size_t output_len) {
  if (!ctx || !cache_c || !h_query || !h_output || !d_w_o) return LLH_ERR_NULL;
  const size_t attention_dim = num_attention_heads * head_dim;
  if (w_rows <= 0 || w_cols <= 0 || (size_t)w_cols != attention_dim || output_len < (size_t)w_rows ||
      w_cols % kMatvecColsMultiple != 0 || !aligned16(d_w_o)) {
    ctx->not_handled++;
    return LLH_NOT_HANDLED;
  }
  return cache_mix_impl(ctx, cache_c, h_query, query_len, row_count, num_attention_heads, num_key_value_heads,
                        head_dim, score_scale, d_w_o, w_rows, h_output, output_len);
}

int llh_select_kv_cache_head_rows_f32_in_place(llh_ctx *ctx, const llh_layer_cache *cache_c, int32_t tensor,
                                               size_t row_count, size_t head_start, size_t head_len,
                                               float *h_output, size_t output_len) {
  if (!ctx || !cache_c || !h_output) return LLH_ERR_NULL;
  auto *cache = const_cast<llh_layer_cache *>(cache_c);
  std::lock_guard<std::mutex> g(cache->mu);
  const size_t vl = cache->vector_len();
  if (tensor != 0 && tensor != 1) return ctx->fail(LLH_ERR_INVALID_SHAPE, "tensor must be 0 (key) or 1 (value)");
  if (row_count > cache->token_count)
    return ctx->fail(LLH_ERR_INVALID_SHAPE, "head row selection row count exceeds the cache");
  if (head_start + head_len > vl) return ctx->fail(LLH_ERR_INVALID_SHAPE, "head row selection range exceeds row length");
  if (output_len < row_count * head_len) return ctx->fail(LLH_ERR_INVALID_SHAPE, "head row selection output buffer too small");
  if (row_count == 0 || head_len == 0) return LLH_OK;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return ctx->hip_fail(e, "hipSetDevice");
  BlockStore &bs = *cache->store;
  std::lock_guard<std::mutex> gs(bs.mu);  // through the stream wait
  const size_t nb = cache->table.size();
  const size_t off_table = kAlign;
  const size_t off_out = off_table + align_up(nb * sizeof(int32_t));
  const size_t out_bytes = row_count * vl * sizeof(float);
  e = cache->scratch.ensure(off_out + out_bytes, off_out + out_bytes);
  if (e != hipSuccess) return ctx->hip_fail(e, "scratch allocation");
  char *hb = static_cast<char *>(cache->scratch.host);
  char *sb = static_cast<char *>(cache->scratch.dev);
  const int32_t zero = 0;
  std::memcpy(hb, &zero, sizeof(zero));
  std::memcpy(hb + off_table, cache->table.data(), nb * sizeof(int32_t));
  e = hipMemcpyAsync(sb, hb, off_out, hipMemcpyHostToDevice, cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "upload");
  // logical row i is ring slot (window_start + i) % max_tokens (layer.rs:1080-1095)
  const int64_t abs_start = (int64_t)cache->window_start;
  GatherArgs a{};
  a.pool = bs.view();
  a.table = reinterpret_cast<const int32_t *>(sb + off_table);
  a.max_blocks = (int32_t)nb;
  a.lo = (int32_t)abs_start;
  a.hi = (int32_t)(abs_start + (int64_t)row_count);
  a.tensor = tensor;
  a.ring_tokens = (int32_t)cache->max_tokens;
  a.out = sb + off_out;
  a.out_f32 = 1;
  a.err = reinterpret_cast<int32_t *>(sb);
  e = launch_gather(a, cache->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(hb + off_out, sb + off_out, out_bytes, hipMemcpyDeviceToHost, cache->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(cache->stream);
  if (e != hipSuccess) return ctx->hip_fail(e, "select head rows");
  const float *rows = reinterpret_cast<const float *>(hb + off_out);
  for (size_t r = 0; r < row_count; r++)
    std::memcpy(h_output + r * head_len, rows + r * vl + head_start, head_len * sizeof(float));
  return LLH_OK;
}

}  // extern "C"
