/*
 * llm_hip.h -- C ABI of the MI355X (gfx950) attention-over-KV-cache library.
 *
 * This is the drop-in boundary for kir-ai's accelerated attention path.  In the
 * reference, the per-layer attention calls cross the `NativeMatvecBackend`
 * trait (crates/llm-backend/src/core/native_matvec.rs:222-769) into the Metal
 * implementation (crates/llm-native-runtime/src/native_matvec.rs:3026-4566).
 * A Rust shim binds the functions below with `extern "C"` and adds a
 * `NativeTextMatvecBackend::Hip` arm that forwards the trait methods here.
 *
 * Conventions
 *   - Every function returns an int status (llh_status); none aborts.
 *   - Pointers named `d_*` are device pointers; `h_*` are host pointers.
 *   - Batched entry points are asynchronous on the given stream (hipStream_t
 *     passed as void*, NULL = the null stream).  Each stream gets its own
 *     device workspace inside the context (split partials, merge descriptors,
 *     projection staging), allocated by the stream's first call and grown when
 *     a call needs more; a stream whose workspace is large enough allocates
 *     nothing (llh_ctx_reserve_stream_workspace sizes it ahead of time).
 *   - Trait-mirror entry points (llh_layer_cache_*, llh_full_attention_*,
 *     llh_append_kv_cache_*) are synchronous, like the reference's awaited
 *     command buffers (crates/llm-metal/src/device/primitives.rs:1325-1338):
 *     each layer cache owns a stream and waits for that stream only.
 *   - Threading (the reference shares one backend process-wide and calls its
 *     &self methods concurrently, crates/llm-native-runtime/src/native_matvec.rs:2787-2819):
 *     a context may be used from several threads at once.  Batched calls on
 *     distinct streams never share device scratch memory; calls on one stream
 *     from several threads are serialised by that stream's workspace lock.
 *     Layer caches and block pools lock themselves; the caches and clones that
 *     share device blocks are serialised on those blocks.  Pools and
 *     descriptors passed to concurrent calls must not be written meanwhile.
 */
#ifndef LLM_HIP_H
#define LLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLH_ABI_VERSION 6  /* 6: head_dim-256 kernels, llh_metrics.d256_decode_calls / generic_decode_calls,
                              gate fields, LLH_KV_F16;
                              5: per-stream device error words, llh_layer_cache_create_from_rows;
                              4: int8 and fp8 pools store their scales as (K, V) pairs */

/* Status codes.  Mirrors MathError / KvCacheError
 * (crates/llm-backend/src/core/math.rs:10-15, crates/llm-kv-cache/src/lib.rs). */
typedef enum llh_status {
  LLH_OK = 0,
  /* "not handled": the Ok(false) of full_attention_cache_mix_f32_in_place
   * (native_matvec.rs:656-668); the caller runs its own per-head path. */
  LLH_NOT_HANDLED = 1,
  LLH_ERR_INVALID_SHAPE = -1, /* MathError::InvalidShape / KvCacheError::InvalidShape */
  LLH_ERR_CAPACITY = -2,      /* KvCacheError::CapacityExceeded */
  LLH_ERR_NON_FINITE = -3,    /* "softmax scores must be finite" (math.rs:485-489), NonFiniteValue */
  LLH_ERR_UNSUPPORTED = -4,   /* KvCacheError::UnsupportedFormat */
  LLH_ERR_DEVICE = -5,        /* HIP runtime failure: caller may record a fallback (native_matvec.rs:2979-2999) */
  LLH_ERR_STALE = -6,         /* block id / revision mismatch (layer.rs:1001-1009) */
  LLH_ERR_NULL = -7,          /* NULL handle or pointer */
  LLH_ERR_INTEGRITY = -8      /* NativeTextDiskCacheError::Integrity (native_text/disk_cache.rs:262-270) */
} llh_status;

/* KV storage formats (crates/llm-kv-cache/src/format.rs:5-21 plus the two
 * quantised device layouts of this build). */
typedef enum llh_kv_format {
  LLH_KV_BF16 = 0,    /* bf16 K and V */
  LLH_KV_INT8 = 1,    /* int8 codes, fp16 scale per (token, kv head): absmax/127 */
  LLH_KV_FP8_E4M3 = 2, /* OCP e4m3fn codes, f32 scale per (block, kv head) for K and for V: absmax/448 */
  LLH_KV_INT8_ROW = 3, /* int8 codes, f32 scale per token row over all kv heads: absmax/127 -- the
                          reference's own int8 layout (crates/llm-kv-cache/src/format.rs:702-759);
                          served by the element-wise kernels */
  LLH_KV_F16 = 4       /* IEEE fp16 K and V: the dtype of the reference's Metal mirror
                          (attention_scores_f16, crates/llm-metal/src/device/shaders/generic.metal:89-118;
                          KvCacheFormat::F16, format.rs:69-120).  Rows are rounded to nearest even;
                          a value beyond the fp16 range is stored as an infinity (as a float -> half
                          conversion does).  The tuned decode and prefill kernels compute q . k on
                          fp16 with each query head (prefill: each query row) scaled into fp16 by a
                          power of two: elements within 2^-28 of the largest |q| are exact, smaller
                          ones err by under 2^-38 of it; softmax weights enter p . v as fp16.  Device
                          pools only: a layer cache of this format is UNSUPPORTED, as
                          LayerKvCache::new_with_config refuses it (layer.rs:399-403) */
} llh_kv_format;

typedef struct llh_ctx llh_ctx;
typedef struct llh_kv_pool llh_kv_pool;
typedef struct llh_layer_cache llh_layer_cache;

/* ------------------------------------------------------------------ */
/* context                                                            */
/* ------------------------------------------------------------------ */

/* Creates a context on HIP device `device`.  Replaces NativeTextMatvecBackend::
 * system_default (crates/llm-native-runtime/src/native_matvec.rs:2823-2832). */
int llh_ctx_create(int device, llh_ctx **out);
int llh_ctx_destroy(llh_ctx *ctx);
/* Message of the last error on this context (like MathError's String); never
 * NULL.  The returned string is the calling thread's copy: it stays valid
 * until this thread's next llh_ctx_last_error call. */
const char *llh_ctx_last_error(const llh_ctx *ctx);
/* Sets the minimum workspace size of every stream of this context (existing
 * ones grow now; a new stream's first call allocates at least this much). */
int llh_ctx_reserve_workspace(llh_ctx *ctx, size_t bytes);
/* Allocates (or grows) the workspace of one stream now, so that its batched
 * calls of at most this size allocate nothing. */
int llh_ctx_reserve_stream_workspace(llh_ctx *ctx, void *stream, size_t bytes);
/* Frees one stream's workspace (after waiting for the device).  Call it before
 * destroying a stream that made batched calls on this context. */
int llh_ctx_release_stream(llh_ctx *ctx, void *stream);

/* Tuning options.  Their initial values come from the environment at
 * llh_ctx_create (the names in parentheses; unset = 0 = automatic) and are
 * never read from it again. */
typedef enum llh_option {
  LLH_OPT_DECODE_KERNEL = 0,         /* (LLH_DECODE_KERNEL: "split" = 1, "stream" = 2) 0 = by step size */
  LLH_OPT_DECODE_SPLIT_BLOCKS = 1,   /* (LLH_DECODE_SPLIT_BLOCKS) blocks per split-K split, 0 = planned */
  LLH_OPT_DECODE_STREAM_WGS = 2,     /* (LLH_DECODE_STREAM_WGS) stream-kernel workgroups, 0 = 2 per CU */
  LLH_OPT_FORCE_GENERIC = 3,         /* (LLH_FORCE_GENERIC) 1 = the element-wise decode and prefill
                                        kernels for every shape */
  LLH_OPT_PREFILL_HEADS_PER_WG = 4,  /* (LLH_PREFILL_HEADS_PER_WG) 1 = one query head per prefill workgroup */
  LLH_OPT_TRAIT_REFERENCE_ORDER = 5, /* (LLH_TRAIT_REFERENCE_ORDER) trait-mirror attention: 0 = the tuned
                                        kernels where the shape allows, 1 = the reference-order kernel always */
  LLH_OPT_COUNT = 6
} llh_option;
int llh_ctx_set_option(llh_ctx *ctx, int32_t option, int32_t value);
int llh_ctx_get_option(const llh_ctx *ctx, int32_t option, int32_t *value);
/* Workspace bytes a llh_paged_decode call with these bounds needs (any head_dim up to 256). */
size_t llh_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len);
/* Fallback/attempt counters, as MetalBackendMetrics' attention counters
 * (crates/llm-native-runtime/src/native_metrics.rs:73-112). */
typedef struct llh_metrics {
  uint64_t decode_calls;
  uint64_t prefill_calls;
  uint64_t append_calls;
  uint64_t not_handled;
  uint64_t device_errors;
  uint64_t shape_errors;
  uint64_t stream_decode_calls; /* decode calls that ran the persistent stream kernel */
  uint64_t trait_tuned_calls;   /* trait-mirror attention calls served by the tuned decode kernels */
  uint64_t generic_prefill_calls; /* prefill calls that ran the element-wise kernel */
  uint64_t fused_append_calls;    /* llh_paged_decode_append calls served by one launch */
  uint64_t stream_slots;          /* streams holding a workspace slot (scratch and error word) now */
  uint64_t workspace_bytes;       /* device bytes of those slots' scratch now */
  uint64_t d256_decode_calls;     /* decode calls that ran the head_dim-256 kernel */
  uint64_t generic_decode_calls;  /* llh_paged_decode* calls that ran the element-wise kernel */
} llh_metrics;
int llh_ctx_metrics(const llh_ctx *ctx, llh_metrics *out);
/* Sticky error flags the batched kernels raise instead of faulting: 1 = a
 * block table entry outside the pool, 2 = a sequence longer than the call's
 * max_seq_len allows, 4 = a non-finite value (score, or a row given to an
 * int8 write / append), 8 = a sequence's attended span needs more blocks than
 * its block-table row holds (the row is read modulo its length, so the span
 * would alias its own blocks).  Each stream has its own flag word (the calls
 * made on it raise flags there; MetalBackendMetrics records fallbacks per
 * call in the reference, native_metrics.rs:81-112), created with the stream's
 * workspace slot; calls that cannot have one (llh_paged_decode_noalloc on a
 * stream without a slot, a stream under graph capture without one) use the
 * context's word.
 * llh_ctx_device_errors waits for the whole device and returns the OR of every
 * word (the context's, every stream's, and those of released streams),
 * optionally clearing them all. */
int llh_ctx_device_errors(llh_ctx *ctx, int32_t *flags, int32_t reset);
/* One stream's flags: waits for that stream only, then reads (and optionally
 * clears) the word of the calls made on it; 0 for a stream that has none. */
int llh_ctx_stream_device_errors(llh_ctx *ctx, void *stream, int32_t *flags, int32_t reset);
/* Kernel timing for measurement: while enabled, each llh_paged_decode /
 * llh_paged_prefill call records a pair of HIP events on its stream around its
 * main kernel (the split-K or stream decode kernel, not the merge; the prefill
 * kernel).
 * llh_ctx_kernel_time waits for the recorded events and returns the summed
 * duration and count for kind 0 = decode, 1 = prefill (reset clears them). */
int llh_ctx_set_kernel_timing(llh_ctx *ctx, int32_t enable);
int llh_ctx_kernel_time(llh_ctx *ctx, int32_t kind, double *total_ms, int64_t *count, int32_t reset);

/* ------------------------------------------------------------------ */
/* paged KV pool (device resident)                                    */
/* ------------------------------------------------------------------ */
/*
 * One pool holds one layer's K and V for many sequences in fixed-size blocks
 * (crates/llm-kv-cache/src/block_pool.rs:159-171 makes block size a pool
 * parameter).  Device layout, block b, kv head h:
 *   K  [n_blocks][kv_heads][block_tokens][head_dim]   token rows
 *   V  [n_blocks][kv_heads][head_dim][block_tokens]   dim rows (transposed)
 *   int8 scales: fp16 [n_blocks][kv_heads][block_tokens][2] in one allocation:
 *                per token the pair (K scale, V scale), so a decode lane reads
 *                its token's two scales with one 4-byte load
 *                (d_v_scales = d_k_scales + 2 bytes; both have a stride of
 *                4 bytes per token)
 *   fp8 scales : f32  [n_blocks][kv_heads][2] in one allocation: the pair
 *                (K scale, V scale) of (block, head), one 8-byte load per
 *                decode unit (d_v_scales = d_k_scales + 4 bytes; both have a
 *                stride of 8 bytes per (block, head))
 *   int8 row scales (LLH_KV_INT8_ROW): f32 [n_blocks][block_tokens] for K and for V
 * Position p of a sequence lives in block_table[(p / block_tokens) % max_blocks]
 * at offset p % block_tokens.  The modulus lets a ring of blocks serve a
 * sliding window (crates/llm-kv-cache/src/layer.rs:765-805).
 */
typedef struct llh_kv_pool_info {
  int32_t format;
  int32_t block_tokens;
  int32_t kv_heads;
  int32_t head_dim;
  int64_t n_blocks;
  void *d_k;
  void *d_v;
  void *d_k_scales; /* NULL for bf16 */
  void *d_v_scales; /* NULL for bf16; int8, fp8: inside d_k_scales' allocation (see above) */
  size_t k_bytes;   /* bytes of d_k (and of d_v) */
  size_t scale_bytes; /* bytes of the K (and of the V) scales; int8, fp8: the allocation at
                         d_k_scales holds both, 2 * scale_bytes, as (K, V) pairs */
} llh_kv_pool_info;

int llh_kv_pool_create(llh_ctx *ctx, int32_t format, int32_t block_tokens, int32_t kv_heads,
                       int32_t head_dim, int64_t n_blocks, llh_kv_pool **out);
int llh_kv_pool_destroy(llh_kv_pool *pool);
int llh_kv_pool_get_info(const llh_kv_pool *pool, llh_kv_pool_info *out);

/* Writes whole blocks, quantising on write.  Replaces the block re-quantisation
 * of LayerInt8KvStore::update_block (crates/llm-kv-cache/src/format.rs:262-276)
 * and the Metal f32->f16 block upload (native_matvec.rs:384-465).
 *   d_blocks [n] pool block indices; d_k, d_v [n][block_tokens][kv_heads][head_dim] bf16.
 * int8: per (token, head) scale = f16(absmax/127), codes with the rounded scale.
 * fp8 : per (block, head) scale = absmax/448 over the block's tokens. */
int llh_kv_write_blocks(llh_ctx *ctx, llh_kv_pool *pool, const int32_t *d_blocks, const void *d_k,
                        const void *d_v, int32_t n, void *stream);

/* Appends token rows at absolute slots (block * block_tokens + offset),
 * quantising on write for int8.  Replaces append_kv_cache_sliding_f32
 * (native_matvec.rs:643-653) and the Metal direct f16/int8 append
 * (crates/llm-native-runtime/src/native_matvec.rs:575-943).
 *   d_slots [n] int64; d_k, d_v [n][kv_heads][head_dim] bf16.
 * fp8 pools (one scale per (block, head) and tensor) re-quantise the block as
 * each token arrives, as the reference re-quantises a block on every int8 append
 * (crates/llm-kv-cache/src/layer.rs:1396-1408): the scale becomes
 * max(old, absmax(row) / 448) and, when it grows, the block's tokens before the
 * new one are re-encoded from their dequantised values; a token at offset 0
 * starts the block afresh.  Tokens of one block in one call are appended in
 * call order.  (So a window ring of fp8 blocks needs window/block_tokens + 1
 * blocks: the offset-0 token must not share its block with live tokens.) */
int llh_kv_append(llh_ctx *ctx, llh_kv_pool *pool, const int64_t *d_slots, const void *d_k,
                  const void *d_v, int32_t n, void *stream);
/* llh_kv_append from f32 rows (d_k, d_v [n][kv_heads][head_dim] f32): the
 * restore side of a disk block, whose tensors are f32 (codec.rs:72-99); the
 * bf16 rounding is round-to-nearest-even, so rows exported from a bf16 pool
 * come back bit for bit. */
int llh_kv_append_f32(llh_ctx *ctx, llh_kv_pool *pool, const int64_t *d_slots, const float *d_k,
                      const float *d_v, int32_t n, void *stream);

/* ------------------------------------------------------------------ */
/* batched paged attention (the hot path)                             */
/* ------------------------------------------------------------------ */

/* Per-step decode descriptor.  The reference calls attention once per sequence
 * (crates/llm-server/src/engine/scheduler.rs:579-712 admits, it does not batch);
 * this descriptor batches one step of many sequences. */
typedef struct llh_decode_desc {
  int32_t num_seqs;
  int32_t num_q_heads;        /* Hq; kv heads come from the pool; Hq % Hkv == 0 */
  int32_t max_blocks_per_seq; /* row stride of d_block_tables */
  int32_t max_seq_len;        /* host-known bound on d_seq_lens (sizes the grid) */
  int32_t window;             /* 0 = full attention; else attend [max(0, len - window), len) */
  int32_t total_tokens_hint;  /* host-known sum of attended tokens (sizes split-K); 0 = unknown */
  const int32_t *d_seq_lens;     /* [num_seqs] tokens incl. the new one (appended first, native_attention.rs:307-309) */
  const int32_t *d_block_tables; /* [num_seqs][max_blocks_per_seq] pool block indices */
  /* NULL, or the attention output gate of Qwen3.5 / 3.6 (attn_output_gate), bf16
   * [num_seqs][num_q_heads][head_dim]: out = attention * sigmoid(gate) element-wise, in f32
   * before the output's bf16 rounding (apply_attention_gate, native_attention.rs:765-781). */
  const void *d_gate;
} llh_decode_desc;

/* One decode step: out[b][h] = softmax(scale * q[b][h] . K^T) V over the
 * sequence's attended positions, GQA kv head = h / (Hq / Hkv)
 * (native_attention.rs:707-773).  d_q, d_out: [num_seqs][Hq][head_dim] bf16. */
int llh_paged_decode(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_q,
                     void *d_out, float score_scale, void *stream);

/* kir-ai's decode step, append then attend (native_attention.rs:307-329), in one
 * call: the same result as llh_kv_append of each sequence's new token, at position
 * d_seq_lens[b] - 1 through its block-table row, followed by llh_paged_decode.
 * d_k_new, d_v_new: [num_seqs][kv_heads][head_dim] bf16 (sequences with
 * d_seq_lens[b] == 0 have none).  bf16 pools on the tuned kernels run it as one
 * launch: the new token is attended from d_k_new / d_v_new and written to its slot
 * by the wavefront that computes the sequence's last block; other pools (the
 * quantised token must be attended as stored) and shapes run the append kernel,
 * then the decode.  The pool is written: unlike llh_paged_decode, concurrent calls
 * must not share the sequences' last blocks. */
int llh_paged_decode_append(llh_ctx *ctx, llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_k_new,
                            const void *d_v_new, const void *d_q, void *d_out, float score_scale, void *stream);

/* llh_paged_decode without any allocation.  No counterpart in the reference:
 * this entry point is for callers that cannot allocate -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  The step's
 * split partials and merge descriptors live in a static device array of the
 * library (LLH_NOALLOC_SCRATCH_BYTES per GPU, held by every GPU the library
 * runs on until the process ends) instead of the stream's workspace; it calls
 * no hipMalloc/hipFree and creates no events (kernel timing does not see it).
 * Same arguments, kernels and results as llh_paged_decode.  A step whose plan
 * needs more scratch than the array holds returns LLH_ERR_CAPACITY (use
 * llh_paged_decode).  All calls on one GPU share the array: calls that overlap
 * on one GPU (other streams, other threads) race on it. */
#define LLH_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int llh_paged_decode_noalloc(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, const void *d_q,
                             void *d_out, float score_scale, void *stream);

/* Chunked prefill over cached prefix blocks.  Sequence b owns query rows
 * [d_chunk_starts[b], d_chunk_starts[b+1]); its context holds d_context_lens[b]
 * tokens (prefix + the chunk, whose K/V are already in the pool).  Row i sits
 * at position context_len - chunk_len + i and attends [lo, pos], lo = window ?
 * pos - window + 1 : 0 (native_attention.rs:356-464: append then attend). */
typedef struct llh_prefill_desc {
  int32_t num_seqs;
  int32_t num_q_heads;
  int32_t max_blocks_per_seq;
  int32_t window;
  int32_t total_q_rows;   /* d_chunk_starts[num_seqs] */
  int32_t max_chunk_len;  /* host-known bound (sizes the grid) */
  const int32_t *d_chunk_starts; /* [num_seqs + 1] */
  const int32_t *d_context_lens; /* [num_seqs] */
  const int32_t *d_block_tables; /* [num_seqs][max_blocks_per_seq] */
  const void *d_gate;            /* NULL, or bf16 [total_q_rows][num_q_heads][head_dim]: out = attention *
                                    sigmoid(gate), as llh_decode_desc.d_gate */
} llh_prefill_desc;

/* d_q, d_out: [total_q_rows][Hq][head_dim] bf16 (2-byte aligned).  Every pool
 * format: int8 / fp8 blocks are dequantised, so the result is attention over
 * the dequantised cache (layer.rs:650-656).  head_dim 128 with 16-token blocks
 * and 16-byte aligned rows runs the MFMA kernel (codes * scale rounded to bf16
 * as the key/value tiles are staged); every other shape with head_dim <= 512
 * runs an element-wise kernel (sequential f32 dot products, online softmax in
 * f32); head_dim > 512 returns LLH_ERR_UNSUPPORTED. */
int llh_paged_prefill(llh_ctx *ctx, const llh_kv_pool *pool, const llh_prefill_desc *desc, const void *d_q,
                      void *d_out, float score_scale, void *stream);

/* Output projection after attention, on the device: the batched form of
 * bf16_matvecs_row_major_f32_flat_inputs (native_matvec.rs:264-272) with the
 * reference's per-row dot (crates/llm-backend/src/core/safetensors/math.rs:66-72).
 * out[i][r] = sum_c W[r][c] * x[i][c]; W bf16 [rows][cols] row-major, x [n][cols]
 * bf16 (x_f32 = 0) or f32 (x_f32 = 1, rounded to bf16 for the MFMA), out f32
 * [n][rows], f32 accumulation.  cols must be a multiple of 128 and W, x 16-byte
 * aligned, else LLH_ERR_UNSUPPORTED. */
int llh_matvec_bf16_f32(llh_ctx *ctx, const void *d_w, int32_t rows, int32_t cols, const void *d_x, int32_t x_f32,
                        int32_t n, float *d_out, void *stream);

/* full_attention_cache_mix_bf16_output_projection_f32_in_place
 * (native_matvec.rs:671-685), batched: one llh_paged_decode step whose bf16
 * attention output stays in the context workspace, then out[b] = W_o attn[b]
 * on the same stream.  W_o bf16 [rows][num_q_heads * head_dim]; out f32
 * [num_seqs][rows]. */
int llh_paged_decode_output_projection(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc,
                                       const void *d_q, const void *d_w_o, int32_t rows, float *d_out,
                                       float score_scale, void *stream);

/* Bit-exact gather of positions [lo, hi) of sequence `seq` through its block
 * table into d_out [hi-lo][kv_heads][head_dim] raw elements (2 bytes bf16,
 * 1 byte int8/fp8); tensor 0 = K, 1 = V.  The gather half of
 * select_kv_cache_head_rows_f32_in_place (native_matvec.rs:619-641) and of
 * select_head_rows_* (crates/llm-metal/src/device/shaders/generic.metal:310-360). */
int llh_debug_gather(llh_ctx *ctx, const llh_kv_pool *pool, const llh_decode_desc *desc, int32_t seq,
                     int32_t lo, int32_t hi, int32_t tensor, void *d_out, void *stream);

/* Decodes `n` raw fp8 e4m3 codes with the kernels' own conversion (f32 out). */
int llh_debug_decode_fp8(llh_ctx *ctx, const uint8_t *d_codes, float *d_out, int32_t n, void *stream);

/* Runs the kernels' fp8 e4m3 encoder (the hardware conversion) and the integer
 * reference rule on every f32 bit pattern but NaNs and stores how many codes differ
 * (a test hook, no reference counterpart; synchronous, allocates 8 bytes). */
int llh_debug_fp8_encode_check(llh_ctx *ctx, uint64_t *h_mismatches);

/* ------------------------------------------------------------------ */
/* trait mirror: LayerKvCache + NativeMatvecBackend attention hooks    */
/* ------------------------------------------------------------------ */

/* LayerKvCache::new_with_config (crates/llm-kv-cache/src/layer.rs:345-400):
 * a ring of `max_tokens` token slots whose storage is paged device blocks.
 * format: LLH_KV_BF16 (the reference's f32 rows are stored as bf16),
 * LLH_KV_INT8 (per (token, head) fp16 scales; the tuned kernels) or
 * LLH_KV_INT8_ROW (the reference's KvCacheFormat::Int8 bit for bit: one f32
 * scale per token row, quantised from the f32 rows; the reference-order
 * kernel).  Errors as the reference: zero sizes -> INVALID_SHAPE, fp8 ->
 * UNSUPPORTED. */
int llh_layer_cache_create(llh_ctx *ctx, size_t max_tokens, size_t kv_heads, size_t head_dim, int32_t format,
                           llh_layer_cache **out);
/* Also releases the workspace slot of the cache's own stream. */
int llh_layer_cache_destroy(llh_layer_cache *cache);

/* A device mirror of a host LayerKvCache that already holds rows:
 * LayerKvCache::from_snapshot (crates/llm-kv-cache/src/layer.rs:467-507, with
 * window_start = 0) and from_prefix_cache_state (layer.rs:544-581) -- the
 * caches the driver restores on a prefix-cache hit
 * (crates/llm-native-runtime/src/native_text/driver.rs:694-703).  The rows are
 * the cache's logical rows (keys() / values(), layer.rs:1046-1052): logical row
 * i goes to ring slot (window_start + i) % max_tokens, stored as appending it
 * would store it (bf16 rounding, int8 quantisation).  The new cache has a
 * fresh id and block ids, and the given revision, token count, tokens seen
 * and window start, so its state and active_blocks() are those of the host
 * cache.  Errors as the reference: a state failing from_prefix_cache_state's
 * checks (zero sizes, token_count > max_tokens, tokens_seen < token_count,
 * window_start >= max_tokens) or rows of the wrong length -> INVALID_SHAPE,
 * non-finite rows of an int8 cache -> NON_FINITE, fp8 -> UNSUPPORTED. */
typedef struct llh_layer_cache_rows {
  uint64_t max_tokens;
  uint64_t kv_heads;
  uint64_t head_dim;
  int32_t format;         /* LLH_KV_BF16, LLH_KV_INT8 or LLH_KV_INT8_ROW */
  uint64_t revision;      /* revision() */
  uint64_t token_count;   /* token_count() */
  uint64_t tokens_seen;   /* next_position() */
  uint64_t window_start;  /* physical slot of logical token 0: active_blocks()[0].physical_token_start() */
  const float *h_keys;    /* [token_count][kv_heads * head_dim] f32 host rows, logical order */
  const float *h_values;
  size_t keys_len;        /* elements of h_keys and of h_values: token_count * kv_heads * head_dim */
} llh_layer_cache_rows;
int llh_layer_cache_create_from_rows(llh_ctx *ctx, const llh_layer_cache_rows *rows, llh_layer_cache **out);
/* Clone with a fresh cache id that shares blocks until written (layer.rs:237-259, block.rs:124-130). */
int llh_layer_cache_clone(const llh_layer_cache *cache, llh_layer_cache **out);
/* clear() (layer.rs:1068-1086) */
int llh_layer_cache_clear(llh_layer_cache *cache);

typedef struct llh_layer_cache_state {
  uint64_t id;            /* LayerKvCache::id() */
  uint64_t revision;      /* revision() */
  uint64_t max_tokens;
  uint64_t kv_heads;
  uint64_t head_dim;
  uint64_t token_count;   /* token_count() */
  uint64_t tokens_seen;   /* next_position() */
  uint64_t window_start;  /* physical slot of logical token 0 */
  uint64_t block_count;   /* device blocks backing the ring */
  int32_t format;
  int32_t block_tokens;
} llh_layer_cache_state;
int llh_layer_cache_get_state(const llh_layer_cache *cache, llh_layer_cache_state *out);

/* LayerKvCacheBlockRun / active_blocks() (layer.rs:158-207,972-1044): runs of
 * logical tokens that are contiguous in one device block. */
typedef struct llh_block_run {
  uint64_t block_id;            /* BlockId (0 = invalid, block_id.rs:11-41) */
  uint64_t block_index;         /* index in the cache's block table */
  uint64_t logical_token_start;
  uint64_t physical_token_start;
  uint64_t block_token_start;
  uint64_t token_count;
} llh_block_run;
int llh_layer_cache_active_blocks(const llh_layer_cache *cache, llh_block_run *h_out, size_t capacity,
                                  size_t *count);
/* block_ids() (layer.rs:954-956) */
int llh_layer_cache_block_ids(const llh_layer_cache *cache, uint64_t *h_out, size_t capacity, size_t *count);

/* NativeMatvecBackend::append_kv_cache_sliding_f32 (native_matvec.rs:643-653):
 * ring append; once full, overwrites the oldest slot (layer.rs:765-805).
 * h_key, h_value: [kv_heads * head_dim] f32 host rows. */
int llh_append_kv_cache_sliding_f32(llh_ctx *ctx, llh_layer_cache *cache, const float *h_key,
                                    const float *h_value, size_t len);
/* LayerKvCache::append (strict; capacity error when full, layer.rs:744-763). */
int llh_append_kv_cache_f32(llh_ctx *ctx, llh_layer_cache *cache, const float *h_key, const float *h_value,
                            size_t len);

/* NativeMatvecBackend::full_attention_cache_mix_f32_in_place
 * (native_matvec.rs:656-668): attends the first `row_count` logical rows.
 * h_query [num_attention_heads * head_dim], h_output [>= same] f32 host.
 * Returns LLH_OK when handled, LLH_NOT_HANDLED for shapes the device path
 * does not take, or an error (shape errors as primitives.rs:1113-1128). */
int llh_full_attention_cache_mix_f32_in_place(llh_ctx *ctx, const llh_layer_cache *cache, const float *h_query,
                                              size_t query_len, size_t row_count, size_t num_attention_heads,
                                              size_t num_key_value_heads, size_t head_dim, float score_scale,
                                              float *h_output, size_t output_len);

/* NativeMatvecBackend::full_attention_cache_mix_bf16_output_projection_f32_in_place
 * (native_matvec.rs:671-685; Metal form crates/llm-native-runtime/src/native_matvec.rs:4418-4492):
 * attention as above, then the o_proj matvec on the device.  d_w_o: device bf16
 * [w_rows][w_cols] (the safetensors tensor, uploaded once by the caller).
 * h_output receives w_rows f32 values.  LLH_NOT_HANDLED (the trait's Ok(false))
 * when w_cols != heads * head_dim, output_len < w_rows, or w_cols is not a
 * multiple of 128. */
int llh_full_attention_cache_mix_bf16_output_projection_f32_in_place(
    llh_ctx *ctx, const llh_layer_cache *cache, const float *h_query, size_t query_len, size_t row_count,
    size_t num_attention_heads, size_t num_key_value_heads, size_t head_dim, float score_scale, const void *d_w_o,
    int32_t w_rows, int32_t w_cols, float *h_output, size_t output_len);

/* NativeMatvecBackend::select_kv_cache_head_rows_f32_in_place
 * (native_matvec.rs:619-641): rows [0, row_count) of one head slice
 * [head_start, head_start + head_len) of the row vector, as f32. */
int llh_select_kv_cache_head_rows_f32_in_place(llh_ctx *ctx, const llh_layer_cache *cache, int32_t tensor,
                                               size_t row_count, size_t head_start, size_t head_len,
                                               float *h_output, size_t output_len);

/* ------------------------------------------------------------------ */
/* paged block allocator: BlockPool, session block tables, prefixes   */
/* ------------------------------------------------------------------ */
/*
 * kir-ai's BlockPool (crates/llm-kv-cache/src/block_pool.rs:38-318,344-896)
 * over the blocks of a device KV pool: block i of the allocator is block i of
 * the llh_kv_pool, so session tables map straight to the int32 rows of
 * llh_decode_desc / llh_prefill_desc.  Every entry point takes the pool's
 * mutex.  Functions that return Option / bool in the reference report through
 * an out parameter (0 id = None; 0/1 flag) and return LLH_OK.
 */
typedef struct llh_block_pool llh_block_pool;

/* SHA-256 (FIPS 180-4) of a byte string. */
int llh_sha256(const void *data, size_t len, uint8_t out[32]);
/* cache_block_chain_hash (crates/llm-kv-cache/src/block.rs:8-33): SHA-256 of
 * "kir-ai-kv-block-chain/v1" || u64le(len) || model_id || u64le(len) ||
 * cache_context || previous_hash[32] || u64le(n) || u32le token ids. */
int llh_cache_block_chain_hash(const char *model_id, size_t model_len, const char *cache_context,
                               size_t context_len, const uint8_t previous_hash[32], const uint32_t *token_ids,
                               size_t n, uint8_t out[32]);

/* BlockPool::new(block_count, block_capacity_tokens, vector_len)
 * (block_pool.rs:151-163, 345-370): bookkeeping only, no payload. */
int llh_block_pool_create_host(size_t block_count, size_t block_capacity_tokens, size_t vector_len,
                               llh_block_pool **out);
/* A BlockPool over every block of a device pool (capacity = the pool's
 * block_tokens, vector_len = kv_heads * head_dim).  The pool must outlive it. */
int llh_block_pool_create(llh_ctx *ctx, llh_kv_pool *pool, llh_block_pool **out);
int llh_block_pool_destroy(llh_block_pool *bp);
const char *llh_block_pool_last_error(const llh_block_pool *bp);

/* total_blocks / free_blocks / allocated_blocks / session_count (block_pool.rs:165-179,193-195) */
typedef struct llh_block_pool_counts {
  uint64_t total_blocks;
  uint64_t free_blocks;
  uint64_t allocated_blocks;
  uint64_t sessions;
} llh_block_pool_counts;
int llh_block_pool_get_counts(const llh_block_pool *bp, llh_block_pool_counts *out);

/* PagedKvCacheMetricsSnapshot (block_pool.rs:99-122) */
typedef struct llh_paged_kv_metrics {
  uint64_t total_blocks, resident_blocks, active_blocks, blocks_in_use, free_blocks, free_list_blocks;
  double pool_utilization_pct;
  uint64_t sessions, session_block_tables, shared_blocks, refcount_total;
  double avg_refcount;
  uint64_t max_refcount, max_refcount_seen, total_refcount_increments, total_cow_clones, cow_bytes_saved;
  uint64_t blocks_evicted_lru, sessions_evicted_lru, eviction_high_water_mark, pool_high_water_blocks;
} llh_paged_kv_metrics;
int llh_block_pool_metrics(const llh_block_pool *bp, llh_paged_kv_metrics *out);

/* CacheBlock metadata (block.rs:36-53) and its device pool index.
 * payload_bytes: bytes of the block's K and V (f32 for host-only pools, as the
 * reference counts them; device bytes incl. scales for device pools). */
typedef struct llh_cache_block_info {
  uint64_t block_id;
  int64_t pool_index;
  uint64_t revision, capacity_tokens, vector_len, token_count, ref_count, last_access, payload_bytes;
  int32_t has_content_hash;
  uint8_t content_hash[32];
} llh_cache_block_info;
/* LLH_ERR_STALE for an id this pool does not hold. */
int llh_block_pool_block_info(const llh_block_pool *bp, uint64_t block_id, llh_cache_block_info *out);

/* allocate / deallocate (= release) / retain / touch / lru_block (block_pool.rs:669-728) */
int llh_block_pool_allocate(llh_block_pool *bp, uint64_t *block_id);
int llh_block_pool_release(llh_block_pool *bp, uint64_t block_id, int32_t *released);
int llh_block_pool_retain(llh_block_pool *bp, uint64_t block_id, int32_t *retained);
int llh_block_pool_touch(llh_block_pool *bp, uint64_t block_id, int32_t *touched);
int llh_block_pool_lru_block(const llh_block_pool *bp, uint64_t *block_id);
/* CacheBlock::set_content_hash via block_mut (block_pool.rs:730-737): only on
 * a block with ref_count 1 (else LLH_ERR_INVALID_SHAPE); hash NULL clears. */
int llh_block_pool_set_content_hash(llh_block_pool *bp, uint64_t block_id, const uint8_t *hash);

/* sessions (block_pool.rs:197-227, 433-481) */
int llh_block_pool_create_session(llh_block_pool *bp, uint64_t *session_id);
int llh_block_pool_release_session(llh_block_pool *bp, uint64_t session_id, int32_t *released);
/* evicts least-recently-used sessions when no block is free */
int llh_block_pool_allocate_for_session(llh_block_pool *bp, uint64_t session_id, uint64_t *block_id);
int llh_block_pool_append_block_to_session(llh_block_pool *bp, uint64_t session_id, uint64_t block_id);
int llh_block_pool_read_session_block(llh_block_pool *bp, uint64_t session_id, size_t index, uint64_t *block_id);
typedef struct llh_session_info {
  uint64_t session_id, created_at, last_access, block_count, owned_block_count;
} llh_session_info;
int llh_block_pool_session_info(const llh_block_pool *bp, uint64_t session_id, llh_session_info *out);
/* The session's table as BlockIds and device pool indices (either may be NULL). */
int llh_block_pool_session_blocks(const llh_block_pool *bp, uint64_t session_id, uint64_t *h_ids,
                                  int32_t *h_pool_indices, size_t capacity, size_t *count);
int llh_block_pool_lru_session(const llh_block_pool *bp, uint64_t *session_id);

/* prefix registry keyed by the terminal chain hash (block_pool.rs:483-519) */
int llh_block_pool_register_prefix(llh_block_pool *bp, const uint8_t prefix_hash[32], const uint64_t *block_ids,
                                   size_t n);
int llh_block_pool_lookup_prefix(const llh_block_pool *bp, const uint8_t prefix_hash[32], uint64_t *h_ids,
                                 size_t capacity, size_t *count, int32_t *found);
int llh_block_pool_attach_prefix_to_session(llh_block_pool *bp, uint64_t session_id, const uint8_t prefix_hash[32],
                                            uint64_t *h_ids, size_t capacity, size_t *count, int32_t *found);
/* copy_on_write_session_block (block_pool.rs:521-603): a shared block is
 * cloned (device payload copy for device pools) into a fresh block that
 * replaces it in this session's table. */
int llh_block_pool_copy_on_write_session_block(llh_block_pool *bp, uint64_t session_id, size_t index,
                                               uint64_t *block_id);

/* payload, device pools only */
/* CacheBlock::append (block.rs:250-272) through block_mut: one token row to
 * the block's next slot (quantised on write for int8); exclusive blocks only. */
int llh_block_pool_append_f32(llh_block_pool *bp, uint64_t block_id, const float *h_key, const float *h_value,
                              size_t len);
/* Records n rows the caller wrote with llh_kv_append at slots
 * pool_index * block_tokens + token_count + i (token_count, hash, revision). */
int llh_block_pool_commit_tokens(llh_block_pool *bp, uint64_t block_id, size_t n);
/* CacheBlock::keys() / values() (block.rs:300-306): token_count rows of
 * vector_len f32 (dequantised); tensor 0 = K, 1 = V. */
int llh_block_pool_read_rows_f32(llh_block_pool *bp, uint64_t block_id, int32_t tensor, float *h_out,
                                 size_t capacity, size_t *count);

/* ---------------------------------------------------------------------------
 * Prefix cache: the driver-side longest-prefix lookup over token ids
 * (NativeTextPrefixCache, crates/llm-native-runtime/src/native_text/prefix_cache.rs:20-336).
 * Entries are keyed by (namespace, exact token sequence) -- the namespace is
 * the caller's serialisation of NativeTextPrefixCacheNamespace
 * (prefix_cache.rs:59-80), compared byte for byte.  A payload is a hidden row
 * (f32) plus opaque 64-bit state handles (here: BlockPool block ids holding the
 * prefix's K/V); its size is 4 * n_hidden + state_bytes (the reference's
 * prefix_cache_entry_bytes).  A successful store takes the cache's own
 * reference to the handles (`retain`, like the reference cloning the caller's
 * caches into the payload), each hit takes one more for the caller (the
 * reference's Arc clone of the hit payload, prefix_cache.rs:256-275), and the
 * cache's reference goes (`release`) when the entry is evicted, replaced or the
 * cache destroyed.  Callbacks run outside the cache's lock.
 * ------------------------------------------------------------------------- */
typedef struct llh_prefix_cache llh_prefix_cache;
typedef void (*llh_prefix_retain_fn)(void *user, const uint64_t *states, size_t n_states);
typedef void (*llh_prefix_release_fn)(void *user, const uint64_t *states, size_t n_states);
/* lookup_compatible's predicate (prefix_cache.rs:223-229): nonzero = reusable */
typedef int (*llh_prefix_compatible_fn)(void *user, const uint64_t *states, size_t n_states);

typedef struct llh_prefix_hit {
  uint64_t token_count; /* 0 = miss */
  uint64_t n_hidden;
  uint64_t n_states;
  uint64_t byte_len;
} llh_prefix_hit;

/* NativeTextPrefixCacheCounters (prefix_cache.rs:170-196); every counter saturates */
typedef struct llh_prefix_cache_counters {
  uint64_t hits, misses, stores, evictions, rejected, reused_tokens;
  uint64_t prefill_chunks, prefill_tokens, checkpoint_stores, checkpoint_store_tokens;
  uint64_t checkpoint_reuse_hits, checkpoint_reused_tokens, shared_prefix_hits, shared_prefix_reused_tokens;
  uint64_t hit_tokens, miss_tokens, avoided_prefill_tokens, entries_scanned, namespace_entries_scanned;
  uint64_t hit_clone_bytes, bytes_stored, bytes_evicted, resident_bytes, resident_entries;
} llh_prefix_cache_counters;

enum {
  LLH_PREFIX_RECORD_PREFILL_CHUNK = 0,        /* record_prefill_chunk (prefix_cache.rs:556-561) */
  LLH_PREFIX_RECORD_CHECKPOINT_STORE = 1,     /* record_checkpoint_store */
  LLH_PREFIX_RECORD_CHECKPOINT_REUSE = 2,     /* record_checkpoint_reuse */
  LLH_PREFIX_RECORD_SHARED_PREFIX_REUSE = 3,  /* record_shared_prefix_reuse */
  LLH_PREFIX_RECORD_HIT = 4,                  /* record_hit for a hit served elsewhere (disk tier) */
  LLH_PREFIX_RECORD_MISS_TOKENS = 5           /* record_miss_tokens */
};

/* NativeTextPrefixCache::new (prefix_cache.rs:204-209) */
int llh_prefix_cache_create(uint64_t max_bytes, llh_prefix_retain_fn retain, llh_prefix_release_fn release,
                            void *user, llh_prefix_cache **out);
int llh_prefix_cache_destroy(llh_prefix_cache *pc);
/* store (prefix_cache.rs:256-336): *stored = 0 for an empty token list or an
 * entry over the whole budget (counted as rejected) */
int llh_prefix_cache_store(llh_prefix_cache *pc, const char *ns, size_t ns_len, const uint32_t *tokens,
                           size_t n_tokens, const float *hidden, size_t n_hidden, const uint64_t *states,
                           size_t n_states, uint64_t state_bytes, int32_t *stored);
/* lookup_compatible (prefix_cache.rs:223-254); compatible = NULL accepts any
 * entry (lookup).  Copies up to hidden_cap / states_cap values out. */
int llh_prefix_cache_lookup(llh_prefix_cache *pc, const char *ns, size_t ns_len, const uint32_t *tokens,
                            size_t n_tokens, llh_prefix_compatible_fn compatible, void *compat_user,
                            llh_prefix_hit *hit, float *hidden_out, size_t hidden_cap, uint64_t *states_out,
                            size_t states_cap);
/* driver-side counters (NativeTextPrefixCacheMetrics::record_*) */
int llh_prefix_cache_record(llh_prefix_cache *pc, int32_t kind, uint64_t tokens);
int llh_prefix_cache_metrics(llh_prefix_cache *pc, llh_prefix_cache_counters *out);
/* introspection for tests: namespace buckets, entries and indexed lengths of
 * one namespace, resident bytes; the index-th entry in LRU order (oldest first) */
int llh_prefix_cache_shape(llh_prefix_cache *pc, const char *ns, size_t ns_len, uint64_t *namespaces,
                           uint64_t *entries_in_ns, uint64_t *indexed_in_ns, uint64_t *used_bytes);
int llh_prefix_cache_lru_entry(llh_prefix_cache *pc, size_t index, char *ns_out, size_t ns_cap, size_t *ns_len,
                               uint32_t *tokens_out, size_t tokens_cap, size_t *n_tokens);

/* ---------------------------------------------------------------------------
 * On-disk prefix KV blocks (the SSD tier behind the prefix cache,
 * crates/llm-native-runtime/src/native_text/disk_cache.rs, disk_cache/io.rs,
 * disk_cache/codec.rs, disk_cache/hashing.rs).  A block file is a safetensors
 * archive: u64le header length, a JSON header with "__metadata__":{"kir_ai":
 * <block metadata JSON>} and one F32 tensor per name ("hidden",
 * "layers.<i>.full.keys", ...), tensors in name order.  The encoder writes the
 * bytes the reference writes for the same content.  Hashes are lowercase hex
 * SHA-256, 64 characters plus NUL.  Errors other than NULL arguments are
 * LLH_ERR_INTEGRITY with the reference's message in llh_disk_last_error().
 * K/V travel as f32 rows: llh_kv_export_rows_f32 reads them out of a device
 * pool, llh_kv_append writes them back.
 * ------------------------------------------------------------------------- */
enum {
  LLH_DISK_LAYER_QWEN_FULL = 0, /* "qwen_full_attention", tensors layers.<i>.full.{keys,values} */
  LLH_DISK_LAYER_GEMMA = 1,     /* "gemma_attention", tensors layers.<i>.attention.{keys,values} */
  LLH_DISK_LAYER_OTHER = 2      /* "qwen_linear_attention": recurrent state, not paged KV (read side only) */
};

/* NativeTextDiskCacheBlockDescriptor (disk_cache.rs:165-217) */
typedef struct llh_disk_block_descriptor {
  char model_hash[65];
  char snapshot_hash[65];
  char model_family[64];
  char namespace_hash[65];
  char previous_block_hash[65];
  char block_hash[65];
  uint64_t block_start;
  uint64_t token_count;
  uint32_t cache_layout_version;
  uint32_t n_layers; /* filled by llh_disk_block_read_descriptor only */
} llh_disk_block_descriptor;

/* NativeTextDiskCacheIdentity (disk_cache.rs:93-147); allowed_namespace_hash may be NULL */
typedef struct llh_disk_identity {
  const char *model_hash;
  const char *snapshot_hash;
  const char *model_family;
  const char *allowed_namespace_hash;
} llh_disk_identity;

/* One full-attention layer of a block (NativeTextDiskFullAttentionLayout,
 * codec.rs:43-55): keys / values are token_count x key_value_heads x head_dim f32 */
typedef struct llh_disk_layer {
  int32_t kind; /* LLH_DISK_LAYER_QWEN_FULL or LLH_DISK_LAYER_GEMMA */
  uint64_t revision, max_tokens, key_value_heads, head_dim, token_count, tokens_seen;
  const float *keys;
  const float *values;
} llh_disk_layer;

typedef struct llh_disk_layer_info {
  int32_t kind;
  uint64_t revision, max_tokens, key_value_heads, head_dim, token_count, tokens_seen;
  uint64_t n_values; /* f32 values per tensor */
} llh_disk_layer_info;

typedef struct llh_disk_block llh_disk_block;

/* message of the calling thread's last LLH_ERR_INTEGRITY from this family */
const char *llh_disk_last_error(void);
/* hash_components (hashing.rs:178-190): label, then (name, value-or-NULL) pairs --
 * the snapshot, model and namespace hashes (hashing.rs:32-128) are this with
 * their labels and component lists */
int llh_disk_hash_components(const char *label, size_t n, const char *const *names, const char *const *values,
                             char out_hex[65]);
/* native_text_disk_block_hash (hashing.rs:130-150) */
int llh_disk_block_hash(const char *model_hash, const char *namespace_hash, const char *previous_block_hash,
                        uint64_t block_start, const uint64_t *tokens, size_t n_tokens, char out_hex[65]);
/* native_text_disk_previous_block_hash (hashing.rs:152-176) */
int llh_disk_previous_block_hash(const char *model_hash, const char *namespace_hash, uint64_t block_start,
                                 uint64_t block_token_count, const uint64_t *prefix_tokens, size_t n_prefix,
                                 char out_hex[65]);
/* NativeTextDiskCacheBlockDescriptor::new (disk_cache.rs:176-217): the block is
 * prefix_tokens[block_start..] */
int llh_disk_block_descriptor_new(const llh_disk_identity *identity, const char *namespace_hash,
                                  uint32_t cache_layout_version, uint64_t block_start, const uint64_t *prefix_tokens,
                                  size_t n_prefix, llh_disk_block_descriptor *out);
/* path_for_descriptor (disk_cache.rs:527-534) below the cache root:
 * <model_hash>/<namespace_hash>/<block_hash[0:2]>/<block_hash>.safetensors */
int llh_disk_block_path(const llh_disk_block_descriptor *desc, char *out, size_t capacity, size_t *length);
/* NativeTextDiskCacheBlock::encode (io.rs:40-69).  out = NULL reports the size
 * in *length; a short buffer is LLH_ERR_CAPACITY. */
int llh_disk_block_encode(const llh_disk_block_descriptor *desc, const float *hidden, size_t n_hidden,
                          const llh_disk_layer *layers, size_t n_layers, uint8_t *out, size_t capacity,
                          size_t *length);
/* Parses a block file (header, metadata, tensor table: io.rs:195-204); the
 * handle keeps its own copy of the bytes. */
int llh_disk_block_open(const uint8_t *bytes, size_t length, llh_disk_block **out);
int llh_disk_block_close(llh_disk_block *blk);
/* decode_descriptor (io.rs:105-121): the metadata's descriptor, after the codec / layout check */
int llh_disk_block_read_descriptor(const llh_disk_block *blk, llh_disk_block_descriptor *out);
/* the checks of NativeTextDiskCacheBlock::decode (io.rs:71-103), in its order */
int llh_disk_block_validate(const llh_disk_block *blk, const llh_disk_block_descriptor *expected,
                            const llh_disk_identity *identity);
/* the hidden row: *count values, up to capacity copied (out may be NULL) */
int llh_disk_block_hidden(const llh_disk_block *blk, float *out, size_t capacity, size_t *count);
/* decode_layer_kv_snapshot (codec.rs:101-130) for layer `index`; up to
 * capacity values of each tensor copied.  LLH_ERR_UNSUPPORTED for a linear
 * attention layer, LLH_ERR_INVALID_SHAPE past the last layer. */
int llh_disk_block_layer(const llh_disk_block *blk, size_t index, llh_disk_layer_info *info, float *keys,
                         float *values, size_t capacity);

/* The checks that join consecutive blocks of one prefix
 * (validate_contiguous_disk_blocks and assemble_layer_kv_prefix_state_blocks,
 * codec.rs:252-322): block starts contiguous from 0, the same layer kinds and
 * KV shapes in every block, the joined rows within each layer's max_tokens.
 * *total_tokens = the prefix length. */
int llh_disk_blocks_assemble_check(const llh_disk_block *const *blocks, size_t n, uint64_t *total_tokens);

/* Reads n token rows (K and V, kv_heads x head_dim each) of a device pool as
 * f32 into d_k / d_v: row i is token slot d_slots[i] (pool block * block_tokens
 * + offset).  Dequantises int8 / fp8 with the block's scales -- the
 * LayerKvCacheSnapshot keys()/values() view the disk encoder consumes
 * (codec.rs:72-99). */
int llh_kv_export_rows_f32(llh_ctx *ctx, const llh_kv_pool *pool, const int64_t *d_slots, int64_t n, float *d_k,
                           float *d_v, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LLM_HIP_H */
