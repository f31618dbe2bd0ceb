/*
 * oracle.h -- CPU restatement of kir-ai's attention-over-KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * kernels in kir-ai_amd/csrc and the CPU baseline timed by bench.py.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (libllm_hip.so) never links, loads or calls it.
 *
 * What it restates (paths relative to the kir-ai reference tree):
 *   - per-head fp32 attention loop     crates/llm-backend/src/core/native_attention.rs:707-773,827-841
 *       matvec                         crates/llm-backend/src/core/math.rs:126-161
 *       softmax                        crates/llm-backend/src/core/math.rs:476-505
 *       weighted sum                   crates/llm-backend/src/core/math.rs:260-287
 *       head-row select                crates/llm-backend/src/core/math.rs:343-383
 *   - decode = append then attend      crates/llm-backend/src/core/native_attention.rs:284-354
 *   - prefill = per token append+attend crates/llm-backend/src/core/native_attention.rs:356-464
 *   - ring KV cache + active runs      crates/llm-kv-cache/src/layer.rs:744-880,972-1044,1080-1162
 *   - int8 row quantisation            crates/llm-kv-cache/src/format.rs:702-759
 *   - sliding window = ring capacity   crates/llm-backend/src/core/qwen/ops/cache.rs:116-121
 *
 * Additions the reference does not have (each pinned independently, see the
 * tests): the paged pool layout the GPU uses, the per-(token, head) fp16-scale
 * int8 layout and the per-(block, head) fp8 e4m3 layout, the seeded PRNG, and
 * a float64 brute-force attention used as a second checker.
 *
 * Arithmetic follows the reference exactly where it is defined: products and
 * sums are separate roundings (build with -ffp-contract=off), sums run
 * sequentially in row order, exp is the C library's expf.
 */
#ifndef KIRAI_ORACLE_H
#define KIRAI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (mirror llm_hip.h) */
#define ORC_OK 0
#define ORC_ERR_INVALID_SHAPE (-1)
#define ORC_ERR_CAPACITY (-2)
#define ORC_ERR_NON_FINITE (-3)

/* KV formats (mirror llm_hip.h) */
#define ORC_KV_BF16 0
#define ORC_KV_INT8 1
#define ORC_KV_FP8_E4M3 2
#define ORC_KV_INT8_ROW 3 /* the reference's own int8 layout: f32 scale per token row over all heads */
#define ORC_KV_F16 4      /* IEEE binary16 elements (KvCacheConfig::f16, format.rs:69-120) */

/* ---------------- scalar conversions ---------------- */
uint16_t orc_f32_to_bf16(float x);   /* round to nearest even, NaN kept quiet */
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_f16(float x);    /* IEEE binary16, round to nearest even */
float orc_f16_to_f32(uint16_t h);
uint8_t orc_f32_to_fp8e4m3(float x); /* OCP E4M3FN, RNE, saturate to +-448 */
float orc_fp8e4m3_to_f32(uint8_t c);
float orc_round_half_away(float x);  /* Rust f32::round */

/* ---------------- seeded counter-based PRNG ----------------
 * value(seed, i): pair j = i/2, u1 = U(mix64(seed + (2j+1)*G)), u2 = U(mix64(seed + (2j+2)*G)),
 * r = sqrt(-2 ln u1), z = (i even) ? r cos(2 pi u2) : r sin(2 pi u2), computed in double,
 * returned as float.  mix64 = splitmix64 finaliser, G = 0x9E3779B97F4A7C15,
 * U(x) = ((x >> 11) + 0.5) * 2^-53. */
uint64_t orc_mix64(uint64_t z);
float orc_normal(uint64_t seed, uint64_t index);
void orc_fill_normal_f32(uint64_t seed, uint64_t offset, size_t n, float *out);
void orc_fill_normal_bf16(uint64_t seed, uint64_t offset, size_t n, uint16_t *out);
/* uniform integer in [lo, hi] from mix64(seed + (index+1)*G) */
int64_t orc_uniform_int(uint64_t seed, uint64_t index, int64_t lo, int64_t hi);
/* Fisher-Yates permutation of 0..n-1 driven by orc_uniform_int(seed, k, ...) */
void orc_permutation(uint64_t seed, int32_t n, int32_t *out);

/* ---------------- reference math (math.rs) ---------------- */
/* matvec_row_major_f32_in_place: out[r] = sum_c w[r*cols+c]*x[c], sequential */
void orc_matvec_row_major(const float *x, const float *w, size_t rows, size_t cols, float *out);
/* safetensors/math.rs:66-72 bf16_dot_f32_scalar, one per row: f32 input, bf16 row-major weights */
void orc_matvec_bf16_f32(const uint16_t *w, size_t rows, size_t cols, const float *x, float *out);
/* softmax_f32_in_place: error on non-finite input or invalid denominator */
int orc_softmax(const float *scores, size_t n, float *out);
/* math.rs:472-474 sigmoid_f32: 1 / (1 + exp(-value)) */
float orc_sigmoid(float value);
/* native_attention.rs:775-781 apply_attention_gate (and the per-head form of :765-770):
 * attended[i] *= sigmoid_f32(gate[i]) for i < n */
void orc_apply_gate(float *attended, const float *gate, size_t n);
/* weighted_sum_f32_in_place */
void orc_weighted_sum(const float *values, const float *weights, size_t rows, size_t vector_len, float *out);
/* select_head_rows_f32_in_place */
void orc_select_head_rows(const float *values, size_t rows, size_t row_len, size_t head_start,
                          size_t head_len, float *out);

/* native_full_attention_mix_from_cache per-head loop.
 * keys/values: logical rows [row_count][kv_heads*head_dim]; query [q_heads*head_dim].
 * Returns ORC_OK, ORC_ERR_INVALID_SHAPE or ORC_ERR_NON_FINITE. */
int orc_attention_mix(const float *query, const float *keys, const float *values, size_t row_count,
                      size_t q_heads, size_t kv_heads, size_t head_dim, float scale, float *out);
/* same contract, float64 brute force (independent checker, not the reference order) */
int orc_attention_mix_f64(const float *query, const float *keys, const float *values,
                          size_t row_count, size_t q_heads, size_t kv_heads, size_t head_dim,
                          double scale, double *out);

/* ---------------- ring KV cache (layer.rs) ---------------- */
typedef struct orc_run {
  int64_t block_index;
  int64_t logical_token_start;
  int64_t physical_token_start;
  int64_t block_token_start;
  int64_t token_count;
} orc_run;

typedef struct orc_ring {
  int64_t max_tokens;
  int64_t vector_len;
  int64_t block_tokens; /* LAYER_KV_BLOCK_TOKENS = 256 in the reference */
  int64_t token_count;
  int64_t tokens_seen;
  int64_t window_start;
  uint64_t revision;
  float *keys;   /* caller storage [max_tokens][vector_len], physical order */
  float *values; /* caller storage [max_tokens][vector_len] */
  orc_run *runs; /* caller storage, capacity run_cap */
  int64_t run_cap;
  int64_t run_count;
} orc_ring;

int orc_ring_init(orc_ring *r, int64_t max_tokens, int64_t vector_len, int64_t block_tokens,
                  float *keys, float *values, orc_run *runs, int64_t run_cap);
/* append_sliding_with_metadata; writes the token index and physical slot */
int orc_ring_append_sliding(orc_ring *r, const float *key, const float *value, int64_t *token_index,
                            int64_t *physical_index);
/* append (strict): capacity error when full */
int orc_ring_append(orc_ring *r, const float *key, const float *value, int64_t *token_index);
/* keys()/values(): logical rows [token_count][vector_len] */
void orc_ring_logical_rows(const orc_ring *r, int tensor, float *out);

/* ---------------- paged pool (device layout) ----------------
 * K  : [n_blocks][kv_heads][block_tokens][head_dim]   (token rows)
 * V  : [n_blocks][kv_heads][head_dim][block_tokens]   (dim rows, i.e. transposed)
 * int8 scales: [n_blocks][kv_heads][block_tokens] fp16 for K and for V
 * fp8 scales : [n_blocks][kv_heads] f32 for K and for V
 * int8 row scales: [n_blocks][block_tokens] f32 for K and for V (format.rs:702-759)
 * Position p of a sequence lives in block table[(p / block_tokens) % n_table],
 * at offset p % block_tokens. */
typedef struct orc_pool {
  int32_t format;
  int32_t block_tokens;
  int32_t kv_heads;
  int32_t head_dim;
  int64_t n_blocks;
  const void *k;
  const void *v;
  const void *k_scales;
  const void *v_scales;
} orc_pool;

/* dequantised element of tensor (0 = K, 1 = V) at (block, head, token-in-block, dim) */
float orc_pool_elem(const orc_pool *p, int tensor, int64_t block, int32_t head, int32_t t, int32_t d);
/* gather logical positions [lo, hi) into row-major f32 rows [hi-lo][kv_heads*head_dim] */
int orc_pool_gather_f32(const orc_pool *p, const int32_t *table, int32_t n_table, int32_t lo,
                        int32_t hi, float *keys_out, float *values_out);
/* gather raw storage bits of tensor into [hi-lo][kv_heads][head_dim] elements
 * (2 bytes for bf16 / f16, 1 byte for int8/fp8) */
int orc_pool_gather_raw(const orc_pool *p, const int32_t *table, int32_t n_table, int32_t lo,
                        int32_t hi, int tensor, void *out);
/* write one token row ([kv_heads*head_dim] f32) into slot (block, t) of a bf16 pool */
int orc_pool_write_bf16(const orc_pool *p, int64_t block, int32_t t, const float *key, const float *value);

/* decode: for every sequence b, attend positions [lo_b, seq_lens[b]) with
 * lo_b = window ? max(0, len - window) : 0, query q[b] (bf16), out f32 [B][Hq][D].
 * threads <= 1 runs the reference's single-threaded loop. */
int orc_paged_decode(const orc_pool *p, int32_t num_seqs, int32_t q_heads, const int32_t *seq_lens,
                     const int32_t *block_tables, int32_t max_blocks, int32_t window,
                     const uint16_t *q_bf16, float scale, float *out, int threads);
/* prefill: sequence b owns query rows [chunk_starts[b], chunk_starts[b+1]); row i of it sits
 * at position context_lens[b] - chunk_len + i and attends [lo(pos), pos]. */
int orc_paged_prefill(const orc_pool *p, int32_t num_seqs, int32_t q_heads, const int32_t *chunk_starts,
                      const int32_t *context_lens, const int32_t *block_tables, int32_t max_blocks,
                      int32_t window, const uint16_t *q_bf16, float scale, float *out, int threads);
/* same prefill restricted to query rows [row_lo, row_hi) of sequence b (bounded CPU timing) */
int orc_paged_prefill_rows(const orc_pool *p, int32_t b, int32_t q_heads, const int32_t *chunk_starts,
                           const int32_t *context_lens, const int32_t *block_tables, int32_t max_blocks,
                           int32_t window, const uint16_t *q_bf16, float scale, float *out,
                           int32_t row_lo, int32_t row_hi, int threads);

/* ---------------- quantisation ---------------- */
/* quantize_int8_rows (format.rs:702-737): per row scale = absmax/127 (0 -> 0),
 * code = clamp(round_half_away(x/scale), -127, 127) */
int orc_quantize_int8_rows(const float *x, size_t rows, size_t vector_len, int8_t *codes, float *scales);
/* dequantize_int8_rows (format.rs:739-759) */
void orc_dequantize_int8_rows(const int8_t *codes, const float *scales, size_t rows, size_t vector_len,
                              float *out);
/* per (token, head) int8 with fp16 scale: s16 = f16(absmax/127), codes quantised with the
 * f16-rounded scale so that storage and dequantisation agree */
int orc_quantize_int8_head(const float *x, int32_t n, int8_t *codes, uint16_t *scale_f16);
/* per (block, head) fp8: scale = absmax/448 over n values (0 -> 0, codes 0), code = e4m3(x/scale) */
int orc_quantize_fp8_block(const float *x, int32_t n, uint8_t *codes, float *scale);
/* Per-token append into one fp8 (block, head) tensor, re-quantising the block as
 * the reference re-quantises a block on every int8 append (layer.rs:1396-1408;
 * fp8 itself has no counterpart there): codes [block_tokens][dim] token-major,
 * *scale the block's scale.  Token `off` = row x [dim]: old = off == 0 ? 0 :
 * *scale; new = max(old, absmax(x) / 448); when new != old the codes of tokens
 * 0 .. off-1 become e4m3((old == 0 ? 0 : e4m3_to_f32(code) * old) / new); the
 * row's codes are new == 0 ? 0 : e4m3(x / new).  Non-finite x -> error. */
int orc_append_fp8_token(uint8_t *codes, int32_t dim, float *scale, int32_t off, const float *x);

#ifdef __cplusplus
}
#endif
#endif
