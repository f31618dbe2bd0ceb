/*
 * oracle.c -- CPU restatement of kir-ai's attention-over-KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline.  The product
 * library never links or calls this file.  Function-level citations are to the
 * kir-ai reference tree; oracle.h lists what is restated and what is added.
 *
 * Build with -ffp-contract=off so that every product and sum rounds separately,
 * as the reference's Rust f32 arithmetic does.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define GOLDEN 0x9E3779B97F4A7C15ULL

/* ------------------------------------------------------------------ */
/* scalar conversions                                                 */
/* ------------------------------------------------------------------ */

static uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

uint16_t orc_f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

uint16_t orc_f32_to_f16(float x) {
  uint32_t u = f32_bits(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t exp = (u >> 23) & 0xffu;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    int shift = 14 - e;
    uint32_t q = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t man = (uint32_t)h & 0x3ffu;
  if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13));
  if (exp == 0) {
    float v = (float)man * (1.0f / 16777216.0f); /* man * 2^-24, exact */
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

float orc_fp8e4m3_to_f32(uint8_t c) {
  int s = c >> 7;
  int e = (c >> 3) & 0xf;
  int m = c & 7;
  float v;
  if (e == 0xf && m == 7) return NAN;
  if (e == 0)
    v = (float)m * (1.0f / 512.0f); /* m/8 * 2^-6 */
  else
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return s ? -v : v;
}

/* orc_fp8e4m3_to_f32 of every code, filled when the library loads (the pool reads
   of an fp8 pool go through it: the same values, without a ldexpf per element) */
static float fp8_table[256];
__attribute__((constructor)) static void fill_fp8_table(void) {
  for (int c = 0; c < 256; c++) fp8_table[c] = orc_fp8e4m3_to_f32((uint8_t)c);
}

uint8_t orc_f32_to_fp8e4m3(float x) {
  uint32_t u = f32_bits(x);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (uint8_t)(sign | 0x7f);
  if (bits_f32(au) >= 448.0f) return (uint8_t)(sign | 0x7e);
  uint32_t exp = au >> 23;
  uint32_t man = au & 0x7fffffu;
  int e = (int)exp - 127 + 7;
  if (e <= 0) {
    if (exp == 0) return sign;
    man |= 0x800000u;
    int shift = 21 - e; /* q = man24 * 2^(e-21) counts units of 2^-9 */
    if (shift > 24) return sign;
    uint32_t q = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint8_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 3) | (man >> 20);
  uint32_t rem = man & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
  if (q > 0x7eu) q = 0x7eu;
  return (uint8_t)(sign | q);
}

float orc_round_half_away(float x) { return roundf(x); }

/* ------------------------------------------------------------------ */
/* PRNG                                                               */
/* ------------------------------------------------------------------ */

uint64_t orc_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

static double u01(uint64_t x) { return ((double)(x >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

float orc_normal(uint64_t seed, uint64_t index) {
  uint64_t j = index >> 1;
  double u1 = u01(orc_mix64(seed + (2 * j + 1) * GOLDEN));
  double u2 = u01(orc_mix64(seed + (2 * j + 2) * GOLDEN));
  double r = sqrt(-2.0 * log(u1));
  double t = 6.283185307179586476925 * u2;
  return (float)((index & 1) ? r * sin(t) : r * cos(t));
}

void orc_fill_normal_f32(uint64_t seed, uint64_t offset, size_t n, float *out) {
  for (size_t i = 0; i < n; i++) out[i] = orc_normal(seed, offset + i);
}

void orc_fill_normal_bf16(uint64_t seed, uint64_t offset, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(orc_normal(seed, offset + i));
}

int64_t orc_uniform_int(uint64_t seed, uint64_t index, int64_t lo, int64_t hi) {
  uint64_t x = orc_mix64(seed + (index + 1) * GOLDEN);
  uint64_t span = (uint64_t)(hi - lo) + 1u;
  return lo + (int64_t)(x % span);
}

void orc_permutation(uint64_t seed, int32_t n, int32_t *out) {
  for (int32_t i = 0; i < n; i++) out[i] = i;
  for (int32_t i = n - 1; i > 0; i--) {
    int32_t j = (int32_t)orc_uniform_int(seed, (uint64_t)i, 0, i);
    int32_t t = out[i];
    out[i] = out[j];
    out[j] = t;
  }
}

/* ------------------------------------------------------------------ */
/* reference math                                                     */
/* ------------------------------------------------------------------ */

/* math.rs:126-161 matvec_row_major_f32_in_place: zip(...).map(w*x).sum() */
void orc_matvec_row_major(const float *x, const float *w, size_t rows, size_t cols, float *out) {
  for (size_t r = 0; r < rows; r++) {
    const float *row = w + r * cols;
    float acc = 0.0f;
    for (size_t c = 0; c < cols; c++) {
      float prod = row[c] * x[c];
      acc = acc + prod;
    }
    out[r] = acc;
  }
}

/* bf16_dot_f32_scalar (crates/llm-backend/src/core/safetensors/math.rs:66-72) per row:
 * out[r] = sum_c bf16(w[r][c]) * x[c], products and sum in f32, in column order
 * (the row matvec of bf16_matvec_rows_f32_in_place, safetensors.rs:915-966). */
void orc_matvec_bf16_f32(const uint16_t *w, size_t rows, size_t cols, const float *x, float *out) {
  for (size_t r = 0; r < rows; r++) {
    const uint16_t *row = w + r * cols;
    float acc = 0.0f;
    for (size_t c = 0; c < cols; c++) {
      float prod = orc_bf16_to_f32(row[c]) * x[c];
      acc = acc + prod;
    }
    out[r] = acc;
  }
}

/* math.rs:476-505 softmax_f32_in_place */
int orc_softmax(const float *scores, size_t n, float *out) {
  if (n == 0) return ORC_OK;
  for (size_t i = 0; i < n; i++)
    if (!isfinite(scores[i])) return ORC_ERR_NON_FINITE;
  float max_score = -INFINITY;
  for (size_t i = 0; i < n; i++) max_score = fmaxf(max_score, scores[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    out[i] = expf(scores[i] - max_score);
    sum = sum + out[i];
  }
  if (sum == 0.0f || !isfinite(sum)) return ORC_ERR_NON_FINITE;
  for (size_t i = 0; i < n; i++) out[i] = out[i] / sum;
  return ORC_OK;
}

/* math.rs:472-474 sigmoid_f32 */
float orc_sigmoid(float value) { return 1.0f / (1.0f + expf(-value)); }

/* native_attention.rs:775-781 apply_attention_gate: each attended value times the
 * sigmoid of its gate (the per-head loop at :765-770 applies the same product) */
void orc_apply_gate(float *attended, const float *gate, size_t n) {
  for (size_t i = 0; i < n; i++) attended[i] = attended[i] * orc_sigmoid(gate[i]);
}

/* math.rs:260-287 weighted_sum_f32_in_place */
void orc_weighted_sum(const float *values, const float *weights, size_t rows, size_t vector_len, float *out) {
  for (size_t d = 0; d < vector_len; d++) out[d] = 0.0f;
  for (size_t r = 0; r < rows; r++) {
    const float *row = values + r * vector_len;
    for (size_t d = 0; d < vector_len; d++) {
      float prod = row[d] * weights[r];
      out[d] = out[d] + prod;
    }
  }
}

/* math.rs:343-383 select_head_rows_f32_in_place */
void orc_select_head_rows(const float *values, size_t rows, size_t row_len, size_t head_start,
                          size_t head_len, float *out) {
  for (size_t r = 0; r < rows; r++)
    memcpy(out + r * head_len, values + r * row_len + head_start, head_len * sizeof(float));
}

/* one head of native_attention.rs:731-771 over head-selected rows [rows][head_dim] */
static int attend_head(const float *q_head, const float *key_rows, const float *value_rows, size_t rows,
                       size_t head_dim, float scale, float *scratch, float *out) {
  float *scores = scratch;
  float *weights = scratch + rows;
  orc_matvec_row_major(q_head, key_rows, rows, head_dim, scores);
  for (size_t r = 0; r < rows; r++) scores[r] = scores[r] * scale; /* :827-841 */
  int st = orc_softmax(scores, rows, weights);
  if (st != ORC_OK) return st;
  orc_weighted_sum(value_rows, weights, rows, head_dim, out);
  return ORC_OK;
}

/* native_attention.rs:707-773 native_full_attention_mix_from_cache (per-head path) */
int orc_attention_mix(const float *query, const float *keys, const float *values, size_t row_count,
                      size_t q_heads, size_t kv_heads, size_t head_dim, float scale, float *out) {
  if (q_heads == 0 || kv_heads == 0 || head_dim == 0 || q_heads % kv_heads != 0)
    return ORC_ERR_INVALID_SHAPE;
  size_t groups = q_heads / kv_heads;
  size_t vector_len = kv_heads * head_dim;
  size_t rows = row_count;
  float *key_rows = (float *)malloc((rows * head_dim + 1) * sizeof(float));
  float *value_rows = (float *)malloc((rows * head_dim + 1) * sizeof(float));
  float *scratch = (float *)malloc((2 * rows + 1) * sizeof(float));
  int st = ORC_OK;
  for (size_t h = 0; h < q_heads && st == ORC_OK; h++) {
    size_t kv = h / groups; /* :732 */
    orc_select_head_rows(keys, rows, vector_len, kv * head_dim, head_dim, key_rows);
    orc_select_head_rows(values, rows, vector_len, kv * head_dim, head_dim, value_rows);
    st = attend_head(query + h * head_dim, key_rows, value_rows, rows, head_dim, scale, scratch,
                     out + h * head_dim);
  }
  free(key_rows);
  free(value_rows);
  free(scratch);
  return st;
}

int orc_attention_mix_f64(const float *query, const float *keys, const float *values,
                          size_t row_count, size_t q_heads, size_t kv_heads, size_t head_dim,
                          double scale, double *out) {
  if (q_heads == 0 || kv_heads == 0 || head_dim == 0 || q_heads % kv_heads != 0)
    return ORC_ERR_INVALID_SHAPE;
  size_t groups = q_heads / kv_heads;
  size_t vector_len = kv_heads * head_dim;
  double *s = (double *)malloc((row_count + 1) * sizeof(double));
  for (size_t h = 0; h < q_heads; h++) {
    size_t kv = h / groups;
    double m = -INFINITY;
    for (size_t r = 0; r < row_count; r++) {
      double acc = 0.0;
      for (size_t d = 0; d < head_dim; d++)
        acc += (double)query[h * head_dim + d] * (double)keys[r * vector_len + kv * head_dim + d];
      s[r] = acc * scale;
      if (!isfinite(s[r])) {
        free(s);
        return ORC_ERR_NON_FINITE;
      }
      if (s[r] > m) m = s[r];
    }
    double l = 0.0;
    for (size_t r = 0; r < row_count; r++) {
      s[r] = exp(s[r] - m);
      l += s[r];
    }
    for (size_t d = 0; d < head_dim; d++) {
      double acc = 0.0;
      for (size_t r = 0; r < row_count; r++) acc += s[r] * (double)values[r * vector_len + kv * head_dim + d];
      out[h * head_dim + d] = row_count ? acc / l : 0.0;
    }
  }
  free(s);
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* ring KV cache (layer.rs)                                           */
/* ------------------------------------------------------------------ */

int orc_ring_init(orc_ring *r, int64_t max_tokens, int64_t vector_len, int64_t block_tokens,
                  float *keys, float *values, orc_run *runs, int64_t run_cap) {
  if (max_tokens <= 0 || vector_len <= 0 || block_tokens <= 0) return ORC_ERR_INVALID_SHAPE;
  memset(r, 0, sizeof(*r));
  r->max_tokens = max_tokens;
  r->vector_len = vector_len;
  r->block_tokens = block_tokens;
  r->keys = keys;
  r->values = values;
  r->runs = runs;
  r->run_cap = run_cap;
  memset(keys, 0, (size_t)(max_tokens * vector_len) * sizeof(float));
  memset(values, 0, (size_t)(max_tokens * vector_len) * sizeof(float));
  return ORC_OK;
}

/* layer.rs:1089-1106 append_active_block_run */
static int ring_append_run(orc_ring *r, int64_t logical, int64_t physical) {
  if (physical >= r->max_tokens) return ORC_ERR_INVALID_SHAPE;
  int64_t block = physical / r->block_tokens;
  int64_t off = physical % r->block_tokens;
  if (r->run_count > 0) {
    orc_run *last = &r->runs[r->run_count - 1];
    if (last->block_index == block && last->logical_token_start + last->token_count == logical &&
        last->physical_token_start + last->token_count == physical &&
        last->block_token_start + last->token_count == off) {
      last->token_count += 1;
      return ORC_OK;
    }
  }
  if (r->run_count >= r->run_cap) return ORC_ERR_CAPACITY;
  orc_run run = {block, logical, physical, off, 1};
  r->runs[r->run_count++] = run;
  return ORC_OK;
}

/* layer.rs:1128-1152 remove_oldest_active_block_token */
static int ring_remove_oldest(orc_ring *r) {
  if (r->run_count == 0) return ORC_ERR_INVALID_SHAPE;
  orc_run *first = &r->runs[0];
  if (first->token_count == 1) {
    memmove(&r->runs[0], &r->runs[1], (size_t)(r->run_count - 1) * sizeof(orc_run));
    r->run_count -= 1;
  } else {
    first->physical_token_start += 1;
    first->block_token_start += 1;
    first->token_count -= 1;
  }
  for (int64_t i = 0; i < r->run_count; i++)
    if (r->runs[i].logical_token_start > 0) r->runs[i].logical_token_start -= 1;
  return ORC_OK;
}

static void ring_write(orc_ring *r, int64_t physical, const float *key, const float *value) {
  memcpy(r->keys + physical * r->vector_len, key, (size_t)r->vector_len * sizeof(float));
  memcpy(r->values + physical * r->vector_len, value, (size_t)r->vector_len * sizeof(float));
}

/* layer.rs:840-880 append_at_end_validated */
static int ring_append_at_end(orc_ring *r, const float *key, const float *value, int64_t *token_index,
                              int64_t *physical_index) {
  if (r->token_count == r->max_tokens) return ORC_ERR_CAPACITY;
  int64_t idx = r->token_count;
  ring_write(r, idx, key, value);
  int st = ring_append_run(r, idx, idx);
  if (st != ORC_OK) return st;
  r->token_count += 1;
  r->tokens_seen += 1;
  r->revision += 1;
  if (token_index) *token_index = idx;
  if (physical_index) *physical_index = idx;
  return ORC_OK;
}

int orc_ring_append(orc_ring *r, const float *key, const float *value, int64_t *token_index) {
  return ring_append_at_end(r, key, value, token_index, NULL);
}

/* layer.rs:765-805 append_sliding_with_metadata */
int orc_ring_append_sliding(orc_ring *r, const float *key, const float *value, int64_t *token_index,
                            int64_t *physical_index) {
  if (r->token_count < r->max_tokens) return ring_append_at_end(r, key, value, token_index, physical_index);
  int64_t physical = r->window_start;
  int64_t idx = r->max_tokens - 1;
  ring_write(r, physical, key, value);
  int st = ring_remove_oldest(r);
  if (st != ORC_OK) return st;
  st = ring_append_run(r, idx, physical);
  if (st != ORC_OK) return st;
  r->window_start = (r->window_start + 1) % r->max_tokens;
  r->tokens_seen += 1;
  r->revision += 1;
  if (token_index) *token_index = idx;
  if (physical_index) *physical_index = physical;
  return ORC_OK;
}

/* layer.rs:1046-1052,1528-1552 keys()/values(): logical order */
void orc_ring_logical_rows(const orc_ring *r, int tensor, float *out) {
  const float *src = tensor ? r->values : r->keys;
  for (int64_t i = 0; i < r->token_count; i++) {
    int64_t physical = (r->window_start + i) % r->max_tokens;
    memcpy(out + i * r->vector_len, src + physical * r->vector_len, (size_t)r->vector_len * sizeof(float));
  }
}

/* ------------------------------------------------------------------ */
/* paged pool                                                         */
/* ------------------------------------------------------------------ */

static int64_t k_index(const orc_pool *p, int64_t block, int32_t head, int32_t t, int32_t d) {
  return (((int64_t)block * p->kv_heads + head) * p->block_tokens + t) * p->head_dim + d;
}

static int64_t v_index(const orc_pool *p, int64_t block, int32_t head, int32_t t, int32_t d) {
  return (((int64_t)block * p->kv_heads + head) * p->head_dim + d) * p->block_tokens + t;
}

float orc_pool_elem(const orc_pool *p, int tensor, int64_t block, int32_t head, int32_t t, int32_t d) {
  int64_t idx = tensor ? v_index(p, block, head, t, d) : k_index(p, block, head, t, d);
  const void *base = tensor ? p->v : p->k;
  const void *scales = tensor ? p->v_scales : p->k_scales;
  switch (p->format) {
    case ORC_KV_BF16:
      return orc_bf16_to_f32(((const uint16_t *)base)[idx]);
    case ORC_KV_INT8: {
      float s = orc_f16_to_f32(((const uint16_t *)scales)[((int64_t)block * p->kv_heads + head) * p->block_tokens + t]);
      return (float)((const int8_t *)base)[idx] * s;
    }
    case ORC_KV_FP8_E4M3: {
      float s = ((const float *)scales)[(int64_t)block * p->kv_heads + head];
      return fp8_table[((const uint8_t *)base)[idx]] * s;
    }
    case ORC_KV_INT8_ROW: /* dequantize_int8_rows (format.rs:739-759): code * row scale */
      return (float)((const int8_t *)base)[idx] * ((const float *)scales)[(int64_t)block * p->block_tokens + t];
    case ORC_KV_F16: /* the f16 element widened to f32 (exact) */
      return orc_f16_to_f32(((const uint16_t *)base)[idx]);
    default:
      return NAN;
  }
}

static int check_table(const orc_pool *p, const int32_t *table, int32_t n_table, int32_t lo, int32_t hi) {
  if (lo < 0 || hi < lo || n_table <= 0) return ORC_ERR_INVALID_SHAPE;
  if (hi == lo) return ORC_OK;
  for (int32_t j = lo / p->block_tokens; j <= (hi - 1) / p->block_tokens; j++) {
    int32_t b = table[j % n_table];
    if (b < 0 || b >= p->n_blocks) return ORC_ERR_INVALID_SHAPE;
  }
  return ORC_OK;
}

int orc_pool_gather_f32(const orc_pool *p, const int32_t *table, int32_t n_table, int32_t lo,
                        int32_t hi, float *keys_out, float *values_out) {
  int st = check_table(p, table, n_table, lo, hi);
  if (st != ORC_OK) return st;
  int64_t vl = (int64_t)p->kv_heads * p->head_dim;
  for (int32_t pos = lo; pos < hi; pos++) {
    int64_t block = table[(pos / p->block_tokens) % n_table];
    int32_t t = pos % p->block_tokens;
    for (int32_t h = 0; h < p->kv_heads; h++)
      for (int32_t d = 0; d < p->head_dim; d++) {
        int64_t o = (int64_t)(pos - lo) * vl + (int64_t)h * p->head_dim + d;
        if (keys_out) keys_out[o] = orc_pool_elem(p, 0, block, h, t, d);
        if (values_out) values_out[o] = orc_pool_elem(p, 1, block, h, t, d);
      }
  }
  return ORC_OK;
}

int orc_pool_gather_raw(const orc_pool *p, const int32_t *table, int32_t n_table, int32_t lo,
                        int32_t hi, int tensor, void *out) {
  int st = check_table(p, table, n_table, lo, hi);
  if (st != ORC_OK) return st;
  int64_t vl = (int64_t)p->kv_heads * p->head_dim;
  for (int32_t pos = lo; pos < hi; pos++) {
    int64_t block = table[(pos / p->block_tokens) % n_table];
    int32_t t = pos % p->block_tokens;
    for (int32_t h = 0; h < p->kv_heads; h++)
      for (int32_t d = 0; d < p->head_dim; d++) {
        int64_t src = tensor ? v_index(p, block, h, t, d) : k_index(p, block, h, t, d);
        int64_t o = (int64_t)(pos - lo) * vl + (int64_t)h * p->head_dim + d;
        const void *base = tensor ? p->v : p->k;
        if (p->format == ORC_KV_BF16 || p->format == ORC_KV_F16)
          ((uint16_t *)out)[o] = ((const uint16_t *)base)[src];
        else
          ((uint8_t *)out)[o] = ((const uint8_t *)base)[src];
      }
  }
  return ORC_OK;
}

int orc_pool_write_bf16(const orc_pool *p, int64_t block, int32_t t, const float *key, const float *value) {
  if (p->format != ORC_KV_BF16 || block < 0 || block >= p->n_blocks || t < 0 || t >= p->block_tokens)
    return ORC_ERR_INVALID_SHAPE;
  uint16_t *k = (uint16_t *)p->k;
  uint16_t *v = (uint16_t *)p->v;
  for (int32_t h = 0; h < p->kv_heads; h++)
    for (int32_t d = 0; d < p->head_dim; d++) {
      k[k_index(p, block, h, t, d)] = orc_f32_to_bf16(key[h * p->head_dim + d]);
      v[v_index(p, block, h, t, d)] = orc_f32_to_bf16(value[h * p->head_dim + d]);
    }
  return ORC_OK;
}

/* One (query row, q head) item: select_kv_cache_head_rows over positions [lo, hi)
 * then the per-head loop of native_attention.rs:731-771. */
static int attend_item(const orc_pool *p, const int32_t *table, int32_t n_table, int32_t lo, int32_t hi,
                       int32_t kv_head, const uint16_t *q_bf16, float scale, float *out) {
  int32_t rows = hi - lo;
  int32_t D = p->head_dim;
  float *q = (float *)malloc((size_t)D * sizeof(float));
  float *key_rows = (float *)malloc(((size_t)rows * D + 1) * sizeof(float));
  float *value_rows = (float *)malloc(((size_t)rows * D + 1) * sizeof(float));
  float *scratch = (float *)malloc(((size_t)rows * 2 + 1) * sizeof(float));
  for (int32_t d = 0; d < D; d++) q[d] = orc_bf16_to_f32(q_bf16[d]);
  for (int32_t pos = lo; pos < hi; pos++) {
    int64_t block = table[(pos / p->block_tokens) % n_table];
    int32_t t = pos % p->block_tokens;
    for (int32_t d = 0; d < D; d++) {
      key_rows[(int64_t)(pos - lo) * D + d] = orc_pool_elem(p, 0, block, kv_head, t, d);
      value_rows[(int64_t)(pos - lo) * D + d] = orc_pool_elem(p, 1, block, kv_head, t, d);
    }
  }
  int st = attend_head(q, key_rows, value_rows, (size_t)rows, (size_t)D, scale, scratch, out);
  free(q);
  free(key_rows);
  free(value_rows);
  free(scratch);
  return st;
}

static int window_lo(int32_t end, int32_t window) {
  if (window <= 0) return 0;
  return end > window ? end - window : 0;
}

int orc_paged_decode(const orc_pool *p, int32_t num_seqs, int32_t q_heads, const int32_t *seq_lens,
                     const int32_t *block_tables, int32_t max_blocks, int32_t window,
                     const uint16_t *q_bf16, float scale, float *out, int threads) {
  if (num_seqs < 0 || q_heads <= 0 || p->kv_heads <= 0 || q_heads % p->kv_heads != 0 || max_blocks <= 0)
    return ORC_ERR_INVALID_SHAPE;
  int32_t groups = q_heads / p->kv_heads;
  int32_t D = p->head_dim;
  for (int32_t b = 0; b < num_seqs; b++) {
    int32_t len = seq_lens[b];
    int st = check_table(p, block_tables + (int64_t)b * max_blocks, max_blocks, window_lo(len, window), len);
    if (st != ORC_OK) return st;
  }
  int64_t items = (int64_t)num_seqs * q_heads;
  int status = ORC_OK;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 1 ? threads : 1) if (threads > 1)
#endif
  for (int64_t it = 0; it < items; it++) {
    int32_t b = (int32_t)(it / q_heads);
    int32_t h = (int32_t)(it % q_heads);
    int32_t len = seq_lens[b];
    int st = attend_item(p, block_tables + (int64_t)b * max_blocks, max_blocks, window_lo(len, window), len,
                         h / groups, q_bf16 + ((int64_t)b * q_heads + h) * D, scale,
                         out + ((int64_t)b * q_heads + h) * D);
    if (st != ORC_OK) {
#ifdef _OPENMP
#pragma omp critical
#endif
      status = st;
    }
  }
  (void)threads;
  return status;
}

int orc_paged_prefill_rows(const orc_pool *p, int32_t b, int32_t q_heads, const int32_t *chunk_starts,
                           const int32_t *context_lens, const int32_t *block_tables, int32_t max_blocks,
                           int32_t window, const uint16_t *q_bf16, float scale, float *out,
                           int32_t row_lo, int32_t row_hi, int threads) {
  if (q_heads <= 0 || p->kv_heads <= 0 || q_heads % p->kv_heads != 0 || max_blocks <= 0)
    return ORC_ERR_INVALID_SHAPE;
  int32_t groups = q_heads / p->kv_heads;
  int32_t D = p->head_dim;
  int32_t c0 = chunk_starts[b];
  int32_t chunk = chunk_starts[b + 1] - c0;
  int32_t ctx = context_lens[b];
  if (chunk < 0 || ctx < chunk || row_lo < 0 || row_hi > chunk) return ORC_ERR_INVALID_SHAPE;
  const int32_t *table = block_tables + (int64_t)b * max_blocks;
  int st0 = check_table(p, table, max_blocks, window_lo(ctx - chunk + row_lo + 1, window), ctx);
  if (st0 != ORC_OK) return st0;
  int64_t items = (int64_t)(row_hi - row_lo) * q_heads;
  int status = ORC_OK;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 1 ? threads : 1) if (threads > 1)
#endif
  for (int64_t it = 0; it < items; it++) {
    int32_t i = row_lo + (int32_t)(it / q_heads);
    int32_t h = (int32_t)(it % q_heads);
    int32_t pos = ctx - chunk + i;
    int64_t row = (int64_t)c0 + i;
    int st = attend_item(p, table, max_blocks, window_lo(pos + 1, window), pos + 1, h / groups,
                         q_bf16 + (row * q_heads + h) * D, scale, out + (row * q_heads + h) * D);
    if (st != ORC_OK) {
#ifdef _OPENMP
#pragma omp critical
#endif
      status = st;
    }
  }
  (void)threads;
  return status;
}

int orc_paged_prefill(const orc_pool *p, int32_t num_seqs, int32_t q_heads, const int32_t *chunk_starts,
                      const int32_t *context_lens, const int32_t *block_tables, int32_t max_blocks,
                      int32_t window, const uint16_t *q_bf16, float scale, float *out, int threads) {
  for (int32_t b = 0; b < num_seqs; b++) {
    int32_t chunk = chunk_starts[b + 1] - chunk_starts[b];
    int st = orc_paged_prefill_rows(p, b, q_heads, chunk_starts, context_lens, block_tables, max_blocks,
                                    window, q_bf16, scale, out, 0, chunk, threads);
    if (st != ORC_OK) return st;
  }
  return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* quantisation                                                       */
/* ------------------------------------------------------------------ */

/* format.rs:702-737 quantize_int8_rows */
int orc_quantize_int8_rows(const float *x, size_t rows, size_t vector_len, int8_t *codes, float *scales) {
  if (rows == 0 || vector_len == 0) return ORC_ERR_INVALID_SHAPE;
  for (size_t r = 0; r < rows; r++) {
    const float *row = x + r * vector_len;
    float max_abs = 0.0f;
    for (size_t i = 0; i < vector_len; i++) {
      if (!isfinite(row[i])) return ORC_ERR_NON_FINITE;
      max_abs = fmaxf(max_abs, fabsf(row[i]));
    }
    float scale = max_abs == 0.0f ? 0.0f : max_abs / 127.0f;
    for (size_t i = 0; i < vector_len; i++) {
      float c = scale == 0.0f ? 0.0f : roundf(row[i] / scale);
      if (c > 127.0f) c = 127.0f;
      if (c < -127.0f) c = -127.0f;
      codes[r * vector_len + i] = (int8_t)c;
    }
    scales[r] = scale;
  }
  return ORC_OK;
}

/* format.rs:739-759 dequantize_int8_rows */
void orc_dequantize_int8_rows(const int8_t *codes, const float *scales, size_t rows, size_t vector_len,
                              float *out) {
  for (size_t r = 0; r < rows; r++)
    for (size_t i = 0; i < vector_len; i++) out[r * vector_len + i] = (float)codes[r * vector_len + i] * scales[r];
}

int orc_quantize_int8_head(const float *x, int32_t n, int8_t *codes, uint16_t *scale_f16) {
  float max_abs = 0.0f;
  for (int32_t i = 0; i < n; i++) {
    if (!isfinite(x[i])) return ORC_ERR_NON_FINITE;
    max_abs = fmaxf(max_abs, fabsf(x[i]));
  }
  uint16_t s16 = orc_f32_to_f16(max_abs == 0.0f ? 0.0f : max_abs / 127.0f);
  float s = orc_f16_to_f32(s16);
  if (!isfinite(s)) return ORC_ERR_NON_FINITE;
  for (int32_t i = 0; i < n; i++) {
    float c = s == 0.0f ? 0.0f : roundf(x[i] / s);
    if (c > 127.0f) c = 127.0f;
    if (c < -127.0f) c = -127.0f;
    codes[i] = (int8_t)c;
  }
  *scale_f16 = s16;
  return ORC_OK;
}

int orc_quantize_fp8_block(const float *x, int32_t n, uint8_t *codes, float *scale) {
  float max_abs = 0.0f;
  for (int32_t i = 0; i < n; i++) {
    if (!isfinite(x[i])) return ORC_ERR_NON_FINITE;
    max_abs = fmaxf(max_abs, fabsf(x[i]));
  }
  float s = max_abs == 0.0f ? 0.0f : max_abs / 448.0f;
  for (int32_t i = 0; i < n; i++) codes[i] = s == 0.0f ? 0 : orc_f32_to_fp8e4m3(x[i] / s);
  *scale = s;
  return ORC_OK;
}

int orc_append_fp8_token(uint8_t *codes, int32_t dim, float *scale, int32_t off, const float *x) {
  float max_abs = 0.0f;
  for (int32_t d = 0; d < dim; d++) {
    if (!isfinite(x[d])) return ORC_ERR_NON_FINITE;
    max_abs = fmaxf(max_abs, fabsf(x[d]));
  }
  const float s_old = off == 0 ? 0.0f : *scale;
  const float cand = max_abs == 0.0f ? 0.0f : max_abs / 448.0f;
  const float s_new = fmaxf(s_old, cand);
  if (s_new != s_old)
    for (int32_t u = 0; u < off; u++)
      for (int32_t d = 0; d < dim; d++) {
        const float v = s_old == 0.0f ? 0.0f : orc_fp8e4m3_to_f32(codes[u * dim + d]) * s_old;
        codes[u * dim + d] = orc_f32_to_fp8e4m3(v / s_new);
      }
  for (int32_t d = 0; d < dim; d++) codes[off * dim + d] = s_new == 0.0f ? 0 : orc_f32_to_fp8e4m3(x[d] / s_new);
  *scale = s_new;
  return ORC_OK;
}
