// KV writes into the paged pool (quantise on write) and the bit-exact gather.
//
// write_blocks: whole blocks from token-major bf16 rows.  Replaces the
//   per-append re-quantisation of a whole block in LayerInt8KvStore::update_block
//   (crates/llm-kv-cache/src/format.rs:262-276) and the f32->f16 block upload
//   of the Metal mirror (crates/llm-native-runtime/src/native_matvec.rs:384-465).
// append: single token rows at absolute slots (the device half of
//   append_kv_cache_sliding_f32, crates/llm-backend/src/core/native_matvec.rs:643-653);
//   fp8 blocks are re-quantised as tokens arrive, as the reference re-quantises
//   a block on every int8 append (crates/llm-kv-cache/src/layer.rs:1396-1408).
// gather: raw elements of a sequence's positions through its block table
//   (select_head_rows_*, crates/llm-metal/src/device/shaders/generic.metal:310-360).
//
// Quantisation arithmetic matches the oracle bit for bit: int8 scale =
// f16(absmax / 127) and codes = clamp(round_half_away(x / scale), -127, 127)
// with the rounded scale (the symmetric rule of format.rs:702-737 at per
// (token, head) granularity); fp8 scale = absmax / 448 per (block, head) and
// codes are OCP e4m3fn, round to nearest even, saturating.
#include "device_common.h"

namespace llh {

namespace {

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Max over the 16 lanes of a DPP row (lanes 16g .. 16g+15), in every lane of
// the row: quad butterflies (quad_perm [1,0,3,2] and [2,3,0,1]), then the row
// rotated by 4 and by 8 lanes.  No LDS round trip.
template <int CTRL>
__device__ __forceinline__ float row_dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, row_dpp<0xB1>(v));
  v = fmaxf(v, row_dpp<0x4E>(v));
  v = fmaxf(v, row_dpp<0x124>(v));
  v = fmaxf(v, row_dpp<0x128>(v));
  return v;
}

// Max over the wavefront, in every lane: the row maxima, then v_permlane16_swap
// and v_permlane32_swap of the register with itself (each leaves one row, or
// half, of every pair in each result register, so the max of the two covers
// the pair).  No LDS round trip.
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
}

// Eight bf16 elements as eight fp16 ones (round to nearest even).
__device__ __forceinline__ uint4 bf16x8_to_f16x8(uint4 w) {
  uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++)
    u[j] = (uint32_t)f32_to_f16_bits(__uint_as_float(u[j] << 16)) |
           ((uint32_t)f32_to_f16_bits(__uint_as_float(u[j] & 0xffff0000u)) << 16);
  return make_uint4(u[0], u[1], u[2], u[3]);
}

// Whole 16-token blocks of head_dim 128, every pool format but int8-row: one
// workgroup of 256 lanes per (block, head).  Lane (t = lane / 16, c = lane % 16)
// loads the 16 B of token t at dims 8c .. 8c+7 of K and of V (coalesced; fp16
// pools convert them in registers), writes K rows straight out, and V is
// transposed through LDS so that every lane then writes 16 B (bf16 / fp16) or
// 8 B (int8 / fp8) of one dim row: every global access is a full,
// coalesced vector access.  int8: the per-(token, head) scale is the 16 lanes'
// absmax, then the same f16 rounding and code rule as the generic kernel; fp8:
// the per-(block, head) scale is the workgroup's absmax / 448, then the generic
// kernel's encode, so both kernels write identical bytes.
__global__ __launch_bounds__(256) void write_blocks_d128_kernel(const WriteBlocksArgs a) {
  constexpr int BT = 16, Dh = 128;
  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int t = tid >> 4, c = tid & 15;
  const int Hkv = a.pool.kv_heads;
  const int blk = a.blocks[i];
  if (blk < 0 || (int64_t)blk >= a.pool.n_blocks) {
    if (tid == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  const size_t src = (((size_t)i * BT + t) * Hkv + h) * Dh + 8 * c;
  uint4 kw = *reinterpret_cast<const uint4 *>(a.k + src);
  uint4 vw = *reinterpret_cast<const uint4 *>(a.v + src);
  const int d = tid >> 1, half = tid & 1;  // the dim row and token half this lane writes after the transpose
  if (is16(a.pool.format)) {
    if (a.pool.format == kF16) {  // each bf16 element widened (exact), then rounded to fp16
      kw = bf16x8_to_f16x8(kw);
      vw = bf16x8_to_f16x8(vw);
    }
    __shared__ uint16_t lv[BT][Dh + 8];
    *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.k_dst) + (bh * BT + t) * Dh + 8 * c) = kw;
    *reinterpret_cast<uint4 *>(&lv[t][8 * c]) = vw;
    __syncthreads();
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
      w[j] = (uint32_t)lv[8 * half + 2 * j][d] | ((uint32_t)lv[8 * half + 2 * j + 1][d] << 16);
    *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.v_dst) + (bh * Dh + d) * BT + 8 * half) =
        make_uint4(w[0], w[1], w[2], w[3]);
    return;
  }
  // quantised blocks: a NaN or an infinity in the block's rows is NonFiniteValue
  // in the reference (format.rs:713-716): flagged, and the block is left as it was.
  // Each wave posts its verdict in LDS; the workgroup reads the four after a barrier
  // the kernel has anyway (fp8: the absmax reduction; int8: the V transpose), before
  // any global store.
  bool bad = false;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t u[2] = {(&kw.x)[j], (&vw.x)[j]};
#pragma unroll
    for (int k = 0; k < 2; k++)
      bad = bad || (u[k] & 0x7f80u) == 0x7f80u || (u[k] & 0x7f800000u) == 0x7f800000u;
  }
  __shared__ __align__(16) uint32_t wave_bad[4];
  {
    const uint32_t wb = __any(bad) ? 1u : 0u;
    if ((tid & 63) == 0) wave_bad[tid >> 6] = wb;
  }
  const auto block_bad = [&]() {
    const uint4 f = *reinterpret_cast<const uint4 *>(wave_bad);
    return (f.x | f.y | f.z | f.w) != 0u;
  };
  __shared__ uint8_t lq[BT][Dh + 16];
  uint32_t codes[2][2];
  uint16_t s16b[2] = {0u, 0u};  // int8: the token's fp16 K and V scales
  if (a.pool.format == kFp8) {
    // one f32 scale per (block, head) and tensor: absmax over the block / 448,
    // codes as the generic kernel computes them (RNE e4m3 of x / scale)
    __shared__ float red[2][4];
    float x[2][8];
    float mx[2] = {0.0f, 0.0f};
#pragma unroll
    for (int tensor = 0; tensor < 2; tensor++) {
      const uint4 wv = tensor ? vw : kw;
      const uint32_t u[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        x[tensor][2 * j] = bf16_to_f32((uint16_t)(u[j] & 0xffffu));
        x[tensor][2 * j + 1] = bf16_to_f32((uint16_t)(u[j] >> 16));
        mx[tensor] = fmaxf(mx[tensor], fmaxf(fabsf(x[tensor][2 * j]), fabsf(x[tensor][2 * j + 1])));
      }
      mx[tensor] = wave_max(mx[tensor]);
      if ((tid & 63) == 0) red[tensor][tid >> 6] = mx[tensor];
    }
    __syncthreads();
    if (block_bad()) {
      if (tid == 0) atomicOr(a.err, kErrNonFinite);
      return;
    }
#pragma unroll
    for (int tensor = 0; tensor < 2; tensor++) {
      const float m = fmaxf(fmaxf(red[tensor][0], red[tensor][1]), fmaxf(red[tensor][2], red[tensor][3]));
      const float sc = m == 0.0f ? 0.0f : __fdiv_rn(m, 448.0f);
      uint32_t q[2] = {0u, 0u};
      if (sc >= 0x1p-90f) {  // block-uniform: the shared-divisor quotient (div_shared)
        const float rr = __fdiv_rn(1.0f, sc);
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; j++) y[j] = div_shared(x[tensor][j], sc, rr);
#pragma unroll
        for (int k = 0; k < 2; k++)
          q[k] = e4m3x2<true>(y[4 * k + 2], y[4 * k + 3], e4m3x2<false>(y[4 * k], y[4 * k + 1], 0u));
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const uint32_t code = sc == 0.0f ? 0u : encode_e4m3(__fdiv_rn(x[tensor][j], sc));
          q[j >> 2] |= code << (8 * (j & 3));
        }
      }
      codes[tensor][0] = q[0];
      codes[tensor][1] = q[1];
      if (tid == 0) reinterpret_cast<float *>(tensor ? a.vs_dst : a.ks_dst)[fp8_scale_index(bh)] = sc;
    }
  } else {
  // int8 with per (token, head) fp16 scales
#pragma unroll
  for (int tensor = 0; tensor < 2; tensor++) {
    const uint4 wv = tensor ? vw : kw;
    const uint32_t u[4] = {wv.x, wv.y, wv.z, wv.w};
    float x[8];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      x[2 * j] = bf16_to_f32((uint16_t)(u[j] & 0xffffu));
      x[2 * j + 1] = bf16_to_f32((uint16_t)(u[j] >> 16));
      mx = fmaxf(mx, fmaxf(fabsf(x[2 * j]), fabsf(x[2 * j + 1])));
    }
    mx = row16_max(mx);  // the token's 16 lanes
    const _Float16 s16 = (_Float16)(mx == 0.0f ? 0.0f : __fdiv_rn(mx, 127.0f));
    const float sc = (float)s16;
    uint32_t q[2] = {0u, 0u};
    if (sc > 0.0f && sc < INFINITY) {  // (per token row) the shared-divisor quotient (div_shared)
      // Rust's round (half away from zero) as trunc(y + copysign(0.5, y)): not that rule
      // for every float, but for every quotient this kernel forms (tests/quotient_check.c);
      // the integer c + 1.5 * 2^23 holds c's two's-complement byte in its low mantissa byte
      const float rr = __fdiv_rn(1.0f, sc);
      uint32_t cb[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float y = div_shared(x[j], sc, rr);
        const float c = __builtin_amdgcn_fmed3f(__builtin_truncf(y + __builtin_copysignf(0.5f, y)), -127.0f, 127.0f);
        cb[j] = __float_as_uint(c + 12582912.0f);
      }
#pragma unroll
      for (int k = 0; k < 2; k++)
        q[k] = __builtin_amdgcn_perm(cb[4 * k + 1], cb[4 * k], 0x0c0c0400u) |
               __builtin_amdgcn_perm(cb[4 * k + 3], cb[4 * k + 2], 0x04000c0cu);
    } else {
#pragma unroll
      for (int j = 0; j < 8; j++) q[j >> 2] |= (uint32_t)(uint8_t)quant_int8(x[j], sc) << (8 * (j & 3));
    }
    codes[tensor][0] = q[0];
    codes[tensor][1] = q[1];
    s16b[tensor] = __builtin_bit_cast(uint16_t, s16);
  }
  }
  // one-byte codes (int8 / fp8): K rows straight out, V transposed through LDS
  *reinterpret_cast<uint2 *>(&lq[t][8 * c]) = make_uint2(codes[1][0], codes[1][1]);
  __syncthreads();
  if (a.pool.format != kFp8 && block_bad()) {  // fp8 checked at its reduction barrier
    if (tid == 0) atomicOr(a.err, kErrNonFinite);
    return;
  }
  *reinterpret_cast<uint2 *>(reinterpret_cast<int8_t *>(a.k_dst) + (bh * BT + t) * Dh + 8 * c) =
      make_uint2(codes[0][0], codes[0][1]);
  if (a.pool.format != kFp8 && c < 2)
    reinterpret_cast<uint16_t *>(c ? a.vs_dst : a.ks_dst)[int8_scale_index(bh, t, BT)] = c ? s16b[1] : s16b[0];
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int j = 0; j < 8; j++) w[j >> 2] |= (uint32_t)lq[8 * half + j][d] << (8 * (j & 3));
  *reinterpret_cast<uint2 *>(reinterpret_cast<int8_t *>(a.v_dst) + (bh * Dh + d) * BT + 8 * half) = make_uint2(w[0], w[1]);
}

// One workgroup per (block i, kv head).  Source rows src[i][t][h][d].
// bf16 / fp16 pools at head_dim 256 (the Qwen3.5 / 3.6 full-attention layers), 16-token
// blocks, 16-byte aligned rows: write_blocks_d128_kernel's 16-bit path at twice the row
// width.  One workgroup of 512 per (block i, kv head); thread tid loads 16 bytes of token
// tid/32's K and V rows (dims 8(tid%32) ..), stores K straight out and V through LDS, then
// writes 16 bytes of V^T dim row tid/2 (tokens 8(tid&1) ..).
__global__ __launch_bounds__(512) void write_blocks16_d256_kernel(const WriteBlocksArgs a) {
  constexpr int BT = 16, Dh = 256;
  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int tid = threadIdx.x;
  const int t = tid >> 5, c = tid & 31;
  const int Hkv = a.pool.kv_heads;
  const int blk = a.blocks[i];
  if (blk < 0 || (int64_t)blk >= a.pool.n_blocks) {
    if (tid == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  const size_t src = (((size_t)i * BT + t) * Hkv + h) * Dh + 8 * c;
  uint4 kw = *reinterpret_cast<const uint4 *>(a.k + src);
  uint4 vw = *reinterpret_cast<const uint4 *>(a.v + src);
  if (a.pool.format == kF16) {  // each bf16 element widened (exact), then rounded to fp16
    kw = bf16x8_to_f16x8(kw);
    vw = bf16x8_to_f16x8(vw);
  }
  __shared__ uint16_t lv[BT][Dh + 8];
  *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.k_dst) + (bh * BT + t) * Dh + 8 * c) = kw;
  *reinterpret_cast<uint4 *>(&lv[t][8 * c]) = vw;
  __syncthreads();
  const int d = tid >> 1, half = tid & 1;
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; j++)
    w[j] = (uint32_t)lv[8 * half + 2 * j][d] | ((uint32_t)lv[8 * half + 2 * j + 1][d] << 16);
  *reinterpret_cast<uint4 *>(reinterpret_cast<uint16_t *>(a.v_dst) + (bh * Dh + d) * BT + 8 * half) =
      make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ __launch_bounds__(256) void write_blocks_kernel(const WriteBlocksArgs a) {
  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  const int blk = a.blocks[i];
  if (blk < 0 || (int64_t)blk >= a.pool.n_blocks) {
    if (threadIdx.x == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  auto src_idx = [&](int t, int d) { return (((size_t)i * BT + t) * Hkv + h) * Dh + d; };
  const int n = BT * Dh;
  if (a.pool.format == kBf16) {
    uint16_t *kd = reinterpret_cast<uint16_t *>(a.k_dst);
    uint16_t *vd = reinterpret_cast<uint16_t *>(a.v_dst);
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
      const int t = e / Dh, d = e % Dh;
      kd[(bh * BT + t) * Dh + d] = a.k[src_idx(t, d)];
      vd[(bh * Dh + d) * BT + t] = a.v[src_idx(t, d)];
    }
    return;
  }
  if (a.pool.format == kF16) {  // the bf16 rows converted (bf16 -> f32 exact, one rounding to fp16)
    uint16_t *kd = reinterpret_cast<uint16_t *>(a.k_dst);
    uint16_t *vd = reinterpret_cast<uint16_t *>(a.v_dst);
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
      const int t = e / Dh, d = e % Dh;
      kd[(bh * BT + t) * Dh + d] = f32_to_f16_bits(bf16_to_f32(a.k[src_idx(t, d)]));
      vd[(bh * Dh + d) * BT + t] = f32_to_f16_bits(bf16_to_f32(a.v[src_idx(t, d)]));
    }
    return;
  }
  {
    // quantised blocks: a NaN or an infinity in the block's rows is flagged
    // (NonFiniteValue, format.rs:713-716) and the block is left as it was
    bool bad = false;
    for (int e = threadIdx.x; e < n; e += blockDim.x)
      bad = bad || !isfinite(bf16_to_f32(a.k[src_idx(e / Dh, e % Dh)])) ||
            !isfinite(bf16_to_f32(a.v[src_idx(e / Dh, e % Dh)]));
    if (__syncthreads_or(bad)) {
      if (threadIdx.x == 0) atomicOr(a.err, kErrNonFinite);
      return;
    }
  }
  if (a.pool.format == kInt8) {
    // one wavefront per token row of this head
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int8_t *kd = reinterpret_cast<int8_t *>(a.k_dst);
    int8_t *vd = reinterpret_cast<int8_t *>(a.v_dst);
    uint16_t *ksd = reinterpret_cast<uint16_t *>(a.ks_dst);
    uint16_t *vsd = reinterpret_cast<uint16_t *>(a.vs_dst);
    for (int t = wave; t < BT; t += blockDim.x / 64) {
      for (int tensor = 0; tensor < 2; tensor++) {
        const uint16_t *src = tensor ? a.v : a.k;
        float mx = 0.0f;
        for (int d = lane; d < Dh; d += 64) mx = fmaxf(mx, fabsf(bf16_to_f32(src[src_idx(t, d)])));
        mx = wave_max(mx);
        const _Float16 s16 = (_Float16)(mx == 0.0f ? 0.0f : __fdiv_rn(mx, 127.0f));
        const float s = (float)s16;
        for (int d = lane; d < Dh; d += 64) {
          const int8_t code = quant_int8(bf16_to_f32(src[src_idx(t, d)]), s);
          if (tensor)
            vd[(bh * Dh + d) * BT + t] = code;
          else
            kd[(bh * BT + t) * Dh + d] = code;
        }
        if (lane == 0) (tensor ? vsd : ksd)[int8_scale_index(bh, t, BT)] = __builtin_bit_cast(uint16_t, s16);
      }
    }
    return;
  }
  // fp8: per (block, head) scale over all tokens of the block
  __shared__ float red[256];
  uint8_t *kd = reinterpret_cast<uint8_t *>(a.k_dst);
  uint8_t *vd = reinterpret_cast<uint8_t *>(a.v_dst);
  for (int tensor = 0; tensor < 2; tensor++) {
    const uint16_t *src = tensor ? a.v : a.k;
    float mx = 0.0f;
    for (int e = threadIdx.x; e < n; e += blockDim.x) mx = fmaxf(mx, fabsf(bf16_to_f32(src[src_idx(e / Dh, e % Dh)])));
    red[threadIdx.x] = mx;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
      if ((int)threadIdx.x < w) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + w]);
      __syncthreads();
    }
    const float s = red[0] == 0.0f ? 0.0f : __fdiv_rn(red[0], 448.0f);
    __syncthreads();
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
      const int t = e / Dh, d = e % Dh;
      const uint8_t code = s == 0.0f ? 0 : encode_e4m3(__fdiv_rn(bf16_to_f32(src[src_idx(t, d)]), s));
      if (tensor)
        vd[(bh * Dh + d) * BT + t] = code;
      else
        kd[(bh * BT + t) * Dh + d] = code;
    }
    if (threadIdx.x == 0) reinterpret_cast<float *>(tensor ? a.vs_dst : a.ks_dst)[fp8_scale_index(bh)] = s;
  }
}

// The reference's own int8 layout (format.rs:702-737): one f32 scale per token
// row over all kv heads, absmax / 127, codes round(x / scale) half away from zero,
// clamped to +-127.  One workgroup per block: wavefront w quantises tokens w,
// w + 4, ... of K, then of V (a row spans every head, so no per-head split).
__global__ __launch_bounds__(256) void write_blocks_row_kernel(const WriteBlocksArgs a) {
  const int i = blockIdx.x;
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int blk = a.blocks[i];
  if (blk < 0 || (int64_t)blk >= a.pool.n_blocks) {
    if (threadIdx.x == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const int vl = Hkv * Dh;
  for (int t = wave; t < BT; t += 4) {
    // a row holding a NaN or an infinity is NonFiniteValue in the reference
    // (format.rs:713-716): flagged, and the token's rows are left as they were
    bool finite = true;
    for (int tensor = 0; tensor < 2; tensor++) {
      const uint16_t *src = (tensor ? a.v : a.k) + ((size_t)i * BT + t) * vl;
      for (int e = lane; e < vl; e += 64) finite = finite && isfinite(bf16_to_f32(src[e]));
    }
    if (__any(!finite)) {
      if (lane == 0) atomicOr(a.err, kErrNonFinite);
      continue;
    }
    for (int tensor = 0; tensor < 2; tensor++) {
      const uint16_t *src = (tensor ? a.v : a.k) + ((size_t)i * BT + t) * vl;  // [h][d] of token t
      float mx = 0.0f;
      for (int e = lane; e < vl; e += 64) mx = fmaxf(mx, fabsf(bf16_to_f32(src[e])));
      mx = wave_max(mx);
      const float s = mx == 0.0f ? 0.0f : __fdiv_rn(mx, 127.0f);
      int8_t *dst = reinterpret_cast<int8_t *>(tensor ? a.v_dst : a.k_dst);
      for (int e = lane; e < vl; e += 64) {
        const int h = e / Dh, d = e % Dh;
        const size_t bh = (size_t)blk * Hkv + h;
        const int8_t code = quant_int8(bf16_to_f32(src[e]), s);
        if (tensor)
          dst[(bh * Dh + d) * BT + t] = code;
        else
          dst[(bh * BT + t) * Dh + d] = code;
      }
      if (lane == 0) reinterpret_cast<float *>(tensor ? a.vs_dst : a.ks_dst)[(size_t)blk * BT + t] = s;
    }
  }
}


// Appends one token row (this wavefront's kv head) into an fp8 block whose
// scale is per (block, head) and tensor: the block's scale becomes
// max(old scale, absmax(row) / 448); when it grows, the block's earlier tokens
// (offsets below `off`) are re-encoded from their dequantised values,
// encode(decode(code) * old / new); a token at offset 0 starts the block
// afresh (old scale 0).  `scale` is the block's current scale (kept in a
// register across the tokens of one block in one call); returns the new one.
template <typename ST, typename LD>
__device__ __forceinline__ float append_fp8_row(uint8_t *dst, bool dim_major, size_t bh, int BT, int Dh, int off,
                                                const ST *src, LD ld, float scale, int lane) {
  const float s_old = off == 0 ? 0.0f : scale;
  float mx = 0.0f;
  for (int d = lane; d < Dh; d += 64) mx = fmaxf(mx, fabsf(ld(src, d)));
  mx = wave_max(mx);
  const float cand = mx == 0.0f ? 0.0f : __fdiv_rn(mx, 448.0f);
  const float s_new = fmaxf(s_old, cand);
  auto at = [&](int u, int d) -> uint8_t & {
    return dim_major ? dst[(bh * Dh + d) * BT + u] : dst[(bh * BT + u) * Dh + d];
  };
  if (s_new != s_old) {
    for (int u = 0; u < off; u++)
      for (int d = lane; d < Dh; d += 64) {
        const float x = s_old == 0.0f ? 0.0f : decode_e4m3(at(u, d)) * s_old;
        at(u, d) = encode_e4m3(__fdiv_rn(x, s_new));
      }
  }
  for (int d = lane; d < Dh; d += 64) at(off, d) = s_new == 0.0f ? 0 : encode_e4m3(__fdiv_rn(ld(src, d), s_new));
  return s_new;
}

// Pool slot of append row i: a.slots[i], or (a.slots null) the new token of
// sequence i, position seq_lens[i] - 1 through its block-table row (kNoSlot when
// seq_lens[i] <= 0).
__device__ __forceinline__ int64_t append_slot(const AppendArgs &a, int i) {
  if (a.slots) return a.slots[i];
  const int pos = a.seq_lens[i] - 1;
  const int bt = a.pool.block_tokens;
  return pos < 0 ? kNoSlot
                 : (int64_t)a.tables[(size_t)i * a.max_blocks + (pos / bt) % a.max_blocks] * bt + pos % bt;
}

// Row element d of a bf16 or f32 source row as f32.
template <typename ST>
__device__ __forceinline__ float src_elem(const ST *p, int d) {
  if constexpr (sizeof(ST) == 4)
    return p[d];
  else
    return bf16_to_f32(p[d]);
}

// fp8 blocks: the tokens of one call that go to block blk are appended by the
// wavefront of the block's first token in call order, all of them, in that
// order (each may rescale the block).  Row i's wavefront returns at once when
// an earlier row of the call goes to the same block.
template <typename ST>
__device__ __forceinline__ void append_fp8_in_order(const AppendArgs &a, int i, int h, int64_t blk, size_t bh,
                                                    int lane) {
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  auto ld = [](const ST *p, int d) -> float { return src_elem<ST>(p, d); };
  for (int j0 = 0; j0 < i; j0 += 64) {
    const int j = j0 + lane;
    const int64_t sj = j < i ? append_slot(a, j) : (int64_t)-1;
    const bool same = sj >= 0 && sj / BT == blk;
    if (__any(same)) return;
  }
  float scale[2] = {reinterpret_cast<const float *>(a.ks_dst)[fp8_scale_index(bh)],
                    reinterpret_cast<const float *>(a.vs_dst)[fp8_scale_index(bh)]};
  // this call's tokens of the block, in call order: the slots are read 64 at a
  // time (one vector load per lane) and walked through a ballot mask
  for (int j0 = i; j0 < a.n; j0 += 64) {
    const int64_t sl = j0 + lane < a.n ? append_slot(a, j0 + lane) : (int64_t)-1;
    uint64_t pending = __ballot(sl >= 0 && sl / BT == blk);
    while (pending) {
      const int k = __builtin_ctzll(pending);
      pending &= pending - 1;
      const int j = j0 + k;
      const int64_t sj = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(sl >> 32), k) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)sl, k));
      const int offj = (int)(sj % BT);
      const ST *kj = reinterpret_cast<const ST *>(a.k) + ((size_t)j * Hkv + h) * Dh;
      const ST *vj = reinterpret_cast<const ST *>(a.v) + ((size_t)j * Hkv + h) * Dh;
      bool finite = true;
      for (int d = lane; d < Dh; d += 64) finite = finite && isfinite(ld(kj, d)) && isfinite(ld(vj, d));
      if (__any(!finite)) {
        if (lane == 0) atomicOr(a.err, kErrNonFinite);
        continue;
      }
      // this wavefront's earlier stores to the block are complete before it reads the block again
      if (j > i) __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
      scale[0] = append_fp8_row(reinterpret_cast<uint8_t *>(a.k_dst), false, bh, BT, Dh, offj, kj, ld, scale[0], lane);
      scale[1] = append_fp8_row(reinterpret_cast<uint8_t *>(a.v_dst), true, bh, BT, Dh, offj, vj, ld, scale[1], lane);
    }
  }
  if (lane == 0) {
    reinterpret_cast<float *>(a.ks_dst)[fp8_scale_index(bh)] = scale[0];
    reinterpret_cast<float *>(a.vs_dst)[fp8_scale_index(bh)] = scale[1];
  }
}

// fp8 blocks of 16 tokens x 128 dims, calls of at most 64 rows: append_kernel's fp8
// result (append_fp8_in_order, append_fp8_row's arithmetic bit for bit) in three
// memory round trips.  The call's slots (one per lane) and the row come first; a row
// that shares its block with a later row of the call takes the in-order path; else
// the block's scales and codes come together, and a scale that grows re-encodes the
// earlier tokens in registers.  Lane l holds K token l/4, bytes 32(l&3) .. +32, and
// V^T dims 2l, 2l + 1 (16 tokens each).
template <typename ST>
__global__ __launch_bounds__(64) void append_fp8_d128_kernel(const AppendArgs a) {
  constexpr int BT = 16, Dh = 128;
  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int Hkv = a.pool.kv_heads;
  const ST *ks = reinterpret_cast<const ST *>(a.k) + ((size_t)i * Hkv + h) * Dh;
  const ST *vs = reinterpret_cast<const ST *>(a.v) + ((size_t)i * Hkv + h) * Dh;
  const int64_t sl = lane < a.n ? append_slot(a, lane) : (int64_t)-1;
  float kx[2], vx[2], vp[2];  // K and V dims lane, lane + 64; V dims 2 lane, 2 lane + 1
#pragma unroll
  for (int r = 0; r < 2; r++) {
    kx[r] = src_elem<ST>(ks, lane + 64 * r);
    vx[r] = src_elem<ST>(vs, lane + 64 * r);
    vp[r] = src_elem<ST>(vs, 2 * lane + r);
  }
  const int64_t slot = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(sl >> 32), i) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)sl, i));
  if (slot == kNoSlot) return;  // a sequence with no new token (fused-append fallback)
  const int64_t blk = slot / BT;
  const int off = (int)(slot % BT);
  if (slot < 0 || blk >= a.pool.n_blocks) {
    if (lane == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  const bool same = sl >= 0 && sl / BT == blk;
  if (__ballot(same && lane < i)) return;  // an earlier row's wavefront appends this one
  if (__ballot(same && lane > i)) {
    append_fp8_in_order<ST>(a, i, h, blk, bh, lane);
    return;
  }
  uint8_t *kd = reinterpret_cast<uint8_t *>(a.k_dst) + bh * BT * Dh;
  uint8_t *vd = reinterpret_cast<uint8_t *>(a.v_dst) + bh * Dh * BT;
  float *ksc = reinterpret_cast<float *>(a.ks_dst) + fp8_scale_index(bh);
  float *vsc = reinterpret_cast<float *>(a.vs_dst) + fp8_scale_index(bh);
  const float sc_k = *ksc, sc_v = *vsc;
  const uint4 kc0 = reinterpret_cast<const uint4 *>(kd)[2 * lane], kc1 = reinterpret_cast<const uint4 *>(kd)[2 * lane + 1];
  const uint4 vc[2] = {reinterpret_cast<const uint4 *>(vd)[2 * lane], reinterpret_cast<const uint4 *>(vd)[2 * lane + 1]};
  if (__any(!(isfinite(kx[0]) && isfinite(kx[1]) && isfinite(vx[0]) && isfinite(vx[1])))) {
    if (lane == 0) atomicOr(a.err, kErrNonFinite);  // NonFiniteValue: the block is left as it was
    return;
  }
  float s_old[2], s_new[2];
#pragma unroll
  for (int tensor = 0; tensor < 2; tensor++) {
    const float *x = tensor ? vx : kx;
    const float mx = wave_max(fmaxf(fabsf(x[0]), fabsf(x[1])));
    const float cand = mx == 0.0f ? 0.0f : __fdiv_rn(mx, 448.0f);
    s_old[tensor] = off == 0 ? 0.0f : (tensor ? sc_v : sc_k);
    s_new[tensor] = fmaxf(s_old[tensor], cand);
  }
  auto enc = [](float v, float s) -> uint32_t { return s == 0.0f ? 0u : encode_e4m3(__fdiv_rn(v, s)); };
  auto recode = [](uint32_t code, float so, float s) -> uint32_t {
    const float x = so == 0.0f ? 0.0f : decode_e4m3(code) * so;
    return encode_e4m3(__fdiv_rn(x, s));
  };
  // K: the scale grew -> tokens before off re-encoded (32 bytes per lane); row off
  if (s_new[0] != s_old[0] && (lane >> 2) < off) {
    uint32_t w[8] = {kc0.x, kc0.y, kc0.z, kc0.w, kc1.x, kc1.y, kc1.z, kc1.w};
#pragma unroll
    for (int e = 0; e < 32; e++) {
      const uint32_t code = recode((w[e >> 2] >> (8 * (e & 3))) & 0xffu, s_old[0], s_new[0]);
      w[e >> 2] = (w[e >> 2] & ~(0xffu << (8 * (e & 3)))) | (code << (8 * (e & 3)));
    }
    reinterpret_cast<uint4 *>(kd)[2 * lane] = make_uint4(w[0], w[1], w[2], w[3]);
    reinterpret_cast<uint4 *>(kd)[2 * lane + 1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
#pragma unroll
  for (int r = 0; r < 2; r++) kd[off * Dh + lane + 64 * r] = (uint8_t)enc(kx[r], s_new[0]);
  // V: the scale grew -> this lane's two dim rows rewritten whole (tokens before
  // off re-encoded, the new token at off); else the new token's byte of each dim
  if (s_new[1] != s_old[1] && off > 0) {
#pragma unroll
    for (int r = 0; r < 2; r++) {
      uint32_t w[4] = {vc[r].x, vc[r].y, vc[r].z, vc[r].w};
#pragma unroll
      for (int u = 0; u < BT; u++) {
        if (u > off) break;
        const uint32_t old = (w[u >> 2] >> (8 * (u & 3))) & 0xffu;
        const uint32_t code = u == off ? enc(vp[r], s_new[1]) : recode(old, s_old[1], s_new[1]);
        w[u >> 2] = (w[u >> 2] & ~(0xffu << (8 * (u & 3)))) | (code << (8 * (u & 3)));
      }
      reinterpret_cast<uint4 *>(vd)[2 * lane + r] = make_uint4(w[0], w[1], w[2], w[3]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 2; r++) vd[(lane + 64 * r) * BT + off] = (uint8_t)enc(vx[r], s_new[1]);
  }
  if (lane == 0) {
    *ksc = s_new[0];
    *vsc = s_new[1];
  }
}

// One wavefront per token row i: the reference's int8 row layout (one f32
// scale over all kv heads of the row; write_blocks_row_kernel's rule).
template <typename ST>
__global__ __launch_bounds__(64) void append_row_kernel(const AppendArgs a) {
  const int i = blockIdx.x;
  const int lane = threadIdx.x;
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  const int64_t slot = append_slot(a, i);
  if (slot == kNoSlot) return;
  const int64_t blk = slot / BT;
  const int off = (int)(slot % BT);
  if (slot < 0 || blk >= a.pool.n_blocks) {
    if (lane == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const int vl = Hkv * Dh;
  auto ld_row = [&](int tensor, int e) -> float {
    const ST *src = reinterpret_cast<const ST *>(tensor ? a.v : a.k) + (size_t)i * vl;
    if constexpr (sizeof(ST) == 4)
      return src[e];
    else
      return bf16_to_f32(src[e]);
  };
  // a row holding a NaN or an infinity is NonFiniteValue in the reference
  // (format.rs:713-716): flagged, and the slot is left as it was
  bool finite = true;
  for (int tensor = 0; tensor < 2; tensor++)
    for (int e = lane; e < vl; e += 64) finite = finite && isfinite(ld_row(tensor, e));
  if (__any(!finite)) {
    if (lane == 0) atomicOr(a.err, kErrNonFinite);
    return;
  }
  for (int tensor = 0; tensor < 2; tensor++) {
    auto ld = [&](int e) -> float { return ld_row(tensor, e); };
    float mx = 0.0f;
    for (int e = lane; e < vl; e += 64) mx = fmaxf(mx, fabsf(ld(e)));
    mx = wave_max(mx);
    const float s = mx == 0.0f ? 0.0f : __fdiv_rn(mx, 127.0f);
    int8_t *dst = reinterpret_cast<int8_t *>(tensor ? a.v_dst : a.k_dst);
    for (int e = lane; e < vl; e += 64) {
      const int h = e / Dh, d = e % Dh;
      const size_t bh = (size_t)blk * Hkv + h;
      const int8_t code = quant_int8(ld(e), s);
      if (tensor)
        dst[(bh * Dh + d) * BT + off] = code;
      else
        dst[(bh * BT + off) * Dh + d] = code;
    }
    if (lane == 0) reinterpret_cast<float *>(tensor ? a.vs_dst : a.ks_dst)[blk * BT + off] = s;
  }
}

// One wavefront per (token row i, kv head).
template <typename ST>
__global__ __launch_bounds__(64) void append_kernel(const AppendArgs a) {
  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int lane = threadIdx.x;
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  const ST *ks = reinterpret_cast<const ST *>(a.k) + ((size_t)i * Hkv + h) * Dh;
  const ST *vs = reinterpret_cast<const ST *>(a.v) + ((size_t)i * Hkv + h) * Dh;
  auto ld = [](const ST *p, int d) -> float {
    if constexpr (sizeof(ST) == 4)
      return p[d];
    else
      return bf16_to_f32(p[d]);
  };
  // head_dim <= 128: the token's rows (two elements per lane) do not depend on
  // the slot, so they are loaded together with it and one memory round trip
  // covers both (the empty asm takes all five values, so neither load is
  // deferred behind the slot checks)
  const bool rows_in_regs = Dh <= 128;
  const int64_t slot = append_slot(a, i);
  uint32_t kraw[2] = {0u, 0u}, vraw[2] = {0u, 0u};  // the elements' bits as stored in k / v
  if (rows_in_regs) {
#pragma unroll
    for (int r = 0; r < 2; r++) {  // unconditional (clamped) loads: all four in flight at once
      const int d = min(lane + 64 * r, Dh - 1);
      if constexpr (sizeof(ST) == 4) {
        kraw[r] = __float_as_uint(ks[d]);
        vraw[r] = __float_as_uint(vs[d]);
      } else {
        kraw[r] = ks[d];
        vraw[r] = vs[d];
      }
    }
  }
  asm volatile("" ::"v"(kraw[0]), "v"(kraw[1]), "v"(vraw[0]), "v"(vraw[1]), "s"(slot));
  float kx[2], vx[2];
#pragma unroll
  for (int r = 0; r < 2; r++) {
    kx[r] = sizeof(ST) == 4 ? __uint_as_float(kraw[r]) : bf16_to_f32((uint16_t)kraw[r]);
    vx[r] = sizeof(ST) == 4 ? __uint_as_float(vraw[r]) : bf16_to_f32((uint16_t)vraw[r]);
  }
  if (slot == kNoSlot) return;  // a sequence with no new token (fused-append fallback)
  const int64_t blk = slot / BT;
  const int off = (int)(slot % BT);
  if (slot < 0 || blk >= a.pool.n_blocks) {
    if (lane == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  // calls f(d, k, v) for each element d of this lane's share of the rows
  auto for_elems = [&](auto f) __attribute__((always_inline)) {
    if (rows_in_regs) {
#pragma unroll
      for (int r = 0; r < 2; r++)
        if (lane + 64 * r < Dh) f(lane + 64 * r, kx[r], vx[r]);
    } else {
      for (int d = lane; d < Dh; d += 64) f(d, ld(ks, d), ld(vs, d));
    }
  };
  if (is16(a.pool.format)) {
    uint16_t *kd = reinterpret_cast<uint16_t *>(a.k_dst);
    uint16_t *vd = reinterpret_cast<uint16_t *>(a.v_dst);
    const bool f16 = a.pool.format == kF16;
    for_elems([&](int d, float k, float v) __attribute__((always_inline)) {
      kd[(bh * BT + off) * Dh + d] = f16 ? f32_to_f16_bits(k) : f32_to_bf16_rne(k);
      vd[(bh * Dh + d) * BT + off] = f16 ? f32_to_f16_bits(v) : f32_to_bf16_rne(v);
    });
    return;
  }
  if (a.pool.format == kFp8) {
    append_fp8_in_order<ST>(a, i, h, blk, bh, lane);
    return;
  }
  // int8 with per (token, head) fp16 scale; a NaN or an infinity in either row
  // is flagged and nothing of the token is written
  int8_t *kd = reinterpret_cast<int8_t *>(a.k_dst);
  int8_t *vd = reinterpret_cast<int8_t *>(a.v_dst);
  bool finite = true;
  for_elems([&](int, float k, float v) __attribute__((always_inline)) { finite = finite && isfinite(k) && isfinite(v); });
  if (__any(!finite)) {
    if (lane == 0) atomicOr(a.err, kErrNonFinite);
    return;
  }
  for (int tensor = 0; tensor < 2; tensor++) {
    float mx = 0.0f;
    for_elems([&](int, float k, float v) __attribute__((always_inline)) { mx = fmaxf(mx, fabsf(tensor ? v : k)); });
    mx = wave_max(mx);
    const _Float16 s16 = (_Float16)(mx == 0.0f ? 0.0f : __fdiv_rn(mx, 127.0f));
    const float s = (float)s16;
    for_elems([&](int d, float k, float v) __attribute__((always_inline)) {
      const int8_t code = quant_int8(tensor ? v : k, s);
      if (tensor)
        vd[(bh * Dh + d) * BT + off] = code;
      else
        kd[(bh * BT + off) * Dh + d] = code;
    });
    if (lane == 0)
      reinterpret_cast<uint16_t *>(tensor ? a.vs_dst : a.ks_dst)[int8_scale_index(bh, off, BT)] =
          __builtin_bit_cast(uint16_t, s16);
  }
}

__device__ __forceinline__ float load_f32(const PoolView &p, const void *base, const void *sc, size_t bh, size_t idx,
                                          int off) {
  if (p.format == kBf16) return bf16_to_f32(reinterpret_cast<const uint16_t *>(base)[idx]);
  if (p.format == kF16) return (float)__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t *>(base)[idx]);
  if (p.format == kInt8) {
    const float s = (float)__builtin_bit_cast(
        _Float16, reinterpret_cast<const uint16_t *>(sc)[int8_scale_index(bh, off, p.block_tokens)]);
    return (float)reinterpret_cast<const int8_t *>(base)[idx] * s;
  }
  if (p.format == kInt8Row)
    return (float)reinterpret_cast<const int8_t *>(base)[idx] *
           reinterpret_cast<const float *>(sc)[(bh / p.kv_heads) * p.block_tokens + off];
  return __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)reinterpret_cast<const uint8_t *>(base)[idx], false)[0] *
         reinterpret_cast<const float *>(sc)[fp8_scale_index(bh)];
}

// One wavefront per (slot, kv head): K and V of that token as f32 rows
// k[i][h][d], v[i][h][d] (V is stored d-major within a block).
__global__ __launch_bounds__(64) void export_rows_kernel(const ExportArgs a) {
  const int i = blockIdx.x;
  const int h = blockIdx.y;
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  const int64_t slot = a.slots[i];
  const int64_t blk = slot / BT;
  const int off = (int)(slot % BT);
  if (slot < 0 || blk >= a.pool.n_blocks) {
    if (threadIdx.x == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  const size_t orow = ((size_t)i * Hkv + h) * Dh;
  for (int d = threadIdx.x; d < Dh; d += 64) {
    a.k[orow + d] = load_f32(a.pool, a.pool.k, a.pool.k_scales, bh, (bh * BT + off) * Dh + d, off);
    a.v[orow + d] = load_f32(a.pool, a.pool.v, a.pool.v_scales, bh, (bh * Dh + d) * BT + off, off);
  }
}

// One wavefront per (position, kv head): raw elements out[pos-lo][h][d].
__global__ __launch_bounds__(64) void gather_kernel(const GatherArgs a) {
  const int r = blockIdx.x;
  const int h = blockIdx.y;
  const int pos = a.lo + r;
  const int BT = a.pool.block_tokens;
  const int Hkv = a.pool.kv_heads;
  const int Dh = a.pool.head_dim;
  int slot_blk, off;
  if (a.ring_tokens > 0) {
    const int slot = pos % a.ring_tokens;
    slot_blk = slot / BT;
    off = slot % BT;
  } else {
    slot_blk = (pos / BT) % a.max_blocks;
    off = pos % BT;
  }
  const int blk = slot_blk < a.max_blocks ? a.table[slot_blk] : -1;
  if (blk < 0 || (int64_t)blk >= a.pool.n_blocks) {
    if (threadIdx.x == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const size_t bh = (size_t)blk * Hkv + h;
  const size_t orow = ((size_t)r * Hkv + h) * Dh;
  const void *base = a.tensor ? a.pool.v : a.pool.k;
  const void *sc = a.tensor ? a.pool.v_scales : a.pool.k_scales;
  for (int d = threadIdx.x; d < Dh; d += 64) {
    const size_t idx = a.tensor ? (bh * Dh + d) * BT + off : (bh * BT + off) * Dh + d;
    if (a.out_f32)
      reinterpret_cast<float *>(a.out)[orow + d] = load_f32(a.pool, base, sc, bh, idx, off);
    else if (is16(a.pool.format))
      reinterpret_cast<uint16_t *>(a.out)[orow + d] = reinterpret_cast<const uint16_t *>(base)[idx];
    else
      reinterpret_cast<uint8_t *>(a.out)[orow + d] = reinterpret_cast<const uint8_t *>(base)[idx];
  }
}

// Every f32 bit pattern but NaNs: the fp8 encoder the kernels use (encode_e4m3,
// v_cvt_pk_fp8_f32 on clamped inputs) against the integer reference rule
// (encode_e4m3_soft); one count per thread, added once.
__global__ __launch_bounds__(256) void fp8_encode_check_kernel(unsigned long long *mismatches) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  unsigned long long bad = 0;
  for (uint64_t i = tid; i < (1ull << 32); i += stride) {
    const float x = __uint_as_float((uint32_t)i);
    if (x != x) continue;
    bad += encode_e4m3(x) != encode_e4m3_soft(x);
  }
  atomicAdd(mismatches, bad);
}

}  // namespace

hipError_t launch_fp8_encode_check(unsigned long long *mismatches, hipStream_t s) {
  hipLaunchKernelGGL(fp8_encode_check_kernel, dim3(8192), dim3(256), 0, s, mismatches);
  return hipGetLastError();
}

hipError_t launch_export_rows(const ExportArgs &a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  hipLaunchKernelGGL(export_rows_kernel, dim3(a.n, a.pool.kv_heads), dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_write_blocks(const WriteBlocksArgs &a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  const bool aligned = reinterpret_cast<uintptr_t>(a.k) % 16 == 0 && reinterpret_cast<uintptr_t>(a.v) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(a.k_dst) % 16 == 0 && reinterpret_cast<uintptr_t>(a.v_dst) % 16 == 0;
  const bool fast = a.pool.head_dim == 128 && a.pool.block_tokens == 16 && a.pool.format != kInt8Row && aligned;
  const bool fast256 = a.pool.head_dim == 256 && a.pool.block_tokens == 16 && is16(a.pool.format) && aligned;
  if (a.pool.format == kInt8Row)
    hipLaunchKernelGGL(write_blocks_row_kernel, dim3(a.n), dim3(256), 0, s, a);
  else if (fast)
    hipLaunchKernelGGL(write_blocks_d128_kernel, dim3(a.n, a.pool.kv_heads), dim3(256), 0, s, a);
  else if (fast256)
    hipLaunchKernelGGL(write_blocks16_d256_kernel, dim3(a.n, a.pool.kv_heads), dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL(write_blocks_kernel, dim3(a.n, a.pool.kv_heads), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_append(const AppendArgs &a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  if (a.pool.format == kInt8Row && a.src_f32)
    hipLaunchKernelGGL(append_row_kernel<float>, dim3(a.n), dim3(64), 0, s, a);
  else if (a.pool.format == kInt8Row)
    hipLaunchKernelGGL(append_row_kernel<uint16_t>, dim3(a.n), dim3(64), 0, s, a);
  else if (a.pool.format == kFp8 && a.pool.head_dim == 128 && a.pool.block_tokens == 16 && a.n <= 64 && a.src_f32)
    hipLaunchKernelGGL(append_fp8_d128_kernel<float>, dim3(a.n, a.pool.kv_heads), dim3(64), 0, s, a);
  else if (a.pool.format == kFp8 && a.pool.head_dim == 128 && a.pool.block_tokens == 16 && a.n <= 64)
    hipLaunchKernelGGL(append_fp8_d128_kernel<uint16_t>, dim3(a.n, a.pool.kv_heads), dim3(64), 0, s, a);
  else if (a.src_f32)
    hipLaunchKernelGGL(append_kernel<float>, dim3(a.n, a.pool.kv_heads), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL(append_kernel<uint16_t>, dim3(a.n, a.pool.kv_heads), dim3(64), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_gather(const GatherArgs &a, hipStream_t s) {
  if (a.hi <= a.lo) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(a.hi - a.lo, a.pool.kv_heads), dim3(64), 0, s, a);
  return hipGetLastError();
}

}  // namespace llh
