// Device helpers shared by the HIP kernels of libllm_hip (decode, prefill, KV writes).
#pragma once

#include "llh_internal.h"

namespace llh {

// f32 -> bf16 bits, round to nearest even; NaN stays NaN (quiet bit set).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// f32 -> fp16 bits, round to nearest even (v_cvt_f16_f32): beyond the fp16 range
// an infinity, NaN stays NaN -- a float -> half conversion.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// int8 code of x with scale s: clamp(round_half_away(x / s), -127, 127), 0 for
// s = 0 -- the symmetric rule of crates/llm-kv-cache/src/format.rs:711-735 (Rust
// f32::round rounds half away from zero, as roundf does).  Shared by the KV
// writes and the fused append of the decode kernels, so both store identical bytes.
__device__ __forceinline__ int8_t quant_int8(float x, float s) {
  if (s == 0.0f) return 0;
  float c = roundf(__fdiv_rn(x, s));
  c = fminf(fmaxf(c, -127.0f), 127.0f);
  return (int8_t)c;
}

// x / s rounded to nearest even for a divisor s > 0 shared by many x, given
// r = RN(1 / s): Markstein's method, q = RN(x r), e = x - q s (exact by fma),
// RN(q + e r), with x's sign (which restores -0).  Three instructions instead of a
// correctly rounded division per element.  Used only where tests/quotient_check.c
// shows exhaustively that its codes equal those of the correctly rounded quotient
// (under IEEE and flush-to-zero arithmetic alike).
__device__ __forceinline__ float div_shared(float x, float s, float r) {
  const float q = __fmul_rn(x, r);
  return __builtin_copysignf(__builtin_fmaf(__builtin_fmaf(-q, s, x), r, q), x);
}

// OCP e4m3fn encode in integer arithmetic: round to nearest even, saturate to
// +-448, NaN -> 0x7f.  The reference rule for encode_e4m3 below
// (llh_debug_fp8_encode_check compares the two on every f32).
__device__ __forceinline__ uint8_t encode_e4m3_soft(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (uint8_t)(sign | 0x7fu);
  if (__uint_as_float(au) >= 448.0f) return (uint8_t)(sign | 0x7eu);
  const uint32_t exp = au >> 23;
  uint32_t man = au & 0x7fffffu;
  const int e = (int)exp - 127 + 7;
  if (e <= 0) {
    if (exp == 0) return (uint8_t)sign;
    man |= 0x800000u;
    const int shift = 21 - e;
    if (shift > 24) return (uint8_t)sign;
    uint32_t q = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint8_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 3) | (man >> 20);
  const uint32_t rem = man & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
  if (q > 0x7eu) q = 0x7eu;
  return (uint8_t)(sign | q);
}

// OCP e4m3fn codes of a and b into bytes 0-1 (HI: bytes 2-3) of old: v_cvt_pk_fp8_f32
// (round to nearest even) on the inputs clamped to +-448, which gives encode_e4m3_soft's
// code for every f32 but NaN (checked exhaustively on gfx950 by
// llh_debug_fp8_encode_check).
template <bool HI>
__device__ __forceinline__ uint32_t e4m3x2(float a, float b, uint32_t old) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, -448.0f, 448.0f),
                                                   __builtin_amdgcn_fmed3f(b, -448.0f, 448.0f), (int)old, HI);
}
__device__ __forceinline__ uint8_t encode_e4m3(float x) { return (uint8_t)e4m3x2<false>(x, 0.0f, 0u); }

// fp8 e4m3 code as f32 (exact).
__device__ __forceinline__ float decode_e4m3(uint32_t code) { return __builtin_amdgcn_cvt_pk_f32_fp8(code, false)[0]; }

// The attention output gate of Qwen3.5 / 3.6 (attn_output_gate): attention * sigmoid(g)
// per output element, sigmoid_f32(g) = 1 / (1 + exp(-g)) (crates/llm-backend/src/core/
// math.rs:472-474, applied at native_attention.rs:765-770,775-781).  gate: bf16 bits, or
// null for no gate.
__device__ __forceinline__ float gated(float v, const uint16_t *gate, size_t idx) {
  if (!gate) return v;
  const float g = __uint_as_float((uint32_t)gate[idx] << 16);
  return v * (1.0f / (1.0f + expf(-g)));
}

// One dequantised K (tensor 0) or V (tensor 1) element of any pool format and
// shape: token t of block blk, kv head h, dim d (K rows token-major, V rows
// dim-major).
__device__ __forceinline__ float pool_elem(const PoolView &p, int tensor, int64_t blk, int h, int t, int d) {
  const int64_t bh = blk * p.kv_heads + h;
  const int64_t idx = tensor ? (bh * p.head_dim + d) * p.block_tokens + t : (bh * p.block_tokens + t) * p.head_dim + d;
  const void *base = tensor ? p.v : p.k;
  const void *sc = tensor ? p.v_scales : p.k_scales;
  if (p.format == kBf16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(base)[idx] << 16);
  if (p.format == kF16) return (float)__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t *>(base)[idx]);
  if (p.format == kInt8) {
    const float s =
        (float)__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t *>(sc)[int8_scale_index(bh, t, p.block_tokens)]);
    return (float)reinterpret_cast<const int8_t *>(base)[idx] * s;
  }
  if (p.format == kInt8Row)  // one f32 scale per token row of the block (all heads)
    return (float)reinterpret_cast<const int8_t *>(base)[idx] * reinterpret_cast<const float *>(sc)[blk * p.block_tokens + t];
  const uint32_t code = reinterpret_cast<const uint8_t *>(base)[idx];
  return __builtin_amdgcn_cvt_pk_f32_fp8(code, false)[0] * reinterpret_cast<const float *>(sc)[fp8_scale_index(bh)];
}

}  // namespace llh
