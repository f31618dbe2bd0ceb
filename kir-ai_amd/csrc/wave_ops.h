// Wavefront-level building blocks of the decode kernels (gfx950, wave64):
// non-temporal loads, packed bf16 arithmetic and DPP / permlane exchanges
// between lanes, all without an LDS round trip.
#pragma once

#include "device_common.h"

namespace llh {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// K/V are read once per step: non-temporal loads keep them from displacing
// the block tables, queries and partials in the caches (measured 8-12% faster
// on MI355X for C2).
__device__ __forceinline__ uint4 ld_nt16(const char *p) {
  const u32x4_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ uint2 ld_nt8(const char *p) {
  const u32x2_t t = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
  return make_uint2(t.x, t.y);
}
__device__ __forceinline__ uint32_t ld_nt4(const char *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Value of lane (l ^ 15) within its 16-lane row: every lane is written, so no
// old value is needed (mov_dpp leaves the destination's prior bits unused).
__device__ __forceinline__ float row_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
}

// Value of lane l ^ 16 / l ^ 32 without an LDS round trip: v_permlane16_swap
// (v_permlane32_swap) of a register with itself leaves the even rows' (low
// half's) values in both rows of each pair in r[0] and the odd rows' (high
// half's) in r[1].
__device__ __forceinline__ float xor16_other(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_other(float v, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((lane & 32) ? r[0] : r[1]);
}

// Sum over the 16 lanes of a DPP row; every lane receives the total.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}

// Sum over each 8-lane half of a DPP row.
__device__ __forceinline__ float row_sum8(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v;
}

// Value of lane n (0..15) of this lane's 16-lane row (DPP row_newbcast).  n
// must fold to a constant: callers pass unrolled loop indices.
__device__ __forceinline__ float row_bcast(float v, int n) {
  const int x = __float_as_int(v);
  switch (n) {
    case 0: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x150, 0xF, 0xF, false));
    case 1: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x151, 0xF, 0xF, false));
    case 2: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x152, 0xF, 0xF, false));
    case 3: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x153, 0xF, 0xF, false));
    case 4: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x154, 0xF, 0xF, false));
    case 5: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x155, 0xF, 0xF, false));
    case 6: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x156, 0xF, 0xF, false));
    case 7: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x157, 0xF, 0xF, false));
    case 8: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x158, 0xF, 0xF, false));
    case 9: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x159, 0xF, 0xF, false));
    case 10: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x15A, 0xF, 0xF, false));
    case 11: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x15B, 0xF, 0xF, false));
    case 12: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x15C, 0xF, 0xF, false));
    case 13: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x15D, 0xF, 0xF, false));
    case 14: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x15E, 0xF, 0xF, false));
    default: return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x15F, 0xF, 0xF, false));
  }
}

// Reduction over the four lanes l, l+4, l+8, l+12 of a 16-lane row (row_ror 4, 8).
__device__ __forceinline__ float row_max_stride4(float v) {
  v = fmaxf(v, dpp<0x124>(v));
  return fmaxf(v, dpp<0x128>(v));
}
__device__ __forceinline__ float row_sum_stride4(float v) {
  v += dpp<0x124>(v);
  return v + dpp<0x128>(v);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});  // round to nearest even
}

// x rounded to bf16 (nearest even), as f32: the value pack_bf16 stores for x
__device__ __forceinline__ float bf16_round(float x) { return bf16_lo(pack_bf16(x, 0.0f)); }

// acc + lo + hi of a packed bf16 pair, exactly (dot product with (1, 1) in f32)
__device__ __forceinline__ float dot2_ones(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair),
                                         __builtin_bit_cast(bf16x2_t, 0x3F803F80u), acc, false);
}

// The same three for packed fp16 pairs (v_dot2_f32_f16, f32 accumulation).
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
}
__device__ __forceinline__ uint32_t pack_f16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, f16x2_t{(_Float16)lo, (_Float16)hi});  // round to nearest even
}
__device__ __forceinline__ float dot2_ones_f16(uint32_t pair, float acc) {
  return dot2_f16(pair, 0x3C003C00u, acc);
}

// Format-generic forms for the 16-bit pools: FMT is kBf16 or kF16.
template <int FMT>
__device__ __forceinline__ float dot2_16(uint32_t a, uint32_t b, float c) {
  if constexpr (FMT == kF16)
    return dot2_f16(a, b, c);
  else
    return dot2_bf16(a, b, c);
}
template <int FMT>
__device__ __forceinline__ uint32_t pack_16(float lo, float hi) {
  if constexpr (FMT == kF16)
    return pack_f16(lo, hi);
  else
    return pack_bf16(lo, hi);
}
template <int FMT>
__device__ __forceinline__ float dot2_ones_16(uint32_t pair, float acc) {
  if constexpr (FMT == kF16)
    return dot2_ones_f16(pair, acc);
  else
    return dot2_ones(pair, acc);
}

// Largest |x| over the bf16 elements of w[0 .. NW), as integer bits: the bits
// of |x| order as integers (NaN above infinity).
template <int NW, int N>
__device__ __forceinline__ int bf16_absmax_bits(const uint32_t (&w)[N]) {
  static_assert(NW <= N, "words");
  typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
  u16x2_t mv = {0, 0};
#pragma unroll
  for (int k = 0; k < NW; k++) mv = __builtin_elementwise_max(mv, __builtin_bit_cast(u16x2_t, w[k] & 0x7fff7fffu));
  return max((int)mv.x, (int)mv.y);
}

// bf16 -> fp16 for q . k against fp16 K.  A query vector whose largest |x| has
// the bits mx is scaled by inv = 2^-e, chosen so that its largest scaled element
// lies in [2^14, 2^15) (no fp16 overflow; e >= -126), and rounded to fp16
// (nearest even): elements within 2^-28 of the largest convert exactly (bf16
// holds 8 significant bits), smaller ones keep an absolute error below 2^-38 of
// it.  step = 2^e (q . k = 2^e * q' . k), NaN when the vector holds an infinity
// or NaN.
struct F16Scaling {
  float inv;
  float step;
};
__device__ __forceinline__ F16Scaling f16_scaling(int mx) {
  const int ex = mx >> 7;                // biased exponent of the largest |x|
  const int inv_b = min(268 - ex, 253);  // biased exponent of 2^-e
  return {__int_as_float(inv_b << 23), ex == 255 ? __builtin_nanf("") : __int_as_float((254 - inv_b) << 23)};
}

// The scaled fp16 pair of a bf16 pair
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w, float inv) {
  return pack_f16(bf16_lo(w) * inv, bf16_hi(w) * inv);
}

// One query head's bf16 words (the first NW of w; the head's dims spread over
// the 16 lanes of a row) as fp16 words (f16_scaling over the head's elements).
// Returns the head's step.
template <int NW, int N>
__device__ __forceinline__ float q_bf16_to_f16(uint32_t (&w)[N]) {
  int mx = bf16_absmax_bits<NW>(w);
  mx = max(mx, __builtin_amdgcn_update_dpp(0, mx, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  mx = max(mx, __builtin_amdgcn_update_dpp(0, mx, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  mx = max(mx, __builtin_amdgcn_update_dpp(0, mx, 0x141, 0xF, 0xF, false));  // row_half_mirror
  mx = max(mx, __builtin_amdgcn_update_dpp(0, mx, 0x140, 0xF, 0xF, false));  // row_mirror
  const F16Scaling sc = f16_scaling(mx);
#pragma unroll
  for (int k = 0; k < NW; k++) w[k] = bf16x2_to_f16x2(w[k], sc.inv);
  return sc.step;
}

}  // namespace llh
