/* Exhaustive check of the shared-divisor quotient of the whole-block KV write kernel
 * (write_blocks_d128_kernel, kir-ai_amd/csrc/kvwrite.hip).
 *
 * The kernel quantises bf16 elements x by a scale s shared by a token row (int8: s is
 * the fp16 scale) or a whole block (fp8: s = RN(absmax / 448) for a bf16 absmax).
 * Instead of a correctly rounded division per element it computes r = RN(1 / s) once
 * and, per element (Markstein's method),
 *     q = RN(x r),  e = fma(-q, s, x) (exact),  x / s ~ copysign(fma(e, r, q), x)
 * (the sign restores -0 for x = -0 and for negative x whose quotient underflows).
 * int8 codes round that quotient as trunc(q + copysign(0.5, q)).
 * The codes must equal those of the correctly rounded x / s.  This program takes every
 * absmax m the kernel can see (every positive finite bf16 value), derives s as the
 * kernel does, and compares the codes of every finite bf16 x with |x| <= m, under IEEE
 * arithmetic and again with subnormals flushed to zero (MXCSR FTZ + DAZ), so the
 * result holds whichever denormal mode the GPU uses.
 *
 *   quotient_check int8   -- s = RN_f16(RN(m / 127)); s = 0 or infinity: exact division
 *   quotient_check fp8    -- s = RN(m / 448); s < 2^-90: exact division
 * Prints the pair and mismatch counts and exits 1 when any code differs.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <immintrin.h>

static float from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* int8 code of a quotient: round half away from zero, clamp to +-127 (quant_int8) */
static int code_int8(float q) {
  float c = roundf(q);
  return (int)fminf(fmaxf(c, -127.0f), 127.0f);
}

/* the kernel's int8 code of its quotient: trunc(q + copysign(0.5, q)), clamped.  Not
 * round-half-away for every float (q = 0.5 - 2^-25 sums to 1), so it is checked here
 * against code_int8 of the exact quotient like the quotient itself */
static int code_int8_kernel(float q) {
  return (int)fminf(fmaxf(truncf(q + copysignf(0.5f, q)), -127.0f), 127.0f);
}

/* OCP e4m3fn code of a quotient, round to nearest even, saturating at +-448 (the
 * kernel's encode) */
static int code_e4m3(float x) {
  const uint32_t u = bits(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return (int)(sign | 0x7fu);
  if (from_bits(au) >= 448.0f) return (int)(sign | 0x7eu);
  const uint32_t ex = au >> 23;
  uint32_t man = au & 0x7fffffu;
  const int e = (int)ex - 127 + 7;
  if (e <= 0) {
    if (ex == 0) return (int)sign;
    man |= 0x800000u;
    const int shift = 21 - e;
    if (shift > 24) return (int)sign;
    uint32_t q = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (int)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 3) | (man >> 20);
  const uint32_t rem = man & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q++;
  if (q > 0x7eu) q = 0x7eu;
  return (int)(sign | q);
}

/* mismatching x for one row / block absmax m (bits mb): every finite bf16 x with
 * |x| <= m, codes of the shared-divisor quotient against codes of RN(x / s) (ref, IEEE) */
static long check_absmax(uint32_t mb, float s, int fp8, int *ref) {
  const float r = 1.0f / s;
  long bad = 0;
  for (uint32_t b = 0; b <= mb; b++) {
    for (int sg = 0; sg < 2; sg++) {
      const float x = from_bits((b << 16) | (sg ? 0x80000000u : 0u));
      const float q = x * r;
      const float e = fmaf(-q, s, x);
      const float m = copysignf(fmaf(e, r, q), x);  /* s > 0: the quotient has x's sign, zeros too */
      const int c = fp8 ? code_e4m3(m) : code_int8_kernel(m);
      bad += c != ref[2 * b + sg];
    }
  }
  return bad;
}

/* the kernel's scale for absmax m, or 0 where it divides exactly instead */
static float kernel_scale(float m, int fp8) {
  if (fp8) {
    const float s = m / 448.0f;
    return s >= 0x1p-90f ? s : 0.0f;
  }
  /* int8: the fp16 scale RN_f16(RN(m / 127)); zero and infinity divide exactly */
  const float s = _cvtsh_ss(_cvtss_sh(m / 127.0f, 0));
  return (s > 0.0f && isfinite(s)) ? s : 0.0f;
}

int main(int argc, char **argv) {
  if (argc < 2 || (strcmp(argv[1], "int8") && strcmp(argv[1], "fp8"))) {
    fprintf(stderr, "usage: quotient_check int8|fp8\n");
    return 2;
  }
  const int fp8 = strcmp(argv[1], "fp8") == 0;
  long pairs = 0, bad_ieee = 0, bad_ftz = 0, exact = 0;
#pragma omp parallel reduction(+ : pairs, bad_ieee, bad_ftz, exact)
  {
    static __thread int ref[2 * 0x7f80];
    const unsigned csr = _mm_getcsr();
#pragma omp for schedule(dynamic, 32)
    for (int mb = 1; mb < 0x7f80; mb++) {  /* every positive finite bf16 absmax */
      const float m = from_bits((uint32_t)mb << 16);
      _mm_setcsr(csr & ~0x8040u); /* IEEE: no FTZ, no DAZ */
      const float s = kernel_scale(m, fp8);
      if (s == 0.0f) {
        exact++;
        continue;
      }
      for (int b = 0; b <= mb; b++)
        for (int sg = 0; sg < 2; sg++) {
          const float x = from_bits(((uint32_t)b << 16) | (sg ? 0x80000000u : 0u));
          ref[2 * b + sg] = fp8 ? code_e4m3(x / s) : code_int8(x / s);
        }
      bad_ieee += check_absmax((uint32_t)mb, s, fp8, ref);
      _mm_setcsr(csr | 0x8040u); /* FTZ + DAZ */
      bad_ftz += check_absmax((uint32_t)mb, s, fp8, ref);
      _mm_setcsr(csr);
      pairs += 2L * (mb + 1);
    }
  }
  printf("%s pairs=%ld exact_division_absmax=%ld mismatches_ieee=%ld mismatches_ftz=%ld\n", argv[1], pairs, exact,
         bad_ieee, bad_ftz);
  return (bad_ieee || bad_ftz) ? 1 : 0;
}
