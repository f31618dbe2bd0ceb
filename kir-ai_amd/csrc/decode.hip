// Paged GQA decode attention for gfx950 (MI355X).
//
// Computes, for every sequence b and query head h of one decode step,
//   out[b][h] = sum_t softmax_t(scale * q[b][h] . K[t][kv]) V[t][kv],  kv = h / (Hq / Hkv)
// over the sequence's attended positions (the per-head loop of
// crates/llm-backend/src/core/native_attention.rs:731-771, with the window rule
// of crates/llm-backend/src/core/qwen/ops/cache.rs:116-121).
//
// Tuned kernel (head_dim 128, 16-token blocks): one workgroup per
// (split, kv head, sequence).  A split is `split_blocks` consecutive blocks of
// the attended range; the four wavefronts take its blocks round-robin.  Every
// K/V byte of the kv head is read once and serves all G = Hq/Hkv query heads.
// The path is HBM-bound and uses no MFMA.
//
// Lane roles inside a wavefront, per 16-token block (K: token rows, V: dim rows):
//   group g = lane / 16 owns tokens 4g .. 4g+3, c = lane % 16.
//   K (bf16): lane loads 16 B of token 4g+i (i = 0..3) at dims 8c .. 8c+7:
//             four 256-B segments per instruction.  q . k runs on packed bf16
//             dot2 with fp32 accumulation, then a 16-lane DPP butterfly.
//   V (bf16): lane loads 8 B = tokens 4g..4g+3 of dim 16j + c (j = 0..7):
//             512 contiguous bytes per instruction.
// Each group keeps its own online-softmax state (running max in log2 units,
// sum, 8 output dims per lane per head); groups, wavefronts and splits are
// merged by log-sum-exp.  The last workgroup of a (sequence, kv head) to finish
// merges the split partials, so one launch produces the output.
#include "llh_internal.h"

namespace llh {

namespace {

constexpr int D = kFastHeadDim;
constexpr int BT = kFastBlockTokens;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
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

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Per-block online-softmax update for one query head of one token group.
// s[4] are scores (log2 units, -inf when masked), w[4] the weights used for V
// (p, or p * value scale); returns p via the array.
__device__ __forceinline__ void online_update(float &m, float &l, float s[4], float &alpha, float p[4]) {
  float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  mx = fmaxf(mx, m);
  const float mref = (mx == -INFINITY) ? 0.0f : mx;
  alpha = fast_exp2(m - mref);
#pragma unroll
  for (int i = 0; i < 4; i++) p[i] = fast_exp2(s[i] - mref);
  l = l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
  m = mx;
}

template <int G, int FMT>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(const DecodeArgs a) {
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  const int Hkv = a.pool.kv_heads;

  const int len = a.seq_lens[b];
  const int lo = a.window > 0 ? max(0, len - a.window) : 0;
  const int first_blk = lo / BT;
  const int n_blk = len > lo ? (len - 1) / BT - first_blk + 1 : 0;
  const int n_splits = (n_blk + a.split_blocks - 1) / a.split_blocks;
  if (n_splits > a.max_splits) {
    if (threadIdx.x == 0 && split == 0) atomicOr(a.err, kErrTooManySplits);
    return;
  }
  if (split >= max(n_splits, 1)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;
  const size_t qrow0 = (size_t)b * a.q_heads + (size_t)kvh * G;

  if (n_blk == 0) {  // empty context: zero output (weighted sum of nothing)
    for (int idx = tid; idx < G * D; idx += kDecodeThreads) a.out[qrow0 * D + idx] = 0;
    return;
  }

  // ---- query ----
  uint32_t qw[G][4];     // bf16 pairs, dims 8c..8c+7 (bf16 K path)
  float qf[G][16];       // f32 dims 16*(lane&7) .. +16 (int8/fp8 K path)
  float qsum[G];
  if constexpr (FMT == kBf16) {
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      const uint4 t = *reinterpret_cast<const uint4 *>(a.q + (qrow0 + gi) * D + c * 8);
      qw[gi][0] = t.x;
      qw[gi][1] = t.y;
      qw[gi][2] = t.z;
      qw[gi][3] = t.w;
    }
  } else {
    const int c8 = lane & 7;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      const uint4 *src = reinterpret_cast<const uint4 *>(a.q + (qrow0 + gi) * D + c8 * 16);
      const uint4 t0 = src[0], t1 = src[1];
      const uint32_t w[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        qf[gi][2 * k] = bf16_lo(w[k]);
        qf[gi][2 * k + 1] = bf16_hi(w[k]);
        s += qf[gi][2 * k] + qf[gi][2 * k + 1];
      }
      qsum[gi] = s;
    }
  }

  float m[G], l[G], wsum[G], o[G][8];
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    m[gi] = -INFINITY;
    l[gi] = 0.0f;
    wsum[gi] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) o[gi][j] = 0.0f;
  }

  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  const int blk_begin = first_blk + split * a.split_blocks;
  const int blk_end = min(blk_begin + a.split_blocks, first_blk + n_blk);
  constexpr int kBlockBytes = (FMT == kBf16 ? 2 : 1) * BT * D;

  for (int jb = blk_begin + wave; jb < blk_end; jb += 4) {
    const int phys = table[jb % a.max_blocks];
    if (phys < 0 || (int64_t)phys >= a.pool.n_blocks) {
      if (lane == 0) atomicOr(a.err, kErrBadBlock);
      continue;
    }
    const size_t bh = (size_t)phys * Hkv + kvh;
    const char *kb = reinterpret_cast<const char *>(a.pool.k) + bh * kBlockBytes;
    const char *vb = reinterpret_cast<const char *>(a.pool.v) + bh * kBlockBytes;
    const int pos0 = jb * BT + 4 * g;
    const bool partial = (jb * BT < lo) || (jb * BT + BT > len);
    bool ok[4];
#pragma unroll
    for (int i = 0; i < 4; i++) ok[i] = (pos0 + i >= lo) && (pos0 + i < len);

    float s[G][4];
    float vf[8][4];  // V values of dims 16j + c, tokens 4g .. 4g+3
    float vsc[4] = {1.0f, 1.0f, 1.0f, 1.0f};

    if constexpr (FMT == kBf16) {
      uint4 kr[4];
#pragma unroll
      for (int i = 0; i < 4; i++) kr[i] = *reinterpret_cast<const uint4 *>(kb + (4 * g + i) * (D * 2) + c * 16);
      uint2 vr[8];
#pragma unroll
      for (int j = 0; j < 8; j++) vr[j] = *reinterpret_cast<const uint2 *>(vb + (16 * j + c) * (BT * 2) + g * 8);
      if (partial) {
        const uint32_t mx = (ok[0] ? 0xffffu : 0u) | (ok[1] ? 0xffff0000u : 0u);
        const uint32_t my = (ok[2] ? 0xffffu : 0u) | (ok[3] ? 0xffff0000u : 0u);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          vr[j].x &= mx;
          vr[j].y &= my;
        }
      }
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float acc = dot2_bf16(kr[i].x, qw[gi][0], 0.0f);
          acc = dot2_bf16(kr[i].y, qw[gi][1], acc);
          acc = dot2_bf16(kr[i].z, qw[gi][2], acc);
          acc = dot2_bf16(kr[i].w, qw[gi][3], acc);
          s[gi][i] = row_sum16(acc) * a.scale_log2e;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; j++) {
        vf[j][0] = bf16_lo(vr[j].x);
        vf[j][1] = bf16_hi(vr[j].x);
        vf[j][2] = bf16_lo(vr[j].y);
        vf[j][3] = bf16_hi(vr[j].y);
      }
    } else {
      // int8 / fp8: K token rows of 128 bytes; lane (g, half hf, c8) holds tokens
      // 4g + 2i + hf (i = 0, 1) at dims 16*c8 .. +16.  V dim rows of 16 bytes;
      // lane holds the 4 bytes of tokens 4g..4g+3 for dims 16j + c.
      const int hf = (lane >> 3) & 1;
      const int c8 = lane & 7;
      uint4 kr[2];
#pragma unroll
      for (int i = 0; i < 2; i++) kr[i] = *reinterpret_cast<const uint4 *>(kb + (4 * g + 2 * i + hf) * D + c8 * 16);
      uint32_t vr[8];
#pragma unroll
      for (int j = 0; j < 8; j++) vr[j] = *reinterpret_cast<const uint32_t *>(vb + (16 * j + c) * BT + g * 4);
      if (partial) {
        const uint32_t mk = (ok[0] ? 0xffu : 0u) | (ok[1] ? 0xff00u : 0u) | (ok[2] ? 0xff0000u : 0u) |
                            (ok[3] ? 0xff000000u : 0u);
#pragma unroll
        for (int j = 0; j < 8; j++) vr[j] &= mk;
      }
      float kscale_own[2];
      if constexpr (FMT == kInt8) {
        const uint16_t *ksp = reinterpret_cast<const uint16_t *>(a.pool.k_scales) + bh * BT + 4 * g;
        const uint16_t *vsp = reinterpret_cast<const uint16_t *>(a.pool.v_scales) + bh * BT + 4 * g;
        const uint2 ks = *reinterpret_cast<const uint2 *>(ksp);
        const uint2 vs = *reinterpret_cast<const uint2 *>(vsp);
        const float k4[4] = {f16_bits_to_f32(ks.x & 0xffffu), f16_bits_to_f32(ks.x >> 16),
                             f16_bits_to_f32(ks.y & 0xffffu), f16_bits_to_f32(ks.y >> 16)};
        vsc[0] = f16_bits_to_f32(vs.x & 0xffffu);
        vsc[1] = f16_bits_to_f32(vs.x >> 16);
        vsc[2] = f16_bits_to_f32(vs.y & 0xffffu);
        vsc[3] = f16_bits_to_f32(vs.y >> 16);
        kscale_own[0] = hf ? k4[1] : k4[0];
        kscale_own[1] = hf ? k4[3] : k4[2];
        // codes as unsigned bytes u = code + 128 (xor 0x80); f32(u) is one convert
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const uint32_t u = vr[j] ^ 0x80808080u;
#pragma unroll
          for (int i = 0; i < 4; i++) vf[j][i] = (float)((u >> (8 * i)) & 0xffu);
        }
      } else {
        const float ksb = reinterpret_cast<const float *>(a.pool.k_scales)[bh];
        const float vsb = reinterpret_cast<const float *>(a.pool.v_scales)[bh];
        kscale_own[0] = ksb;
        kscale_own[1] = ksb;
        vsc[0] = vsc[1] = vsc[2] = vsc[3] = vsb;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const auto lo2 = __builtin_amdgcn_cvt_pk_f32_fp8(vr[j], false);
          const auto hi2 = __builtin_amdgcn_cvt_pk_f32_fp8(vr[j], true);
          vf[j][0] = lo2[0];
          vf[j][1] = lo2[1];
          vf[j][2] = hi2[0];
          vf[j][3] = hi2[1];
        }
      }
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        float own[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const uint32_t w[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
          float acc = 0.0f;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            if constexpr (FMT == kInt8) {
              const uint32_t u = w[k] ^ 0x80808080u;
#pragma unroll
              for (int n = 0; n < 4; n++) acc += qf[gi][4 * k + n] * (float)((u >> (8 * n)) & 0xffu);
            } else {
              const auto lo2 = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], false);
              const auto hi2 = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], true);
              acc += qf[gi][4 * k + 0] * lo2[0];
              acc += qf[gi][4 * k + 1] * lo2[1];
              acc += qf[gi][4 * k + 2] * hi2[0];
              acc += qf[gi][4 * k + 3] * hi2[1];
            }
          }
          if constexpr (FMT == kInt8) acc -= 128.0f * qsum[gi];
          own[i] = row_sum8(acc) * kscale_own[i] * a.scale_log2e;
        }
        const float oth0 = dpp<0x140>(own[0]);  // row_mirror swaps the two 8-lane halves
        const float oth1 = dpp<0x140>(own[1]);
        s[gi][0] = hf ? oth0 : own[0];
        s[gi][1] = hf ? own[0] : oth0;
        s[gi][2] = hf ? oth1 : own[1];
        s[gi][3] = hf ? own[1] : oth1;
      }
    }

    if (partial) {
#pragma unroll
      for (int gi = 0; gi < G; gi++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (!ok[i]) s[gi][i] = -INFINITY;
    }

#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      float p[4], alpha;
      online_update(m[gi], l[gi], s[gi], alpha, p);
      float w[4];
#pragma unroll
      for (int i = 0; i < 4; i++) w[i] = (FMT == kBf16) ? p[i] : (ok[i] ? p[i] * vsc[i] : 0.0f);
      if constexpr (FMT == kInt8) wsum[gi] = wsum[gi] * alpha + ((w[0] + w[1]) + (w[2] + w[3]));
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float acc = o[gi][j] * alpha;
        acc += w[0] * vf[j][0];
        acc += w[1] * vf[j][1];
        acc += w[2] * vf[j][2];
        acc += w[3] * vf[j][3];
        o[gi][j] = acc;
      }
    }
  }

  // ---- merge the four token groups of the wavefront ----
  __shared__ float s_o[4][G][D];
  __shared__ float s_m[4][G];
  __shared__ float s_l[4][G];
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    if constexpr (FMT == kInt8) {
#pragma unroll
      for (int j = 0; j < 8; j++) o[gi][j] -= 128.0f * wsum[gi];
    }
    float mm = fmaxf(m[gi], __shfl_xor(m[gi], 16));
    mm = fmaxf(mm, __shfl_xor(mm, 32));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    const float f = fast_exp2(m[gi] - mref);
    float ll = l[gi] * f;
    ll += __shfl_xor(ll, 16);
    ll += __shfl_xor(ll, 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float v = o[gi][j] * f;
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      o[gi][j] = v;
    }
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < 8; j++) s_o[wave][gi][16 * j + c] = o[gi][j];
      if (c == 0) {
        s_m[wave][gi] = mm;
        s_l[wave][gi] = ll;
      }
    }
  }
  __syncthreads();

  // ---- merge the four wavefronts; write output or the split partial ----
  const size_t part0 = qrow0 * a.max_splits;  // partial row of (b, first q head of group, split 0)
  for (int idx = tid; idx < G * D; idx += kDecodeThreads) {
    const int gi = idx / D;
    const int d = idx % D;
    float mm = fmaxf(fmaxf(s_m[0][gi], s_m[1][gi]), fmaxf(s_m[2][gi], s_m[3][gi]));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    float ll = 0.0f, oo = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float f = fast_exp2(s_m[w][gi] - mref);
      ll += s_l[w][gi] * f;
      oo += s_o[w][gi][d] * f;
    }
    if (n_splits == 1) {
      a.out[(qrow0 + gi) * D + d] = f32_to_bf16_rne(oo / ll);
    } else {
      const size_t row = part0 + (size_t)gi * a.max_splits + split;
      a.ws_o[row * D + d] = oo;
      if (d == 0) a.ws_ml[row] = make_float2(mm, ll);
    }
  }
  if (n_splits == 1) return;

  // ---- last workgroup of this (sequence, kv head) merges the splits ----
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const int prev = atomicAdd(&a.counters[(size_t)b * Hkv + kvh], 1);
    s_last = (prev == n_splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid == 0) a.counters[(size_t)b * Hkv + kvh] = 0;
  for (int idx = tid; idx < G * D; idx += kDecodeThreads) {
    const int gi = idx / D;
    const int d = idx % D;
    const size_t row0 = part0 + (size_t)gi * a.max_splits;
    float mm = -INFINITY;
    for (int sp = 0; sp < n_splits; sp++) mm = fmaxf(mm, __builtin_nontemporal_load(&a.ws_ml[row0 + sp].x));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    float ll = 0.0f, oo = 0.0f;
    for (int sp = 0; sp < n_splits; sp++) {
      const float mx = __builtin_nontemporal_load(&a.ws_ml[row0 + sp].x);
      const float lx = __builtin_nontemporal_load(&a.ws_ml[row0 + sp].y);
      const float f = fast_exp2(mx - mref);
      ll += lx * f;
      oo += __builtin_nontemporal_load(&a.ws_o[(row0 + sp) * D + d]) * f;
    }
    a.out[(qrow0 + gi) * D + d] = f32_to_bf16_rne(oo / ll);
  }
}

// ---------------------------------------------------------------------------
// Reference-order decode for any shape: one workgroup per (q head, sequence).
// Scores in reference order (sequential dot over d, then * scale), softmax by
// max-subtract / exp / sum / divide, weighted sum sequential over rows
// (math.rs:126-161, 476-505, 260-287).  Used by the LayerKvCache trait mirror
// and for shapes the tuned kernel does not take.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float load_as_f32(const void *p, size_t i);
template <>
__device__ __forceinline__ float load_as_f32<float>(const void *p, size_t i) {
  return reinterpret_cast<const float *>(p)[i];
}
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const void *p, size_t i) {
  return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(p)[i] << 16);
}

__device__ __forceinline__ float pool_elem(const PoolView &p, int tensor, int64_t blk, int h, int t, int d) {
  const int64_t bh = blk * p.kv_heads + h;
  const int64_t idx = tensor ? (bh * p.head_dim + d) * p.block_tokens + t : (bh * p.block_tokens + t) * p.head_dim + d;
  const void *base = tensor ? p.v : p.k;
  const void *sc = tensor ? p.v_scales : p.k_scales;
  if (p.format == kBf16) return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(base)[idx] << 16);
  if (p.format == kInt8) {
    const float s = (float)__builtin_bit_cast(_Float16, reinterpret_cast<const uint16_t *>(sc)[bh * p.block_tokens + t]);
    return (float)reinterpret_cast<const int8_t *>(base)[idx] * s;
  }
  const uint32_t code = reinterpret_cast<const uint8_t *>(base)[idx];
  return __builtin_amdgcn_cvt_pk_f32_fp8(code, false)[0] * reinterpret_cast<const float *>(sc)[bh];
}

__device__ __forceinline__ bool slot_of(const GenericDecodeArgs &a, const int32_t *table, int pos, int64_t &blk,
                                        int &off) {
  const int bt = a.pool.block_tokens;
  int slot_blk;
  if (a.ring_tokens > 0) {
    const int slot = pos % a.ring_tokens;
    slot_blk = slot / bt;
    off = slot % bt;
    if (slot_blk >= a.max_blocks) return false;
  } else {
    slot_blk = (pos / bt) % a.max_blocks;
    off = pos % bt;
  }
  blk = table[slot_blk];
  return blk >= 0 && blk < a.pool.n_blocks;
}

template <typename QT, typename OT>
__global__ __launch_bounds__(256) void decode_generic_kernel(const GenericDecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int D_ = a.pool.head_dim;
  const int groups = a.q_heads / a.pool.kv_heads;
  const int kvh = h / groups;
  const int end = a.seq_lens[b];
  const int start = a.starts ? a.starts[b] : (a.window > 0 ? max(0, end - a.window) : 0);
  const int rows = max(0, end - start);
  if (rows > a.score_stride) {  // longer than the call's max_seq_len allows: the score scratch would overflow
    if (threadIdx.x == 0) atomicOr(a.err, kErrTooManySplits);
    return;
  }
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  const size_t qoff = ((size_t)b * a.q_heads + h) * D_;
  float *sc = a.scores + ((size_t)b * a.q_heads + h) * a.score_stride;
  __shared__ float red[256];
  __shared__ int s_bad;
  if (threadIdx.x == 0) s_bad = 0;
  __syncthreads();

  float lmax = -INFINITY;
  for (int r = threadIdx.x; r < rows; r += blockDim.x) {
    int64_t blk;
    int off;
    float s = 0.0f;
    if (!slot_of(a, table, start + r, blk, off)) {
      atomicOr(&s_bad, 1);
    } else {
      for (int d = 0; d < D_; d++) {
        const float prod = __fmul_rn(pool_elem(a.pool, 0, blk, kvh, off, d), load_as_f32<QT>(a.q, qoff + d));
        s = __fadd_rn(s, prod);
      }
    }
    s = __fmul_rn(s, a.scale);
    if (!isfinite(s)) atomicOr(&s_bad, 2);
    sc[r] = s;
    lmax = fmaxf(lmax, s);
  }
  red[threadIdx.x] = lmax;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + w]);
    __syncthreads();
  }
  const float mx = red[0];
  __syncthreads();
  float lsum = 0.0f;
  for (int r = threadIdx.x; r < rows; r += blockDim.x) {
    const float e = expf(__fsub_rn(sc[r], mx));
    sc[r] = e;
    lsum += e;
  }
  red[threadIdx.x] = lsum;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  const float sum = red[0];
  if (threadIdx.x == 0) {
    if (s_bad & 1) atomicOr(a.err, kErrBadBlock);
    if ((s_bad & 2) || (rows > 0 && (sum == 0.0f || !isfinite(sum)))) atomicOr(a.err, kErrNonFinite);
  }
  for (int d = threadIdx.x; d < D_; d += blockDim.x) {
    float acc = 0.0f;
    for (int r = 0; r < rows; r++) {
      int64_t blk;
      int off;
      if (!slot_of(a, table, start + r, blk, off)) continue;
      const float w = __fdiv_rn(sc[r], sum);
      acc = __fadd_rn(acc, __fmul_rn(pool_elem(a.pool, 1, blk, kvh, off, d), w));
    }
    if constexpr (sizeof(OT) == 4)
      reinterpret_cast<float *>(a.out)[qoff + d] = acc;
    else
      reinterpret_cast<uint16_t *>(a.out)[qoff + d] = f32_to_bf16_rne(acc);
  }
}

__global__ void decode_fp8_kernel(const uint8_t *codes, float *out, int32_t n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)codes[i], false)[0];
}

template <int G, int FMT>
hipError_t launch_decode_t(const DecodeArgs &a, int max_seq_len, hipStream_t s) {
  const int max_blk = (max_seq_len + BT - 1) / BT + 1;
  const int grid_x = max(1, (max_blk + a.split_blocks - 1) / a.split_blocks);
  dim3 grid(min(grid_x, a.max_splits), a.pool.kv_heads, a.num_seqs);
  hipLaunchKernelGGL((paged_decode_kernel<G, FMT>), grid, dim3(kDecodeThreads), 0, s, a);
  return hipGetLastError();
}

template <int G>
hipError_t launch_decode_fmt(const DecodeArgs &a, int max_seq_len, hipStream_t s) {
  switch (a.pool.format) {
    case kBf16:
      return launch_decode_t<G, kBf16>(a, max_seq_len, s);
    case kInt8:
      return launch_decode_t<G, kInt8>(a, max_seq_len, s);
    case kFp8:
      return launch_decode_t<G, kFp8>(a, max_seq_len, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_decode(const DecodeArgs &a, int group, int max_seq_len, hipStream_t s) {
  switch (group) {
    case 1:
      return launch_decode_fmt<1>(a, max_seq_len, s);
    case 2:
      return launch_decode_fmt<2>(a, max_seq_len, s);
    case 4:
      return launch_decode_fmt<4>(a, max_seq_len, s);
    case 8:
      return launch_decode_fmt<8>(a, max_seq_len, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_decode_generic(const GenericDecodeArgs &a, int q_f32, int out_f32, hipStream_t s) {
  dim3 grid(a.q_heads, a.num_seqs);
  if (q_f32 && out_f32)
    hipLaunchKernelGGL((decode_generic_kernel<float, float>), grid, dim3(256), 0, s, a);
  else if (q_f32)
    hipLaunchKernelGGL((decode_generic_kernel<float, uint16_t>), grid, dim3(256), 0, s, a);
  else if (out_f32)
    hipLaunchKernelGGL((decode_generic_kernel<uint16_t, float>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((decode_generic_kernel<uint16_t, uint16_t>), grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_decode_fp8(const uint8_t *codes, float *out, int32_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(decode_fp8_kernel, dim3((n + 255) / 256), dim3(256), 0, s, codes, out, n);
  return hipGetLastError();
}

}  // namespace llh
