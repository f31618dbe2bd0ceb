// Paged GQA decode attention for gfx950 (MI355X).
//
// Computes, for every sequence b and query head h of one decode step,
//   out[b][h] = sum_t softmax_t(scale * q[b][h] . K[t][kv]) V[t][kv],  kv = h / (Hq / Hkv)
// over the sequence's attended positions (the per-head loop of
// crates/llm-backend/src/core/native_attention.rs:731-771, with the window rule
// of crates/llm-backend/src/core/qwen/ops/cache.rs:116-121).
//
// Tuned path (head_dim 128, 16-token blocks), two launches:
//   1. paged_decode_kernel: one workgroup per (split, kv head, sequence).  A
//      split is `split_blocks` consecutive blocks of the attended range; the
//      four wavefronts take its blocks round-robin, double-buffering the loads
//      of the next block behind the math of the current one.  Every K/V byte of
//      the kv head is read once and serves all G = Hq/Hkv query heads.  A
//      single-split sequence writes its output directly; otherwise each split
//      writes (max, sum, unnormalised output) partials.
//   2. decode_merge_kernel: log-sum-exp merge of the partials.
// The launch boundary makes the partials visible to the merge: no device-scope
// fence runs inside a workgroup (on gfx950 such a fence writes back and
// invalidates the whole L2 of the XCD, and those serialise).
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
// merged by log-sum-exp.
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

// Raw registers of one block for one wavefront.
template <int FMT>
struct BlockRegs;

template <>
struct BlockRegs<kBf16> {
  uint4 k[4];
  uint2 v[8];
  bool valid;
};

template <int FMT>
struct BlockRegs {
  uint4 k[2];
  uint32_t v[8];
  uint2 ks;   // int8: fp16 scales of tokens 4g..4g+3
  uint2 vs;
  float ksb;  // fp8: per (block, head) scales
  float vsb;
  bool valid;
};

// Issues the loads of block `phys` (wave-uniform) into r.
template <int FMT>
__device__ __forceinline__ void load_block(const DecodeArgs &a, int phys, int kvh, int lane, BlockRegs<FMT> &r) {
  const int g = lane >> 4;
  const int c = lane & 15;
  r.valid = phys >= 0 && (int64_t)phys < a.pool.n_blocks;
  if (!r.valid) return;
  constexpr int kBlockBytes = (FMT == kBf16 ? 2 : 1) * BT * D;
  const size_t bh = (size_t)phys * a.pool.kv_heads + kvh;
  const char *kb = reinterpret_cast<const char *>(a.pool.k) + bh * kBlockBytes;
  const char *vb = reinterpret_cast<const char *>(a.pool.v) + bh * kBlockBytes;
  if constexpr (FMT == kBf16) {
#pragma unroll
    for (int i = 0; i < 4; i++) r.k[i] = *reinterpret_cast<const uint4 *>(kb + (4 * g + i) * (D * 2) + c * 16);
#pragma unroll
    for (int j = 0; j < 8; j++) r.v[j] = *reinterpret_cast<const uint2 *>(vb + (16 * j + c) * (BT * 2) + g * 8);
  } else {
    const int hf = (lane >> 3) & 1;
    const int c8 = lane & 7;
#pragma unroll
    for (int i = 0; i < 2; i++) r.k[i] = *reinterpret_cast<const uint4 *>(kb + (4 * g + 2 * i + hf) * D + c8 * 16);
#pragma unroll
    for (int j = 0; j < 8; j++) r.v[j] = *reinterpret_cast<const uint32_t *>(vb + (16 * j + c) * BT + g * 4);
    if constexpr (FMT == kInt8) {
      r.ks = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.pool.k_scales) + bh * BT + 4 * g);
      r.vs = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(a.pool.v_scales) + bh * BT + 4 * g);
    } else {
      r.ksb = reinterpret_cast<const float *>(a.pool.k_scales)[bh];
      r.vsb = reinterpret_cast<const float *>(a.pool.v_scales)[bh];
    }
  }
}

// Per-group online-softmax state for G query heads.
template <int G>
struct SoftmaxState {
  float m[G];
  float l[G];
  float wsum[G];  // int8 only: running sum of p * value scale (offset-128 correction)
  float o[G][8];
};

template <int G, int FMT>
__device__ __forceinline__ void compute_block(const DecodeArgs &a, const BlockRegs<FMT> &r, int jb, int lo, int len,
                                              int lane, const uint32_t (&qw)[G][4], const float (&qf)[G][16],
                                              const float (&qsum)[G], SoftmaxState<G> &st) {
  if (!r.valid) {
    if (lane == 0) atomicOr(a.err, kErrBadBlock);
    return;
  }
  const int g = lane >> 4;
  const int pos0 = jb * BT + 4 * g;
  const bool partial = (jb * BT < lo) || (jb * BT + BT > len);
  bool ok[4];
#pragma unroll
  for (int i = 0; i < 4; i++) ok[i] = (pos0 + i >= lo) && (pos0 + i < len);

  float s[G][4];
  float vf[8][4];  // V values of dims 16j + c, tokens 4g .. 4g+3
  float vsc[4] = {1.0f, 1.0f, 1.0f, 1.0f};

  if constexpr (FMT == kBf16) {
    uint2 vr[8];
#pragma unroll
    for (int j = 0; j < 8; j++) vr[j] = r.v[j];
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
        float acc = dot2_bf16(r.k[i].x, qw[gi][0], 0.0f);
        acc = dot2_bf16(r.k[i].y, qw[gi][1], acc);
        acc = dot2_bf16(r.k[i].z, qw[gi][2], acc);
        acc = dot2_bf16(r.k[i].w, qw[gi][3], acc);
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
    uint32_t vr[8];
#pragma unroll
    for (int j = 0; j < 8; j++) vr[j] = r.v[j];
    if (partial) {
      const uint32_t mk = (ok[0] ? 0xffu : 0u) | (ok[1] ? 0xff00u : 0u) | (ok[2] ? 0xff0000u : 0u) |
                          (ok[3] ? 0xff000000u : 0u);
#pragma unroll
      for (int j = 0; j < 8; j++) vr[j] &= mk;
    }
    float kscale_own[2];
    if constexpr (FMT == kInt8) {
      const float k4[4] = {f16_bits_to_f32(r.ks.x & 0xffffu), f16_bits_to_f32(r.ks.x >> 16),
                           f16_bits_to_f32(r.ks.y & 0xffffu), f16_bits_to_f32(r.ks.y >> 16)};
      vsc[0] = f16_bits_to_f32(r.vs.x & 0xffffu);
      vsc[1] = f16_bits_to_f32(r.vs.x >> 16);
      vsc[2] = f16_bits_to_f32(r.vs.y & 0xffffu);
      vsc[3] = f16_bits_to_f32(r.vs.y >> 16);
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
      kscale_own[0] = r.ksb;
      kscale_own[1] = r.ksb;
      vsc[0] = vsc[1] = vsc[2] = vsc[3] = r.vsb;
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
        const uint32_t w[4] = {r.k[i].x, r.k[i].y, r.k[i].z, r.k[i].w};
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
    float mx = fmaxf(fmaxf(s[gi][0], s[gi][1]), fmaxf(s[gi][2], s[gi][3]));
    mx = fmaxf(mx, st.m[gi]);
    const float mref = (mx == -INFINITY) ? 0.0f : mx;
    const float alpha = fast_exp2(st.m[gi] - mref);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = fast_exp2(s[gi][i] - mref);
    st.l[gi] = st.l[gi] * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    st.m[gi] = mx;
    float w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = (FMT == kBf16) ? p[i] : (ok[i] ? p[i] * vsc[i] : 0.0f);
    if constexpr (FMT == kInt8) st.wsum[gi] = st.wsum[gi] * alpha + ((w[0] + w[1]) + (w[2] + w[3]));
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float acc = st.o[gi][j] * alpha;
      acc += w[0] * vf[j][0];
      acc += w[1] * vf[j][1];
      acc += w[2] * vf[j][2];
      acc += w[3] * vf[j][3];
      st.o[gi][j] = acc;
    }
  }
}

__device__ __forceinline__ void seq_range(const DecodeArgs &a, int b, int &len, int &lo, int &first_blk, int &n_blk,
                                          int &n_splits) {
  len = a.seq_lens[b];
  lo = a.window > 0 ? max(0, len - a.window) : 0;
  first_blk = lo / BT;
  n_blk = len > lo ? (len - 1) / BT - first_blk + 1 : 0;
  n_splits = (n_blk + a.split_blocks - 1) / a.split_blocks;
}

template <int G, int FMT>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(const DecodeArgs a) {
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  int len, lo, first_blk, n_blk, n_splits;
  seq_range(a, b, len, lo, first_blk, n_blk, n_splits);
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

  // ---- this wavefront's blocks and their pool indices (one load, read back per block) ----
  const int blk_begin = first_blk + split * a.split_blocks;
  const int blk_end = min(blk_begin + a.split_blocks, first_blk + n_blk);
  const int nbw = max(0, (blk_end - blk_begin - wave + 3) / 4);  // <= split_blocks / 4 <= 64
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  const int my_entry = lane < nbw ? table[(blk_begin + wave + 4 * lane) % a.max_blocks] : -1;

  // ---- query ----
  uint32_t qw[G][4];  // bf16 pairs, dims 8c..8c+7 (bf16 K path)
  float qf[G][16];    // f32 dims 16*(lane&7) .. +16 (int8/fp8 K path)
  float qsum[G];
  if constexpr (FMT == kBf16) {
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      const uint4 t = *reinterpret_cast<const uint4 *>(a.q + (qrow0 + gi) * D + c * 8);
      qw[gi][0] = t.x;
      qw[gi][1] = t.y;
      qw[gi][2] = t.z;
      qw[gi][3] = t.w;
      qsum[gi] = 0.0f;
#pragma unroll
      for (int k = 0; k < 16; k++) qf[gi][k] = 0.0f;
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
#pragma unroll
      for (int k = 0; k < 4; k++) qw[gi][k] = 0u;
    }
  }

  SoftmaxState<G> st;
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    st.m[gi] = -INFINITY;
    st.l[gi] = 0.0f;
    st.wsum[gi] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) st.o[gi][j] = 0.0f;
  }

  // ---- double-buffered block loop: loads of block k+1 overlap the math of block k ----
  BlockRegs<FMT> ra, rb;
  if (nbw > 0) load_block<FMT>(a, __builtin_amdgcn_readlane(my_entry, 0), kvh, lane, ra);
  for (int k = 0; k < nbw; k += 2) {
    if (k + 1 < nbw) load_block<FMT>(a, __builtin_amdgcn_readlane(my_entry, k + 1), kvh, lane, rb);
    compute_block<G, FMT>(a, ra, blk_begin + wave + 4 * k, lo, len, lane, qw, qf, qsum, st);
    if (k + 1 < nbw) {
      if (k + 2 < nbw) load_block<FMT>(a, __builtin_amdgcn_readlane(my_entry, k + 2), kvh, lane, ra);
      compute_block<G, FMT>(a, rb, blk_begin + wave + 4 * (k + 1), lo, len, lane, qw, qf, qsum, st);
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
      for (int j = 0; j < 8; j++) st.o[gi][j] -= 128.0f * st.wsum[gi];
    }
    float mm = fmaxf(st.m[gi], __shfl_xor(st.m[gi], 16));
    mm = fmaxf(mm, __shfl_xor(mm, 32));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    const float f = fast_exp2(st.m[gi] - mref);
    float ll = st.l[gi] * f;
    ll += __shfl_xor(ll, 16);
    ll += __shfl_xor(ll, 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float v = st.o[gi][j] * f;
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      st.o[gi][j] = v;
    }
    if (g == 0) {
#pragma unroll
      for (int j = 0; j < 8; j++) s_o[wave][gi][16 * j + c] = st.o[gi][j];
      if (c == 0) {
        s_m[wave][gi] = mm;
        s_l[wave][gi] = ll;
      }
    }
  }
  __syncthreads();

  // ---- merge the four wavefronts; write the output or this split's partial ----
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
      const size_t row = (qrow0 + gi) * a.max_splits + split;
      a.ws_o[row * D + d] = oo;
      if (d == 0) a.ws_ml[row] = make_float2(mm, ll);
    }
  }
}

// Log-sum-exp merge of the split partials: one workgroup of 128 lanes (one per
// dim) per (query head, sequence) whose sequence used more than one split.
__global__ __launch_bounds__(D) void decode_merge_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  int len, lo, first_blk, n_blk, n_splits;
  seq_range(a, b, len, lo, first_blk, n_blk, n_splits);
  if (n_splits <= 1 || n_splits > a.max_splits) return;
  const int d = threadIdx.x;
  const size_t row0 = ((size_t)b * a.q_heads + h) * a.max_splits;
  float mm = -INFINITY;
  for (int sp = 0; sp < n_splits; sp++) mm = fmaxf(mm, a.ws_ml[row0 + sp].x);
  const float mref = (mm == -INFINITY) ? 0.0f : mm;
  float ll = 0.0f, oo = 0.0f;
  for (int sp = 0; sp < n_splits; sp++) {
    const float2 ml = a.ws_ml[row0 + sp];
    const float f = fast_exp2(ml.x - mref);
    ll += ml.y * f;
    oo += a.ws_o[(row0 + sp) * D + d] * f;
  }
  a.out[((size_t)b * a.q_heads + h) * D + d] = f32_to_bf16_rne(oo / ll);
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
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.max_splits <= 1) return e;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(a.q_heads, a.num_seqs), dim3(D), 0, s, a);
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
