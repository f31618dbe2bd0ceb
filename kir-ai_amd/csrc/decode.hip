// Paged GQA decode attention for gfx950 (MI355X).
//
// Computes, for every sequence b and query head h of one decode step,
//   out[b][h] = sum_t softmax_t(scale * q[b][h] . K[t][kv]) V[t][kv],  kv = h / (Hq / Hkv)
// over the sequence's attended positions (the per-head loop of
// crates/llm-backend/src/core/native_attention.rs:731-771, with the window rule
// of crates/llm-backend/src/core/qwen/ops/cache.rs:116-121).
//
// Tuned path (head_dim 128, 16-token blocks), two kernels over the same
// per-block math (load_block / compute_block):
//  * paged_decode_stream_kernel (large batches): a persistent grid whose
//    wavefronts each stream an equal, contiguous range of one sequence's
//    (kv head, block) units; see its own comment.
//  * paged_decode_kernel (small batches: fewer than 8 units per stream
//    wavefront): one workgroup per (split, kv head, sequence).  A split is `split_blocks`
// consecutive blocks of the attended range; the four wavefronts take its blocks
// round-robin, double-buffering the loads of the next block behind the math of
// the current one.  Every K/V byte of the kv head is read once and serves all
// G = Hq/Hkv query heads.  A single-split sequence writes its output directly;
// otherwise each split writes (max, sum, unnormalised output) partials that a
// second launch (decode_merge_kernel) merges by log-sum-exp.
// The path is HBM-bound and uses no MFMA.
//
// Lane roles inside a wavefront, per 16-token block (K: token rows, V: dim rows):
//   group g = lane / 16 owns tokens 4g .. 4g+3, c = lane % 16.
//   K (bf16): lane loads 16 B of token 4g+i (i = 0..3) at dims 8c .. 8c+7:
//             four 256-B segments per instruction.  q . k runs on packed bf16
//             dot2 with fp32 accumulation, then a 16-lane DPP butterfly.
//   V (bf16): lane loads 8 B = tokens 4g..4g+3 of dim 16j + c (j = 0..7):
//             512 contiguous bytes per instruction (int8 / fp8: 4 B, 256).
//   K (int8 / fp8, G <= 4, token-lane layout): lane 4tq + c4 of row g loads
//             the 32 B of token 4g + tq at dims 32c4 .. 32c4+31 and scores that
//             token for head c4 % G after a 4-lane butterfly (see kTokenLanes);
//   K (int8 / fp8, G = 8): lane loads 16 B of tokens 4g + 2i + hf at dims
//             16 (c % 8) .. +16, then an 8-lane butterfly and a row mirror.
// Each group keeps its own online-softmax state (running max in log2 units,
// sum, 8 output dims per lane per head); groups, wavefronts and splits are
// merged by log-sum-exp.
#include "device_common.h"
#include "wave_ops.h"
#include "stream_partition.h"

namespace llh {

namespace {

constexpr int D = kFastHeadDim;
constexpr int BT = kFastBlockTokens;

// int8 / fp8 pools with G <= 4 query heads per kv head use the token-lane
// layout for q . k: lane 16g + 4tq + c holds token 4g + tq of the block at
// dims 32c .. 32c+31 and scores that token for head c % G, so every score is
// computed (and exponentiated) once per wavefront instead of once per lane of
// a 16-lane row.  Other shapes keep the row layout (16 dims of two tokens per
// lane).  V is laid out the same way in both.
template <int G, int FMT>
constexpr bool kTokenLanes = !is16(FMT) && G <= 4;
// q words (packed bf16 pairs; fp16 pairs on fp16 pools) per lane and head
template <int G, int FMT>
constexpr int kQWords = kTokenLanes<G, FMT> ? 16 : 8;

// Raw registers of one block for one wavefront.
template <int FMT>
struct BlockRegs;

// 16-bit pools (bf16, fp16): 16 bytes of each of 4 K token rows, 8 bytes of
// each of 8 V dim rows
struct BlockRegs16 {
  uint4 k[4];
  uint2 v[8];
  bool valid;
};
template <>
struct BlockRegs<kBf16> : BlockRegs16 {};
template <>
struct BlockRegs<kF16> : BlockRegs16 {};

template <int FMT>
struct BlockRegs {
  uint4 k[2];
  uint32_t v[8];
  // int8: fp16 (K scale, V scale) pairs, one per word: the lane's own token in
  // the token-lane layout (x only), tokens 4g..4g+3 in the row layout
  uint4 sc;
  float ksb;  // fp8: per (block, head) scales
  float vsb;
  bool valid;
};

// Issues the loads of block `phys` (wave-uniform) into r.  The loads are
// unconditional: an entry outside the pool reads pool block 0 instead and is
// marked invalid, and compute_block consumes (and masks) it like any other
// block, so no control-flow path leaves loads in flight past the math, which
// would make the compiler wait for every outstanding load before the next issue.
template <int FMT, bool TL>
__device__ __forceinline__ void load_block(const DecodeArgs &a, int phys, int kvh, int lane, BlockRegs<FMT> &r) {
  const int g = lane >> 4;
  const int c = lane & 15;
  r.valid = phys >= 0 && (int64_t)phys < a.pool.n_blocks;
  if (!r.valid) phys = 0;
  constexpr int kBlockBytes = (is16(FMT) ? 2 : 1) * BT * D;
  const size_t bh = (size_t)phys * a.pool.kv_heads + kvh;
  const char *kb = reinterpret_cast<const char *>(a.pool.k) + bh * kBlockBytes;
  const char *vb = reinterpret_cast<const char *>(a.pool.v) + bh * kBlockBytes;
  if constexpr (is16(FMT)) {
#pragma unroll
    for (int i = 0; i < 4; i++) r.k[i] = ld_nt16(kb + (4 * g + i) * (D * 2) + c * 16);
#pragma unroll
    for (int j = 0; j < 8; j++) r.v[j] = ld_nt8(vb + (16 * j + c) * (BT * 2) + g * 8);
  } else {
    if constexpr (TL) {
      // token 4g + tq, dims 32c .. 32c+31: the 32 bytes at lane * 32
#pragma unroll
      for (int i = 0; i < 2; i++) r.k[i] = ld_nt16(kb + lane * 32 + i * 16);
    } else {
      const int hf = (lane >> 3) & 1;
      const int c8 = lane & 7;
#pragma unroll
      for (int i = 0; i < 2; i++) r.k[i] = ld_nt16(kb + (4 * g + 2 * i + hf) * D + c8 * 16);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) r.v[j] = ld_nt4(vb + (16 * j + c) * BT + g * 4);
    if constexpr (FMT == kInt8) {
      const uint16_t *sp = reinterpret_cast<const uint16_t *>(a.pool.k_scales);
      if constexpr (TL) {
        r.sc.x = *reinterpret_cast<const uint32_t *>(sp + int8_scale_index(bh, 4 * g + ((lane >> 2) & 3), BT));
      } else {
        r.sc = *reinterpret_cast<const uint4 *>(sp + int8_scale_index(bh, 4 * g, BT));
      }
    } else {
      // the block-head's (K, V) scale pair: bh is wave-uniform, so a scalar load
      // (constant address space: nothing writes the scales during the launch)
      typedef const __attribute__((address_space(4))) float scale_elem_t;
      const scale_elem_t *sp = (const scale_elem_t *)a.pool.k_scales + fp8_scale_index(bh);
      r.ksb = sp[0];
      r.vsb = sp[1];
    }
  }
}

// Per-group online-softmax state for G query heads.
template <int G>
struct SoftmaxState {
  float m[G];
  float l[G];
  float o[G][8];
  // token-lane layout: running max and weight sum of this lane's head (c % G)
  // in its row; folded into m / l by finalize_state
  float m_own;
  float l_own;
};

template <int G>
__device__ __forceinline__ void reset_state(SoftmaxState<G> &st) {
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    st.m[gi] = -INFINITY;
    st.l[gi] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) st.o[gi][j] = 0.0f;
  }
  st.m_own = -INFINITY;
  st.l_own = 0.0f;
}

// Token-lane layout: makes m[gi] and l[gi] the row's running max and weight
// sum of head gi in every lane of the row, as the row layout keeps them.
template <int G, int FMT>
__device__ __forceinline__ void finalize_state(SoftmaxState<G> &st) {
  if constexpr (kTokenLanes<G, FMT>) {
    const float lr = row_sum_stride4(st.l_own);  // the row's four tokens of this lane's head
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      st.m[gi] = row_bcast(st.m_own, gi);  // row lane gi: token 0 of the row, head gi
      st.l[gi] = row_bcast(lr, gi);
    }
  }
}


// Two signed int8 codes (bytes b, b+1 of w) as a packed bf16 pair (exact).
__device__ __forceinline__ uint32_t i8x2_to_bf16(uint32_t w, int b) {
  return pack_bf16((float)(int8_t)(w >> (8 * b)), (float)(int8_t)(w >> (8 * b + 8)));
}

// Two OCP e4m3 codes (bytes 2*HI, 2*HI+1 of w) as a packed bf16 pair (exact).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

// One V word of a quantized pool (dim 16j + c, tokens 4g..4g+3) as two packed
// bf16 pairs: (token 0, token 1) and (token 2, token 3).
template <int FMT>
__device__ __forceinline__ void v_code_pairs(uint32_t w, uint32_t &p01, uint32_t &p23) {
  if constexpr (FMT == kInt8) {
    p01 = i8x2_to_bf16(w, 0);
    p23 = i8x2_to_bf16(w, 2);
  } else {
    p01 = fp8x2_to_bf16<false>(w);
    p23 = fp8x2_to_bf16<true>(w);
  }
}

// One 16-token block for the G query heads of this wavefront's kv head.
// q . k and p . v run on packed bf16 dot2 with fp32 accumulation: K, V and q
// are exact in bf16 (int8 and e4m3 codes convert exactly).  fp16 pools run
// the same steps on packed fp16 dot2 against q in fp16 (q_bf16_to_f16: each
// head's scores carry its step 2^e) with fp16 softmax weights.  The exception is
// q . k on int8 pools in the token-lane layout, which runs on v_dot4_i32_i8
// against q in 16-bit fixed point (prep_q; qstep is the fixed-point step of
// this lane's head).  The softmax weights p (times the value scale for
// int8/fp8) are rounded to bf16 for the p . v products, and the softmax
// denominator sums exactly those rounded weights (divided by the value scale
// for int8/fp8), so the output is a weighted mean of the attended values whose
// weights sum to one.
template <int G, int FMT>
__device__ __forceinline__ void compute_block(const DecodeArgs &a, const BlockRegs<FMT> &r, int jb, int lo, int len,
                                              int lane, const uint32_t (&qw)[G][kQWords<G, FMT>], float qstep,
                                              SoftmaxState<G> &st) {
  if (!r.valid && lane == 0) atomicOr(a.err, kErrBadBlock);  // its tokens are all masked below
  const int g = lane >> 4;
  const bool partial = (jb * BT < lo) || (jb * BT + BT > len) || !r.valid;
  bool ok[4] = {true, true, true, true};
  uint32_t vmask[2] = {0xffffffffu, 0xffffffffu};  // zero V of tokens outside [lo, len) (slots may hold garbage)
  if (partial) {
    const int pos0 = jb * BT + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; i++) ok[i] = (pos0 + i >= lo) && (pos0 + i < len) && r.valid;
    if constexpr (is16(FMT)) {
      vmask[0] = (ok[0] ? 0xffffu : 0u) | (ok[1] ? 0xffff0000u : 0u);
      vmask[1] = (ok[2] ? 0xffffu : 0u) | (ok[3] ? 0xffff0000u : 0u);
    } else {
      vmask[0] = (ok[0] ? 0xffu : 0u) | (ok[1] ? 0xff00u : 0u) | (ok[2] ? 0xff0000u : 0u) | (ok[3] ? 0xff000000u : 0u);
    }
  }

  uint32_t w01[G], w23[G];
  if constexpr (kTokenLanes<G, FMT>) {
    // this lane: token 4g + tq of the row, dims 32c4 .. 32c4+31, scores head c4 % G
    const int tq = (lane >> 2) & 3;
    const int c4 = lane & 3;
    const bool ok_own = !partial || ((jb * BT + 4 * g + tq >= lo) && (jb * BT + 4 * g + tq < len) && r.valid);
    // q . k of this token for every head over the lane's 32 dims, summed over
    // the token's four lanes (quad_perm butterflies: all four get the sum)
    float s_own = 0.0f;
    if constexpr (FMT == kInt8) {
      // the codes against q's fixed-point words (prep_q): 256 (hi . k) + lo . k,
      // exact in int32 (|sum| < 2^29), times the head's step 2^e
      const uint32_t kw[8] = {r.k[0].x, r.k[0].y, r.k[0].z, r.k[0].w, r.k[1].x, r.k[1].y, r.k[1].z, r.k[1].w};
      int s_int = 0;
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        int acc = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) acc = __builtin_amdgcn_sdot4((int)kw[k], (int)qw[gi][k], acc, false);
        acc *= 256;
#pragma unroll
        for (int k = 0; k < 8; k++) acc = __builtin_amdgcn_sdot4((int)kw[k], (int)qw[gi][8 + k], acc, false);
        acc += dpp_i32<0xB1>(acc);
        acc += dpp_i32<0x4E>(acc);
        if (gi == 0 || (c4 & (G - 1)) == gi) s_int = acc;
      }
      s_own = (float)s_int * qstep;
    } else {
      uint32_t kp[16];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t w[4] = {r.k[i].x, r.k[i].y, r.k[i].z, r.k[i].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          kp[8 * i + 2 * k] = fp8x2_to_bf16<false>(w[k]);
          kp[8 * i + 2 * k + 1] = fp8x2_to_bf16<true>(w[k]);
        }
      }
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) acc = dot2_bf16(kp[k], qw[gi][k], acc);
        acc += dpp<0xB1>(acc);  // quad_perm [1,0,3,2]
        acc += dpp<0x4E>(acc);  // quad_perm [2,3,0,1]
        if (gi == 0 || (c4 & (G - 1)) == gi) s_own = acc;
      }
    }
    float ks_own, vs_own;
    if constexpr (FMT == kInt8) {
      ks_own = f16_bits_to_f32(r.sc.x & 0xffffu);
      vs_own = f16_bits_to_f32(r.sc.x >> 16);
    } else {
      ks_own = r.ksb;
      vs_own = r.vsb;
    }
    s_own *= ks_own * a.scale_log2e;
    if (!ok_own) {
      s_own = -INFINITY;
      vs_own = 0.0f;  // its scale bits may be garbage: keep 0 * garbage out of the sums
    }
    // lazy running max per (row, head), as in the row layout; the lanes of a
    // row that score one head see the same row max
    const float tmax = row_max_stride4(s_own);
    const bool grow = tmax > st.m_own + 8.0f;  // true on the first block with a finite score
    if (__any(grow)) {
      const float nm = grow ? tmax : st.m_own;
      const float alpha = grow ? fast_exp2(st.m_own - nm) : 1.0f;  // 0 when st.m_own = -inf
      st.m_own = nm;
      st.l_own *= alpha;
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        const float al = row_bcast(alpha, gi);  // row lane gi scores head gi
#pragma unroll
        for (int j = 0; j < 8; j++) st.o[gi][j] *= al;
      }
    }
    const float mref = (st.m_own == -INFINITY) ? 0.0f : st.m_own;
    const float p = fast_exp2(s_own - mref);
    const float wv = p * vs_own;
    // the normaliser sums the weights p . v really applies to the dequantised value
    // (code * scale): bf16(p * scale) / scale, the same bf16 rounding as the packs below
    st.l_own += vs_own != 0.0f ? bf16_round(wv) * __builtin_amdgcn_rcpf(vs_own) : p;
    // every lane of the row gathers the row's 4 tokens' value weights of each
    // head: each lane packs its weight with the next token's (same head, 4 lanes
    // on: DPP row_shl:4), so the pairs (t0, t1) and (t2, t3) of head gi sit in
    // row lanes gi and 8 + gi and one broadcast per pair reaches the row
    const uint32_t pr = pack_bf16(wv, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(wv), 0x104, 0xF, 0xF,
                                                                              false)));
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      w01[gi] = __float_as_uint(row_bcast(__uint_as_float(pr), gi));
      w23[gi] = __float_as_uint(row_bcast(__uint_as_float(pr), 8 + gi));
    }
  } else {
    float s[G][4];
    float vsc[4] = {1.0f, 1.0f, 1.0f, 1.0f};

    if constexpr (is16(FMT)) {
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        // fp16: word 4 holds the head's q step (prep_q)
        const float sc = FMT == kF16 ? a.scale_log2e * __uint_as_float(qw[gi][4]) : a.scale_log2e;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float acc = dot2_16<FMT>(r.k[i].x, qw[gi][0], 0.0f);
          acc = dot2_16<FMT>(r.k[i].y, qw[gi][1], acc);
          acc = dot2_16<FMT>(r.k[i].z, qw[gi][2], acc);
          acc = dot2_16<FMT>(r.k[i].w, qw[gi][3], acc);
          s[gi][i] = row_sum16(acc) * sc;
        }
      }
    } else {
      // int8 / fp8: K token rows of 128 bytes; lane (g, half hf, c8) holds tokens
      // 4g + 2i + hf (i = 0, 1) at dims 16*c8 .. +16.  V dim rows of 16 bytes;
      // lane holds the 4 bytes of tokens 4g..4g+3 for dims 16j + c.
      const int hf = (lane >> 3) & 1;
      float kscale_own[2];
      if constexpr (FMT == kInt8) {
        const uint32_t pr[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
        float k4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          k4[i] = f16_bits_to_f32(pr[i] & 0xffffu);
          vsc[i] = f16_bits_to_f32(pr[i] >> 16);
        }
        kscale_own[0] = (hf ? k4[1] : k4[0]) * a.scale_log2e;
        kscale_own[1] = (hf ? k4[3] : k4[2]) * a.scale_log2e;
      } else {
        kscale_own[0] = kscale_own[1] = r.ksb * a.scale_log2e;
        vsc[0] = vsc[1] = vsc[2] = vsc[3] = r.vsb;
      }
      float own[G][2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint32_t w[4] = {r.k[i].x, r.k[i].y, r.k[i].z, r.k[i].w};
        uint32_t kp[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          if constexpr (FMT == kInt8) {
            kp[2 * k] = i8x2_to_bf16(w[k], 0);
            kp[2 * k + 1] = i8x2_to_bf16(w[k], 2);
          } else {
            kp[2 * k] = fp8x2_to_bf16<false>(w[k]);
            kp[2 * k + 1] = fp8x2_to_bf16<true>(w[k]);
          }
        }
#pragma unroll
        for (int gi = 0; gi < G; gi++) {
          float acc = 0.0f;
#pragma unroll
          for (int k = 0; k < 8; k++) acc = dot2_bf16(kp[k], qw[gi][k], acc);
          own[gi][i] = row_sum8(acc) * kscale_own[i];
        }
      }
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        const float oth0 = row_mirror(own[gi][0]);  // swaps the two 8-lane halves of a row
        const float oth1 = row_mirror(own[gi][1]);
        s[gi][0] = hf ? oth0 : own[gi][0];
        s[gi][1] = hf ? own[gi][0] : oth0;
        s[gi][2] = hf ? oth1 : own[gi][1];
        s[gi][3] = hf ? own[gi][1] : oth1;
      }
    }

    if (partial) {
#pragma unroll
      for (int gi = 0; gi < G; gi++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (!ok[i]) s[gi][i] = -INFINITY;
      // slots outside [lo, len) may hold any scale bits: zero their weights' scale
      // (their V codes are masked too) so that 0 * garbage cannot reach the sums
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (!ok[i]) vsc[i] = 0.0f;
    }

    // Online softmax per head with a lazy reference max (log2 units): st.m only
    // moves when a score exceeds it by more than 8, so the weights stay <= 2^8 and
    // the accumulators are rescaled on few blocks (a wavefront-uniform branch).
    // Any reference max gives the same softmax; the partials carry theirs.
    bool grow[G];
    bool any_grow = false;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      const float tmax = fmaxf(fmaxf(s[gi][0], s[gi][1]), fmaxf(s[gi][2], s[gi][3]));
      grow[gi] = tmax > st.m[gi] + 8.0f;  // true on the first block with a finite score
      any_grow |= grow[gi];
    }
    if (__any(any_grow)) {
#pragma unroll
      for (int gi = 0; gi < G; gi++) {
        const float tmax = fmaxf(fmaxf(s[gi][0], s[gi][1]), fmaxf(s[gi][2], s[gi][3]));
        const float nm = grow[gi] ? tmax : st.m[gi];
        const float alpha = grow[gi] ? fast_exp2(st.m[gi] - nm) : 1.0f;  // 0 when st.m = -inf
        st.m[gi] = nm;
        st.l[gi] *= alpha;
#pragma unroll
        for (int j = 0; j < 8; j++) st.o[gi][j] *= alpha;
      }
    }
    // quantized: the normaliser counts weight bf16(p * s) / s per token (see below)
    float vinv[4];
    if constexpr (!is16(FMT)) {
#pragma unroll
      for (int i = 0; i < 4; i++) vinv[i] = vsc[i] != 0.0f ? __builtin_amdgcn_rcpf(vsc[i]) : 0.0f;
    }
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      const float mref = (st.m[gi] == -INFINITY) ? 0.0f : st.m[gi];
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; i++) p[i] = fast_exp2(s[gi][i] - mref);
      if constexpr (is16(FMT)) {
        w01[gi] = pack_16<FMT>(p[0], p[1]);
        w23[gi] = pack_16<FMT>(p[2], p[3]);
        // the normaliser sums exactly the 16-bit weights that enter p . v
        st.l[gi] = dot2_ones_16<FMT>(w23[gi], dot2_ones_16<FMT>(w01[gi], st.l[gi]));
      } else {
        w01[gi] = pack_bf16(p[0] * vsc[0], p[1] * vsc[1]);
        w23[gi] = pack_bf16(p[2] * vsc[2], p[3] * vsc[3]);
        // p . v multiplies the codes by bf16(p * s): on the dequantised value
        // (code * s) that is the weight bf16(p * s) / s, which the normaliser sums
        // (a token whose scale is 0 has a zero value and keeps its weight p)
        const float r[4] = {bf16_lo(w01[gi]), bf16_hi(w01[gi]), bf16_lo(w23[gi]), bf16_hi(w23[gi])};
        float lsum = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) lsum += vsc[i] != 0.0f ? r[i] * vinv[i] : p[i];
        st.l[gi] += lsum;
      }
    }
  }
  // p . v over this lane's 8 dims; V of tokens outside [lo, len) is zeroed
  // first (only partial blocks pay the masks)
  if constexpr (is16(FMT)) {
    uint2 vv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) vv[j] = r.v[j];
    if (partial) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        vv[j].x &= vmask[0];
        vv[j].y &= vmask[1];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int gi = 0; gi < G; gi++)
        st.o[gi][j] = dot2_16<FMT>(vv[j].y, w23[gi], dot2_16<FMT>(vv[j].x, w01[gi], st.o[gi][j]));
  } else {
    uint32_t vv[8];
#pragma unroll
    for (int j = 0; j < 8; j++) vv[j] = r.v[j];
    if (partial) {
#pragma unroll
      for (int j = 0; j < 8; j++) vv[j] &= vmask[0];
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t v01, v23;
      v_code_pairs<FMT>(vv[j], v01, v23);
#pragma unroll
      for (int gi = 0; gi < G; gi++) st.o[gi][j] = dot2_bf16(v23, w23[gi], dot2_bf16(v01, w01[gi], st.o[gi][j]));
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

// The query words of this lane: 16-bit K rows, dims 8c..8c+7 (c = lane & 15);
// int8 / fp8 row layout, dims 16 * (lane & 7) .. +16; token-lane layout, dims
// 32 * (lane & 3) .. +32.
template <int G, int FMT>
__device__ __forceinline__ void load_q(const DecodeArgs &a, size_t qrow0, int lane,
                                       uint32_t (&qw)[G][kQWords<G, FMT>]) {
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    if constexpr (is16(FMT)) {
      const uint4 t = *reinterpret_cast<const uint4 *>(a.q + (qrow0 + gi) * D + (lane & 15) * 8);
      qw[gi][0] = t.x;
      qw[gi][1] = t.y;
      qw[gi][2] = t.z;
      qw[gi][3] = t.w;
      qw[gi][4] = qw[gi][5] = qw[gi][6] = qw[gi][7] = 0u;
    } else {
      constexpr int N = kQWords<G, FMT> / 4;  // uint4 per head
      const uint4 *src = reinterpret_cast<const uint4 *>(a.q + (qrow0 + gi) * D + (lane & (16 / N - 1)) * 8 * N);
#pragma unroll
      for (int i = 0; i < N; i++) {
        const uint4 t = src[i];
        qw[gi][4 * i] = t.x;
        qw[gi][4 * i + 1] = t.y;
        qw[gi][4 * i + 2] = t.z;
        qw[gi][4 * i + 3] = t.w;
      }
    }
  }
}

// Turns the bf16 q words of load_q into the operands compute_block uses and
// returns this lane's fixed-point step (1 where q stays bf16).  Split from the
// loads so that a caller can issue its next block's loads in between.
//
// fp16 pools: each head's q becomes fp16 words (q_bf16_to_f16) and its step
// goes to the head's word 4 (unused by the row layout's q . k), wave-uniform.
//
// int8 pools in the token-lane layout take q . k on v_dot4_i32_i8: each head's
// q becomes q16 = round(q * 2^-e) with e = exponent(max |q|) - 13, so |q16| <=
// 16320 and |q - q16 * 2^e| <= 2^-14 * max |q| (bf16 elements within 2^-6 of
// the largest one's binade are exact).  Words k = 0..7 then hold
// hi = floor((q16 + 128) / 256) and words 8..15 lo = q16 - 256 hi (both in int8
// range) for dims 32c + 4k .. +3, the dims of the lane's K word k, so that
// q . k = 2^e (256 hi . k + lo . k) in int32 without rounding.  The step is NaN
// when the head's q holds an infinity or NaN, so its scores are NaN as in f32.
template <int G, int FMT>
__device__ __forceinline__ float prep_q(int lane, uint32_t (&qw)[G][kQWords<G, FMT>]) {
  if constexpr (FMT == kInt8 && kTokenLanes<G, FMT>) {
    typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
    // q * 2^-e + 1.5 * 2^23 + 128, rounded once (fma): the float's low 16 bits
    // are q16 + 128 in two's complement, byte 0 = lo + 128, byte 1 = hi
    constexpr float kRound = 12583040.0f;
    float own = 1.0f;
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      u16x2_t mv = {0, 0};
#pragma unroll
      for (int k = 0; k < 16; k++)
        mv = __builtin_elementwise_max(mv, __builtin_bit_cast(u16x2_t, qw[gi][k] & 0x7fff7fffu));
      // |q| bits order as integers (NaN above infinity); the head's 128 dims lie in the lane's quad
      int mx = max((int)mv.x, (int)mv.y);
      mx = max(mx, dpp_i32<0xB1>(mx));
      mx = max(mx, dpp_i32<0x4E>(mx));
      const int ex = mx >> 7;                  // biased exponent of the largest |q|
      const int inv_b = min(267 - ex, 253);    // 2^-e, with e >= -126
      const float inv = __int_as_float(inv_b << 23);
      const float step = ex == 255 ? __builtin_nanf("") : __int_as_float((254 - inv_b) << 23);
      uint32_t t[16];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint32_t p0 = qw[gi][2 * k], p1 = qw[gi][2 * k + 1];
        const uint32_t f0 = __float_as_uint(fmaf(bf16_lo(p0), inv, kRound));
        const uint32_t f1 = __float_as_uint(fmaf(bf16_hi(p0), inv, kRound));
        const uint32_t f2 = __float_as_uint(fmaf(bf16_lo(p1), inv, kRound));
        const uint32_t f3 = __float_as_uint(fmaf(bf16_hi(p1), inv, kRound));
        // bytes (hi0, hi1, lo0 + 128, lo1 + 128) and (hi2, hi3, lo2 + 128, lo3 + 128)
        const uint32_t t01 = __builtin_amdgcn_perm(f1, f0, 0x04000501u);
        const uint32_t t23 = __builtin_amdgcn_perm(f3, f2, 0x04000501u);
        t[k] = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
        t[8 + k] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
      }
#pragma unroll
      for (int k = 0; k < 16; k++) qw[gi][k] = t[k];
      if (gi == 0 || ((lane & 3) & (G - 1)) == gi) own = step;
    }
    return own;
  } else if constexpr (FMT == kF16) {
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      const float step = q_bf16_to_f16<4>(qw[gi]);  // every row holds the same q: uniform over the wave
      qw[gi][4] = __builtin_amdgcn_readfirstlane(__float_as_uint(step));
    }
    return 1.0f;
  } else {
    return 1.0f;
  }
}

// Fused append, bf16 pools (row layout): adds sequence b's new token (position
// len - 1, which the pool part of the step masks out) from a.k_new / a.v_new to
// this wavefront's state, in row 0 (lanes 0..15) as one more token of that row,
// with the same bf16 weight and normaliser rule as compute_block; then writes
// the token to its pool slot (nothing reads that slot during the launch: the
// block holding it is computed by this wavefront only, which already has it).
// This lane's share of a sequence's new K / V rows: K dims 8c .. 8c+7, V dims
// 16j + c (low halves), as the row layout holds a block's tokens.
struct NewToken {
  uint4 k;
  uint32_t v[8];
  int blk;  // block-table entry of the block that receives the token (the segment's last unit's)
};

__device__ __forceinline__ void load_new_token(const DecodeArgs &a, int b, int kvh, int lane, NewToken &nt, int blk) {
  const int c = lane & 15;
  nt.blk = blk;
  const size_t row = (size_t)b * a.pool.kv_heads + kvh;
  nt.k = *reinterpret_cast<const uint4 *>(a.k_new + row * D + 8 * c);
#pragma unroll
  for (int j = 0; j < 8; j++) nt.v[j] = a.v_new[row * D + 16 * j + c];
}

// Writes a sequence's new token (position len - 1) into its pool slot: K as
// one 256-byte row, V as one 2-byte element in each of the 128 dim rows.
__device__ __forceinline__ void store_new_token(const DecodeArgs &a, int kvh, int len, int lane, const NewToken &nt) {
  const int g = lane >> 4;
  const int c = lane & 15;
  const int pos = len - 1;
  const int e = nt.blk;
  if (g == 0 && e >= 0 && (int64_t)e < a.pool.n_blocks) {
    const size_t bh = (size_t)e * a.pool.kv_heads + kvh;
    uint16_t *kd = const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(a.pool.k));
    uint16_t *vd = const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(a.pool.v));
    *reinterpret_cast<uint4 *>(kd + (bh * BT + pos % BT) * D + 8 * c) = nt.k;
#pragma unroll
    for (int j = 0; j < 8; j++) vd[(bh * D + 16 * j + c) * BT + pos % BT] = (uint16_t)nt.v[j];
  }
}

// Adds the new token to the state (STORE: and writes it to the pool).
template <int G, bool STORE = true>
__device__ __forceinline__ void add_new_token(const DecodeArgs &a, SoftmaxState<G> &st, int b, int kvh, int len,
                                              int lane, const uint32_t (&qw)[G][kQWords<G, kBf16>],
                                              const NewToken &nt) {
  const int g = lane >> 4;
  const uint4 kn = nt.k;
  const uint32_t(&vn)[8] = nt.v;
  float s[G];
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    float acc = dot2_bf16(kn.x, qw[gi][0], 0.0f);
    acc = dot2_bf16(kn.y, qw[gi][1], acc);
    acc = dot2_bf16(kn.z, qw[gi][2], acc);
    acc = dot2_bf16(kn.w, qw[gi][3], acc);
    s[gi] = row_sum16(acc) * a.scale_log2e;
  }
  if (g == 0) {
#pragma unroll
    for (int gi = 0; gi < G; gi++) {
      if (s[gi] > st.m[gi] + 8.0f) {  // the lazy reference max of compute_block
        const float alpha = fast_exp2(st.m[gi] - s[gi]);  // 0 when st.m = -inf
        st.m[gi] = s[gi];
        st.l[gi] *= alpha;
#pragma unroll
        for (int j = 0; j < 8; j++) st.o[gi][j] *= alpha;
      }
      const float mref = (st.m[gi] == -INFINITY) ? 0.0f : st.m[gi];
      const uint32_t w = pack_bf16(fast_exp2(s[gi] - mref), 0.0f);
      st.l[gi] = dot2_ones(w, st.l[gi]);
#pragma unroll
      for (int j = 0; j < 8; j++) st.o[gi][j] = dot2_bf16(vn[j], w, st.o[gi][j]);
    }
  }
  if constexpr (STORE) store_new_token(a, kvh, len, lane, nt);
}

// ---------------------------------------------------------------------------
// Fused append for int8 / fp8 pools.  The new token must be attended as stored
// (quantised), so the wavefront that computes the sequence's last block
// quantises it exactly as append_kernel would -- int8: codes with the fp16
// scale absmax / 127 of the token's head row; fp8: the block's scale becomes
// max(old, absmax / 448) (restarted at offset 0) and, when it grows, the
// block's earlier tokens are re-encoded from their dequantised values -- patches
// the codes and scales into the block registers it loaded from the pool (whose
// slot of the new position is stale), attends the block, and writes the token
// (and re-encoded tokens) back.  The pool ends byte-identical to llh_kv_append,
// and the attention equals the two calls' (the same registers meet the same
// arithmetic).  A non-finite row is flagged and not appended, as append_kernel
// does.
// Each lane holds two dims of the new rows (2l, 2l+1 of K and of V, one bf16
// pair each); the codes reach the lanes that hold the slot in the block layout
// through ds_bpermute.
struct NewTokenQ {
  uint32_t k2, v2;  // bf16 pairs: dims 2 * lane, 2 * lane + 1
  int blk;          // block-table entry of the block that receives the token
};

__device__ __forceinline__ void load_new_token_q(const DecodeArgs &a, int b, int kvh, int lane, NewTokenQ &nt,
                                                 int blk) {
  const size_t row = ((size_t)b * a.pool.kv_heads + kvh) * D;
  nt.blk = blk;
  nt.k2 = reinterpret_cast<const uint32_t *>(a.k_new + row)[lane];
  nt.v2 = reinterpret_cast<const uint32_t *>(a.v_new + row)[lane];
}

// Max over the wavefront, in every lane (DPP within rows, then row exchanges).
__device__ __forceinline__ float wave_max_f(float v, int lane) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  v = fmaxf(v, xor16_other(v, lane));
  return fmaxf(v, xor32_other(v, lane));
}

__device__ __forceinline__ uint32_t bperm(uint32_t v, int src_lane) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane << 2, (int)v);
}

// Re-encodes the fp8 codes of a 16-byte run from scale s_old to s_new (append_fp8_row's
// rule, encode(decode(code) * s_old / s_new)); byte i is re-encoded when bit i of mask is set.
// (The bytes of a word are walked by a loop that is not unrolled: the path is rare, and
// 64 unrolled software encodes per lane would bloat the decode loop's code.)
__device__ __forceinline__ uint32_t fp8_rescale_word(uint32_t w, float s_old, float s_new, uint32_t mask4) {
#pragma unroll 1
  for (int i = 0; i < 4; i++)
    if (mask4 & (1u << i)) {
      const uint32_t code = (w >> (8 * i)) & 0xffu;
      const float x = s_old == 0.0f ? 0.0f : decode_e4m3(code) * s_old;
      const uint32_t nc = encode_e4m3(__fdiv_rn(x, s_new));
      w = (w & ~(0xffu << (8 * i))) | (nc << (8 * i));
    }
  return w;
}
__device__ __forceinline__ uint4 fp8_rescale16(uint4 w, float s_old, float s_new, uint32_t mask) {
  return make_uint4(fp8_rescale_word(w.x, s_old, s_new, mask & 15u), fp8_rescale_word(w.y, s_old, s_new, (mask >> 4) & 15u),
                    fp8_rescale_word(w.z, s_old, s_new, (mask >> 8) & 15u),
                    fp8_rescale_word(w.w, s_old, s_new, (mask >> 12) & 15u));
}

// fp8 block scale growth (rare): the append done in the pool itself, as append_fp8_row
// does it -- tokens before `off` re-encoded (K: lane = token lane / 4, dims 32 (lane % 4)
// .. + 31; V: dim rows 2 lane, 2 lane + 1, tokens 0 .. off - 1), the new token's codes
// (kc / vc: dims 2 lane, 2 lane + 1) and the scale pair written -- then the block's codes
// read back into r.  Called by the whole wavefront (uniform condition).
template <int FMT, bool TL>
__device__ __forceinline__ void fp8_append_in_pool(const DecodeArgs &a, BlockRegs<FMT> &r, int blk, int kvh, int off,
                                                   float ks_old, float ks, float vs_old, float vs, uint32_t kc,
                                                   uint32_t vc, int lane) {
  const size_t bh = (size_t)blk * a.pool.kv_heads + kvh;
  uint8_t *kb = const_cast<uint8_t *>(reinterpret_cast<const uint8_t *>(a.pool.k)) + bh * (BT * D);
  uint8_t *vb = const_cast<uint8_t *>(reinterpret_cast<const uint8_t *>(a.pool.v)) + bh * (BT * D);
  const int tok = lane >> 2;
  uint4 k0 = *reinterpret_cast<const uint4 *>(kb + lane * 32);
  uint4 k1 = *reinterpret_cast<const uint4 *>(kb + lane * 32 + 16);
  uint4 v0 = *reinterpret_cast<const uint4 *>(vb + (2 * lane) * BT);
  uint4 v1 = *reinterpret_cast<const uint4 *>(vb + (2 * lane + 1) * BT);
  if (ks != ks_old && tok < off) {
    k0 = fp8_rescale16(k0, ks_old, ks, 0xffffu);
    k1 = fp8_rescale16(k1, ks_old, ks, 0xffffu);
  }
  if (vs != vs_old) {
    const uint32_t m = (1u << off) - 1u;
    v0 = fp8_rescale16(v0, vs_old, vs, m);
    v1 = fp8_rescale16(v1, vs_old, vs, m);
  }
  *reinterpret_cast<uint4 *>(kb + lane * 32) = k0;
  *reinterpret_cast<uint4 *>(kb + lane * 32 + 16) = k1;
  *reinterpret_cast<uint4 *>(vb + (2 * lane) * BT) = v0;
  *reinterpret_cast<uint4 *>(vb + (2 * lane + 1) * BT) = v1;
  // the new token: K row bytes 2 lane, 2 lane + 1; V byte `off` of dim rows 2 lane, 2 lane + 1
  *reinterpret_cast<uint16_t *>(kb + off * D + 2 * lane) = (uint16_t)kc;
  vb[(2 * lane) * BT + off] = (uint8_t)(vc & 0xffu);
  vb[(2 * lane + 1) * BT + off] = (uint8_t)(vc >> 8);
  if (lane == 0)
    *reinterpret_cast<float2 *>(const_cast<float *>(reinterpret_cast<const float *>(a.pool.k_scales)) +
                                fp8_scale_index(bh)) = make_float2(ks, vs);
  // this wavefront's stores are complete before it reads the block again
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  const bool valid = r.valid;
  load_block<FMT, TL>(a, blk, kvh, lane, r);
  r.valid = valid;
  r.ksb = ks;  // (the scalar load of load_block may read the scale pair through the scalar cache)
  r.vsb = vs;
}

// What a patched block writes back to the pool after it is computed.
struct NewTokenStore {
  bool any;          // this wavefront appends (finite rows, valid block)
  uint32_t k_rows;   // token-lane layout: the lane's token row is written; row layout: bit i = r.k[i]
  uint32_t v_words;  // the lane's V words are written (its group holds a changed token)
  bool scale;        // this lane writes the scale pair(s)
};

// Patches the new token (offset off of block r) into the registers; returns what to store.
template <int G, int FMT>
__device__ __forceinline__ NewTokenStore patch_new_token_q(const DecodeArgs &a, BlockRegs<FMT> &r,
                                                           const NewTokenQ &nt, int kvh, int off, int lane) {
  static_assert(FMT == kInt8 || FMT == kFp8, "quantised pools");
  constexpr bool TL = kTokenLanes<G, FMT>;
  NewTokenStore out{false, 0u, 0u, false};
  const int g = lane >> 4;
  const int c = lane & 15;
  const float kx[2] = {bf16_lo(nt.k2), bf16_hi(nt.k2)};
  const float vx[2] = {bf16_lo(nt.v2), bf16_hi(nt.v2)};
  const bool finite = isfinite(kx[0]) && isfinite(kx[1]) && isfinite(vx[0]) && isfinite(vx[1]);
  if (__any(!finite)) {  // append_kernel: NonFiniteValue, nothing of the token written
    if (lane == 0) atomicOr(a.err, kErrNonFinite);
    return out;
  }
  if (!r.valid) return out;  // the append flags the slot (compute_block flags the block)
  const float kmax = wave_max_f(fmaxf(fabsf(kx[0]), fabsf(kx[1])), lane);
  const float vmax = wave_max_f(fmaxf(fabsf(vx[0]), fabsf(vx[1])), lane);
  float ks, vs;            // the token's scales
  float ks_old = 0.0f, vs_old = 0.0f;
  uint32_t s16pair = 0u;   // int8: the (K, V) fp16 scale pair
  if constexpr (FMT == kInt8) {
    const _Float16 k16 = (_Float16)(kmax == 0.0f ? 0.0f : __fdiv_rn(kmax, 127.0f));
    const _Float16 v16 = (_Float16)(vmax == 0.0f ? 0.0f : __fdiv_rn(vmax, 127.0f));
    ks = (float)k16;
    vs = (float)v16;
    s16pair = (uint32_t)__builtin_bit_cast(uint16_t, k16) | ((uint32_t)__builtin_bit_cast(uint16_t, v16) << 16);
  } else {
    ks_old = off == 0 ? 0.0f : r.ksb;
    vs_old = off == 0 ? 0.0f : r.vsb;
    ks = fmaxf(ks_old, kmax == 0.0f ? 0.0f : __fdiv_rn(kmax, 448.0f));
    vs = fmaxf(vs_old, vmax == 0.0f ? 0.0f : __fdiv_rn(vmax, 448.0f));
  }
  auto code = [&](float x, float sc) -> uint32_t {
    if constexpr (FMT == kInt8)
      return (uint32_t)(uint8_t)quant_int8(x, sc);
    else
      return sc == 0.0f ? 0u : (uint32_t)encode_e4m3(__fdiv_rn(x, sc));
  };
  // this lane's two codes of each row (dims 2 * lane, 2 * lane + 1)
  const uint32_t kc = code(kx[0], ks) | (code(kx[1], ks) << 8);
  const uint32_t vc = code(vx[0], vs) | (code(vx[1], vs) << 8);
  if constexpr (FMT == kFp8) {
    if (off > 0 && (ks != ks_old || vs != vs_old)) {  // the block's scale grows: the rare path, in the pool
      fp8_append_in_pool<FMT, TL>(a, r, nt.blk, kvh, off, ks_old, ks, vs_old, vs, kc, vc, lane);
      return out;  // written already
    }
  }
  // ---- K ----
  if constexpr (TL) {
    // lane 16g + 4tq + c4 holds token 4g + tq at dims 32 c4 .. + 31: codes of lanes 16 c4 .. + 15
    const int c4 = lane & 3;
    const int tok = 4 * g + ((lane >> 2) & 3);
    uint32_t w[8];
#pragma unroll
    for (int m = 0; m < 8; m++)
      w[m] = (bperm(kc, 16 * c4 + 2 * m) & 0xffffu) | (bperm(kc, 16 * c4 + 2 * m + 1) << 16);
    if (tok == off) {
      r.k[0] = make_uint4(w[0], w[1], w[2], w[3]);
      r.k[1] = make_uint4(w[4], w[5], w[6], w[7]);
      out.k_rows = 1u;
      if constexpr (FMT == kInt8) {
        r.sc.x = s16pair;
        out.scale = c4 == 0;
      }
    }
  } else {
    // lane 16g + 8hf + c8 holds tokens 4g + 2i + hf (i = 0, 1) at dims 16 c8 .. + 15: codes of lanes 8 c8 .. + 7
    const int hf = (lane >> 3) & 1;
    const int c8 = lane & 7;
    uint32_t w[4];
#pragma unroll
    for (int m = 0; m < 4; m++)
      w[m] = (bperm(kc, 8 * c8 + 2 * m) & 0xffffu) | (bperm(kc, 8 * c8 + 2 * m + 1) << 16);
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int tok = 4 * g + 2 * i + hf;
      if (tok == off) {
        r.k[i] = make_uint4(w[0], w[1], w[2], w[3]);
        out.k_rows |= 1u << i;
      }
    }
    if constexpr (FMT == kInt8) {
      if (g == off / 4) {
        if ((off & 3) == 0) r.sc.x = s16pair;
        if ((off & 3) == 1) r.sc.y = s16pair;
        if ((off & 3) == 2) r.sc.z = s16pair;
        if ((off & 3) == 3) r.sc.w = s16pair;
        out.scale = (lane & 15) == 0;
      }
    }
  }
  // ---- V: lane (g, c) holds tokens 4g .. 4g+3 (bytes) of dims 16j + c ----
  const int shift = 8 * (off & 3);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int dim = 16 * j + c;
    const uint32_t cv = (bperm(vc, dim >> 1) >> (8 * (dim & 1))) & 0xffu;
    if (g == off / 4) r.v[j] = (r.v[j] & ~(0xffu << shift)) | (cv << shift);
  }
  out.v_words = g == off / 4 ? 1u : 0u;
  if constexpr (FMT == kFp8) {
    r.ksb = ks;
    r.vsb = vs;
    out.scale = lane == 0;
  }
  out.any = true;
  return out;
}

// Writes what patch_new_token_q changed (block nt.blk, kv head kvh, offset off).
template <int G, int FMT>
__device__ __forceinline__ void store_new_token_q(const DecodeArgs &a, const BlockRegs<FMT> &r, const NewTokenQ &nt,
                                                  const NewTokenStore &w, int kvh, int off, int lane) {
  if (!w.any) return;
  constexpr bool TL = kTokenLanes<G, FMT>;
  const int g = lane >> 4;
  const int c = lane & 15;
  const size_t bh = (size_t)nt.blk * a.pool.kv_heads + kvh;
  char *kb = const_cast<char *>(reinterpret_cast<const char *>(a.pool.k)) + bh * (BT * D);
  char *vb = const_cast<char *>(reinterpret_cast<const char *>(a.pool.v)) + bh * (BT * D);
  if constexpr (TL) {
    if (w.k_rows) {
      *reinterpret_cast<uint4 *>(kb + lane * 32) = r.k[0];
      *reinterpret_cast<uint4 *>(kb + lane * 32 + 16) = r.k[1];
    }
  } else {
    const int hf = (lane >> 3) & 1;
    const int c8 = lane & 7;
#pragma unroll
    for (int i = 0; i < 2; i++)
      if (w.k_rows & (1u << i)) *reinterpret_cast<uint4 *>(kb + (4 * g + 2 * i + hf) * D + c8 * 16) = r.k[i];
  }
  if (w.v_words) {
#pragma unroll
    for (int j = 0; j < 8; j++) *reinterpret_cast<uint32_t *>(vb + (16 * j + c) * BT + g * 4) = r.v[j];
  }
  if (w.scale) {
    if constexpr (FMT == kInt8) {
      uint32_t pair;
      if constexpr (TL) {
        pair = r.sc.x;
      } else {
        const uint32_t p4[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
        pair = p4[off & 3];
      }
      uint16_t *sp = const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(a.pool.k_scales));
      *reinterpret_cast<uint32_t *>(sp + int8_scale_index(bh, off, BT)) = pair;
    } else {
      float *sp = const_cast<float *>(reinterpret_cast<const float *>(a.pool.k_scales));
      *reinterpret_cast<float2 *>(sp + fp8_scale_index(bh)) = make_float2(r.ksb, r.vsb);
    }
  }
}

// The new-token registers of the fused append: bf16 rows as the row layout holds
// a block (NewToken), or two dims per lane for quantised pools (NewTokenQ).
template <int FMT>
struct NtOf {
  typedef NewTokenQ type;
};
template <>
struct NtOf<kBf16> {
  typedef NewToken type;
};
__device__ __forceinline__ void load_nt(const DecodeArgs &a, int b, int kvh, int lane, NewToken &nt, int blk) {
  load_new_token(a, b, kvh, lane, nt, blk);
}
__device__ __forceinline__ void load_nt(const DecodeArgs &a, int b, int kvh, int lane, NewTokenQ &nt, int blk) {
  load_new_token_q(a, b, kvh, lane, nt, blk);
}

template <int G, int FMT, bool FUSED = false>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(const DecodeArgs a) {
  // consecutive workgroups are consecutive splits of one (kv head, sequence):
  // they share its query rows and block-table row in L2 (measured faster on
  // MI355X than dispatching all first splits first)
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  int len, lo, first_blk, n_blk, n_splits;
  seq_range(a, b, len, lo, first_blk, n_blk, n_splits);
  if (n_splits > a.max_splits) {
    if (threadIdx.x == 0 && split == 0) atomicOr(a.err, kErrTooManySplits);
    return;
  }
  if (len - lo > a.max_blocks * BT) {  // the span would alias its own table entries
    if (threadIdx.x == 0 && split == 0) atomicOr(a.err, kErrSpan);
    return;
  }
  if (split >= max(n_splits, 1)) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keeps the block loop scalar
  const int g = lane >> 4;
  const int c = lane & 15;
  const size_t qrow0 = (size_t)b * a.q_heads + (size_t)kvh * G;

  if (n_blk == 0) {  // empty context: zero output (weighted sum of nothing)
    for (int idx = tid; idx < G * D; idx += kDecodeThreads) a.out[qrow0 * D + idx] = 0;
    return;
  }

  // ---- this wavefront's blocks: every 4th block of the split ----
  const int blk_begin = first_blk + split * a.split_blocks;
  const int blk_end = min(blk_begin + a.split_blocks, first_blk + n_blk);
  const int nbw = max(0, (blk_end - blk_begin - wave + 3) / 4);
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  // pool index of block k of this wavefront: a scalar load from the block-table
  // row (no one writes it during the launch), fetched one block ahead, so the
  // waits before the math cover K/V loads only
  typedef const __attribute__((address_space(4))) int32_t table_elem_t;
  const table_elem_t *stable = (const table_elem_t *)table;
  auto entry = [&](int k) __attribute__((always_inline)) -> int {
    return stable[(blk_begin + wave + 4 * k) % a.max_blocks];
  };

  constexpr bool TL = kTokenLanes<G, FMT>;
  uint32_t qw[G][kQWords<G, FMT>];
  load_q<G, FMT>(a, qrow0, lane, qw);

  SoftmaxState<G> st;
  reset_state(st);
  // fused append, bf16: the pool part attends [lo, len - 1) and the new token comes from
  // a.k_new; int8 / fp8: the token is quantised into the registers of the block that
  // receives it, which is then attended up to len as stored
  constexpr bool fused = FUSED;
  constexpr bool qfused = FUSED && FMT != kBf16;
  const int len_kv = fused && !qfused ? len - 1 : len;
  // the wavefront that walks the sequence's last block takes the new token: its rows
  // are loaded now, ahead of the block loop
  const int last_blk = first_blk + n_blk - 1;
  const bool takes_new = fused && last_blk >= blk_begin && last_blk < blk_end && (last_blk - blk_begin) % 4 == wave;
  typename NtOf<FMT>::type nt;
  if (takes_new) load_nt(a, b, kvh, lane, nt, stable[((len - 1) / BT) % a.max_blocks]);

  // ---- two-stage block pipeline: block k+1's loads are in flight during block k's math ----
  float qstep = 1.0f;
  if (nbw > 0) {
    BlockRegs<FMT> r[2];
    load_block<FMT, TL>(a, entry(0), kvh, lane, r[0]);
    qstep = prep_q<G, FMT>(lane, qw);
    int e_next = nbw > 1 ? entry(1) : -1;
    // every step inside the loop issues the next block's loads before its math,
    // so the wait before the math always leaves them in flight
    auto step = [&](int k, BlockRegs<FMT> &cur, BlockRegs<FMT> &nxt, bool issue) __attribute__((always_inline)) {
      if (issue) {
        load_block<FMT, TL>(a, e_next, kvh, lane, nxt);
        e_next = k + 2 < nbw ? entry(k + 2) : -1;
      }
      // int8 / fp8 fused append: the block that receives the new token gets it patched in
      // first (one compute_block below either way: the block math is not duplicated)
      NewTokenStore nw{false, 0u, 0u, false};
      const bool patch = qfused && takes_new && blk_begin + wave + 4 * k == last_blk;
      if constexpr (qfused)
        if (patch) nw = patch_new_token_q<G, FMT>(a, cur, nt, kvh, (len - 1) % BT, lane);
      compute_block<G, FMT>(a, cur, blk_begin + wave + 4 * k, lo, len_kv, lane, qw, qstep, st);
      if constexpr (qfused)
        if (patch) store_new_token_q<G, FMT>(a, cur, nt, nw, kvh, (len - 1) % BT, lane);
    };
    int k = 0;
    for (; k + 2 < nbw; k += 2) {
      step(k, r[0], r[1], true);
      step(k + 1, r[1], r[0], true);
    }
    if (k + 1 < nbw) {
      step(k, r[0], r[1], true);
      step(k + 1, r[1], r[0], false);
    } else {
      step(k, r[0], r[1], false);
    }
  }

  if constexpr (FMT == kBf16)
    if (takes_new) add_new_token<G>(a, st, b, kvh, len, lane, qw, nt);

  // ---- merge the four token groups of the wavefront ----
  finalize_state<G, FMT>(st);
  __shared__ float s_o[4][G][D];
  __shared__ float s_m[4][G];
  __shared__ float s_l[4][G];
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    float mm = fmaxf(st.m[gi], xor16_other(st.m[gi], lane));
    mm = fmaxf(mm, xor32_other(mm, lane));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    const float f = fast_exp2(st.m[gi] - mref);
    float ll = st.l[gi] * f;
    ll += xor16_other(ll, lane);
    ll += xor32_other(ll, lane);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float v = st.o[gi][j] * f;
      v += xor16_other(v, lane);
      v += xor32_other(v, lane);
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
      a.out[(qrow0 + gi) * D + d] = f32_to_bf16_rne(gated(oo / ll, a.gate, (qrow0 + gi) * D + d));
    } else {
      const size_t row = (qrow0 + gi) * a.max_splits + split;
      a.ws_o[row * D + d] = oo;
      if (d == 0) a.ws_ml[row] = make_float2(mm, ll);
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent stream decode.
//
// The attended blocks of one (sequence, kv head) are that segment's "units".
// All units of the step, U of them, are ordered (sequence, kv head, block) and
// wavefront w < W' = min(W, U) of the W in the grid streams the contiguous
// range [w * U / W', (w + 1) * U / W'), across kv-head and sequence
// boundaries, loading one unit ahead of the math.  Every wavefront has the same number of units to
// within one however ragged the lengths are, there is no workgroup barrier and
// no wait on another workgroup, so results do not depend on how many
// workgroups are resident at once (the default grid is all resident).
//
// A segment that lies wholly inside one wavefront's range is written out
// directly.  A segment cut between wavefronts leaves one (max, sum, output)
// partial per wavefront in slot 2w (the wavefront's first segment) or 2w + 1
// (its last); the wavefront that holds the segment's first unit records
// (first slot, count) in seg_desc and decode_stream_merge_kernel merges them.
// ---------------------------------------------------------------------------
// Ends a segment: merges the wavefront's four token groups, then writes the
// bf16 output (complete segment) or the partial in `slot`; resets the state.
template <int G>
__device__ __forceinline__ void stream_flush(const DecodeArgs &a, SoftmaxState<G> &st, int b, int kvh, bool complete,
                                             int slot, int lane) {
  const int g = lane >> 4;
  const int c = lane & 15;
  const size_t qrow0 = (size_t)b * a.q_heads + (size_t)kvh * G;
#pragma unroll
  for (int gi = 0; gi < G; gi++) {
    float mm = fmaxf(st.m[gi], xor16_other(st.m[gi], lane));
    mm = fmaxf(mm, xor32_other(mm, lane));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    const float f = fast_exp2(st.m[gi] - mref);
    float ll = st.l[gi] * f;
    ll += xor16_other(ll, lane);
    ll += xor32_other(ll, lane);
    float o2[2];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float v = st.o[gi][j] * f;
      v += xor16_other(v, lane);
      v += xor32_other(v, lane);
      if (j == 2 * g) o2[0] = v;
      if (j == 2 * g + 1) o2[1] = v;
    }
    // every group now holds the totals; group g writes dims 16j + c for j = 2g, 2g + 1
    if (complete) {
      const float inv = 1.0f / ll;
      const size_t o0 = (qrow0 + gi) * D + 16 * (2 * g) + c;
      a.out[o0] = f32_to_bf16_rne(gated(o2[0] * inv, a.gate, o0));
      a.out[o0 + 16] = f32_to_bf16_rne(gated(o2[1] * inv, a.gate, o0 + 16));
    } else {
      const size_t row = (size_t)slot * G + gi;
      a.ws_o[row * D + 16 * (2 * g) + c] = o2[0];
      a.ws_o[row * D + 16 * (2 * g + 1) + c] = o2[1];
      if (lane == 0) a.ws_ml[row] = make_float2(mm, ll);
    }
  }
  reset_state(st);
}

// Waves per SIMD the stream kernel is built for: two (its grid of two workgroups
// per CU all resident) for up to four query heads per kv head; the quantised fused
// append's extra registers would otherwise push it to one.
template <int G>
constexpr int kStreamWavesPerSimd = G <= 4 ? 2 : 1;

template <int G, int FMT, bool FUSED = false>
__global__ __launch_bounds__(kDecodeThreads) __attribute__((amdgpu_waves_per_eu(kStreamWavesPerSimd<G>)))
void paged_decode_stream_kernel(const DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  // wave-uniform (readfirstlane): the partition, cursors and branches stay scalar
  const int w = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int W = gridDim.x * 4;
  const int Hkv = a.pool.kv_heads;
  const int B = a.num_seqs;
  const int len0 = lane < B ? a.seq_lens[lane] : 0;  // sequences 0..63, one per lane
  int bad_flags;
  const StreamRange sr = stream_range(a, W, w, lane, len0, &bad_flags);
  if (bad_flags) {
    if (w == 0 && lane == 0) atomicOr(a.err, bad_flags);
    return;
  }
  // empty sequences: zero output (weighted sum of nothing), nothing to merge
  // (lengths of sequences 0..63 come from len0's lanes: no load on the way to
  // the first unit)
  for (int b = w; b < B; b += W) {
    if (attended_blocks(a, b < 64 ? __builtin_amdgcn_readlane(len0, b) : a.seq_lens[b]) == 0) {
      for (int idx = lane; idx < a.q_heads * D; idx += 64) a.out[(size_t)b * a.q_heads * D + idx] = 0;
      for (int idx = lane; idx < 2 * Hkv; idx += 64) a.seg_desc[(size_t)b * Hkv * 2 + idx] = 0;
    }
  }
  const int n = __builtin_amdgcn_readfirstlane(sr.n);
  if (n == 0) return;
  const int U = __builtin_amdgcn_readfirstlane(sr.U);
  const int Wu = __builtin_amdgcn_readfirstlane(sr.Wu);
  // fused append, bf16: the pool part attends [lo, len - 1) and the new token comes from
  // a.k_new; int8 / fp8: the token is quantised into the registers of the segment's last
  // unit (the block that receives it), which is attended up to len as stored
  constexpr bool fused = FUSED;
  constexpr bool qfused = FUSED && FMT != kBf16;

  // Lengths, block-table entries: scalar loads (constant address space: no
  // one writes them during the launch), so the waits before the math cover
  // K/V loads only.  Sequences 0..63 take their length from len0's lanes.
  const stream_const_i32 *stable = (const stream_const_i32 *)a.tables;
  auto advance = [&](UnitCursor &c) __attribute__((always_inline)) { cursor_advance(a, len0, c); };
  const UnitCursor c0 = cursor_at(a, len0, sr);
  // three cursors: the next block-table entry to fetch (one unit ahead of the
  // loads), the next unit to load, the next unit to compute
  UnitCursor E = c0, L = c0, C = c0;
  auto next_entry = [&]() __attribute__((always_inline)) -> int {
    const int e = stable[(size_t)E.b * a.max_blocks + E.tab];
    advance(E);
    return e;
  };

  bool seg_from_start = C.j == 0;
  bool first_seg = true;
  bool need_q = false;
  constexpr bool TL = kTokenLanes<G, FMT>;
  uint32_t qw[G][kQWords<G, FMT>];
  load_q<G, FMT>(a, (size_t)C.b * a.q_heads + (size_t)C.kvh * G, lane, qw);

  BlockRegs<FMT> r[2];
  const int e_first = next_entry();
  load_block<FMT, TL>(a, e_first, L.kvh, lane, r[0]);
  // fused append: a segment's new-token rows are loaded with its last unit, into
  // the buffer that travels with that unit's registers (r[0] / r[1]), with that
  // unit's block-table entry (the block the token goes to)
  typedef typename NtOf<FMT>::type NT;
  NT nt[2];
  NewToken pend;  // bf16: a computed segment's new token, not yet written to the pool
  int pend_kvh = 0, pend_len = 0;
  bool have_pend = false;
  if constexpr (fused)
    if (L.j == L.nb - 1) load_nt(a, L.b, L.kvh, lane, nt[0], e_first);
  float qstep = prep_q<G, FMT>(lane, qw);
  int e_next = n > 1 ? next_entry() : -1;
  advance(L);
  SoftmaxState<G> st;
  reset_state(st);

  auto end_segment = [&](bool complete) __attribute__((always_inline)) {
    const int slot = w * 2 + (first_seg ? 0 : 1);
    finalize_state<G, FMT>(st);
    stream_flush<G>(a, st, C.b, C.kvh, complete, slot, lane);
    if (lane == 0 && (complete || seg_from_start)) {
      // this wavefront holds the segment's first unit: record how to merge it
      int2 d = make_int2(0, 0);
      if (!complete) d = make_int2(slot, wave_of_unit(C.base + (C.kvh + 1) * C.nb - 1, U, Wu) - w + 1);
      reinterpret_cast<int2 *>(a.seg_desc)[(size_t)C.b * Hkv + C.kvh] = d;
    }
    first_seg = false;
  };

  // One unit: a new segment's q is loaded first, then unit k+1's loads are
  // issued, then q is prepared (prep_q) and unit k is computed.  Every step
  // inside the loop issues the next unit's loads after any q load, so the wait
  // before the math always leaves the next unit's loads in flight.
  auto step = [&](int k, BlockRegs<FMT> &cur, BlockRegs<FMT> &nxt, NT &cur_nt, NT &nxt_nt, bool issue)
                  __attribute__((always_inline)) {
    const bool new_q = need_q;
    if (new_q) load_q<G, FMT>(a, (size_t)C.b * a.q_heads + (size_t)C.kvh * G, lane, qw);
    if (issue) {
      load_block<FMT, TL>(a, e_next, L.kvh, lane, nxt);
      if constexpr (fused)
        if (L.j == L.nb - 1) load_nt(a, L.b, L.kvh, lane, nxt_nt, e_next);
      e_next = k + 2 < n ? next_entry() : -1;
      advance(L);
    }
    if (new_q) {
      qstep = prep_q<G, FMT>(lane, qw);
      need_q = false;
    }
    // int8 / fp8 fused append: the segment's last unit (the block that receives the new
    // token) gets it patched in first (one compute_block either way)
    NewTokenStore nw{false, 0u, 0u, false};
    if constexpr (qfused)
      if (C.j == C.nb - 1) nw = patch_new_token_q<G, FMT>(a, cur, cur_nt, C.kvh, (C.len - 1) % BT, lane);
    compute_block<G, FMT>(a, cur, C.lo / BT + C.j, C.lo, fused && !qfused ? C.len - 1 : C.len, lane, qw, qstep, st);
    if constexpr (qfused)
      if (C.j == C.nb - 1) store_new_token_q<G, FMT>(a, cur, cur_nt, nw, C.kvh, (C.len - 1) % BT, lane);
    if (C.j == C.nb - 1) {  // the segment ends with this unit
      if constexpr (fused && FMT == kBf16) {
          if constexpr (G > 4) {
            add_new_token<G, true>(a, st, C.b, C.kvh, C.len, lane, qw, cur_nt);  // no registers to spare
          } else {
            // The token's pool write waits for the end of the range (or the range's
            // next new token): stores count in vmcnt like loads, so one issued in
            // the loop would be waited for by the next unit's load wait.
            add_new_token<G, false>(a, st, C.b, C.kvh, C.len, lane, qw, cur_nt);
            if (have_pend) store_new_token(a, pend_kvh, pend_len, lane, pend);
            pend = cur_nt;
            pend_kvh = C.kvh;
            pend_len = C.len;
            have_pend = true;
          }
        }
      end_segment(seg_from_start);
      seg_from_start = true;
      need_q = true;
    }
    advance(C);
  };
  int k = 0;
  for (; k + 2 < n; k += 2) {
    step(k, r[0], r[1], nt[0], nt[1], true);
    step(k + 1, r[1], r[0], nt[1], nt[0], true);
  }
  if (k + 1 < n) {
    step(k, r[0], r[1], nt[0], nt[1], true);
    step(k + 1, r[1], r[0], nt[1], nt[0], false);
  } else {
    step(k, r[0], r[1], nt[0], nt[1], false);
  }
  if (C.j != 0) end_segment(false);  // the range ends inside a segment
  if constexpr (FMT == kBf16)
    if (fused && have_pend) store_new_token(a, pend_kvh, pend_len, lane, pend);
}

// One round of the stream merge over partials i0 .. i0+cnt-1 (1 <= cnt <= N <=
// 64) of a cut segment.  Every dim and every (max, sum) pair of the round is
// loaded before any is used: dims past the last partial re-read the last one
// and get weight 0, lane j loads pair j, and the weights reach all lanes by
// readlane.  The merge launch is latency-bound, so this keeps it at two
// dependent memory round trips (descriptor, then partials).
template <int G, int N>
__device__ __forceinline__ void stream_merge_round(const DecodeArgs &a, int first_slot, int wf, int gi, int i0, int cnt,
                                                   int lane, float &mm, float &ll, float &o0, float &o1) {
  // partial k of the segment: the first wavefront's slot, then the later wavefronts' first-segment slots
  auto row_of = [&](int k) { return (size_t)(k == 0 ? first_slot : (wf + k) * 2) * G + gi; };
  const float2 ml = a.ws_ml[row_of(i0 + min(lane, cnt - 1))];
  float a0[N], a1[N];
#pragma unroll
  for (int i = 0; i < N; i++) {
    const size_t row = row_of(i0 + min(i, cnt - 1));
    a0[i] = a.ws_o[row * D + lane];
    a1[i] = a.ws_o[row * D + 64 + lane];
  }
  __builtin_amdgcn_sched_barrier(0);  // every load of the round is issued before the first wait
  static_assert(N == 16 || N == 32, "one or two DPP rows of partials");
  // max and sum over lanes 0 .. N-1: DPP within rows, then a row exchange (no LDS)
  const float m = lane < cnt ? ml.x : -INFINITY;
  float nm = m;
  nm = fmaxf(nm, dpp<0xB1>(nm));   // quad_perm [1,0,3,2]
  nm = fmaxf(nm, dpp<0x4E>(nm));   // quad_perm [2,3,0,1]
  nm = fmaxf(nm, dpp<0x141>(nm));  // row_half_mirror
  nm = fmaxf(nm, dpp<0x140>(nm));  // row_mirror
  if constexpr (N == 32) nm = fmaxf(nm, xor16_other(nm, lane));
  nm = fmaxf(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(nm))), mm);
  const float mref = (nm == -INFINITY) ? 0.0f : nm;
  const float f = fast_exp2(m - mref);  // 0 on lanes past the last partial
  float ls = row_sum16(ml.y * f);
  if constexpr (N == 32) ls += xor16_other(ls, lane);
  const float f0 = fast_exp2(mm - mref);
  ll = ll * f0 + __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ls)));
  o0 *= f0;
  o1 *= f0;
#pragma unroll
  for (int i = 0; i < N; i++) {
    const float fi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), i));
    o0 += a0[i] * fi;
    o1 += a1[i] * fi;
  }
  mm = nm;
}

// Merges the partials of the stream kernel's cut segments: one wavefront per
// (query head, sequence), two dims per lane; up to 16 partials in one round,
// more in rounds of 32.
template <int G>
__global__ __launch_bounds__(64) void decode_stream_merge_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int kvh = h / G;
  const int gi = h - kvh * G;
  const int2 d = reinterpret_cast<const int2 *>(a.seg_desc)[(size_t)b * a.pool.kv_heads + kvh];
  const int W = a.stream_wgs * 4;
  const int wf = d.x >> 1;
  // written by the stream kernel; a call it aborted (error flags) may leave any
  // values, so only descriptors naming slots of this grid are followed
  if (d.y < 2 || d.x < 0 || d.x >= 2 * W || wf + d.y > W) return;
  float mm = -INFINITY, ll = 0.0f, o0 = 0.0f, o1 = 0.0f;
  if (d.y <= 16) {
    stream_merge_round<G, 16>(a, d.x, wf, gi, 0, d.y, lane, mm, ll, o0, o1);
  } else {
#pragma unroll 1
    for (int i0 = 0; i0 < d.y; i0 += 32)
      stream_merge_round<G, 32>(a, d.x, wf, gi, i0, min(32, d.y - i0), lane, mm, ll, o0, o1);
  }
  const float inv = 1.0f / ll;
  const size_t orow = (size_t)b * a.q_heads + h;
  a.out[orow * D + lane] = f32_to_bf16_rne(gated(o0 * inv, a.gate, orow * D + lane));
  a.out[orow * D + 64 + lane] = f32_to_bf16_rne(gated(o1 * inv, a.gate, orow * D + 64 + lane));
}

// Log-sum-exp merge of the split partials: one workgroup of 128 lanes (one per
// dim) per (query head, sequence) whose sequence used more than one split.
// The merge is latency-bound, so it is laid out as few dependent memory round
// trips as possible: up to 128 splits from one round of loads
// (merge_in_registers); beyond that the partials of the first 96 splits are
// loaded together with the (max, sum) pairs, the pairs are reduced through
// LDS, and any remaining partials follow 32 at a time.
constexpr int kMergeMaxSplits = 1024;
constexpr int kMergeOneRound = 128;  // splits merged from one round of loads, all in registers
constexpr int kMergePrefetch = 96;   // partials loaded up front on the LDS path

// Merge of n <= N <= 128 splits from one round of loads, all in registers.
// Partial rows past the last split re-read the last split (no branch between
// the loads and their use, so they are all in flight at once) and are weighted
// 0.  The (max, sum) pairs are spread over the lanes: lane i of each wavefront
// loads those of splits i and 64 + i with vector loads, the wavefront reduces
// them with DPP and row exchanges, and the split weights reach every lane
// through LDS.  (Loaded as uniform values they became scalar loads, and
// the scalar queue's depth split them into several dependent rounds: a merge
// of 64 splits took ~7 us.)
template <int N>
__device__ __forceinline__ void merge_in_registers(const DecodeArgs &a, size_t row0, int last, int d, size_t orow) {
  static_assert(N <= 128, "at most two (max, sum) pairs per lane");
  constexpr int P = (N + 63) / 64;  // pairs per lane
  float o_sp[N];
#pragma unroll
  for (int i = 0; i < N; i++) o_sp[i] = a.ws_o[(row0 + min(i, last)) * D + d];
  const int li = d & 63;
  float mx[P], ly[P];
#pragma unroll
  for (int p = 0; p < P; p++) {
    const float2 ml = a.ws_ml[row0 + min(64 * p + li, last)];
    mx[p] = 64 * p + li <= last ? ml.x : -INFINITY;
    ly[p] = ml.y;
  }
  // wavefront max and sum: DPP within rows of 16, then row exchanges (no LDS)
  float mm = mx[0];
#pragma unroll
  for (int p = 1; p < P; p++) mm = fmaxf(mm, mx[p]);
  mm = fmaxf(mm, dpp<0xB1>(mm));   // quad_perm [1,0,3,2]
  mm = fmaxf(mm, dpp<0x4E>(mm));   // quad_perm [2,3,0,1]
  mm = fmaxf(mm, dpp<0x141>(mm));  // row_half_mirror
  mm = fmaxf(mm, dpp<0x140>(mm));  // row_mirror
  mm = fmaxf(mm, xor16_other(mm, li));
  mm = fmaxf(mm, xor32_other(mm, li));
  const float mref = (mm == -INFINITY) ? 0.0f : mm;
  float f[P];
  float lsum = 0.0f;
#pragma unroll
  for (int p = 0; p < P; p++) {
    f[p] = 64 * p + li <= last ? fast_exp2(mx[p] - mref) : 0.0f;
    lsum += ly[p] * f[p];
  }
  float ll = row_sum16(lsum);
  ll += xor16_other(ll, li);
  ll += xor32_other(ll, li);
  // the weights to every lane through LDS (broadcast reads)
  __shared__ __attribute__((aligned(16))) float s_w[N];
  if (d < 64) {
#pragma unroll
    for (int p = 0; p < P; p++)
      if (64 * p + li < N) s_w[64 * p + li] = f[p];
  }
  __syncthreads();
  float oo = 0.0f;
#pragma unroll
  for (int i = 0; i < N; i++) oo += o_sp[i] * s_w[i];
  a.out[orow * D + d] = f32_to_bf16_rne(gated(oo / ll, a.gate, orow * D + d));
}

__global__ __launch_bounds__(D) void decode_merge_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  int len, lo, first_blk, n_blk, n_splits;
  seq_range(a, b, len, lo, first_blk, n_blk, n_splits);
  if (n_splits <= 1 || n_splits > a.max_splits || n_splits > kMergeMaxSplits || len - lo > a.max_blocks * BT) return;
  const int d = threadIdx.x;
  const size_t row0 = ((size_t)b * a.q_heads + h) * a.max_splits;
  const size_t orow = (size_t)b * a.q_heads + h;
  const int last = n_splits - 1;
  if (n_splits <= 8) return merge_in_registers<8>(a, row0, last, d, orow);
  if (n_splits <= 16) return merge_in_registers<16>(a, row0, last, d, orow);
  if (n_splits <= 32) return merge_in_registers<32>(a, row0, last, d, orow);
  if (n_splits <= 64) return merge_in_registers<64>(a, row0, last, d, orow);
  if (n_splits <= kMergeOneRound) return merge_in_registers<kMergeOneRound>(a, row0, last, d, orow);
  // partials of the first splits: in flight while the (max, sum) pairs are reduced
  float o_pre[kMergePrefetch];
#pragma unroll
  for (int i = 0; i < kMergePrefetch; i++) o_pre[i] = a.ws_o[(row0 + min(i, last)) * D + d];
  __shared__ float s_f[kMergeMaxSplits];
  __shared__ float s_l[kMergeMaxSplits];
  __shared__ float s_red[2];
  float lm = -INFINITY;
  for (int sp = d; sp < n_splits; sp += D) {
    const float2 ml = a.ws_ml[row0 + sp];
    s_f[sp] = ml.x;
    s_l[sp] = ml.y;
    lm = fmaxf(lm, ml.x);
  }
  // max over the workgroup (two wavefronts)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) lm = fmaxf(lm, __shfl_xor(lm, o));
  if ((d & 63) == 0) s_red[d >> 6] = lm;
  __syncthreads();
  const float mm = fmaxf(s_red[0], s_red[1]);
  const float mref = (mm == -INFINITY) ? 0.0f : mm;
  float ll = 0.0f;
  for (int sp = d; sp < n_splits; sp += D) {
    const float f = fast_exp2(s_f[sp] - mref);
    ll += s_l[sp] * f;
    s_f[sp] = f;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ll += __shfl_xor(ll, o);
  __syncthreads();
  if ((d & 63) == 0) s_red[d >> 6] = ll;
  __syncthreads();
  const float l_tot = s_red[0] + s_red[1];
  float oo = 0.0f;
#pragma unroll
  for (int i = 0; i < kMergePrefetch; i++) oo += o_pre[i] * (i <= last ? s_f[min(i, last)] : 0.0f);
  for (int sp0 = kMergePrefetch; sp0 < n_splits; sp0 += 32) {
    float o_sp[32];
#pragma unroll
    for (int i = 0; i < 32; i++) o_sp[i] = a.ws_o[(row0 + min(sp0 + i, last)) * D + d];
#pragma unroll
    for (int i = 0; i < 32; i++) oo += o_sp[i] * (sp0 + i <= last ? s_f[min(sp0 + i, last)] : 0.0f);
  }
  a.out[orow * D + d] = f32_to_bf16_rne(gated(oo / l_tot, a.gate, orow * D + d));
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
  if (a.ring_tokens == 0 && (int64_t)rows > (int64_t)a.max_blocks * a.pool.block_tokens) {
    if (threadIdx.x == 0) atomicOr(a.err, kErrSpan);  // the span would alias its own table entries
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
    acc = gated(acc, a.gate, qoff + d);
    if constexpr (sizeof(OT) == 4)
      reinterpret_cast<float *>(a.out)[qoff + d] = acc;
    else
      reinterpret_cast<uint16_t *>(a.out)[qoff + d] = f32_to_bf16_rne(acc);
  }
}

__global__ void decode_fp8_kernel(const uint8_t *codes, float *out, int32_t n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = bf16_lo(fp8x2_to_bf16<false>((uint32_t)codes[i]));
}

template <int G, int FMT, bool FUSED>
hipError_t launch_decode_t(const DecodeArgs &a, int max_seq_len, hipStream_t s, void *hu, LaunchHook hook) {
  const int max_blk = (max_seq_len + BT - 1) / BT + 1;
  const int grid_x = max(1, (max_blk + a.split_blocks - 1) / a.split_blocks);
  if (hook) hook(hu, 0, s);
  if (a.stream_wgs > 0) {
    // fp8 appends on the stream plan go through the append kernel (the host never
    // asks for this instantiation)
    if constexpr (FUSED && FMT == kFp8) {
      return hipErrorInvalidValue;
    } else {
      hipLaunchKernelGGL((paged_decode_stream_kernel<G, FMT, FUSED>), dim3(a.stream_wgs), dim3(kDecodeThreads), 0,
                         s, a);
    }
    hipError_t e = hipGetLastError();
    if (hook) hook(hu, 1, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((decode_stream_merge_kernel<G>), dim3(a.q_heads, a.num_seqs), dim3(64), 0, s, a);
    return hipGetLastError();
  }
  dim3 grid(min(grid_x, a.max_splits), a.pool.kv_heads, a.num_seqs);
  hipLaunchKernelGGL((paged_decode_kernel<G, FMT, FUSED>), grid, dim3(kDecodeThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (hook) hook(hu, 1, s);
  if (e != hipSuccess || a.max_splits <= 1) return e;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(a.q_heads, a.num_seqs), dim3(D), 0, s, a);
  return hipGetLastError();
}

template <int G>
hipError_t launch_decode_fmt(const DecodeArgs &a, int max_seq_len, hipStream_t s, void *hu, LaunchHook hook) {
  switch (a.pool.format) {
    case kBf16:  // a.k_new: fused append of each sequence's new token
      return a.k_new ? launch_decode_t<G, kBf16, true>(a, max_seq_len, s, hu, hook)
                     : launch_decode_t<G, kBf16, false>(a, max_seq_len, s, hu, hook);
    case kInt8:
      return a.k_new ? launch_decode_t<G, kInt8, true>(a, max_seq_len, s, hu, hook)
                     : launch_decode_t<G, kInt8, false>(a, max_seq_len, s, hu, hook);
    case kFp8:
      return a.k_new ? launch_decode_t<G, kFp8, true>(a, max_seq_len, s, hu, hook)
                     : launch_decode_t<G, kFp8, false>(a, max_seq_len, s, hu, hook);
    case kF16:  // appends go through the append kernel (the host never sets a.k_new here)
      if (a.k_new) return hipErrorInvalidValue;
      return launch_decode_t<G, kF16, false>(a, max_seq_len, s, hu, hook);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_decode(const DecodeArgs &a, int group, int max_seq_len, hipStream_t s, void *hu, LaunchHook hook) {
  switch (group) {
    case 1:
      return launch_decode_fmt<1>(a, max_seq_len, s, hu, hook);
    case 2:
      return launch_decode_fmt<2>(a, max_seq_len, s, hu, hook);
    case 4:
      return launch_decode_fmt<4>(a, max_seq_len, s, hu, hook);
    case 8:
      return launch_decode_fmt<8>(a, max_seq_len, s, hu, hook);
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
