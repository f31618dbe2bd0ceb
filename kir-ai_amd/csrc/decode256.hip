// Paged GQA decode attention for head_dim 256 on gfx950 (MI355X): the
// full-attention layers of Qwen3.5 / 3.6 (fixtures/qwen36/config.json: 16 query
// heads, 2 kv heads, head_dim 256, so G = 8 query heads per kv head), bf16 or fp16
// K/V in 16-token blocks (fp16: each head's q is scaled into fp16 by a power of two
// chosen from its largest magnitude, undone on the scores).  Same contract as the head_dim-128 kernels in decode.hip: per
// sequence b and query head h,
//   out[b][h] = sum_t softmax_t(scale * q[b][h] . K[t][kv]) V[t][kv]
// over the attended positions [lo, len) (crates/llm-backend/src/core/
// native_attention.rs:731-771; window rule qwen/ops/cache.rs:116-121), times
// sigmoid(gate) when the call carries a gate (native_attention.rs:765-781).
//
// Two launch shapes over the same per-block math:
// * split-K: one workgroup per (split, kv head, sequence); a split is
//   `split_blocks` consecutive blocks and its four wavefronts take them
//   round-robin.  A single-split sequence writes its output directly, otherwise
//   decode_merge_d256_kernel merges the splits' (max, sum, output) partials.
// * persistent stream (paged_decode_d256_stream_kernel): the step's units
//   (sequence, kv head, block) cut into equal consecutive ranges, one per
//   wavefront of a grid that fills every SIMD (stream_partition.h), as the
//   head_dim-128 stream kernel does; decode_stream_merge_d256_kernel merges the
//   segments cut between wavefronts.
//
// Lane roles per block (64 lanes, row g = lane / 16, c = lane % 16):
//   K: lane loads token 4g + i (i = 0..3) at dims 8c..8c+7 and 128+8c..+7
//      (two 256-byte runs per instruction and row) and forms 32 partial dot
//      products (8 heads x 4 tokens) over its 16 dims.  Query slot s of lane c
//      holds head s ^ fold(c), fold linear over the bits of c, so the 16-lane
//      sum becomes a reduce-scatter of three DPP adds on 16, 8 and 4 values
//      (row_mirror, row_half_mirror, quad swap) and one lane-pair exchange:
//      afterwards lane c holds the scores of head fold(c) for tokens
//      4g + 2 (c % 2) + {0, 1}, each computed once per wavefront.
//   V: lane owns dims 64 j + lane (j = 0..3), all 16 tokens (two 16-byte
//      loads per dim row): no two lanes accumulate the same output element.
//   The 64 packed weight pairs (8 heads x 8 token pairs, one per lane, in the pool's
//   16-bit format)
//   reach every lane as scalar registers (v_readlane), the scalar operand of
//   p . v's dot2 instructions.
// Running max / sum live in the 8 lanes that score a head; outputs in
// registers (8 heads x 4 dims per lane).  HBM-bound; no MFMA.
#include "device_common.h"
#include "stream_partition.h"
#include "wave_ops.h"

namespace llh {

namespace {

constexpr int D2 = kD256HeadDim;
constexpr int BT = kFastBlockTokens;
constexpr int G2 = kD256Group;
constexpr int kBlockBytes2 = BT * D2 * 2;  // one (block, kv head) of K (and of V), bf16
constexpr int kMerge256MaxSplits = 64;

// Head of query slot 0 in lane c of a row (and of slot s: s ^ fold(c)).  fold is
// linear over GF(2) in the bits of c with fold(15) = 4, fold(7) = 2, fold(2) = 1
// and fold(1) = 0: the lane that a reduce step pairs c with (c ^ 15, c ^ 7,
// c ^ 2, c ^ 1) holds the same head in the slot 4, 2, 1 (0) places away.
__host__ __device__ constexpr int fold(int c) {
  return ((c >> 1) & 1) ^ (((c >> 2) & 1) * 3) ^ (((c >> 3) & 1) * 6);
}
// The lane pair (2x, 2x + 1) of a row whose slot-0 head is h.
__host__ __device__ constexpr int pair_of_head(int h) {
  int x = 0;
  while (fold(2 * x) != h) x++;
  return x;
}
static_assert(fold(15) == 4 && fold(7) == 2 && fold(2) == 1 && fold(1) == 0, "reduce-scatter pairing");

struct Kregs {
  uint4 k[8];  // token 4g + i/2 ... : k[2i] dims 8c..8c+7, k[2i+1] dims 128+8c..+7
};
struct Vregs {
  uint4 v[8];  // v[2j + h]: dim 64j + lane, tokens 8h .. 8h+7
};

__device__ __forceinline__ const char *block_base(const void *base, int phys, int kvh, int kv_heads) {
  return reinterpret_cast<const char *>(base) + ((size_t)phys * kv_heads + kvh) * kBlockBytes2;
}

__device__ __forceinline__ void load_k(const DecodeArgs &a, int phys, int kvh, int lane, Kregs &r) {
  const char *kb = block_base(a.pool.k, phys, kvh, a.pool.kv_heads) + (lane >> 4) * 4 * (D2 * 2) + (lane & 15) * 16;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    r.k[2 * i] = ld_nt16(kb + i * (D2 * 2));
    r.k[2 * i + 1] = ld_nt16(kb + i * (D2 * 2) + 256);
  }
}

__device__ __forceinline__ void load_v(const DecodeArgs &a, int phys, int kvh, int lane, Vregs &r) {
  const char *vb = block_base(a.pool.v, phys, kvh, a.pool.kv_heads) + lane * (BT * 2);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    r.v[2 * j] = ld_nt16(vb + j * 64 * (BT * 2));
    r.v[2 * j + 1] = ld_nt16(vb + j * 64 * (BT * 2) + 16);
  }
}

struct State256 {
  float m;        // running max (log2 units) of this lane's head fold(c)
  float l;        // this lane's share of that head's weight sum
  float o[G2][4]; // head h, dim 64j + lane
};

// First half of one block: scores, online softmax.  jb: the block's index in the
// sequence (positions 16 jb ..); valid: its table entry is inside the pool.
// Returns this lane's packed weight pair (head fold(c), tokens 4g + 2 (c % 2) + {0, 1})
// and, per token pair, the mask that zeroes V of unattended tokens.
// FMT: kBf16, or kF16 (fp16 blocks, q scaled per head into fp16 by prep_q256_f16).
// sscale: the score scale in log2 units, scale_log2e (times this lane's head's step
// over fp16 blocks).
template <int FMT>
__device__ __forceinline__ uint32_t block_scores(const DecodeArgs &a, const Kregs &kr, bool valid, int jb, int lo,
                                                 int len, int lane, const uint32_t (&qw)[G2][8], State256 &st,
                                                 uint32_t (&vm)[8], float sscale) {
  const int g = lane >> 4;
  const int b0 = lane & 1;
  // ---- partial q . k: slot s, token 4g + i, over this lane's 16 dims ----
  float p[G2][4];
#pragma unroll
  for (int s = 0; s < G2; s++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint4 lo4 = kr.k[2 * i], hi4 = kr.k[2 * i + 1];
      float acc = dot2_16<FMT>(lo4.x, qw[s][0], 0.0f);
      acc = dot2_16<FMT>(lo4.y, qw[s][1], acc);
      acc = dot2_16<FMT>(lo4.z, qw[s][2], acc);
      acc = dot2_16<FMT>(lo4.w, qw[s][3], acc);
      acc = dot2_16<FMT>(hi4.x, qw[s][4], acc);
      acc = dot2_16<FMT>(hi4.y, qw[s][5], acc);
      acc = dot2_16<FMT>(hi4.z, qw[s][6], acc);
      acc = dot2_16<FMT>(hi4.w, qw[s][7], acc);
      p[s][i] = acc;
    }
  // ---- reduce-scatter over the row (see fold) ----
#pragma unroll
  for (int s = 0; s < 4; s++)
#pragma unroll
    for (int i = 0; i < 4; i++) p[s][i] += row_mirror(p[s + 4][i]);
#pragma unroll
  for (int s = 0; s < 2; s++)
#pragma unroll
    for (int i = 0; i < 4; i++) p[s][i] += dpp<0x141>(p[s + 2][i]);  // row_half_mirror
#pragma unroll
  for (int i = 0; i < 4; i++) p[0][i] += dpp<0x4E>(p[1][i]);  // quad_perm [2,3,0,1]
  float sc[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const float keep = b0 ? p[0][2 + k] : p[0][k];
    const float send = b0 ? p[0][k] : p[0][2 + k];
    sc[k] = (keep + dpp<0xB1>(send)) * sscale;  // quad_perm [1,0,3,2]
  }
  // ---- mask: tokens outside [lo, len) or in a block outside the pool ----
  const bool partial = (jb * BT < lo) || (jb * BT + BT > len) || !valid;
  // per token pair of V: zero what is not attended (slots may hold garbage)
#pragma unroll
  for (int t = 0; t < 8; t++) vm[t] = 0xffffffffu;
  if (partial) {
    const int pos = jb * BT + 4 * g + 2 * b0;
#pragma unroll
    for (int k = 0; k < 2; k++)
      if (!(valid && pos + k >= lo && pos + k < len)) sc[k] = -INFINITY;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const int p0 = jb * BT + 2 * t;
      const bool ok0 = valid && p0 >= lo && p0 < len;
      const bool ok1 = valid && p0 + 1 >= lo && p0 + 1 < len;
      vm[t] = (ok0 ? 0xffffu : 0u) | (ok1 ? 0xffff0000u : 0u);
    }
  }
  // ---- online softmax per head (the 8 lanes of a head agree on every value) ----
  float mx = fmaxf(sc[0], sc[1]);
  mx = fmaxf(mx, dpp<0xB1>(mx));
  mx = fmaxf(mx, xor16_other(mx, lane));
  mx = fmaxf(mx, xor32_other(mx, lane));
  const bool grow = mx > st.m + 8.0f;  // lazy rescale: weights stay below 2^8; true on the first finite block
  if (__any(grow)) {
    const float nm = grow ? mx : st.m;
    const float alpha = grow ? fast_exp2(st.m - nm) : 1.0f;  // 0 when st.m = -inf
    st.m = nm;
    st.l *= alpha;
#pragma unroll
    for (int h = 0; h < G2; h++) {
      const float al = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), 2 * pair_of_head(h)));
#pragma unroll
      for (int j = 0; j < 4; j++) st.o[h][j] *= al;
    }
  }
  const float mref = (st.m == -INFINITY) ? 0.0f : st.m;
  const uint32_t w = pack_16<FMT>(fast_exp2(sc[0] - mref), fast_exp2(sc[1] - mref));
  st.l = dot2_ones_16<FMT>(w, st.l);  // the normaliser sums exactly the bf16 weights that enter p . v
  return w;
}

// Second half: p . v over this lane's 4 dims for every head, head h's weights as
// scalars read from the lanes that hold them.
template <int FMT>
__device__ __forceinline__ void block_accumulate(const Vregs &vr, uint32_t w, const uint32_t (&vm)[8], State256 &st) {
  uint32_t vv[4][8];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint4 a0 = vr.v[2 * j], a1 = vr.v[2 * j + 1];
    vv[j][0] = a0.x & vm[0];
    vv[j][1] = a0.y & vm[1];
    vv[j][2] = a0.z & vm[2];
    vv[j][3] = a0.w & vm[3];
    vv[j][4] = a1.x & vm[4];
    vv[j][5] = a1.y & vm[5];
    vv[j][6] = a1.z & vm[6];
    vv[j][7] = a1.w & vm[7];
  }
#pragma unroll
  for (int h = 0; h < G2; h++) {
    uint32_t sw[8];  // pair t of head h: lane 16 (t / 2) + 2 pair_of_head(h) + t % 2
#pragma unroll
    for (int t = 0; t < 8; t++)
      sw[t] = (uint32_t)__builtin_amdgcn_readlane((int)w, 16 * (t >> 1) + 2 * pair_of_head(h) + (t & 1));
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float acc = st.o[h][j];
#pragma unroll
      for (int t = 0; t < 8; t++) acc = dot2_16<FMT>(vv[j][t], sw[t], acc);
      st.o[h][j] = acc;
    }
  }
}

// Query slot s of this lane: head s ^ fold(c), dims 8c..8c+7 and 128+8c..+7 of
// the kv head whose first query row is qrow0.
__device__ __forceinline__ void load_q256(const DecodeArgs &a, size_t qrow0, int lane, uint32_t (&qw)[G2][8]) {
  const int c = lane & 15;
#pragma unroll
  for (int s = 0; s < G2; s++) {
    const uint16_t *qr = a.q + (qrow0 + (size_t)(s ^ fold(c))) * D2 + 8 * c;
    const uint4 x = *reinterpret_cast<const uint4 *>(qr);
    const uint4 y = *reinterpret_cast<const uint4 *>(qr + 128);
    qw[s][0] = x.x, qw[s][1] = x.y, qw[s][2] = x.z, qw[s][3] = x.w;
    qw[s][4] = y.x, qw[s][5] = y.y, qw[s][6] = y.z, qw[s][7] = y.w;
  }
}

// One step of a max over the row's 16 lanes for every slot: the partner lane c ^ d
// (DPP CTRL) holds this lane's head of slot s (s ^ fold(c)) in its slot s ^ fold(d).
template <int CTRL, int FD>
__device__ __forceinline__ void row_max_step(int (&m)[G2]) {
  int t[G2];
#pragma unroll
  for (int s = 0; s < G2; s++) t[s] = __builtin_amdgcn_update_dpp(0, m[s ^ FD], CTRL, 0xF, 0xF, false);
#pragma unroll
  for (int s = 0; s < G2; s++) m[s] = max(m[s], t[s]);
}

// fp16 blocks: q of each head scaled into fp16 by its own power of two over its 256
// dims (f16_scaling).  The row reduction runs in slot order (row_max_step); slot 0
// holds head fold(c), the head this lane scores, whose step is returned: it
// multiplies this lane's scores.
__device__ __forceinline__ float prep_q256_f16(uint32_t (&qw)[G2][8]) {
  int m[G2];
#pragma unroll
  for (int s = 0; s < G2; s++) m[s] = bf16_absmax_bits<8>(qw[s]);
  row_max_step<0xB1, fold(1)>(m);   // quad_perm [1,0,3,2]: c ^ 1
  row_max_step<0x4E, fold(2)>(m);   // quad_perm [2,3,0,1]: c ^ 2
  row_max_step<0x141, fold(7)>(m);  // row_half_mirror: c ^ 7
  row_max_step<0x140, fold(15)>(m); // row_mirror: c ^ 15
#pragma unroll
  for (int s = 0; s < G2; s++) {
    const float iv = f16_scaling(m[s]).inv;
#pragma unroll
    for (int k = 0; k < 8; k++) qw[s][k] = bf16x2_to_f16x2(qw[s][k], iv);
  }
  return f16_scaling(m[0]).step;
}

__device__ __forceinline__ void reset256(State256 &st) {
  st.m = -INFINITY;
  st.l = 0.0f;
#pragma unroll
  for (int h = 0; h < G2; h++)
#pragma unroll
    for (int j = 0; j < 4; j++) st.o[h][j] = 0.0f;
}

__device__ __forceinline__ void seq_range256(const DecodeArgs &a, int b, int &len, int &lo, int &first_blk,
                                             int &n_blk, int &n_splits) {
  len = a.seq_lens[b];
  lo = a.window > 0 ? max(0, len - a.window) : 0;
  first_blk = lo / BT;
  n_blk = len > lo ? (len - 1) / BT - first_blk + 1 : 0;
  n_splits = (n_blk + a.split_blocks - 1) / a.split_blocks;
}

template <int FMT>
__global__ __launch_bounds__(kDecodeThreads, 2) void paged_decode_d256_kernel(const DecodeArgs a) {
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  int len, lo, first_blk, n_blk, n_splits;
  seq_range256(a, b, len, lo, first_blk, n_blk, n_splits);
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
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const size_t qrow0 = (size_t)b * a.q_heads + (size_t)kvh * G2;
  if (n_blk == 0) {  // empty context: zero output (weighted sum of nothing)
    for (int idx = tid; idx < G2 * D2; idx += kDecodeThreads) a.out[qrow0 * D2 + idx] = 0;
    return;
  }

  const int blk_begin = first_blk + split * a.split_blocks;
  const int blk_end = min(blk_begin + a.split_blocks, first_blk + n_blk);
  const int nbw = max(0, (blk_end - blk_begin - wave + 3) / 4);
  typedef const __attribute__((address_space(4))) int32_t table_elem_t;
  const table_elem_t *stable = (const table_elem_t *)(a.tables + (size_t)b * a.max_blocks);
  auto entry = [&](int k) __attribute__((always_inline)) -> int {
    return stable[(blk_begin + wave + 4 * k) % a.max_blocks];
  };

  uint32_t qw[G2][8];
  load_q256(a, qrow0, lane, qw);
  float sscale = a.scale_log2e;
  if constexpr (FMT == kF16) sscale *= prep_q256_f16(qw);
  State256 st;
  reset256(st);

  if (nbw > 0) {
    // K of the next block loads behind this block's p . v, V of the next block
    // behind the next block's q . k: one block's registers, always a load in flight
    int e = entry(0);
    bool valid = e >= 0 && (int64_t)e < a.pool.n_blocks;
    int phys = valid ? e : 0;
    Kregs kr;
    Vregs vr;
    load_k(a, phys, kvh, lane, kr);
    // K before V, as in the loop, so the loop's first wait (for K) leaves V in flight
    __builtin_amdgcn_sched_barrier(0);
    load_v(a, phys, kvh, lane, vr);
    // A block outside the pool is masked and flagged after the loop (a store in
    // the loop would make every wait there wait for all loads in flight), and
    // the last block is peeled off (loads under a condition made the compiler
    // copy the block registers every iteration, waiting for loads in flight).
    bool bad = false;
    int k = 0;
    for (; k + 1 < nbw; k++) {
      bad |= !valid;
      uint32_t vm[8];
      const uint32_t w = block_scores<FMT>(a, kr, valid, blk_begin + wave + 4 * k, lo, len, lane, qw, st, vm, sscale);
      e = entry(k + 1);
      valid = e >= 0 && (int64_t)e < a.pool.n_blocks;
      phys = valid ? e : 0;
      load_k(a, phys, kvh, lane, kr);
      // nothing of p . v (which waits for V) moves above the K loads
      __builtin_amdgcn_sched_barrier(0);
      block_accumulate<FMT>(vr, w, vm, st);
      load_v(a, phys, kvh, lane, vr);
    }
    bad |= !valid;
    uint32_t vm[8];
    const uint32_t w = block_scores<FMT>(a, kr, valid, blk_begin + wave + 4 * k, lo, len, lane, qw, st, vm, sscale);
    block_accumulate<FMT>(vr, w, vm, st);
    if (bad && lane == 0) atomicOr(a.err, kErrBadBlock);
  }

  // ---- wavefront totals, then merge the four wavefronts through LDS ----
  float l = st.l + dpp<0xB1>(st.l);
  l += xor16_other(l, lane);
  l += xor32_other(l, lane);
  __shared__ float s_o[4][G2][D2];
  __shared__ float s_m[4][G2];
  __shared__ float s_l[4][G2];
#pragma unroll
  for (int h = 0; h < G2; h++)
#pragma unroll
    for (int j = 0; j < 4; j++) s_o[wave][h][64 * j + lane] = st.o[h][j];
  if (lane < 16 && (lane & 1) == 0) {
    s_m[wave][fold(lane)] = st.m;
    s_l[wave][fold(lane)] = l;
  }
  __syncthreads();
  for (int idx = tid; idx < G2 * D2; idx += kDecodeThreads) {
    const int gi = idx / D2;
    const int d = idx % D2;
    const float mm = fmaxf(fmaxf(s_m[0][gi], s_m[1][gi]), fmaxf(s_m[2][gi], s_m[3][gi]));
    const float mref = (mm == -INFINITY) ? 0.0f : mm;
    float ll = 0.0f, oo = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float f = fast_exp2(s_m[w][gi] - mref);
      ll += s_l[w][gi] * f;
      oo += s_o[w][gi][d] * f;
    }
    if (n_splits == 1) {
      a.out[(qrow0 + gi) * D2 + d] = f32_to_bf16_rne(gated(oo / ll, a.gate, (qrow0 + gi) * D2 + d));
    } else {
      const size_t row = (qrow0 + gi) * a.max_splits + split;
      a.ws_o[row * D2 + d] = oo;
      if (d == 0) a.ws_ml[row] = make_float2(mm, ll);
    }
  }
}

// Merge of n <= N <= 64 split partials of one (sequence, query head): every
// partial row in flight at once, the (max, sum) pairs one per lane, reduced
// with DPP and row exchanges; split weights reach the lanes through v_readlane.
template <int N>
__device__ __forceinline__ void merge256(const DecodeArgs &a, size_t row0, int last, int d, size_t orow) {
  float o_sp[N];
#pragma unroll
  for (int i = 0; i < N; i++) o_sp[i] = a.ws_o[(row0 + min(i, last)) * D2 + d];
  const int li = d & 63;
  const float2 ml = a.ws_ml[row0 + min(li, last)];
  const float mx = li <= last ? ml.x : -INFINITY;
  float mm = fmaxf(mx, dpp<0xB1>(mx));
  mm = fmaxf(mm, dpp<0x4E>(mm));
  mm = fmaxf(mm, dpp<0x141>(mm));
  mm = fmaxf(mm, dpp<0x140>(mm));
  mm = fmaxf(mm, xor16_other(mm, li));
  mm = fmaxf(mm, xor32_other(mm, li));
  const float mref = (mm == -INFINITY) ? 0.0f : mm;
  const float f = li <= last ? fast_exp2(mx - mref) : 0.0f;
  float ll = f * ml.y;
  ll = row_sum16(ll);
  ll += xor16_other(ll, li);
  ll += xor32_other(ll, li);
  float oo = 0.0f;
#pragma unroll
  for (int i = 0; i < N; i++) oo += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), i)) * o_sp[i];
  a.out[orow * D2 + d] = f32_to_bf16_rne(gated(oo / ll, a.gate, orow * D2 + d));
}

__global__ __launch_bounds__(D2) void decode_merge_d256_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  int len, lo, first_blk, n_blk, n_splits;
  seq_range256(a, b, len, lo, first_blk, n_blk, n_splits);
  if (n_splits <= 1 || n_splits > a.max_splits || n_splits > kMerge256MaxSplits || len - lo > a.max_blocks * BT)
    return;
  const int d = threadIdx.x;
  const size_t row0 = ((size_t)b * a.q_heads + h) * a.max_splits;
  const size_t orow = (size_t)b * a.q_heads + h;
  const int last = n_splits - 1;
  if (n_splits <= 8) return merge256<8>(a, row0, last, d, orow);
  if (n_splits <= 16) return merge256<16>(a, row0, last, d, orow);
  if (n_splits <= 32) return merge256<32>(a, row0, last, d, orow);
  return merge256<64>(a, row0, last, d, orow);
}

// ---------------------------------------------------------------------------
// Persistent stream form.  Wavefront w of the grid takes units [r0, r0 + n) of
// the step (stream_partition.h) and walks them with the split-K kernel's
// register pipeline (one block's registers, the next block's K loading behind
// this block's p . v and its V behind the next q . k).  A segment (sequence, kv
// head) that ends inside the range is flushed by this wavefront alone (no LDS,
// no barrier): its bf16 output when the segment also began inside the range,
// else a (max, sum, output) partial in slot 2w (the wavefront's first segment)
// or 2w + 1 (its last), and the wavefront that holds the segment's first unit
// records (first slot, pieces) in seg_desc for decode_stream_merge_d256_kernel.
// ---------------------------------------------------------------------------

// Ends a segment: head h's (max, sum) from the lanes that score it (their
// 8-lane sum for the sum), the outputs as every lane holds them (dims 64j + lane).
__device__ __forceinline__ void flush256(const DecodeArgs &a, State256 &st, int b, int kvh, bool complete, int slot,
                                         int lane) {
  float l = st.l + dpp<0xB1>(st.l);
  l += xor16_other(l, lane);
  l += xor32_other(l, lane);
  const size_t qrow0 = (size_t)b * a.q_heads + (size_t)kvh * G2;
#pragma unroll
  for (int h = 0; h < G2; h++) {
    const int src = 2 * pair_of_head(h);
    const float mh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(st.m), src));
    const float lh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), src));
    if (complete) {
      const float inv = 1.0f / lh;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const size_t o = (qrow0 + h) * D2 + 64 * j + lane;
        a.out[o] = f32_to_bf16_rne(gated(st.o[h][j] * inv, a.gate, o));
      }
    } else {
      const size_t row = (size_t)slot * G2 + h;
#pragma unroll
      for (int j = 0; j < 4; j++) a.ws_o[row * D2 + 64 * j + lane] = st.o[h][j];
      if (lane == 0) a.ws_ml[row] = make_float2(mh, lh);
    }
  }
  reset256(st);
}

// ---- fused append (llh_paged_decode_append, bf16 pools) ----
// kir-ai appends the new token, then attends (native_attention.rs:307-329).  Here the
// wavefront that computes the block receiving the token (its segment's last unit) puts
// the token's bf16 bits into the registers it loaded that block into and stores them to
// the token's slot -- a slot no other wavefront reads during the launch -- so the step
// attends exactly what the append kernel would have stored.  A block entry outside the
// pool is flagged (as the append kernel flags it) and nothing is written.

// The new token's K at this lane's dims (8c .., 128 + 8c ..) and V at dims 64j + lane
// (two per word), for sequence b, kv head kvh.
__device__ __forceinline__ void load_new_k(const DecodeArgs &a, int b, int kvh, int lane, uint4 (&nk)[2]) {
  const uint16_t *kn = a.k_new + ((size_t)b * a.pool.kv_heads + kvh) * D2 + 8 * (lane & 15);
  nk[0] = *reinterpret_cast<const uint4 *>(kn);
  nk[1] = *reinterpret_cast<const uint4 *>(kn + 128);
}
__device__ __forceinline__ void load_new_v(const DecodeArgs &a, int b, int kvh, int lane, uint32_t (&nv)[2]) {
  const uint16_t *vn = a.v_new + ((size_t)b * a.pool.kv_heads + kvh) * D2 + lane;
  nv[0] = (uint32_t)vn[0] | ((uint32_t)vn[64] << 16);
  nv[1] = (uint32_t)vn[128] | ((uint32_t)vn[192] << 16);
}
// Token off of the block in kr / vr replaced by the new token (lanes of row off / 4 hold
// its K as kr.k[2 (off % 4)], kr.k[2 (off % 4) + 1]; element off % 8 of vr.v[2j + off / 8]).
// (Selects on every register, so the arrays stay in registers: an index that is not a
// compile-time constant would put them in scratch.)
__device__ __forceinline__ uint4 sel4(bool c, const uint4 &a, const uint4 &b) {
  return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}
__device__ __forceinline__ void patch_new_k(Kregs &kr, const uint4 (&nk)[2], int off, int lane) {
  const bool row = (lane >> 4) == (off >> 2);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const bool hit = row && i == (off & 3);
    kr.k[2 * i] = sel4(hit, nk[0], kr.k[2 * i]);
    kr.k[2 * i + 1] = sel4(hit, nk[1], kr.k[2 * i + 1]);
  }
}
__device__ __forceinline__ void patch_new_v(Vregs &vr, const uint32_t (&nv)[2], int off) {
  const int word = (off & 7) >> 1, sh = 16 * (off & 1);
  const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t x = ((nv[j >> 1] >> (16 * (j & 1))) & 0xffffu) << sh;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const bool h = hh == (off >> 3);
      uint4 &r = vr.v[2 * j + hh];
      r.x = (h && word == 0) ? ((r.x & keep) | x) : r.x;
      r.y = (h && word == 1) ? ((r.y & keep) | x) : r.y;
      r.z = (h && word == 2) ? ((r.z & keep) | x) : r.z;
      r.w = (h && word == 3) ? ((r.w & keep) | x) : r.w;
    }
  }
}
// fp16 pools: the new token's bf16 words as the append kernel stores them (each
// element widened exactly, then rounded to nearest even), converted at the patch,
// where the rows are first used.
__device__ __forceinline__ uint32_t bf16x2_as_f16x2(uint32_t w) { return pack_f16(bf16_lo(w), bf16_hi(w)); }
template <int FMT>
__device__ __forceinline__ void new_k_words(uint4 (&nk)[2]) {
  if constexpr (FMT == kF16)
#pragma unroll
    for (int i = 0; i < 2; i++)
      nk[i] = make_uint4(bf16x2_as_f16x2(nk[i].x), bf16x2_as_f16x2(nk[i].y), bf16x2_as_f16x2(nk[i].z),
                         bf16x2_as_f16x2(nk[i].w));
}
template <int FMT>
__device__ __forceinline__ void new_v_words(uint32_t (&nv)[2]) {
  if constexpr (FMT == kF16)
#pragma unroll
    for (int i = 0; i < 2; i++) nv[i] = bf16x2_as_f16x2(nv[i]);
}

// The new token into its pool slot (block phys, kv head kvh, offset off), from the
// registers the patch used: K from the 16 lanes of row 0 (each holds dims 8c .. and
// 128 + 8c ..), V from every lane (dims 64j + lane).  Written by the wavefront that
// computes the block, at the patch, so no other wavefront waits on it.
__device__ __forceinline__ void store_new_k(const DecodeArgs &a, int phys, int kvh, int off, const uint4 (&nk)[2],
                                            int lane) {
  if (lane >= 16) return;
  char *kb = const_cast<char *>(block_base(a.pool.k, phys, kvh, a.pool.kv_heads)) + off * (D2 * 2) + 16 * lane;
  *reinterpret_cast<uint4 *>(kb) = nk[0];
  *reinterpret_cast<uint4 *>(kb + 256) = nk[1];
}
__device__ __forceinline__ void store_new_v(const DecodeArgs &a, int phys, int kvh, int off, const uint32_t (&nv)[2],
                                            int lane) {
  uint16_t *vb = reinterpret_cast<uint16_t *>(const_cast<char *>(block_base(a.pool.v, phys, kvh, a.pool.kv_heads)));
#pragma unroll
  for (int j = 0; j < 4; j++) vb[(64 * j + lane) * BT + off] = (uint16_t)(nv[j >> 1] >> (16 * (j & 1)));
}

template <int FMT, bool FUSED>
__global__ __launch_bounds__(kDecodeThreads, 2) void paged_decode_d256_stream_kernel(const DecodeArgs a) {
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
  for (int b = w; b < B; b += W) {
    if (attended_blocks(a, b < 64 ? __builtin_amdgcn_readlane(len0, b) : a.seq_lens[b]) == 0) {
      for (int idx = lane; idx < a.q_heads * D2; idx += 64) a.out[(size_t)b * a.q_heads * D2 + idx] = 0;
      for (int idx = lane; idx < 2 * Hkv; idx += 64) a.seg_desc[(size_t)b * Hkv * 2 + idx] = 0;
    }
  }
  const int n = __builtin_amdgcn_readfirstlane(sr.n);
  if (n == 0) return;
  const int U = __builtin_amdgcn_readfirstlane(sr.U);
  const int Wu = __builtin_amdgcn_readfirstlane(sr.Wu);
  const stream_const_i32 *stable = (const stream_const_i32 *)a.tables;
  // cursors: the next block-table entry to fetch (one unit ahead of the loads),
  // the next unit to load, the unit being computed
  UnitCursor C = cursor_at(a, len0, sr);
  UnitCursor L = C, E = C;
  auto next_entry = [&]() __attribute__((always_inline)) -> int {
    const int e = stable[(size_t)E.b * a.max_blocks + E.tab];
    cursor_advance(a, len0, E);
    return e;
  };
  uint32_t qw[G2][8];
  load_q256(a, (size_t)C.b * a.q_heads + (size_t)C.kvh * G2, lane, qw);
  float sscale = a.scale_log2e;
  bool q_new = true;  // fp16: qw holds a segment's bf16 q not yet scaled
  int e = next_entry();
  bool valid = e >= 0 && (int64_t)e < a.pool.n_blocks;
  Kregs kr;
  Vregs vr;
  uint4 nk[2];      // fused: the new token's rows for the unit in kr / vr when it is its segment's last
  uint32_t nv[2];
  load_k(a, valid ? e : 0, L.kvh, lane, kr);
  if constexpr (FUSED)
    if (L.j == L.nb - 1) load_new_k(a, L.b, L.kvh, lane, nk);
  __builtin_amdgcn_sched_barrier(0);  // K before V, as in the loop
  load_v(a, valid ? e : 0, L.kvh, lane, vr);
  if constexpr (FUSED)
    if (L.j == L.nb - 1) load_new_v(a, L.b, L.kvh, lane, nv);
  cursor_advance(a, len0, L);
  int e_next = n > 1 ? next_entry() : -1;
  int cphys = valid ? e : 0;  // the block of unit C

  State256 st;
  reset256(st);
  bool seg_from_start = C.j == 0;
  bool first_seg = true;
  auto end_segment = [&](bool complete) __attribute__((always_inline)) {
    const int slot = w * 2 + (first_seg ? 0 : 1);
    flush256(a, st, C.b, C.kvh, complete, slot, lane);
    if (lane == 0 && (complete || seg_from_start)) {
      // this wavefront holds the segment's first unit: record how to merge it
      int2 d = make_int2(0, 0);
      if (!complete) d = make_int2(slot, wave_of_unit(C.base + (C.kvh + 1) * C.nb - 1, U, Wu) - w + 1);
      reinterpret_cast<int2 *>(a.seg_desc)[(size_t)C.b * Hkv + C.kvh] = d;
    }
    first_seg = false;
  };

  // Units 0 .. n-2 issue the next unit's loads; the last is peeled off (loads
  // under a condition would make the compiler wait for every load in flight).
  // A segment's last unit loads the next segment's q (its registers are free
  // after the scores) before the next unit's V, so the next scores wait for K
  // and q only; an entry outside the pool is masked and flagged after the loop.
  bool bad = false;
  for (int k = 0; k + 1 < n; k++) {
    bad |= !valid;
    uint32_t vm[8];
    const bool seg_end = C.j == C.nb - 1;  // then unit L starts the next segment
    const bool cvalid = valid;
    if constexpr (FUSED)
      if (seg_end) {
        new_k_words<FMT>(nk);
        patch_new_k(kr, nk, (C.len - 1) % BT, lane);
        if (cvalid) store_new_k(a, cphys, C.kvh, (C.len - 1) % BT, nk, lane);
      }
    if constexpr (FMT == kF16)
      if (q_new) {
        sscale = a.scale_log2e * prep_q256_f16(qw);
        q_new = false;
      }
    const uint32_t wp = block_scores<FMT>(a, kr, valid, C.lo / BT + C.j, C.lo, C.len, lane, qw, st, vm, sscale);
    valid = e_next >= 0 && (int64_t)e_next < a.pool.n_blocks;
    const int phys = valid ? e_next : 0;
    load_k(a, phys, L.kvh, lane, kr);
    if constexpr (FUSED)
      if (L.j == L.nb - 1) load_new_k(a, L.b, L.kvh, lane, nk);
    if (seg_end) {
      load_q256(a, (size_t)L.b * a.q_heads + (size_t)L.kvh * G2, lane, qw);
      q_new = true;
    }
    // nothing of p . v (which waits for V) moves above the K loads
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FUSED)
      if (seg_end) {
        new_v_words<FMT>(nv);
        patch_new_v(vr, nv, (C.len - 1) % BT);
        if (cvalid) store_new_v(a, cphys, C.kvh, (C.len - 1) % BT, nv, lane);
      }
    block_accumulate<FMT>(vr, wp, vm, st);
    if (seg_end) {
      end_segment(seg_from_start);
      seg_from_start = true;
    }
    load_v(a, phys, L.kvh, lane, vr);
    if constexpr (FUSED)
      if (L.j == L.nb - 1) load_new_v(a, L.b, L.kvh, lane, nv);
    cursor_advance(a, len0, L);
    e_next = k + 2 < n ? next_entry() : -1;
    cursor_advance(a, len0, C);
    cphys = phys;
  }
  bad |= !valid;
  {
    uint32_t vm[8];
    if constexpr (FUSED)
      if (C.j == C.nb - 1) {
        new_k_words<FMT>(nk);
        patch_new_k(kr, nk, (C.len - 1) % BT, lane);
        if (valid) store_new_k(a, cphys, C.kvh, (C.len - 1) % BT, nk, lane);
      }
    if constexpr (FMT == kF16)
      if (q_new) {
        sscale = a.scale_log2e * prep_q256_f16(qw);
        q_new = false;
      }
    const uint32_t wp = block_scores<FMT>(a, kr, valid, C.lo / BT + C.j, C.lo, C.len, lane, qw, st, vm, sscale);
    if constexpr (FUSED)
      if (C.j == C.nb - 1) {
        new_v_words<FMT>(nv);
        patch_new_v(vr, nv, (C.len - 1) % BT);
        if (valid) store_new_v(a, cphys, C.kvh, (C.len - 1) % BT, nv, lane);
      }
    block_accumulate<FMT>(vr, wp, vm, st);
  }
  // the range ends with the segment (complete if it also began here) or inside it
  end_segment(C.j == C.nb - 1 && seg_from_start);
  if (bad && lane == 0) atomicOr(a.err, kErrBadBlock);
}

// One round of the stream merge over pieces i0 .. i0+cnt-1 (1 <= cnt <= N) of a
// cut segment, one dim per thread: every partial of the round is loaded before
// any is used (pieces past the last re-read it and get weight 0), lane j of each
// wavefront loads piece j's (max, sum), and the weights reach all lanes by
// readlane -- two dependent memory round trips (descriptor, then partials).
template <int N>
__device__ __forceinline__ void stream_merge256_round(const DecodeArgs &a, int first_slot, int wf, int gi, int i0,
                                                      int cnt, int d, float &mm, float &ll, float &oo) {
  static_assert(N == 16 || N == 32, "one or two DPP rows of pieces");
  const int lane = d & 63;
  // piece k of the segment: the first wavefront's slot, then the later wavefronts' first-segment slots
  auto row_of = [&](int k) { return (size_t)(k == 0 ? first_slot : (wf + k) * 2) * G2 + gi; };
  const float2 ml = a.ws_ml[row_of(i0 + min(lane, cnt - 1))];
  float ov[N];
#pragma unroll
  for (int i = 0; i < N; i++) ov[i] = a.ws_o[row_of(i0 + min(i, cnt - 1)) * D2 + d];
  __builtin_amdgcn_sched_barrier(0);
  const float m = lane < cnt ? ml.x : -INFINITY;
  float nm = m;
  nm = fmaxf(nm, dpp<0xB1>(nm));   // quad_perm [1,0,3,2]
  nm = fmaxf(nm, dpp<0x4E>(nm));   // quad_perm [2,3,0,1]
  nm = fmaxf(nm, dpp<0x141>(nm));  // row_half_mirror
  nm = fmaxf(nm, dpp<0x140>(nm));  // row_mirror
  if constexpr (N == 32) nm = fmaxf(nm, xor16_other(nm, lane));
  nm = fmaxf(__int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(nm))), mm);
  const float mref = (nm == -INFINITY) ? 0.0f : nm;
  const float f = fast_exp2(m - mref);  // 0 on lanes past the last piece
  float ls = row_sum16(ml.y * f);
  if constexpr (N == 32) ls += xor16_other(ls, lane);
  const float f0 = fast_exp2(mm - mref);
  ll = ll * f0 + __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ls)));
  oo *= f0;
#pragma unroll
  for (int i = 0; i < N; i++) oo += ov[i] * __int_as_float(__builtin_amdgcn_readlane(__float_as_int(f), i));
  mm = nm;
}

// Merges the stream kernel's cut segments: one workgroup of 256 threads (one per
// dim) per (query head, sequence); up to 16 pieces in one round, more in rounds
// of 32.
__global__ __launch_bounds__(D2) void decode_stream_merge_d256_kernel(const DecodeArgs a) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int kvh = h / G2;
  const int gi = h - kvh * G2;
  const int2 sd = reinterpret_cast<const int2 *>(a.seg_desc)[(size_t)b * a.pool.kv_heads + kvh];
  const int W = a.stream_wgs * 4;
  const int wf = sd.x >> 1;
  // written by the stream kernel; a call it aborted (error flags) may leave any
  // values, so only descriptors naming slots of this grid are followed
  if (sd.y < 2 || sd.x < 0 || sd.x >= 2 * W || wf + sd.y > W) return;
  float mm = -INFINITY, ll = 0.0f, oo = 0.0f;
  if (sd.y <= 16) {
    stream_merge256_round<16>(a, sd.x, wf, gi, 0, sd.y, d, mm, ll, oo);
  } else {
#pragma unroll 1
    for (int i0 = 0; i0 < sd.y; i0 += 32) stream_merge256_round<32>(a, sd.x, wf, gi, i0, min(32, sd.y - i0), d, mm, ll, oo);
  }
  const size_t o = ((size_t)b * a.q_heads + h) * D2 + d;
  a.out[o] = f32_to_bf16_rne(gated(oo / ll, a.gate, o));
}

}  // namespace

hipError_t launch_decode_d256(const DecodeArgs &a, int max_seq_len, hipStream_t s, void *hu, LaunchHook hook) {
  if (a.stream_wgs > 0) {
    if (hook) hook(hu, 0, s);
    if (a.pool.format == kF16 && a.k_new)
      hipLaunchKernelGGL((paged_decode_d256_stream_kernel<kF16, true>), dim3(a.stream_wgs), dim3(kDecodeThreads), 0,
                         s, a);
    else if (a.pool.format == kF16)
      hipLaunchKernelGGL((paged_decode_d256_stream_kernel<kF16, false>), dim3(a.stream_wgs), dim3(kDecodeThreads), 0,
                         s, a);
    else if (a.k_new)
      hipLaunchKernelGGL((paged_decode_d256_stream_kernel<kBf16, true>), dim3(a.stream_wgs), dim3(kDecodeThreads), 0,
                         s, a);
    else
      hipLaunchKernelGGL((paged_decode_d256_stream_kernel<kBf16, false>), dim3(a.stream_wgs), dim3(kDecodeThreads), 0,
                         s, a);
    hipError_t e = hipGetLastError();
    if (hook) hook(hu, 1, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(decode_stream_merge_d256_kernel, dim3(a.q_heads, a.num_seqs), dim3(D2), 0, s, a);
    return hipGetLastError();
  }
  if (a.max_splits > kMerge256MaxSplits) return hipErrorInvalidValue;
  const int max_blk = (max_seq_len + BT - 1) / BT + 1;
  const int grid_x = max(1, (max_blk + a.split_blocks - 1) / a.split_blocks);
  if (hook) hook(hu, 0, s);
  dim3 grid(min(grid_x, a.max_splits), a.pool.kv_heads, a.num_seqs);
  if (a.pool.format == kF16)
    hipLaunchKernelGGL(paged_decode_d256_kernel<kF16>, grid, dim3(kDecodeThreads), 0, s, a);
  else
    hipLaunchKernelGGL(paged_decode_d256_kernel<kBf16>, grid, dim3(kDecodeThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (hook) hook(hu, 1, s);
  if (e != hipSuccess || a.max_splits <= 1) return e;
  hipLaunchKernelGGL(decode_merge_d256_kernel, dim3(a.q_heads, a.num_seqs), dim3(D2), 0, s, a);
  return hipGetLastError();
}

}  // namespace llh
