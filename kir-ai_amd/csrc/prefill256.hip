// Chunked causal prefill at head_dim 256 on gfx950 MFMA: the Qwen3.5 / 3.6
// full-attention layers (fixtures/qwen36/config.json: head_dim 256), bf16 pools
// of 16-token blocks.  Same contract as paged_prefill_kernel (prefill.hip):
// query row i of a chunk sits at pos = context_len - chunk_len + i and attends
// [lo(pos), pos] (crates/llm-backend/src/core/native_attention.rs:356-464),
// times sigmoid(gate) when the call carries one (native_attention.rs:765-781).
//
// Same dataflow as the head_dim-128 kernel -- S^T = K Q^T and O^T += V^T P^T on
// v_mfma_f32_32x32x16_bf16, P^T taken straight from the S^T accumulators, V^T
// read from the dim-major pool layout, K/V tiles of 64 keys double-buffered in
// LDS, online softmax in log2 units with a lazy rescale -- at twice the row
// width: a wavefront holds its 32 query rows' Q^T (16 k-steps, 64 registers)
// and O^T (8 blocks of 32 dims, 128 accumulators), a tile is 64 MFMAs per
// wavefront, two tile buffers take 146 KB of LDS.  One query head per
// workgroup of 4 wavefronts, one workgroup per CU (one wavefront per SIMD, up
// to 512 registers each): the per-wavefront state of head_dim 256 does not fit
// the 256 registers two wavefronts per SIMD would leave.
#include "device_common.h"

namespace llh {

namespace {

constexpr int D = kD256HeadDim;
constexpr int BT = kFastBlockTokens;
constexpr int BM = 128;          // query rows per workgroup
constexpr int BN = 64;           // key positions per tile
constexpr int KBLK = BN / BT;    // pool blocks per tile
constexpr int K_STRIDE = D + 8;  // bf16 elements per K row in LDS (528 B)
constexpr int V_STRIDE = BT + 4; // bf16 elements per V^T row in LDS (40 B)
constexpr int K_TILE = BN * K_STRIDE;
constexpr int V_TILE = KBLK * D * V_STRIDE;
constexpr int kThreads = 256;

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)a, (__bf16)b});  // round to nearest even
}

__device__ __forceinline__ f32x16_t mfma32(const u32x4_t &a, const u32x4_t &b, const f32x16_t &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                  0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Value of lane (l ^ 32) (v_permlane32_swap: no LDS round trip).
__device__ __forceinline__ float xor32_other(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ float dot2_ones(uint32_t pair, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pair),
                                         __builtin_bit_cast(bf16x2_t, 0x3F803F80u), acc, false);
}

// One thread's share of a tile: for each of the 4 blocks, K of token tid/16
// at dims 8(tid%16).. and 128 + 8(tid%16).., and V^T of dims tid/2 and
// 128 + tid/2 at tokens 8(tid&1).. (16 bytes each).
struct Tile256 {
  u32x4_t k[KBLK][2];
  u32x4_t v[KBLK][2];
};

// Block-table entries of the tile starting at kt: lane kb holds block kb's
// entry (lanes repeat mod KBLK); an in-bounds table read, one tile ahead.
__device__ __forceinline__ int fetch_entries(const PrefillArgs &a, const int32_t *table, int kt, int lane) {
  return table[(kt / BT + (lane & (KBLK - 1))) % a.max_blocks];
}

// Issues the tile's loads, all unconditional (an unneeded block or one outside
// the pool reads block 0 and is zeroed when stored); returns the mask of
// blocks to use.  `bad` collects needed blocks with an out-of-pool entry.
__device__ __forceinline__ uint32_t load_tile(const PrefillArgs &a, int entries, int kvh, int kt, int ctx, int klo,
                                              int tid, Tile256 &r, bool &bad) {
  uint32_t use_mask = 0;
#pragma unroll
  for (int kb = 0; kb < KBLK; kb++) {
    const int bpos = kt + kb * BT;
    const bool needed = bpos < ctx && bpos + BT > klo;
    const int phys = __builtin_amdgcn_readlane(entries, kb);
    const bool ok = phys >= 0 && (int64_t)phys < a.pool.n_blocks;
    bad |= needed && !ok;
    const bool use = needed && ok;
    use_mask |= use ? (1u << kb) : 0u;
    const size_t base = ((size_t)(use ? phys : 0) * a.pool.kv_heads + kvh) * (BT * D);
    const uint16_t *kp = reinterpret_cast<const uint16_t *>(a.pool.k) + base + (tid >> 4) * D + (tid & 15) * 8;
    const uint16_t *vp = reinterpret_cast<const uint16_t *>(a.pool.v) + base + (tid >> 1) * BT + (tid & 1) * 8;
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      r.k[kb][hf] = *reinterpret_cast<const u32x4_t *>(kp + hf * 128);
      r.v[kb][hf] = *reinterpret_cast<const u32x4_t *>(vp + hf * 128 * BT);
    }
  }
  return use_mask;
}

// Stores a tile to LDS: K rows as loaded (unattended keys are masked in the
// scores), V^T zeroed for unused blocks and tokens at or past the context end
// (P = 0 times a non-finite V would poison the accumulators).
__device__ __forceinline__ void store_tile(uint16_t *k_lds, uint16_t *v_lds, int tid, const Tile256 &r,
                                           uint32_t use_mask, int kt, int ctx) {
  const bool tail = kt + BN > ctx;
#pragma unroll
  for (int kb = 0; kb < KBLK; kb++) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      *reinterpret_cast<u32x4_t *>(&k_lds[(kb * BT + (tid >> 4)) * K_STRIDE + hf * 128 + (tid & 15) * 8]) =
          r.k[kb][hf];
      u32x4_t v = r.v[kb][hf];
      if (!(use_mask & (1u << kb))) v = u32x4_t{0u, 0u, 0u, 0u};
      if (tail) {
        const int valid = ctx - (kt + kb * BT + (tid & 1) * 8);  // tokens of this 8-run inside the context
        v[0] &= (valid > 0 ? 0x0000ffffu : 0u) | (valid > 1 ? 0xffff0000u : 0u);
        v[1] &= (valid > 2 ? 0x0000ffffu : 0u) | (valid > 3 ? 0xffff0000u : 0u);
        v[2] &= (valid > 4 ? 0x0000ffffu : 0u) | (valid > 5 ? 0xffff0000u : 0u);
        v[3] &= (valid > 6 ? 0x0000ffffu : 0u) | (valid > 7 ? 0xffff0000u : 0u);
      }
      uint16_t *dst = &v_lds[(kb * D + hf * 128 + (tid >> 1)) * V_STRIDE + (tid & 1) * 8];
      *reinterpret_cast<uint2 *>(dst) = make_uint2(v[0], v[1]);
      *reinterpret_cast<uint2 *>(dst + 4) = make_uint2(v[2], v[3]);
    }
  }
}

__global__ __launch_bounds__(kThreads, 1) void paged_prefill_d256_kernel(const PrefillArgs a) {
  // ---- XCD-aware logical work item (as the head_dim-128 kernel) ----
  const int Hq = a.q_heads;
  const int Hkv = a.pool.kv_heads;
  const int GW = Hq / Hkv;  // workgroups per (kv head, query tile): one per query head
  const int n_items = a.q_tiles * Hkv * GW * a.num_seqs;
  const int per_xcd = (n_items + 7) / 8;
  const int per_group = a.q_tiles * GW;
  const int di = blockIdx.x / 8;
  int local = di;
  if (per_xcd % per_group == 0) {
    const int groups = per_xcd / per_group;
    local = ((di / GW) % groups) * per_group + (a.q_tiles - 1 - di / (groups * GW)) * GW + di % GW;
  }
  const int w = (blockIdx.x % 8) * per_xcd + local;
  if (w >= n_items) return;
  const int tile = (w / GW) % a.q_tiles;
  const int kvh = (w / (GW * a.q_tiles)) % Hkv;
  const int b = w / (GW * a.q_tiles * Hkv);
  const int qh = kvh * GW + w % GW;

  const int c0 = a.chunk_starts[b];
  const int chunk = a.chunk_starts[b + 1] - c0;
  const int ctx = a.context_lens[b];
  const int i0 = tile * BM;
  if (i0 >= chunk || chunk <= 0 || ctx < chunk) return;
  {
    // every key of the chunk's first row through the last must be resident at once
    const int first_lo = a.window > 0 ? max(0, ctx - chunk - a.window + 1) : 0;
    if (ctx - first_lo > a.max_blocks * BT) {
      if (threadIdx.x == 0 && tile == 0) atomicOr(a.err, kErrSpan);
      return;
    }
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const int col = lane & 31;
  const int prefix = ctx - chunk;
  const int rows_wg = min(BM, chunk - i0);
  const int qpos_first = prefix + i0;
  const int qpos_last = prefix + i0 + rows_wg - 1;
  const int my_row = i0 + wave * 32 + col;
  const bool row_ok = my_row < chunk;
  const int my_pos = prefix + my_row;
  const int my_lo = a.window > 0 ? max(0, my_pos - a.window + 1) : 0;

  // ---- Q^T operand: 16 k-steps of 16 dims; lane holds dims 16ks + 8h .. +8 of its row ----
  u32x4_t qb[16];
  {
    const uint16_t *qrow = a.q + ((size_t)(c0 + (row_ok ? my_row : 0)) * Hq + qh) * D;
#pragma unroll
    for (int ks = 0; ks < 16; ks++) {
      u32x4_t t = *reinterpret_cast<const u32x4_t *>(qrow + ks * 16 + h * 8);
      if (!row_ok) t = u32x4_t{0u, 0u, 0u, 0u};
      qb[ks] = t;
    }
  }

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][K_TILE];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][V_TILE];

  f32x16_t oacc[8];
#pragma unroll
  for (int mt = 0; mt < 8; mt++)
#pragma unroll
    for (int j = 0; j < 16; j++) oacc[mt][j] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const int klo = a.window > 0 ? max(0, qpos_first - a.window + 1) : 0;
  const int khi = qpos_last + 1;  // exclusive
  const int t_begin = (klo / BN) * BN;
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  const int wrow0 = i0 + wave * 32;
  const int wpos_first = prefix + wrow0;
  const int wpos_last = prefix + min(wrow0 + 31, chunk - 1);
  const int wlo_first = a.window > 0 ? max(0, wpos_first - a.window + 1) : 0;
  const int wlo_last = a.window > 0 ? max(0, wpos_last - a.window + 1) : 0;
  const bool wave_live = wrow0 < chunk;

  Tile256 next;
  bool bad = false;
  uint32_t use_next = load_tile(a, fetch_entries(a, table, t_begin, lane), kvh, t_begin, ctx, klo, tid, next, bad);
  int ent_next = fetch_entries(a, table, t_begin + BN, lane);
  store_tile(k_lds[0], v_lds[0], tid, next, use_next, t_begin, ctx);
  __syncthreads();

  // The O^T accumulators live in AGPRs, where only the MFMAs touch them: the rare
  // rescale (a row's max grew by more than 16 in log2 units) leaves the tile loop,
  // multiplies them, and re-enters at the same tile, reissuing its loads and
  // recomputing its scores.  (A rescale inside the loop made the compiler copy
  // all 128 accumulators out of and back into AGPRs on every tile.)
  int buf = 0;
  int kt = t_begin;
  for (;;) {
  bool rescale = false;
  float m_next = m_run;  // this lane's new running max when leaving to rescale
  for (; kt < khi; kt += BN, buf ^= 1) {
    const bool has_next = kt + BN < khi;
    if (has_next)  // in flight during the math
      use_next = load_tile(a, ent_next, kvh, kt + BN, ctx, klo, tid, next, bad);
    ent_next = fetch_entries(a, table, kt + 2 * BN, lane);

    if (wave_live && kt <= wpos_last && kt + BN > wlo_first) {
      const uint16_t *kl = k_lds[buf];
      const uint16_t *vl = v_lds[buf];
      // ---- S^T = K Q^T for two 32-key sub-tiles (their chains interleaved) ----
      f32x16_t sacc[2];
#pragma unroll
      for (int st = 0; st < 2; st++)
#pragma unroll
        for (int j = 0; j < 16; j++) sacc[st][j] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 16; ks++)
#pragma unroll
        for (int st = 0; st < 2; st++) {
          const u32x4_t ka = *reinterpret_cast<const u32x4_t *>(&kl[(st * 32 + col) * K_STRIDE + ks * 16 + h * 8]);
          sacc[st] = mfma32(ka, qb[ks], sacc[st]);
        }

      // ---- scale, mask, online softmax (as the head_dim-128 kernel) ----
      const bool need_mask = (kt + BN - 1 > wpos_first) || (kt < wlo_last) || (kt + BN > ctx);
      const float c = a.scale_log2e;
      float c_exp = c;
      float tmax = -INFINITY;
      if (need_mask) {
#pragma unroll
        for (int st = 0; st < 2; st++) {
#pragma unroll
          for (int j = 0; j < 16; j++) {
            float s = sacc[st][j] * c;
            const int kp = kt + st * 32 + 8 * (j >> 2) + 4 * h + (j & 3);
            if (kp > my_pos || kp < my_lo || kp >= ctx || !row_ok) s = -INFINITY;
            sacc[st][j] = s;
            tmax = fmaxf(tmax, s);
          }
        }
        c_exp = 1.0f;
      } else if (c >= 0.0f) {
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
          for (int j = 0; j < 16; j++) tmax = fmaxf(tmax, sacc[st][j]);
        tmax *= c;
      } else {
        float tmin = INFINITY;
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
          for (int j = 0; j < 16; j++) tmin = fminf(tmin, sacc[st][j]);
        tmax = tmin * c;
      }
      // Raw scores beyond 2^26 (log2 units) once scaled: tmax, a rounded product, can
      // fall below the fma's exact product c * s by more than the weights' headroom
      // (|error| <= |tmax| 2^-24), so those tiles scale first, as masked tiles do:
      // every score rounds as tmax did and the largest weight is exactly 1.
      if (!need_mask && __any(fabsf(tmax) > 0x1p26f)) {
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
          for (int j = 0; j < 16; j++) sacc[st][j] *= c;
        c_exp = 1.0f;
      }
      tmax = fmaxf(tmax, xor32_other(tmax));
      const float m_cand = fmaxf(m_run, tmax);
      // a row without a finite score yet takes the tile's max (its accumulators are
      // still zero); a row whose max grows by more than 16 needs a rescale first
      const bool grow = m_run != -INFINITY && m_cand > m_run + 16.0f;
      if (__any(grow)) {
        m_next = grow ? m_cand : m_run;
        rescale = true;
        break;
      }
      if (m_run == -INFINITY) m_run = m_cand;
      const float mref = (m_run == -INFINITY) ? 0.0f : m_run;
      u32x4_t pb[4];
#pragma unroll
      for (int st = 0; st < 2; st++) {
        float p[16];
#pragma unroll
        for (int j = 0; j < 16; j++) p[j] = fast_exp2(__builtin_fmaf(sacc[st][j], c_exp, -mref));
#pragma unroll
        for (int q = 0; q < 2; q++)
          pb[2 * st + q] = u32x4_t{pack_bf16(p[8 * q + 0], p[8 * q + 1]), pack_bf16(p[8 * q + 2], p[8 * q + 3]),
                                   pack_bf16(p[8 * q + 4], p[8 * q + 5]), pack_bf16(p[8 * q + 6], p[8 * q + 7])};
      }
      float psum = 0.0f;  // row sums of exactly the bf16 weights that enter P V
#pragma unroll
      for (int kb = 0; kb < KBLK; kb++)
#pragma unroll
        for (int e = 0; e < 4; e++) psum = dot2_ones(pb[kb][e], psum);
      l_run += psum;

      // ---- O^T += V^T P^T over 8 blocks of 32 dims ----
#pragma unroll
      for (int kb = 0; kb < KBLK; kb++) {
#pragma unroll
        for (int mt = 0; mt < 8; mt++) {
          const uint16_t *vrow = &vl[(kb * D + mt * 32 + col) * V_STRIDE];
          const uint2 lo4 = *reinterpret_cast<const uint2 *>(vrow + 4 * h);
          const uint2 hi4 = *reinterpret_cast<const uint2 *>(vrow + 8 + 4 * h);
          oacc[mt] = mfma32(u32x4_t{lo4.x, lo4.y, hi4.x, hi4.y}, pb[kb], oacc[mt]);
        }
      }
    }

    if (has_next) store_tile(k_lds[buf ^ 1], v_lds[buf ^ 1], tid, next, use_next, kt + BN, ctx);
    __syncthreads();  // next tile visible; this tile no longer read
  }
  if (!rescale) break;
  {
    const float alpha = fast_exp2(m_run - m_next);  // 1 for rows that did not grow
    m_run = m_next;
    l_run *= alpha;
#pragma unroll
    for (int mt = 0; mt < 8; mt++)
#pragma unroll
      for (int j = 0; j < 16; j++) oacc[mt][j] *= alpha;
    ent_next = fetch_entries(a, table, kt + BN, lane);  // the re-entered tile's next-tile entries
  }
  }

  // ---- normalise and store: lane holds dims 32mt + 8(j/4) + 4h + (j%4) of its row ----
  if (bad && tid == 0) atomicOr(a.err, kErrBadBlock);  // a needed block was missing: its keys read as zeros
  const float l_tot = l_run + xor32_other(l_run);
  if (!row_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  const size_t obase = ((size_t)(c0 + my_row) * Hq + qh) * D;
  uint16_t *orow = a.out + obase;
#pragma unroll
  for (int mt = 0; mt < 8; mt++) {
#pragma unroll
    for (int jq = 0; jq < 4; jq++) {
      const int d0 = mt * 32 + jq * 8 + 4 * h;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; e++) v[e] = gated(oacc[mt][4 * jq + e] * inv, a.gate, obase + d0 + e);
      *reinterpret_cast<uint2 *>(orow + d0) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
    }
  }
}

}  // namespace

hipError_t launch_prefill_d256(const PrefillArgs &a, hipStream_t s) {
  const int n_items = a.q_tiles * a.q_heads * a.num_seqs;
  const int grid = (n_items + 7) / 8 * 8;
  hipLaunchKernelGGL(paged_prefill_d256_kernel, dim3(grid), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace llh
