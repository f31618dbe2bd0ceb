// Chunked causal prefill at head_dim 256 on gfx950 MFMA: the Qwen3.5 / 3.6
// full-attention layers (fixtures/qwen36/config.json: head_dim 256), bf16 pools
// of 16-token blocks.  Same contract as paged_prefill_kernel (prefill.hip):
// query row i of a chunk sits at pos = context_len - chunk_len + i and attends
// [lo(pos), pos] (crates/llm-backend/src/core/native_attention.rs:356-464),
// times sigmoid(gate) when the call carries one (native_attention.rs:765-781).
//
// S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32_bf16, P^T taken straight
// from the S^T accumulators, V^T read from the dim-major pool layout, K/V tiles of
// 64 keys double-buffered in LDS, online softmax in log2 units with a lazy
// rescale.  A wavefront owns 16 query rows: their Q^T (8 k-steps of 32 dims, 32
// registers), O^T (16 blocks of 16 dims, 64 accumulators) and S^T (4 blocks of 16
// keys, 16 accumulators) fit the 256 registers of two wavefronts per SIMD, so one
// workgroup of 8 wavefronts (128 rows of one query head) per CU keeps two
// wavefronts on every SIMD to cover each other's LDS and exponent latency.  (With
// 32-row tiles on the 32x32x16 form the same state needs ~450 registers and leaves
// one wavefront per SIMD.)
//
// MFMA operand layouts (16x16x32, bf16): A 16 x 32, lane l holds row l%16, k
// 8(l/16)..+8; B 32 x 16, lane l holds column l%16, k 8(l/16)..+8; D 16 x 16, lane
// l holds column l%16, rows 4(l/16)..+4.  So S^T block kb gives lane l the scores
// of keys 16kb + 4g .. +4 (g = l/16) for query row l%16, and the P^T operand of a
// 32-key step s takes keys {32s + 4g .. +4, 32s + 16 + 4g .. +4} in its k-slots
// 8g..8g+7; the V^T operand reads the same keys (one 16-byte LDS read).
#include "device_common.h"
#include "wave_ops.h"

namespace llh {

namespace {

constexpr int D = kD256HeadDim;
constexpr int BT = kFastBlockTokens;
constexpr int ROWS = 16;            // query rows per wavefront
constexpr int WAVES = 8;
constexpr int BM = ROWS * WAVES;    // query rows per workgroup (the host's q_tiles unit)
constexpr int BN = 64;              // key positions per tile
constexpr int KBLK = BN / BT;       // pool blocks per tile
constexpr int K_TILE = BN * D;      // K rows unpadded; 16-byte chunk c of key row t sits at c ^ (t & 15)
constexpr int V_ROW = 2 * BT;          // bf16 elements per V^T dim row of one 32-key step in LDS
constexpr int V_STEP = D * V_ROW;      // one 32-key step (two blocks) of V^T
constexpr int V_TILE = 2 * V_STEP;
constexpr int kThreads = 64 * WAVES;
static_assert(BM == 128, "q_tiles is computed for 128-row query tiles");
constexpr int PF_S = 8;  // K fragment reads kept in flight ahead of the S^T MFMAs
constexpr int PF_V = 6;  // V^T fragment reads kept in flight ahead of the P V MFMAs

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;

// 16x16x32 MFMA on packed 16-bit operands: fp16 for fp16 pools (OP = kF16), else bf16
template <int OP>
__device__ __forceinline__ f32x4_t mfma16(const u32x4_t &a, const u32x4_t &b, const f32x4_t &c) {
  if constexpr (OP == kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                    c, 0, 0, 0);
}

// Scheduling order for a region of N LDS reads feeding N MFMAs: AHEAD reads,
// then one MFMA and one read at a time, then the last AHEAD MFMAs -- so AHEAD
// fragment reads stay in flight (left to itself the scheduler keeps one or two,
// exposing the LDS latency on every MFMA).
template <int N, int AHEAD>
__device__ __forceinline__ void reads_ahead_of_mfma() {
  constexpr int kMfma = 0x008, kDsRead = 0x100;  // sched_group_barrier instruction classes
  __builtin_amdgcn_sched_group_barrier(kDsRead, AHEAD, 0);
#pragma unroll
  for (int i = 0; i < N - AHEAD; i++) {
    __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(kMfma, AHEAD, 0);
}

// Value of lane (l ^ 32) (v_permlane32_swap: no LDS round trip).
__device__ __forceinline__ float xor32_other(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Reduction over the four lanes l%16 + 16g that hold one query row.
__device__ __forceinline__ float row_max4(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, xor32_other(v));
}
__device__ __forceinline__ float row_sum4(float v) {
  v += __shfl_xor(v, 16);
  return v + xor32_other(v);
}

// V^T in LDS, per 32-key step s (blocks 2s, 2s+1): a 64-byte row per dim holding,
// for each 4-token chunk g, chunk g of block 2s then chunk g of block 2s+1 -- the
// 16 bytes one lane's A operand takes (keys 32s + 4g .. +4, 32s + 16 + 4g .. +4).
// Dim row d keeps chunk pair g at pair g ^ v_swz(d), so the lanes of one 16-byte
// read (dims 16db + r, one g) and of one 16-byte store (4 dims x 4 pairs) cover
// the banks once.
__device__ __forceinline__ int v_swz(int dim) { return ((dim >> 2) ^ (dim & 2)) & 3; }

// One thread's share of a tile: for each of the 4 blocks, 16 bytes of K at
// token tid/32, dims 8(tid%32).. (the thread's 16-byte slot of the block's 8 KiB),
// and 8 bytes of V^T (tokens 4(tid&3) .. +4) at dims tid/4 and 128 + tid/4.
struct Tile256 {
  u32x4_t k[KBLK];
  uint2 v[KBLK][2];
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
    r.k[kb] = *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const uint16_t *>(a.pool.k) + base + tid * 8);
    const uint16_t *vp = reinterpret_cast<const uint16_t *>(a.pool.v) + base + tid * 4;
    r.v[kb][0] = *reinterpret_cast<const uint2 *>(vp);
    r.v[kb][1] = *reinterpret_cast<const uint2 *>(vp + 128 * BT);
  }
  return use_mask;
}

// Stores a tile to LDS: K rows as loaded (unattended keys are masked in the
// scores), V^T zeroed for unused blocks and tokens at or past the context end
// (P = 0 times a non-finite V would poison the accumulators).
__device__ __forceinline__ void store_tile(uint16_t *k_lds, uint16_t *v_lds, int tid, const Tile256 &r,
                                           uint32_t use_mask, int kt, int ctx) {
  const bool tail = kt + BN > ctx;
  const int g = tid & 3;
#pragma unroll
  for (int kb = 0; kb < KBLK; kb++)
    *reinterpret_cast<u32x4_t *>(&k_lds[(kb * BT + (tid >> 5)) * D + (((tid & 31) ^ (tid >> 5)) * 8)]) = r.k[kb];
#pragma unroll
  for (int s = 0; s < 2; s++) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      uint2 c[2];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int kb = 2 * s + e;
        uint2 v = r.v[kb][hf];
        if (!(use_mask & (1u << kb))) v = make_uint2(0u, 0u);
        if (tail) {
          const int valid = ctx - (kt + kb * BT + 4 * g);  // tokens of this 4-run inside the context
          v.x &= (valid > 0 ? 0x0000ffffu : 0u) | (valid > 1 ? 0xffff0000u : 0u);
          v.y &= (valid > 2 ? 0x0000ffffu : 0u) | (valid > 3 ? 0xffff0000u : 0u);
        }
        c[e] = v;
      }
      const int dim = (tid >> 2) + 128 * hf;
      *reinterpret_cast<u32x4_t *>(&v_lds[s * V_STEP + dim * V_ROW + 8 * (g ^ v_swz(dim))]) =
          u32x4_t{c[0].x, c[0].y, c[1].x, c[1].y};
    }
  }
}

template <int FMT>
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
  const int g = lane >> 4;   // k-slot group of the MFMA operands
  const int r = lane & 15;   // query row of the wavefront; also the A-operand row
  const int prefix = ctx - chunk;
  const int rows_wg = min(BM, chunk - i0);
  const int qpos_first = prefix + i0;
  const int qpos_last = prefix + i0 + rows_wg - 1;
  const int my_row = i0 + wave * ROWS + r;
  const bool row_ok = my_row < chunk;
  const int my_pos = prefix + my_row;
  const int my_lo = a.window > 0 ? max(0, my_pos - a.window + 1) : 0;

  // ---- Q^T operand: 8 k-steps of 32 dims; lane holds dims 32ks + 8g .. +8 of its row ----
  u32x4_t qb[8];
  {
    const uint16_t *qrow = a.q + ((size_t)(c0 + (row_ok ? my_row : 0)) * Hq + qh) * D;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      u32x4_t t = *reinterpret_cast<const u32x4_t *>(qrow + ks * 32 + g * 8);
      if (!row_ok) t = u32x4_t{0u, 0u, 0u, 0u};
      qb[ks] = t;
    }
  }
  // fp16 pools: the row's q in fp16, scaled by 2^-e over its 256 dims (held by lanes
  // r, r + 16, r + 32, r + 48); its scores carry the step 2^e
  float qstep = 1.0f;
  if constexpr (FMT == kF16) {
    uint32_t w[32];
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int e = 0; e < 4; e++) w[4 * ks + e] = qb[ks][e];
    int mx = bf16_absmax_bits<32>(w);
    mx = max(mx, __shfl_xor(mx, 16));
    mx = max(mx, __float_as_int(xor32_other(__int_as_float(mx))));
    const F16Scaling sc = f16_scaling(mx);
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int e = 0; e < 4; e++) qb[ks][e] = bf16x2_to_f16x2(w[4 * ks + e], sc.inv);
    qstep = sc.step;
  }

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][K_TILE];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][V_TILE];

  f32x4_t oacc[16];
#pragma unroll
  for (int db = 0; db < 16; db++) oacc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const int klo = a.window > 0 ? max(0, qpos_first - a.window + 1) : 0;
  const int khi = qpos_last + 1;  // exclusive
  const int t_begin = (klo / BN) * BN;
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  const int wrow0 = i0 + wave * ROWS;
  const int wpos_first = prefix + wrow0;
  const int wpos_last = prefix + min(wrow0 + ROWS - 1, chunk - 1);
  const int wlo_first = a.window > 0 ? max(0, wpos_first - a.window + 1) : 0;
  const int wlo_last = a.window > 0 ? max(0, wpos_last - a.window + 1) : 0;
  const bool wave_live = wrow0 < chunk;
  const int vsw = 8 * (g ^ v_swz(r));  // element offset of this lane's V^T chunk pair (dims 16db + r)

  Tile256 next;
  bool bad = false;
  uint32_t use_next = load_tile(a, fetch_entries(a, table, t_begin, lane), kvh, t_begin, ctx, klo, tid, next, bad);
  int ent_next = fetch_entries(a, table, t_begin + BN, lane);
  store_tile(k_lds[0], v_lds[0], tid, next, use_next, t_begin, ctx);
  __syncthreads();

  int buf = 0;
  for (int kt = t_begin; kt < khi; kt += BN, buf ^= 1) {
    const bool has_next = kt + BN < khi;
    if (has_next)  // in flight during the math
      use_next = load_tile(a, ent_next, kvh, kt + BN, ctx, klo, tid, next, bad);
    ent_next = fetch_entries(a, table, kt + 2 * BN, lane);

    if (wave_live && kt <= wpos_last && kt + BN > wlo_first) {
      const uint16_t *kl = k_lds[buf];
      const uint16_t *vl = v_lds[buf];
      // ---- S^T = K Q^T: four 16-key blocks, four independent chains ----
      f32x4_t sacc[KBLK];
#pragma unroll
      for (int kb = 0; kb < KBLK; kb++) sacc[kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int kb = 0; kb < KBLK; kb++) {
          const u32x4_t ka = *reinterpret_cast<const u32x4_t *>(&kl[(kb * BT + r) * D + (((ks * 4 + g) ^ r) * 8)]);
          sacc[kb] = mfma16<FMT>(ka, qb[ks], sacc[kb]);
        }
      reads_ahead_of_mfma<KBLK * 8, PF_S>();

      // ---- scale, mask, online softmax (as the head_dim-128 kernel) ----
      const bool need_mask = (kt + BN - 1 > wpos_first) || (kt < wlo_last) || (kt + BN > ctx);
      const float c = a.scale_log2e * qstep;
      float c_exp = c;
      float tmax = -INFINITY;
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < KBLK; kb++) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float s = sacc[kb][i] * c;
            const int kp = kt + kb * BT + 4 * g + i;
            if (kp > my_pos || kp < my_lo || kp >= ctx || !row_ok) s = -INFINITY;
            sacc[kb][i] = s;
            tmax = fmaxf(tmax, s);
          }
        }
        c_exp = 1.0f;
      } else if (c >= 0.0f) {
#pragma unroll
        for (int kb = 0; kb < KBLK; kb++)
#pragma unroll
          for (int i = 0; i < 4; i++) tmax = fmaxf(tmax, sacc[kb][i]);
        tmax *= c;
      } else {
        float tmin = INFINITY;
#pragma unroll
        for (int kb = 0; kb < KBLK; kb++)
#pragma unroll
          for (int i = 0; i < 4; i++) tmin = fminf(tmin, sacc[kb][i]);
        tmax = tmin * c;
      }
      // Raw scores beyond 2^26 (log2 units) once scaled: tmax, a rounded product, can
      // fall below the fma's exact product c * s by more than the weights' headroom
      // (|error| <= |tmax| 2^-24), so those tiles scale first, as masked tiles do:
      // every score rounds as tmax did and the largest weight is exactly 1.
      if (!need_mask && __any(fabsf(tmax) > 0x1p26f)) {
#pragma unroll
        for (int kb = 0; kb < KBLK; kb++)
#pragma unroll
          for (int i = 0; i < 4; i++) sacc[kb][i] *= c;
        c_exp = 1.0f;
      }
      tmax = row_max4(tmax);
      const float m_cand = fmaxf(m_run, tmax);
      // a row without a finite score yet takes the tile's max (its accumulators are
      // still zero); a row whose max grows by more than 16 is rescaled first, so
      // the weights stay below 2^16
      const bool grow = m_run != -INFINITY && m_cand > m_run + 16.0f;
      if (__any(grow)) {
        const float m_new = grow ? m_cand : m_run;
        const float alpha = fast_exp2(m_run - m_new);  // 1 for rows that did not grow
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 16; db++) oacc[db] *= alpha;
      }
      if (m_run == -INFINITY) m_run = m_cand;
      const float mref = (m_run == -INFINITY) ? 0.0f : m_run;
      u32x4_t pb[2];
      float psum = 0.0f;  // row sums of exactly the bf16 weights that enter P V
#pragma unroll
      for (int s = 0; s < 2; s++) {
        float p[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          p[i] = fast_exp2(__builtin_fmaf(sacc[2 * s][i], c_exp, -mref));
          p[4 + i] = fast_exp2(__builtin_fmaf(sacc[2 * s + 1][i], c_exp, -mref));
        }
        pb[s] = u32x4_t{pack_16<FMT>(p[0], p[1]), pack_16<FMT>(p[2], p[3]), pack_16<FMT>(p[4], p[5]),
                        pack_16<FMT>(p[6], p[7])};
#pragma unroll
        for (int e = 0; e < 4; e++) psum = dot2_ones_16<FMT>(pb[s][e], psum);
      }
      l_run += psum;

      // ---- O^T += V^T P^T over 16 blocks of 16 dims, two 32-key steps ----
#pragma unroll
      for (int s = 0; s < 2; s++) {
#pragma unroll
        for (int db = 0; db < 16; db++) {
          const u32x4_t va = *reinterpret_cast<const u32x4_t *>(&vl[s * V_STEP + (db * 16 + r) * V_ROW + vsw]);
          oacc[db] = mfma16<FMT>(va, pb[s], oacc[db]);
        }
      }
      reads_ahead_of_mfma<2 * 16, PF_V>();
    }

    if (has_next) store_tile(k_lds[buf ^ 1], v_lds[buf ^ 1], tid, next, use_next, kt + BN, ctx);
    __syncthreads();  // next tile visible; this tile no longer read
  }

  // ---- normalise and store: lane holds dims 16db + 4g .. +4 of its row ----
  if (bad && tid == 0) atomicOr(a.err, kErrBadBlock);  // a needed block was missing: its keys read as zeros
  const float l_tot = row_sum4(l_run);
  if (!row_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  const size_t obase = ((size_t)(c0 + my_row) * Hq + qh) * D;
  uint16_t *orow = a.out + obase;
#pragma unroll
  for (int db = 0; db < 16; db++) {
    const int d0 = db * 16 + 4 * g;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = gated(oacc[db][e] * inv, a.gate, obase + d0 + e);
    *reinterpret_cast<uint2 *>(orow + d0) = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
  }
}

}  // namespace

hipError_t launch_prefill_d256(const PrefillArgs &a, hipStream_t s) {
  const int n_items = a.q_tiles * a.q_heads * a.num_seqs;
  const int grid = (n_items + 7) / 8 * 8;
  if (a.pool.format == kF16)
    hipLaunchKernelGGL(paged_prefill_d256_kernel<kF16>, dim3(grid), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(paged_prefill_d256_kernel<kBf16>, dim3(grid), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace llh
