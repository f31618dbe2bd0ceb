// Chunked causal prefill over cached prefix blocks, on gfx950 MFMA.
//
// For each sequence, query row i of the chunk sits at position
// pos = context_len - chunk_len + i and attends positions [lo(pos), pos]
// (causal inside the chunk, full attention to the cached prefix, optional
// sliding window).  This is the result of the reference's per-token
// "append then attend" loop (crates/llm-backend/src/core/native_attention.rs:356-464)
// computed as one dense pass.
//
// One workgroup = 128 query rows of one query head (4 wavefronts x 32 rows).
// Key tiles of 64 positions (4 pool blocks) are staged in LDS, double
// buffered: while the wavefronts run the MFMAs of tile t, every lane already
// holds its share of tile t+1 in registers, and stores it to the other buffer
// afterwards (one barrier per tile).  When a kv head's group is even, one
// workgroup of 8 wavefronts runs two of its query heads over the same K/V
// tiles (half the tile loads and LDS stores per FLOP).  Tiles wholly outside the window or past
// the last query are never loaded, and only tiles that straddle a boundary are
// masked.
//
// Work mapping: workgroups are dispatched round-robin over the 8 XCDs, each
// with its own L2.  The launch maps workgroup L to logical work item
// w = (L % 8) * ceil(N / 8) + L / 8, and logical items run (sequence, kv head,
// query tile, query head in group) with the head fastest, so each XCD works on
// few (sequence, kv head) pairs at a time and their K/V tiles stay in its L2.
//
// int8 / fp8 pools are dequantised while a tile is stored to LDS (code * scale in
// f32, rounded to bf16), so the MFMA path is the same for every format: the
// result is attention over the dequantised cache, as the reference attends its
// int8 cache after dequantising it (crates/llm-kv-cache/src/layer.rs:650-656).
// fp16 pools keep K and V in fp16 and run v_mfma_f32_32x32x16_f16 instead, with
// each query row scaled into fp16 by a power of two (f16_scaling) whose step
// multiplies that row's scores, and fp16 softmax weights.
//
// Per wavefront, with v_mfma_f32_32x32x16_bf16:
//   S^T[key][query] = K Q^T       A = K rows (token-major pool layout)
//                                 B = Q^T    (held in registers)
//   O^T[dim][query] += V^T P^T    A = V^T    (the pool stores V dim-major)
//                                 B = P^T    (exp'd S^T accumulators, packed to bf16)
// The accumulator layout of S^T (lane = query column, 16 key rows per lane)
// is exactly the B-operand layout P^T needs when the key order inside each
// 16-key step is {4h..4h+3, 8+4h..8+4h+3} for lane half h; the V^T operand is
// read from LDS with the same key order, so no transpose is ever done.
// Softmax statistics are kept per query column in log2 units (online softmax).
#include "wave_ops.h"

namespace llh {

namespace {

constexpr int D = kFastHeadDim;
constexpr int BT = kFastBlockTokens;
constexpr int BM = 128;          // query rows per workgroup
constexpr int BN = 64;           // key positions per tile
constexpr int KBLK = BN / BT;    // pool blocks per tile
constexpr int K_STRIDE = D + 8;  // bf16 elements per K row in LDS (272 B: conflict-free b128 reads)
constexpr int V_STRIDE = BT + 4; // bf16 elements per V^T row in LDS (40 B: conflict-free b64 reads)
constexpr int K_TILE = BN * K_STRIDE;        // bf16 elements of one K tile in LDS
constexpr int V_TILE = KBLK * D * V_STRIDE;  // bf16 elements of one V^T tile in LDS

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

// 32x32x16 MFMA on packed 16-bit operands: fp16 for fp16 pools (OP = kF16),
// bf16 for every other format
template <int OP>
__device__ __forceinline__ f32x16_t mfma32(const u32x4_t &a, const u32x4_t &b, const f32x16_t &c) {
  if constexpr (OP == kF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                    c, 0, 0, 0);
}

// One lane's share of a key tile: for each of the 4 blocks, the K elements of
// token tid/16 at dims 8*(tid%16).. and the V^T elements of dim tid/2 at tokens
// 8*(tid&1)..: 16 B each for bf16 / fp16 pools; for int8 / fp8 pools 8 B of codes
// each plus the scales they need (int8: the fp16 scale of the K token and the
// eight of the V tokens; fp8: the block's f32 K and V scales), dequantised to
// bf16 when the tile is stored to LDS.
template <int FMT, int NB>
struct TileRegs;

template <int NB>
struct TileRegs16 {
  u32x4_t k[NB];
  u32x4_t v[NB];
};
template <int NB>
struct TileRegs<kBf16, NB> : TileRegs16<NB> {};
template <int NB>
struct TileRegs<kF16, NB> : TileRegs16<NB> {};

template <int FMT, int NB>
struct TileRegs {
  uint2 k[NB];
  uint2 v[NB];
  uint32_t ks[NB];  // int8: fp16 bits of the K token's scale; fp8: f32 bits of the block's K scale
  uint4 vs[NB][2];  // int8: the (K, V) fp16 scale pairs of tokens 8*(tid&1) .. +7; fp8: [0].x = f32 bits of the V scale
};

// Block-table entries of the tile starting at kt: lane kb of every wavefront
// holds the entry of the tile's block kb (lanes repeat mod KBLK).  Always an
// in-bounds table read (the index is taken mod max_blocks), issued one tile
// ahead so the table read never sits on the critical path.
__device__ __forceinline__ int fetch_entries(const PrefillArgs &a, const int32_t *table, int kt, int lane) {
  return table[(kt / BT + (lane & (KBLK - 1))) % a.max_blocks];
}

// Issues the tile's K/V loads.  Every load is unconditional (blocks that are not
// needed, or whose entry is outside the pool, read block 0 and are zeroed when
// stored to LDS), so no branch or conditional memory operation sits between
// the prefetch and the math that overlaps it.  `bad` collects needed blocks
// with an out-of-pool entry (flagged once, at the end of the kernel).
template <int FMT, int NB>
__device__ __forceinline__ uint32_t load_tile(const PrefillArgs &a, int entries, int kvh, int kt, int ctx, int klo,
                                              int tid, int kb0, TileRegs<FMT, NB> &r, bool &bad) {
  const int Hkv = a.pool.kv_heads;
  uint32_t use_mask = 0;
#pragma unroll
  for (int i = 0; i < NB; i++) {
    const int kb = kb0 + i;
    const int bpos = kt + kb * BT;
    const bool needed = bpos < ctx && bpos + BT > klo;
    const int phys = __builtin_amdgcn_readlane(entries, kb);
    const bool ok = phys >= 0 && (int64_t)phys < a.pool.n_blocks;
    bad |= needed && !ok;
    const bool use = needed && ok;
    use_mask |= use ? (1u << i) : 0u;
    const size_t bh = (size_t)(use ? phys : 0) * Hkv + kvh;
    const size_t base = bh * (BT * D);  // elements of this block-head
    if constexpr (is16(FMT)) {
      r.k[i] = *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const uint16_t *>(a.pool.k) + base +
                                                (tid >> 4) * D + (tid & 15) * 8);
      r.v[i] = *reinterpret_cast<const u32x4_t *>(reinterpret_cast<const uint16_t *>(a.pool.v) + base +
                                                (tid >> 1) * BT + (tid & 1) * 8);
    } else {
      r.k[i] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(a.pool.k) + base + (tid >> 4) * D +
                                                (tid & 15) * 8);
      r.v[i] = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint8_t *>(a.pool.v) + base +
                                                (tid >> 1) * BT + (tid & 1) * 8);
      if constexpr (FMT == kInt8) {
        r.ks[i] = reinterpret_cast<const uint16_t *>(a.pool.k_scales)[int8_scale_index(bh, tid >> 4, BT)];
        const uint4 *sp = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(a.pool.k_scales) +
                                                          int8_scale_index(bh, (tid & 1) * 8, BT));
        r.vs[i][0] = sp[0];
        r.vs[i][1] = sp[1];
      } else {
        const uint2 s2 = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint32_t *>(a.pool.k_scales) +
                                                          fp8_scale_index(bh));
        r.ks[i] = s2.x;
        r.vs[i][0].x = s2.y;
      }
    }
  }
  return use_mask;
}

__device__ __forceinline__ float half_bits_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Element e (0..7) of eight int8 / e4m3 codes as f32 (exact).
template <int FMT>
__device__ __forceinline__ float code_f32(const uint2 &w, int e) {
  const uint32_t word = e < 4 ? w.x : w.y;
  if constexpr (FMT == kInt8) {
    return (float)(int8_t)(word >> (8 * (e & 3)));
  } else {
    const auto f = (e & 2) ? __builtin_amdgcn_cvt_pk_f32_fp8(word, true) : __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
    return f[e & 1];
  }
}

// The tile's K and V^T elements of this lane as 16-bit MFMA operands: the
// stored elements of bf16 / fp16 pools; for int8 / fp8 the dequantised value
// (code * scale in f32) rounded to bf16 (nearest even).
template <int FMT, int NB>
__device__ __forceinline__ void tile_operands(const TileRegs<FMT, NB> &r, int i, u32x4_t &k, u32x4_t &v) {
  if constexpr (is16(FMT)) {
    k = r.k[i];
    v = r.v[i];
  } else {
    float kf[8], vf[8];
    const float ks = FMT == kInt8 ? half_bits_f32(r.ks[i]) : __uint_as_float(r.ks[i]);
#pragma unroll
    for (int e = 0; e < 8; e++) kf[e] = code_f32<FMT>(r.k[i], e) * ks;
    if constexpr (FMT == kInt8) {
      const uint32_t pr[8] = {r.vs[i][0].x, r.vs[i][0].y, r.vs[i][0].z, r.vs[i][0].w,
                              r.vs[i][1].x, r.vs[i][1].y, r.vs[i][1].z, r.vs[i][1].w};
#pragma unroll
      for (int e = 0; e < 8; e++) vf[e] = code_f32<FMT>(r.v[i], e) * half_bits_f32(pr[e] >> 16);
    } else {
      const float vs = __uint_as_float(r.vs[i][0].x);
#pragma unroll
      for (int e = 0; e < 8; e++) vf[e] = code_f32<FMT>(r.v[i], e) * vs;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      k[q] = pack_bf16(kf[2 * q], kf[2 * q + 1]);
      v[q] = pack_bf16(vf[2 * q], vf[2 * q + 1]);
    }
  }
}

// Stores a tile to LDS.  K rows are stored as loaded (keys that are not
// attended are masked to -inf in the scores, whatever K holds); V^T is zeroed
// for unused blocks and for tokens at or past the context end, because
// P = 0 times a non-finite V would still poison the accumulators.
template <int FMT, int NB>
__device__ __forceinline__ void store_tile(uint16_t *k_lds, uint16_t *v_lds, int tid, int kb0,
                                           const TileRegs<FMT, NB> &r, uint32_t use_mask, int kt, int ctx) {
  const bool tail = kt + BN > ctx;  // the tile reaches the end of the context (uniform)
#pragma unroll
  for (int i = 0; i < NB; i++) {
    const int kb = kb0 + i;
    u32x4_t kk, v;
    tile_operands<FMT, NB>(r, i, kk, v);
    *reinterpret_cast<u32x4_t *>(&k_lds[(kb * BT + (tid >> 4)) * K_STRIDE + (tid & 15) * 8]) = kk;
    if (!(use_mask & (1u << i))) v = u32x4_t{0u, 0u, 0u, 0u};
    if (tail) {
      const int valid = ctx - (kt + kb * BT + (tid & 1) * 8);  // tokens of this 8-run inside the context
      v[0] &= (valid > 0 ? 0x0000ffffu : 0u) | (valid > 1 ? 0xffff0000u : 0u);
      v[1] &= (valid > 2 ? 0x0000ffffu : 0u) | (valid > 3 ? 0xffff0000u : 0u);
      v[2] &= (valid > 4 ? 0x0000ffffu : 0u) | (valid > 5 ? 0xffff0000u : 0u);
      v[3] &= (valid > 6 ? 0x0000ffffu : 0u) | (valid > 7 ? 0xffff0000u : 0u);
    }
    uint16_t *dst = &v_lds[(kb * D + (tid >> 1)) * V_STRIDE + (tid & 1) * 8];
    *reinterpret_cast<uint2 *>(dst) = make_uint2(v[0], v[1]);
    *reinterpret_cast<uint2 *>(dst + 4) = make_uint2(v[2], v[3]);
  }
}

template <int HPW, int FMT>
__global__ __launch_bounds__(kPrefillThreads * HPW, 2 / HPW) void paged_prefill_kernel(const PrefillArgs a) {
  // ---- XCD-aware logical work item ----
  const int Hq = a.q_heads;
  const int Hkv = a.pool.kv_heads;
  const int GW = Hq / Hkv / HPW;  // workgroups per (kv head, query tile)
  const int n_items = a.q_tiles * Hkv * GW * a.num_seqs;
  const int per_xcd = (n_items + 7) / 8;
  // Within one XCD's items, the longest go first: when its block of items is
  // whole (sequence, kv head) groups, dispatch i takes tile q_tiles-1-r of
  // group g (r = i / (groups * GW)), so the first round runs the tiles with
  // the longest causal reach and the last round the shortest.
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
  const int qh = (kvh * GW + w % GW) * HPW + (threadIdx.x >> 8);  // this wavefront's query head

  const int c0 = a.chunk_starts[b];
  const int chunk = a.chunk_starts[b + 1] - c0;
  const int ctx = a.context_lens[b];
  const int i0 = tile * BM;
  if (i0 >= chunk || chunk <= 0 || ctx < chunk) return;
  {
    // every key of the chunk's first row through the last must be resident at once:
    // a longer span would alias its own table entries (rows are read modulo max_blocks)
    const int first_lo = a.window > 0 ? max(0, ctx - chunk - a.window + 1) : 0;
    if (ctx - first_lo > a.max_blocks * BT) {
      if (threadIdx.x == 0 && tile == 0) atomicOr(a.err, kErrSpan);
      return;
    }
  }

  const int tid = threadIdx.x;
  const int ltid = tid & (kPrefillThreads - 1);  // thread index within the head's 4 wavefronts
  const int kb0 = (tid / kPrefillThreads) * (KBLK / HPW);  // first tile block this thread loads
  const int lane = tid & 63;
  const int wave = ltid >> 6;
  const int h = lane >> 5;     // lane half
  const int col = lane & 31;   // query column of this lane
  const int prefix = ctx - chunk;

  // rows of this workgroup and of this wavefront
  const int rows_wg = min(BM, chunk - i0);
  const int qpos_first = prefix + i0;                 // position of the first row
  const int qpos_last = prefix + i0 + rows_wg - 1;    // position of the last valid row
  const int my_row = i0 + wave * 32 + col;            // chunk row of this lane's query
  const bool row_ok = my_row < chunk;
  const int my_pos = prefix + my_row;
  const int my_lo = a.window > 0 ? max(0, my_pos - a.window + 1) : 0;

  // ---- Q^T operand: 8 k-steps of 16 dims; lane holds dims 16ks + 8h .. +8 of its row ----
  u32x4_t qb[8];
  {
    const uint16_t *qrow = a.q + ((size_t)(c0 + (row_ok ? my_row : 0)) * Hq + qh) * D;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      u32x4_t t = *reinterpret_cast<const u32x4_t *>(qrow + ks * 16 + h * 8);
      if (!row_ok) t = u32x4_t{0u, 0u, 0u, 0u};
      qb[ks] = t;
    }
  }
  // fp16 pools: the row's q in fp16, scaled by 2^-e over its 128 dims (this lane
  // and lane ^ 32 hold them); its scores carry the step 2^e
  constexpr int OP = FMT == kF16 ? kF16 : kBf16;
  float qstep = 1.0f;
  if constexpr (FMT == kF16) {
    uint32_t w[32];
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int e = 0; e < 4; e++) w[4 * ks + e] = qb[ks][e];
    int mx = bf16_absmax_bits<32>(w);
    mx = max(mx, __float_as_int(xor32_other(__int_as_float(mx), lane)));
    const F16Scaling sc = f16_scaling(mx);
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
      for (int e = 0; e < 4; e++) qb[ks][e] = bf16x2_to_f16x2(w[4 * ks + e], sc.inv);
    qstep = sc.step;
  }

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][K_TILE];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][V_TILE];

  f32x16_t oacc[4];
#pragma unroll
  for (int mt = 0; mt < 4; mt++)
#pragma unroll
    for (int j = 0; j < 16; j++) oacc[mt][j] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  // key range of the workgroup
  const int klo = a.window > 0 ? max(0, qpos_first - a.window + 1) : 0;
  const int khi = qpos_last + 1;  // exclusive
  const int t_begin = (klo / BN) * BN;
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  // wavefront-level bounds for masking decisions
  const int wrow0 = i0 + wave * 32;
  const int wpos_first = prefix + wrow0;
  const int wpos_last = prefix + min(wrow0 + 31, chunk - 1);
  const int wlo_first = a.window > 0 ? max(0, wpos_first - a.window + 1) : 0;
  const int wlo_last = a.window > 0 ? max(0, wpos_last - a.window + 1) : 0;
  const bool wave_live = wrow0 < chunk;

  TileRegs<FMT, KBLK / HPW> next;
  bool bad = false;
  uint32_t use_next =
      load_tile(a, fetch_entries(a, table, t_begin, lane), kvh, t_begin, ctx, klo, ltid, kb0, next, bad);
  int ent_next = fetch_entries(a, table, t_begin + BN, lane);
  store_tile(k_lds[0], v_lds[0], ltid, kb0, next, use_next, t_begin, ctx);
  __syncthreads();

  int buf = 0;
  for (int kt = t_begin; kt < khi; kt += BN, buf ^= 1) {
    const bool has_next = kt + BN < khi;
    if (has_next)  // in flight during the math
      use_next = load_tile(a, ent_next, kvh, kt + BN, ctx, klo, ltid, kb0, next, bad);
    // entries of the tile after next, issued behind this tile's loads
    ent_next = fetch_entries(a, table, kt + 2 * BN, lane);

    // tile needed by this wavefront?
    if (wave_live && kt <= wpos_last && kt + BN > wlo_first) {
      const uint16_t *kl = k_lds[buf];
      const uint16_t *vl = v_lds[buf];
      // ---- S^T = K Q^T for two 32-key sub-tiles ----
      f32x16_t sacc[2];
#pragma unroll
      for (int st = 0; st < 2; st++) {
#pragma unroll
        for (int j = 0; j < 16; j++) sacc[st][j] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
          const u32x4_t ka = *reinterpret_cast<const u32x4_t *>(&kl[(st * 32 + col) * K_STRIDE + ks * 16 + h * 8]);
          sacc[st] = mfma32<OP>(ka, qb[ks], sacc[st]);
        }
      }

      // ---- scale, mask, online softmax ----
      // Unmasked tiles keep raw scores: the row max is taken on them and the
      // scale (log2 units) is folded into the exp2 argument, fma(s, c, -m).
      // Masked tiles are scaled first, then masked with -inf (c_exp = 1).
      const bool need_mask = (kt + BN - 1 > wpos_first) || (kt < wlo_last) || (kt + BN > ctx);
      const float c = a.scale_log2e * qstep;
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
      } else if (c >= 0.0f) {  // c * max(s) == max(c * s) for c >= 0, exactly
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
      tmax = fmaxf(tmax, xor32_other(tmax, lane));
      // Lazy rescale: the reference max m_run only moves when a row's max grows
      // by more than 8 (log2 units), so p <= 2^8 and the accumulators are
      // rescaled on few tiles.  The result is the same softmax (any reference
      // max gives it) with no risk of overflow in f32 / bf16 / fp16.
      const float m_cand = fmaxf(m_run, tmax);
      const bool grow = m_cand > m_run + 8.0f;  // true on the first finite tile
      if (__any(grow)) {
        const float alpha = grow ? fast_exp2(m_run - m_cand) : 1.0f;  // 0 when m_run = -inf
        m_run = grow ? m_cand : m_run;
        l_run *= alpha;
#pragma unroll
        for (int mt = 0; mt < 4; mt++)
#pragma unroll
          for (int j = 0; j < 16; j++) oacc[mt][j] *= alpha;
      }
      const float mref = (m_run == -INFINITY) ? 0.0f : m_run;
      u32x4_t pb[4];  // P^T operands for the 4 16-key steps (one pool block each)
#pragma unroll
      for (int st = 0; st < 2; st++) {
        float p[16];
#pragma unroll
        for (int j = 0; j < 16; j++) p[j] = fast_exp2(__builtin_fmaf(sacc[st][j], c_exp, -mref));
#pragma unroll
        for (int q = 0; q < 2; q++)
          pb[2 * st + q] = u32x4_t{pack_16<OP>(p[8 * q + 0], p[8 * q + 1]), pack_16<OP>(p[8 * q + 2], p[8 * q + 3]),
                                   pack_16<OP>(p[8 * q + 4], p[8 * q + 5]), pack_16<OP>(p[8 * q + 6], p[8 * q + 7])};
      }
      // row sums of exactly the 16-bit weights that enter P V (dot2 with (1, 1))
      float psum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < KBLK; kb++)
#pragma unroll
        for (int e = 0; e < 4; e++) psum = dot2_ones_16<OP>(pb[kb][e], psum);
      l_run += psum;

      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int kb = 0; kb < KBLK; kb++) {
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
          const uint16_t *vrow = &vl[(kb * D + mt * 32 + col) * V_STRIDE];
          const uint2 lo4 = *reinterpret_cast<const uint2 *>(vrow + 4 * h);
          const uint2 hi4 = *reinterpret_cast<const uint2 *>(vrow + 8 + 4 * h);
          oacc[mt] = mfma32<OP>(u32x4_t{lo4.x, lo4.y, hi4.x, hi4.y}, pb[kb], oacc[mt]);
        }
      }
    }

    if (has_next) store_tile(k_lds[buf ^ 1], v_lds[buf ^ 1], ltid, kb0, next, use_next, kt + BN, ctx);
    __syncthreads();  // next tile visible; this tile no longer read
  }

  // ---- normalise and store: lane holds dims 32mt + 8(j/4) + 4h + (j%4) of its row ----
  if (bad && tid == 0) atomicOr(a.err, kErrBadBlock);  // a needed block was missing: its keys read as zeros
  const float l_tot = l_run + xor32_other(l_run, lane);
  if (!row_ok) return;
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  const size_t obase = ((size_t)(c0 + my_row) * Hq + qh) * D;
  uint16_t *orow = a.out + obase;
#pragma unroll
  for (int mt = 0; mt < 4; mt++) {
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

template <int FMT>
void launch_prefill_fmt(const PrefillArgs &a, int variant, int grid, hipStream_t s) {
  if (variant == kPrefillTwoHeads)
    hipLaunchKernelGGL((paged_prefill_kernel<2, FMT>), dim3(grid), dim3(2 * kPrefillThreads), 0, s, a);
  else
    hipLaunchKernelGGL((paged_prefill_kernel<1, FMT>), dim3(grid), dim3(kPrefillThreads), 0, s, a);
}

// Prefill for every shape the tuned kernel does not take (head_dim != 128,
// block size != 16, q / output rows not 16-byte aligned), and for the
// force-generic option.  One workgroup per (chunk row, query head) attends
// [lo(pos), pos] in chunks of 256 keys: scores are sequential f32 dot
// products (the reference's order), softmax is online in f32 with expf, and
// the pool is read element-wise in any format, dequantised.
__global__ __launch_bounds__(256) void prefill_generic_kernel(const PrefillArgs a) {
  const int r = blockIdx.x;  // global chunk row
  const int h = blockIdx.y;  // query head
  const int tid = threadIdx.x;
  // the sequence of row r: the last b with chunk_starts[b] <= r
  int lo_b = 0, hi_b = a.num_seqs;
  while (hi_b - lo_b > 1) {
    const int mid = (lo_b + hi_b) / 2;
    if (a.chunk_starts[mid] <= r) lo_b = mid;
    else hi_b = mid;
  }
  const int b = lo_b;
  const int c0 = a.chunk_starts[b];
  const int chunk = a.chunk_starts[b + 1] - c0;
  const int ctx = a.context_lens[b];
  const int i = r - c0;
  if (i < 0 || i >= chunk || ctx < chunk) return;
  const int bt = a.pool.block_tokens;
  const int Dh = a.pool.head_dim;
  const int Hq = a.q_heads;
  {
    const int first_lo = a.window > 0 ? max(0, ctx - chunk - a.window + 1) : 0;
    if ((int64_t)(ctx - first_lo) > (int64_t)a.max_blocks * bt) {  // would alias its own table entries
      if (tid == 0 && i == 0 && h == 0) atomicOr(a.err, kErrSpan);
      return;
    }
  }
  const int pos = ctx - chunk + i;
  const int lo = a.window > 0 ? max(0, pos - a.window + 1) : 0;
  const int kvh = h / (Hq / a.pool.kv_heads);
  const int32_t *table = a.tables + (size_t)b * a.max_blocks;
  const size_t row = ((size_t)r * Hq + h) * Dh;

  __shared__ float qs[kGenericPrefillMaxDim];
  __shared__ float w[256];
  __shared__ float red[256];
  __shared__ int64_t kblk[256];
  __shared__ int koff[256];
  __shared__ int s_bad;
  for (int d = tid; d < Dh; d += 256) qs[d] = __uint_as_float((uint32_t)a.q[row + d] << 16);
  if (tid == 0) s_bad = 0;
  __syncthreads();

  float m = -INFINITY, l = 0.0f;
  float acc[kGenericPrefillMaxDim / 256] = {};
  for (int k0 = lo; k0 <= pos; k0 += 256) {
    const int n = min(256, pos - k0 + 1);
    float s = -INFINITY;
    if (tid < n) {
      const int kp = k0 + tid;
      const int64_t blk = table[(kp / bt) % a.max_blocks];
      const int off = kp % bt;
      kblk[tid] = blk;
      koff[tid] = off;
      if (blk >= 0 && blk < a.pool.n_blocks) {
        float dot = 0.0f;
        for (int d = 0; d < Dh; d++) dot = __fadd_rn(dot, __fmul_rn(pool_elem(a.pool, 0, blk, kvh, off, d), qs[d]));
        s = __fmul_rn(dot, a.scale);
      } else {
        atomicOr(&s_bad, 1);
      }
    }
    red[tid] = s;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
      if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
      __syncthreads();
    }
    const float m_new = fmaxf(m, red[0]);
    __syncthreads();
    const float alpha = m == -INFINITY ? 0.0f : expf(__fsub_rn(m, m_new));
    const float e = s == -INFINITY ? 0.0f : expf(__fsub_rn(s, m_new));
    w[tid] = e;
    red[tid] = e;
    __syncthreads();
    for (int st = 128; st > 0; st >>= 1) {
      if (tid < st) red[tid] += red[tid + st];
      __syncthreads();
    }
    l = l * alpha + red[0];
    m = m_new;
#pragma unroll
    for (int j = 0; j < kGenericPrefillMaxDim / 256; j++) {
      const int d = tid + 256 * j;
      if (d >= Dh) break;
      float o = acc[j] * alpha;
      for (int t = 0; t < n; t++)
        if (w[t] != 0.0f) o = __fadd_rn(o, __fmul_rn(w[t], pool_elem(a.pool, 1, kblk[t], kvh, koff[t], d)));
      acc[j] = o;
    }
    __syncthreads();  // w, kblk, koff and red are rewritten by the next chunk
  }
  if (tid == 0 && s_bad) atomicOr(a.err, kErrBadBlock);
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int j = 0; j < kGenericPrefillMaxDim / 256; j++) {
    const int d = tid + 256 * j;
    if (d < Dh) a.out[row + d] = f32_to_bf16_rne(gated(acc[j] * inv, a.gate, row + d));
  }
}

}  // namespace

hipError_t launch_prefill(const PrefillArgs &a, int variant, hipStream_t s) {
  const int n_items = a.q_tiles * (a.q_heads / (variant == kPrefillOneHead ? 1 : 2)) * a.num_seqs;
  const int grid = (n_items + 7) / 8 * 8;
  switch (a.pool.format) {
    case kBf16:
      launch_prefill_fmt<kBf16>(a, variant, grid, s);
      break;
    case kInt8:
      launch_prefill_fmt<kInt8>(a, variant, grid, s);
      break;
    case kFp8:
      launch_prefill_fmt<kFp8>(a, variant, grid, s);
      break;
    case kF16:
      launch_prefill_fmt<kF16>(a, variant, grid, s);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_prefill_generic(const PrefillArgs &a, int total_rows, hipStream_t s) {
  if (total_rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_generic_kernel, dim3(total_rows, a.q_heads), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace llh
