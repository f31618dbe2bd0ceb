// Internal declarations shared by the HIP kernels and the host API of libllm_hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace llh {

constexpr int kFastHeadDim = 128;   // head_dim of the tuned kernels
constexpr int kD256HeadDim = 256;   // head_dim of the tuned G = 8 bf16 / fp16 decode kernels (decode256.hip)
constexpr int kD256Group = 8;        // their query heads per kv head
constexpr int kFastBlockTokens = 16;  // block_tokens of the tuned kernels
constexpr int kDecodeThreads = 256;   // 4 wavefronts
constexpr int kPrefillThreads = 256;  // 4 wavefronts, 32 query rows each
constexpr int kMatvecWaves = 8;       // wavefronts (K slices) per output-projection workgroup
constexpr int kMatvecColsMultiple = kMatvecWaves * 16;  // cols the projection kernel takes

enum KvFormat : int32_t { kBf16 = 0, kInt8 = 1, kFp8 = 2, kInt8Row = 3, kF16 = 4 };
// 16-bit element formats: bf16 and fp16 share the block layout and load paths
__host__ __device__ constexpr bool is16(int fmt) { return fmt == kBf16 || fmt == kF16; }

// int8 (per (token, head)) scales: one allocation holding, for each (block,
// head) bh and token t, the fp16 pair (K scale, V scale).  A decode lane reads
// its token's two scales with one 4-byte load and a block-head's 16 pairs are
// one 64-byte run.  The pool's V scale pointer is the K scale pointer + one
// fp16 (kInt8VScaleOffsetBytes); index of token t's scale of bh in either.
constexpr size_t kInt8VScaleOffsetBytes = 2;
__host__ __device__ constexpr size_t int8_scale_index(size_t bh, int t, int block_tokens) {
  return (bh * (size_t)block_tokens + (size_t)t) * 2;
}

// fp8 (per (block, head)) scales: one allocation holding, for each (block,
// head) bh, the f32 pair (K scale, V scale), read with one 8-byte load per
// decode unit.  The V scale pointer is the K scale pointer + one f32; index of
// bh's scale in either.
constexpr size_t kFp8VScaleOffsetBytes = 4;
__host__ __device__ constexpr size_t fp8_scale_index(size_t bh) { return bh * 2; }

// Device error flags (bit set by kernels, read back by the host).
enum ErrFlag : int32_t {
  kErrBadBlock = 1,      // block table entry outside the pool
  kErrTooManySplits = 2, // a sequence needed more split-K partials than the grid was sized for
  kErrNonFinite = 4,     // non-finite score (softmax_f32 contract)
  kErrSpan = 8,          // a sequence attends more tokens than its block-table row holds
};

struct PoolView {
  int32_t format;
  int32_t block_tokens;
  int32_t kv_heads;
  int32_t head_dim;
  int64_t n_blocks;
  const void *k;
  const void *v;
  const void *k_scales;
  const void *v_scales;
};

// Split-K decode over the tuned shape (head_dim 128, 16-token blocks).
struct DecodeArgs {
  PoolView pool;
  const uint16_t *q;        // [B][Hq][D] bf16 (D = 128, or 256 on the head_dim-256 kernel)
  uint16_t *out;            // [B][Hq][D] bf16
  const int32_t *seq_lens;  // [B]
  const int32_t *tables;    // [B][max_blocks]
  float *ws_o;              // [B][Hq][max_splits][D]
  float2 *ws_ml;            // [B][Hq][max_splits]  (running max in log2 units, sum)
  int32_t *err;             // error flags
  int32_t num_seqs;
  int32_t q_heads;
  int32_t max_blocks;
  int32_t window;
  int32_t split_blocks;     // blocks per split
  int32_t max_splits;
  int32_t stream_wgs;       // >0: persistent stream kernel over this many workgroups (split fields unused)
  int32_t max_seq_len;      // host bound on seq_lens (stream kernel: longer lengths raise kErrTooManySplits)
  int32_t *seg_desc;        // stream kernel: [B][Hkv][2] (first partial slot, partial count; 0 = written)
  float scale_log2e;        // score_scale * log2(e)
  // fused append (bf16 pools): each sequence's new token (position len - 1), [B][Hkv][128]
  // bf16, is attended from here and written to its pool slot by the wavefront that
  // computes the sequence's last block; null: plain decode
  const uint16_t *k_new;
  const uint16_t *v_new;
  const uint16_t *gate;     // null, or [B][Hq][D] bf16: out = attention * sigmoid(gate)
};

// Reference-order decode for any head_dim / block size / group size.
struct GenericDecodeArgs {
  PoolView pool;
  const void *q;            // [B][Hq][D], f32 or bf16
  void *out;                // [B][Hq][D], f32 or bf16
  const int32_t *seq_lens;  // [B] end positions (exclusive)
  const int32_t *starts;    // [B] first attended position, or null (then window rule)
  const int32_t *tables;
  float *scores;            // [B][Hq][score_stride] scratch
  int32_t *err;
  int32_t num_seqs;
  int32_t q_heads;
  int32_t max_blocks;
  int32_t window;
  int32_t ring_tokens;      // >0: position p lives in slot p % ring_tokens (ring cache mirror)
  int32_t score_stride;
  float scale;
  const uint16_t *gate;     // null, or [B][Hq][D] bf16: out = attention * sigmoid(gate)
};

struct PrefillArgs {
  PoolView pool;
  const uint16_t *q;        // [T][Hq][128]
  uint16_t *out;            // [T][Hq][128]
  const int32_t *chunk_starts;
  const int32_t *context_lens;
  const int32_t *tables;
  int32_t *err;
  int32_t num_seqs;
  int32_t q_heads;
  int32_t max_blocks;
  int32_t window;
  int32_t q_tiles;          // tiles of 128 rows per sequence in the grid
  float scale_log2e;
  float scale;              // score_scale (generic kernel)
  const uint16_t *gate;     // null, or [T][Hq][D] bf16: out = attention * sigmoid(gate)
};

struct WriteBlocksArgs {
  PoolView pool;
  void *k_dst;
  void *v_dst;
  void *ks_dst;
  void *vs_dst;
  const int32_t *blocks;    // [n]
  const uint16_t *k;        // [n][BT][Hkv][D] bf16
  const uint16_t *v;
  int32_t n;
  int32_t *err;
};

struct AppendArgs {
  PoolView pool;
  void *k_dst;
  void *v_dst;
  void *ks_dst;
  void *vs_dst;
  const int64_t *slots;     // [n] block * BT + offset, or null: row i is sequence i's new token
  const void *k;            // [n][Hkv][D], bf16 or f32
  const void *v;
  int32_t n;
  int32_t src_f32;
  int32_t *err;
  // slots == null: row i goes to position seq_lens[i] - 1 through table row i
  // (no row when seq_lens[i] <= 0), as the decode step's new token
  const int32_t *seq_lens;
  const int32_t *tables;
  int32_t max_blocks;
};

struct GatherArgs {
  PoolView pool;
  const int32_t *table;     // one sequence's row
  int32_t max_blocks;
  int32_t lo;
  int32_t hi;
  int32_t tensor;
  int32_t ring_tokens;
  int32_t out_f32;          // 1: dequantised f32 elements, 0: raw storage elements
  void *out;
  int32_t *err;
};

struct ExportArgs {
  PoolView pool;
  const int64_t *slots;     // [n] block * BT + offset
  float *k;                 // [n][Hkv][D] f32
  float *v;
  int32_t n;
  int32_t *err;
};

struct MatvecArgs {
  const uint16_t *w;        // [rows][cols] bf16, row-major
  const void *x;            // [n][ldx] bf16 or f32
  float *out;               // [n][ldo] f32
  int32_t rows;
  int32_t cols;             // multiple of kMatvecColsMultiple
  int32_t n;
  int32_t ldx;
  int32_t ldo;
  int32_t x_f32;
  int32_t ksplit;           // > 1: K split over this many workgroups, partials summed by a second launch
  float *partial;           // ksplit > 1: [ksplit][n][ldo] f32 workspace
};

// K split of the projection for a grid of about one workgroup per CU (1 = none);
// the partial workspace then holds ksplit * n * ldo floats.
int matvec_ksplit(int rows, int cols, int n, int cus);

// launchers (return hipError_t of the launch)
// `hook(user, 0, s)` runs just before and `hook(user, 1, s)` just after the main
// decode kernel is enqueued (before the merge): kernel timing records events there.
typedef void (*LaunchHook)(void *user, int phase, hipStream_t s);
hipError_t launch_decode(const DecodeArgs &a, int group, int max_seq_len, hipStream_t s, void *hook_user = nullptr,
                         LaunchHook hook = nullptr);
// head_dim 256, G = 8, bf16 pools, split-K (a.stream_wgs = 0, a.max_splits <= 64, no fused append)
hipError_t launch_decode_d256(const DecodeArgs &a, int max_seq_len, hipStream_t s, void *hook_user = nullptr,
                              LaunchHook hook = nullptr);
hipError_t launch_decode_generic(const GenericDecodeArgs &a, int q_f32, int out_f32, hipStream_t s);
// heads_per_wg: query heads of one kv head that share a workgroup's K/V tiles (1 or 2; 2 needs an even group)
// prefill kernels: one query head per workgroup, or two heads of a kv head
// sharing the K/V tiles
enum { kPrefillOneHead = 1, kPrefillTwoHeads = 2 };
hipError_t launch_prefill(const PrefillArgs &a, int variant, hipStream_t s);
// head_dim 256, bf16 pools, 16-token blocks (one query head per workgroup)
hipError_t launch_prefill_d256(const PrefillArgs &a, hipStream_t s);
constexpr int kGenericPrefillMaxDim = 512;  // head_dim bound of the generic prefill kernel
// Element-wise prefill for every other shape (any head_dim <= 512, block size,
// row alignment); total_rows = chunk_starts[num_seqs].
hipError_t launch_prefill_generic(const PrefillArgs &a, int total_rows, hipStream_t s);
hipError_t launch_write_blocks(const WriteBlocksArgs &a, hipStream_t s);
hipError_t launch_append(const AppendArgs &a, hipStream_t s);
// no new token for a sequence whose length is <= 0 (the append kernel skips its row)
constexpr int64_t kNoSlot = INT64_MIN;
hipError_t launch_gather(const GatherArgs &a, hipStream_t s);
hipError_t launch_export_rows(const ExportArgs &a, hipStream_t s);
hipError_t launch_decode_fp8(const uint8_t *codes, float *out, int32_t n, hipStream_t s);
// adds to *mismatches the f32 values (NaNs excepted) whose fp8 code from the kernels'
// encoder differs from the integer reference rule
hipError_t launch_fp8_encode_check(unsigned long long *mismatches, hipStream_t s);
hipError_t launch_matvec_bf16(const MatvecArgs &a, hipStream_t s);

}  // namespace llh
