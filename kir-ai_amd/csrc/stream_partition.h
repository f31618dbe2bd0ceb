// The persistent stream partition of a decode step, shared by the head_dim-128
// and head_dim-256 stream kernels: a step's units (sequence, kv head, attended
// block) in that order, cut into equal consecutive ranges, one per wavefront;
// the wavefront's cursors walk its range.  Every function is a pure function of
// the step's lengths, computed by every wavefront alike.
#pragma once

#include "device_common.h"

namespace llh {

__device__ __forceinline__ int attended_blocks(const DecodeArgs &a, int len) {
  const int lo = a.window > 0 ? max(0, len - a.window) : 0;
  return len > lo ? (len - 1) / kFastBlockTokens - lo / kFastBlockTokens + 1 : 0;
}

// Inclusive prefix sum over the wavefront in the VALU (DPP, no LDS round trip):
// a Hillis-Steele scan inside each 16-lane row (row_shr 1, 2, 4, 8), then row
// 15's last lane added to rows 1 and 3 and lane 31 to rows 2 and 3 (row_bcast).
// Lanes whose source is outside the row, and rows outside the row mask, add 0.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

__device__ __forceinline__ int wave_sum(int v) { return __builtin_amdgcn_readlane(wave_incl_scan(v), 63); }

// floor(x / d) for x < 2^63, d > 0: 32-bit division when x fits (the usual
// case; a 64-bit division is several times longer and sits on the path to the
// first load)
__device__ __forceinline__ int div_u64(unsigned long long x, unsigned d) {
  return (int)((x >> 32) == 0 ? (unsigned)x / d : x / d);
}

// First global unit of wavefront omega's range [omega * U / W, (omega + 1) * U / W).
__device__ __forceinline__ int range_begin(int omega, int U, int W) {
  return div_u64((unsigned long long)omega * (unsigned)U, (unsigned)W);
}

// The wavefront whose range holds global unit r.
__device__ __forceinline__ int wave_of_unit(int r, int U, int W) {
  return div_u64((unsigned long long)(r + 1) * (unsigned)W + (unsigned)U - 1u, (unsigned)U) - 1;
}

// Attended tokens of a sequence of length len.
__device__ __forceinline__ int attended_tokens(const DecodeArgs &a, int len) {
  return a.window > 0 ? min(len, a.window) : len;
}

// This wavefront's share of the step, a pure function of seq_lens that every
// wavefront computes (lane l of a 64-sequence chunk reads sequence l; len0 is
// chunk 0, already loaded).  The ranges are cut for Wu = min(W, U) wavefronts,
// so that every range is non-empty and the pieces of a cut segment lie in
// consecutive wavefronts (the merge reads them so); wavefronts w >= Wu idle.
struct StreamRange {
  int U;     // units of the step
  int Wu;    // wavefronts that take units
  int r0;    // first global unit of the range
  int n;     // units in the range (0: none)
  int b;     // sequence of unit r0
  int base;  // global index of that sequence's first unit
};

// Sets *bad_flags to kErrTooManySplits when a length exceeds the host's
// max_seq_len bound and to kErrSpan when a sequence attends more tokens than
// its table row holds (then n = 0).
__device__ __forceinline__ StreamRange stream_range(const DecodeArgs &a, int W, int w, int lane, int len0,
                                                    int *bad_flags) {
  const int B = a.num_seqs;
  const int Hkv = a.pool.kv_heads;
  const int row_tokens = a.max_blocks * kFastBlockTokens;
  int blocks = 0;
  bool too_long = false, span = false;
  for (int cb = 0; cb < B; cb += 64) {
    const int len = cb == 0 ? len0 : (cb + lane < B ? a.seq_lens[cb + lane] : 0);
    blocks += wave_sum(attended_blocks(a, len));
    too_long |= __ballot(len > a.max_seq_len) != 0;
    span |= __ballot(attended_tokens(a, len) > row_tokens) != 0;
  }
  *bad_flags = (too_long ? kErrTooManySplits : 0) | (span ? kErrSpan : 0);
  StreamRange r = {blocks * Hkv, min(W, blocks * Hkv), 0, 0, -1, 0};
  if (*bad_flags || r.U == 0 || w >= r.Wu) return r;
  r.r0 = range_begin(w, r.U, r.Wu);
  r.n = range_begin(w + 1, r.U, r.Wu) - r.r0;
  // the sequence whose units hold r0: inclusive scan of units per sequence
  int before = 0;  // units of the chunks already scanned
  for (int cb = 0; cb < B; cb += 64) {
    const int len = cb == 0 ? len0 : (cb + lane < B ? a.seq_lens[cb + lane] : 0);
    const int ub = Hkv * attended_blocks(a, len);
    const int incl = before + wave_incl_scan(ub);
    const unsigned long long hit = __ballot(r.r0 >= incl - ub && r.r0 < incl);
    if (hit) {
      const int src = __ffsll((long long)hit) - 1;
      r.b = cb + src;
      r.base = __builtin_amdgcn_readlane(incl - ub, src);
      return r;
    }
    before = __builtin_amdgcn_readlane(incl, 63);
  }
  r.n = 0;  // not reached: r0 < U lies in some sequence
  return r;
}

// A position in the stream order (all fields wave-uniform): sequence b, kv
// head kvh, attended block j of the sequence's nb; base is the global index of
// (b, 0, 0) and tab the block-table index of block j.
struct UnitCursor {
  int b, kvh, j, nb;
  int len, lo;     // the sequence's length and first attended position
  int tab, tab0;   // table index of block j and of block 0: (lo / kFastBlockTokens + j) % max_blocks
  int base;
};

// Lengths and block-table entries as scalar loads (constant address space: no one
// writes them during the launch), so the waits before the math cover K/V loads only.
typedef const __attribute__((address_space(4))) int32_t stream_const_i32;

// Sets c to sequence b: its length from len0's lanes (sequences 0..63, one per
// lane) or a scalar load, its attended blocks and the table index of its first.
__device__ __forceinline__ void cursor_set_seq(const DecodeArgs &a, int len0, UnitCursor &c, int b) {
  c.b = b;
  c.len = b < 64 ? __builtin_amdgcn_readlane(len0, b) : ((const stream_const_i32 *)a.seq_lens)[b];
  c.nb = attended_blocks(a, c.len);
  c.lo = a.window > 0 ? max(0, c.len - a.window) : 0;
  c.tab0 = (c.lo / kFastBlockTokens) % a.max_blocks;
}

// The next unit in stream order; past the last sequence nb stays 0 and nothing is read.
__device__ __forceinline__ void cursor_advance(const DecodeArgs &a, int len0, UnitCursor &c) {
  if (++c.j < c.nb) {
    if (++c.tab == a.max_blocks) c.tab = 0;
    return;
  }
  c.j = 0;
  c.tab = c.tab0;
  if (++c.kvh < a.pool.kv_heads) return;
  c.kvh = 0;
  c.base += a.pool.kv_heads * c.nb;
  for (;;) {
    if (++c.b >= a.num_seqs) {
      c.nb = 0;
      return;
    }
    cursor_set_seq(a, len0, c, c.b);
    if (c.nb > 0) {
      c.tab = c.tab0;
      return;
    }
  }
}

// The cursor at the first unit of a wavefront's range.
__device__ __forceinline__ UnitCursor cursor_at(const DecodeArgs &a, int len0, const StreamRange &sr) {
  UnitCursor c;
  cursor_set_seq(a, len0, c, __builtin_amdgcn_readfirstlane(sr.b));
  c.base = __builtin_amdgcn_readfirstlane(sr.base);
  const int u = __builtin_amdgcn_readfirstlane(sr.r0) - c.base;
  c.kvh = u / c.nb;
  c.j = u - c.kvh * c.nb;
  c.tab = c.tab0 + c.j;
  if (c.tab >= a.max_blocks) c.tab -= a.max_blocks;
  return c;
}

}  // namespace llh
