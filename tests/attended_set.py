"""Position-coded probe of the attended set (block-table gather and masking).

With q = 0 every attended token scores exactly 0, so its softmax weight is
exactly 1 (in f32 and in bf16) and the attention output is the plain mean of
the attended value rows.  Value rows are one-hot codes of the token's absolute
position: the row of position p in kv head h is 1.0 at dim code(p, h) and 0
elsewhere, so output dim d of a query head is

    out[d] = count(attended p with code(p, h) == d) * v / n

(n = attended tokens, v = the stored value of 1.0 after quantisation).  The
integer counts are recovered from the bf16 output (count = round(out * n / v))
and compared exactly with the counts of the set the reference attends: the
sequence's positions [max(0, len - W), len) for decode, [max(0, pos - W + 1),
pos] for a prefill row at position pos (crates/llm-backend/src/core/qwen/ops/
cache.rs:116-121; crates/llm-backend/src/core/native_attention.rs:307-329,
400-461).  A dropped, duplicated or swapped block, a wrong table index, a
token masked in or out at a block edge, or a window off by one position
changes some count (tests/test_attended_set_probe.py shows each on the CPU
oracle).  Four codes, one per kv head modulo 4, each balanced over the 128
dims so that no count exceeds n / 128 for long spans:

  0: block index           (p >> 4) & 127
  1: token index           p & 127                      (offset inside the block)
  2: folded block index    ((p >> 4) ^ (p >> 11)) & 127 (tells block j from j + 128)
  3: mixed                 ((p >> 4) * 37 + (p & 15) * 11) & 127

The recovery is exact while counts stay below 128 (bf16 keeps 8 significant
bits: a count c is off by at most c * 2^-9 before rounding).
"""
from __future__ import annotations

import numpy as np

D = 128
BT = 16
ONE_BF16 = 0x3F80


def code(pos, kvh: int):
    """Dim index of the one-hot value row of position(s) pos in kv head kvh
    (numpy or torch integer arrays)."""
    c = kvh % 4
    if c == 0:
        return (pos >> 4) & 127
    if c == 1:
        return pos & 127
    if c == 2:
        return ((pos >> 4) ^ (pos >> 11)) & 127
    return ((pos >> 4) * 37 + (pos & 15) * 11) & 127


def coded_rows(lo: int, hi: int, kv_heads: int, dims: int = D, code_base: int = 0) -> np.ndarray:
    """Value rows of positions [lo, hi): uint16 bf16 [hi-lo][kv_heads][dims]; kv head h
    carries code code_base + h (modulo 4) in dims 0..127, zeros above."""
    pos = np.arange(lo, hi, dtype=np.int64)
    r = np.zeros((hi - lo, kv_heads, dims), np.uint16)
    for h in range(kv_heads):
        r[np.arange(hi - lo), h, code(pos, code_base + h)] = ONE_BF16
    return r


def counts(lo: int, hi: int, kv_heads: int, code_base: int = 0) -> np.ndarray:
    """int64 [kv_heads][128]: how many positions of [lo, hi) carry each code."""
    pos = np.arange(max(lo, 0), max(hi, lo, 0), dtype=np.int64)
    return np.stack([np.bincount(code(pos, code_base + h), minlength=D)[:D] for h in range(kv_heads)])


def prefix_counts(lo: int, hi: int, kv_heads: int, code_base: int = 0) -> np.ndarray:
    """int32 [kv_heads][hi - lo + 1][128]: counts of positions [lo, lo + i) for every i."""
    pos = np.arange(lo, hi, dtype=np.int64)
    out = np.zeros((kv_heads, hi - lo + 1, D), np.int32)
    for h in range(kv_heads):
        one_hot = np.zeros((hi - lo, D), np.int32)
        one_hot[np.arange(hi - lo), code(pos, code_base + h)] = 1
        out[h, 1:] = np.cumsum(one_hot, axis=0)
    return out


def recover(out_f32: np.ndarray, n: int, value: float) -> np.ndarray:
    """Counts from output rows [..., 128] of a set of n tokens whose stored value is `value`;
    asserts that every recovered count is unambiguous (within 0.3 of an integer)."""
    if n == 0:
        assert np.all(out_f32 == 0.0), "an empty set must give a zero output"
        return np.zeros(out_f32.shape, np.int64)
    r = out_f32.astype(np.float64) * n / value
    c = np.rint(r)
    assert np.all(np.abs(r - c) < 0.3), f"ambiguous recovery: max distance {np.abs(r - c).max():.3f}"
    return c.astype(np.int64)


def expected_decode(seq_lens, window: int, q_heads: int, kv_heads: int, code_base: int = 0):
    """(counts [B][Hq][128], n [B]) of the decode step's attended sets."""
    lens = np.asarray(seq_lens, np.int64)
    G = q_heads // kv_heads
    out = np.zeros((lens.size, q_heads, D), np.int64)
    n = np.zeros(lens.size, np.int64)
    for b, L in enumerate(lens):
        lo = max(0, int(L) - window) if window > 0 else 0
        n[b] = int(L) - lo
        c = counts(lo, int(L), kv_heads, code_base)
        out[b] = np.repeat(c, G, axis=0)
    return out, n


def check_decode(out_bf16_bits: np.ndarray, seq_lens, window: int, q_heads: int, kv_heads: int, value: float,
                 what: str = "", head_dim: int = D, code_base: int = 0) -> None:
    """Recovered counts of every (sequence, query head) equal the reference set's, exactly
    (head_dim > 128: the dims above 128, whose value rows are zero, must be exactly 0)."""
    from oracle import bf16_to_f32

    lens = np.asarray(seq_lens, np.int64)
    got = bf16_to_f32(np.ascontiguousarray(out_bf16_bits).ravel()).reshape(lens.size, q_heads, head_dim)
    if head_dim > D:
        assert np.all(got[:, :, D:] == 0.0), f"{what}: dims above {D} must be zero"
        got = got[:, :, :D]
    exp, n = expected_decode(lens, window, q_heads, kv_heads, code_base)
    for b in range(lens.size):
        rec = recover(got[b], int(n[b]), value)
        if not np.array_equal(rec, exp[b]):
            h = int(np.argwhere(np.any(rec != exp[b], axis=1))[0][0])
            d = np.flatnonzero(rec[h] != exp[b][h])[:4]
            raise AssertionError(f"{what}: attended set differs for sequence {b} (len {int(lens[b])}), q head {h}: "
                                 f"dims {d.tolist()} counts {rec[h][d].tolist()} expected {exp[b][h][d].tolist()}")


def check_prefill(out_bf16_bits: np.ndarray, chunk_starts, context_lens, window: int, q_heads: int, kv_heads: int,
                  value: float, what: str = "", head_dim: int = D, code_base: int = 0) -> None:
    """Every chunk row's recovered counts equal those of [lo(pos), pos], exactly (head_dim >
    128: the dims above 128, whose value rows are zero, must be exactly 0)."""
    from oracle import bf16_to_f32

    cs = np.asarray(chunk_starts, np.int64)
    cl = np.asarray(context_lens, np.int64)
    G = q_heads // kv_heads
    got = bf16_to_f32(np.ascontiguousarray(out_bf16_bits).ravel()).reshape(int(cs[-1]), q_heads, head_dim)
    if head_dim > D:
        assert np.all(got[:, :, D:] == 0.0), f"{what}: dims above {D} must be zero"
        got = got[:, :, :D]
    for b in range(cl.size):
        chunk = int(cs[b + 1] - cs[b])
        if chunk == 0:
            continue
        pos = int(cl[b]) - chunk + np.arange(chunk)
        lo = np.maximum(0, pos - window + 1) if window > 0 else np.zeros_like(pos)
        base = int(lo.min())
        pc = prefix_counts(base, int(pos.max()) + 1, kv_heads, code_base)  # [Hkv][span + 1][128]
        exp = pc[:, pos + 1 - base] - pc[:, lo - base]          # [Hkv][chunk][128]
        n = (pos + 1 - lo).astype(np.float64)
        rows = got[cs[b]:cs[b + 1]].astype(np.float64)           # [chunk][Hq][128]
        for h in range(q_heads):
            r = rows[:, h, :] * n[:, None] / value
            c = np.rint(r)
            assert np.all(np.abs(r - c) < 0.3), f"{what}: ambiguous recovery, sequence {b} head {h}"
            bad = np.argwhere(c.astype(np.int64) != exp[h // G])
            if bad.size:
                i, d = (int(x) for x in bad[0])
                raise AssertionError(f"{what}: attended set differs for sequence {b}, row {i} (position {pos[i]}), "
                                     f"q head {h}, dim {d}: count {int(c[i, d])} expected {int(exp[h // G][i, d])}")
