"""Per-step descriptors for the BASELINE workloads (host side, numpy).

The reference has no batched step descriptor: its scheduler admits one request
per backend call (crates/llm-server/src/engine/scheduler.rs:579-712).  These
helpers build what the device kernels consume: int32 block tables into one
shared block pool, per-sequence lengths, and the token-major source blocks
that llh_kv_write_blocks quantises into the pool.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

SEED_BASE = 0x6B69722D00  # "kir-" + config index


@dataclass
class PagedBatch:
    seq_lens: np.ndarray      # int32 [B] context tokens (incl. the new token for decode)
    tables: np.ndarray        # int32 [B][max_blocks] pool block indices
    n_blocks: int             # pool size
    block_tokens: int
    first_block: np.ndarray   # int32 [B] first logical block resident in the pool (window skipping)

    @property
    def max_blocks(self) -> int:
        return int(self.tables.shape[1])


def paged_batch(seq_lens, block_tokens: int = 16, free_frac: float = 0.10, seed: int = 0,
                resident_from=None) -> PagedBatch:
    """Block tables that are a seeded random permutation of one shared pool.

    The pool holds ceil((1 + free_frac) * total_blocks) blocks; sequence b owns
    ceil(len_b / block_tokens) of them, taken in permuted order.  When
    `resident_from[b]` is given, logical blocks before it are not backed by the
    pool (their table entries are -1): the kernels must never touch them.
    """
    lens = np.asarray(seq_lens, dtype=np.int64)
    nblk = (lens + block_tokens - 1) // block_tokens
    first = np.zeros(lens.size, dtype=np.int64) if resident_from is None else np.asarray(resident_from, np.int64)
    need = int(np.sum(np.maximum(nblk - first, 0)))
    n_pool = max(1, int(np.ceil((1.0 + free_frac) * need)))
    rng = np.random.Generator(np.random.PCG64(seed))
    perm = rng.permutation(n_pool).astype(np.int32)
    max_blocks = max(1, int(nblk.max()) if lens.size else 1)
    tables = np.full((lens.size, max_blocks), -1, dtype=np.int32)
    cur = 0
    for b in range(lens.size):
        k = int(max(nblk[b] - first[b], 0))
        tables[b, first[b]:first[b] + k] = perm[cur:cur + k]
        cur += k
    return PagedBatch(lens.astype(np.int32), tables, n_pool, block_tokens, first.astype(np.int32))


def uniform_lengths(n: int, lo: int, hi: int, seed: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(lo, hi + 1, size=n).astype(np.int32)


def block_sources(batch: PagedBatch, rows_fn, kv_heads: int, head_dim: int):
    """Token-major source blocks for llh_kv_write_blocks.

    rows_fn(b, lo, hi) -> uint16/array [hi-lo][kv_heads][head_dim] rows of
    sequence b.  Returns (block_ids int32 [n], src [n][BT][Hkv][D]) covering every
    resident block; tokens past a sequence's length are zero."""
    bt = batch.block_tokens
    ids, chunks = [], []
    for b in range(batch.seq_lens.size):
        L = int(batch.seq_lens[b])
        for j in range(int(batch.first_block[b]), (L + bt - 1) // bt):
            blk = int(batch.tables[b, j])
            lo, hi = j * bt, min(L, (j + 1) * bt)
            src = np.zeros((bt, kv_heads, head_dim), dtype=np.uint16)
            src[: hi - lo] = rows_fn(b, lo, hi)
            ids.append(blk)
            chunks.append(src)
    if not ids:
        return np.zeros(0, np.int32), np.zeros((0, bt, kv_heads, head_dim), np.uint16)
    return np.asarray(ids, dtype=np.int32), np.stack(chunks)
