"""The head_dim-256 MFMA prefill kernel (prefill256.hip): Qwen3.5 / 3.6 full-attention
layers (fixtures/qwen36/config.json: 16 query heads, 2 kv heads, head_dim 256), bf16 blocks
of 16 tokens.  Every row of ragged chunks over cached prefixes against the oracle (the
per-token append-then-attend of crates/llm-backend/src/core/native_attention.rs:356-464,
head_dim from the call), with and without a window and the output gate
(native_attention.rs:765-781); the attended set of every row bit-exactly with the
position-coded probe (tests/attended_set.py)."""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from attended_set import check_prefill, coded_rows
from helpers import assert_parity, from_dev_bf16, magnitude_rows, rows_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu

D = 256
BT = 16
HQ, HKV = 16, 2


def run(ctx, prefix, chunk, window, seed, gate=False, coded=False, q_magnitudes=False, fmt=llm_hip.KV_BF16):
    """Prefill of `chunk` rows after `prefix` cached ones per sequence; returns (out, ref) with
    ref None for the coded probe (q = 0, V one-hot position codes); q scaled by
    helpers.magnitude_rows with q_magnitudes; fmt: the pool's element type (bf16 or fp16,
    the rows rounded to it on write)."""
    import torch

    ctxlen = [p + c for p, c in zip(prefix, chunk)]
    batch = workloads.paged_batch(ctxlen, BT, 0.10, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, HKV, D), HKV, D)
    if coded:
        _, sv = workloads.block_sources(batch, lambda b, lo, hi: coded_rows(lo, hi, HKV, D, 2), HKV, D)
    else:
        _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, HKV, D), HKV, D)
    pool = ctx.pool(fmt, BT, HKV, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    starts = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    T = int(starts[-1])
    q = np.zeros(T * HQ * D, np.uint16) if coded else oracle.normal_bf16(seed + 3, T * HQ * D)
    if q_magnitudes:
        q = magnitude_rows(q, HQ, D)
    g = oracle.f32_to_bf16(oracle.bf16_to_f32(oracle.normal_bf16(seed + 4, T * HQ * D)) * np.float32(2.0)) \
        if gate else None
    out = torch.full((T * HQ * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    desc = ctx.prefill_desc(to_dev(starts), to_dev(batch.seq_lens), to_dev(batch.tables), HQ, max(chunk), window,
                            total_q_rows=T, gate=to_dev(g) if gate else None)
    scale = 1.0 / math.sqrt(D)
    before = ctx.metrics()["generic_prefill_calls"]
    ctx.paged_prefill(pool, desc, to_dev(q), out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    assert ctx.metrics()["generic_prefill_calls"] == before, "the element-wise kernel ran"
    if coded:
        return from_dev_bf16(out), (starts, batch.seq_lens)
    opool = oracle.Pool.from_raw(fmt, BT, HKV, D, batch.n_blocks, pool.raw())
    st, ref = opool.prefill(HQ, starts, batch.seq_lens, batch.tables, window, q, scale, threads=16)
    assert st == oracle.OK
    if gate:
        ref = oracle.apply_gate(ref, oracle.bf16_to_f32(g))
    return from_dev_bf16(out), ref


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_F16])
@pytest.mark.parametrize("window", [0, 90])
def test_prefill256_ragged_full_oracle(ctx, window, fmt):
    """Ragged chunks (an empty one, one of a single row, one past a tile) over prefixes of
    0 .. 1536 tokens, every row against the oracle; bf16 and fp16 pools (fp16: both products
    on the fp16 MFMA, each query row scaled into fp16 by its own power of two)."""
    out, ref = run(ctx, [0, 300, 1000, 1536, 7], [130, 64, 257, 17, 0], window, 41 + window, fmt=fmt)
    assert_parity(out, ref, what=f"prefill d256 W={window} fmt={fmt}")


@pytest.mark.parametrize("window", [0, 64])
def test_prefill256_tile_boundaries(ctx, window):
    """Chunk lengths either side of a wavefront's 16 rows and a workgroup's 128 (1, 15, 16,
    127, 128, 129, 255: wavefronts with no rows, partly filled workgroups) over prefixes
    either side of a 64-key tile (63, 64, 65, 0, 1, 127, 16), every row against the oracle."""
    out, ref = run(ctx, [63, 64, 65, 0, 1, 127, 16], [1, 15, 16, 127, 128, 129, 255], window, 47 + window)
    assert_parity(out, ref, what=f"prefill d256 tile boundaries W={window}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_F16])
def test_prefill256_query_magnitudes(ctx, fmt):
    """Query rows from bf16 subnormal to 1e30 (scores to ~1e31 in log2 units): tiles whose
    scaled max passes 2^26 scale their scores before the exponent; over fp16 blocks each row's
    power-of-two scaling keeps q in fp16's range."""
    out, ref = run(ctx, [300, 0], [200, 129], 0, 95, q_magnitudes=True, fmt=fmt)
    assert_parity(out, ref, what=f"prefill d256 query magnitudes fmt={fmt}")


def test_prefill256_qwen36_chunk(ctx):
    """A Qwen3.6-shaped chunk: 2 sequences of a 1536-token prefix + a 512-token chunk."""
    out, ref = run(ctx, [1536, 1536], [512, 512], 0, 43)
    assert_parity(out, ref, what="prefill d256 1536+512")


@pytest.mark.parametrize("window", [0, 300])
def test_prefill256_gate(ctx, window):
    out, ref = run(ctx, [100, 333], [70, 130], window, 44, gate=True)
    assert_parity(out, ref, what=f"gated prefill d256 W={window}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_F16])
@pytest.mark.parametrize("window", [0, 1, 17, 100])
def test_prefill256_attended_set(ctx, window, fmt):
    out, (starts, lens) = run(ctx, [100, 1000, 0], [37, 200, 129], window, 45, coded=True, fmt=fmt)
    check_prefill(out, starts, lens, window, HQ, HKV, 1.0, f"prefill d256 W={window}", head_dim=D, code_base=2)
