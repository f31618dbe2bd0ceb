"""Chunked causal prefill over cached prefix blocks (MFMA) vs the oracle.

Row i of a chunk sits at position prefix + i and attends [lo, pos]: the result
of the reference's per-token "append then attend" loop
(crates/llm-backend/src/core/native_attention.rs:400-461).  At the BASELINE
sizes the oracle checks sampled rows (tile edges included) and every row is
checked against the decode kernel at that row's position (a separate kernel
with a separate reduction order); small ragged cases are checked in full.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, magnitude_rows, rows_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu

D = 128
BT = 16


def build(ctx, prefix, chunk, Hq, Hkv, window, seed, resident_from=None, fmt=llm_hip.KV_BF16):
    import torch

    ctxlen = [p + c for p, c in zip(prefix, chunk)]
    first = None if resident_from is None else [r // BT for r in resident_from]
    batch = workloads.paged_batch(ctxlen, BT, 0.10, seed, first)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, D), Hkv, D)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, D), Hkv, D)
    pool = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    starts = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q = oracle.normal_bf16(seed + 3, int(starts[-1]) * Hq * D)
    d_starts, d_lens, d_tab = to_dev(starts), to_dev(batch.seq_lens), to_dev(batch.tables)
    desc = ctx.prefill_desc(d_starts, d_lens, d_tab, Hq, max(chunk), window, total_q_rows=int(starts[-1]))
    d_q = to_dev(q)
    d_out = torch.full((int(starts[-1]) * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    scale = 1.0 / math.sqrt(D)
    ctx.paged_prefill(pool, desc, d_q, d_out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    return batch, pool, starts, q, from_dev_bf16(d_out), scale


def decode_every_row(ctx, batch, pool, starts, prefix, chunk, q, Hq, window, scale):
    """Each prefill row as one decode sequence of length pos + 1 sharing its parent's table."""
    import torch

    lens, tabs = [], []
    for b in range(len(chunk)):
        for i in range(chunk[b]):
            lens.append(prefix[b] + i + 1)
            tabs.append(batch.tables[b])
    lens = np.array(lens, np.int32)
    tabs = np.stack(tabs).astype(np.int32)
    d_lens, d_tab = to_dev(lens), to_dev(tabs)
    desc = ctx.decode_desc(d_lens, d_tab, Hq, int(lens.max()), window)
    d_out = torch.empty(lens.size * Hq * D, dtype=torch.int16, device="cuda")
    ctx.paged_decode(pool, desc, to_dev(q), d_out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    return from_dev_bf16(d_out)


def oracle_rows(pool, batch, starts, Hq, Hkv, window, q, scale, rows_per_seq, fmt=llm_hip.KV_BF16):
    opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
    out = np.zeros(int(starts[-1]) * Hq * D, np.float32)
    picked = []
    for b in range(batch.seq_lens.size):
        for r in rows_per_seq[b]:
            st = opool.prefill_rows(b, Hq, starts, batch.seq_lens, batch.tables, window, q, scale, r, r + 1, out,
                                    threads=16)
            assert st == oracle.OK
            picked.append(int(starts[b]) + r)
    return out.reshape(-1, Hq * D), picked


def sample_rows(chunk):
    base = {0, 1, 31, 32, 63, 64, 127, 128, 129, 255, 256, 383, 384, chunk - 2, chunk - 1}
    return sorted(r for r in base if 0 <= r < chunk)


@pytest.mark.parametrize("case", ["C3", "C4"])
def test_prefill_baseline_configs(ctx, case):
    if case == "C3":  # configs[2]: 8 x (1536 cached + 512 new), Hq32/Hkv4, causal in chunk
        prefix, chunk, Hq, Hkv, W, res = [1536] * 8, [512] * 8, 32, 4, 0, None
    else:  # configs[3] prefill: 4 x (31744 + 1024), window 4096, blocks before the window absent
        prefix, chunk, Hq, Hkv, W = [31744] * 4, [1024] * 4, 16, 8, 4096
        res = [31744 - W + 1] * 4
    seed = workloads.SEED_BASE + (2 if case == "C3" else 3)
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, W, seed, res)
    ref, picked = oracle_rows(pool, batch, starts, Hq, Hkv, W, q, scale, [sample_rows(c) for c in chunk])
    got = out.reshape(-1, Hq * D)
    assert_parity(got[picked], ref[picked], what=f"{case} sampled rows vs oracle")
    dec = decode_every_row(ctx, batch, pool, starts, prefix, chunk, q, Hq, W, scale)
    assert_parity(out, oracle.bf16_to_f32(dec), what=f"{case} all rows vs decode kernel")


@pytest.mark.parametrize("W", [0, 37, 200])
def test_prefill_ragged_full_oracle(ctx, W):
    prefix = [0, 17, 1000, 3, 64]
    chunk = [1, 5, 130, 300, 64]
    Hq, Hkv = 16, 8
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, W, 50 + W)
    opool = oracle.Pool.from_raw(llm_hip.KV_BF16, BT, Hkv, D, batch.n_blocks, pool.raw())
    st, ref = opool.prefill(Hq, starts, batch.seq_lens, batch.tables, W, q, scale, threads=16)
    assert st == oracle.OK
    assert_parity(out, ref, what=f"ragged W={W}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (32, 4), (16, 1), (12, 4)])
def test_prefill_gqa_groups(ctx, Hq, Hkv):
    """Groups of 1 and 3 run one query head per workgroup, even groups two."""
    prefix, chunk = [40, 0], [100, 129]
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, 0, Hq + Hkv)
    opool = oracle.Pool.from_raw(llm_hip.KV_BF16, BT, Hkv, D, batch.n_blocks, pool.raw())
    st, ref = opool.prefill(Hq, starts, batch.seq_lens, batch.tables, 0, q, scale, threads=16)
    assert st == oracle.OK
    assert_parity(out, ref, what=f"Hq={Hq} Hkv={Hkv}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_prefill_quantized_c3_shape(ctx, fmt):
    """configs[2]'s shape over int8 (fp16 scale per (token, head)) and fp8 e4m3 (f32 scale per
    (block, head)) blocks, dequantised in the tile load: sampled rows against the oracle's
    dequantise-then-attend loop, every row against the decode kernel on the same pool."""
    prefix, chunk, Hq, Hkv = [1536] * 8, [512] * 8, 32, 4
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, 0, workloads.SEED_BASE + 2 + fmt,
                                               fmt=fmt)
    ref, picked = oracle_rows(pool, batch, starts, Hq, Hkv, 0, q, scale, [sample_rows(c) for c in chunk], fmt)
    got = out.reshape(-1, Hq * D)
    assert_parity(got[picked], ref[picked], what=f"C3 fmt={fmt} sampled rows vs oracle")
    dec = decode_every_row(ctx, batch, pool, starts, prefix, chunk, q, Hq, 0, scale)
    assert_parity(out, oracle.bf16_to_f32(dec), what=f"C3 fmt={fmt} all rows vs decode kernel")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
@pytest.mark.parametrize("W", [0, 37])
def test_prefill_quantized_ragged_full_oracle(ctx, fmt, W):
    prefix = [0, 17, 1000, 3, 64]
    chunk = [1, 5, 130, 300, 64]
    Hq, Hkv = 16, 8
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, W, 70 + W + fmt, fmt=fmt)
    opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
    st, ref = opool.prefill(Hq, starts, batch.seq_lens, batch.tables, W, q, scale, threads=16)
    assert st == oracle.OK
    assert_parity(out, ref, what=f"ragged fmt={fmt} W={W}")


def build_shape(ctx, prefix, chunk, Hq, Hkv, window, seed, head_dim, bt, fmt=llm_hip.KV_BF16, misalign=False,
                q_magnitudes=False):
    """Any pool shape: the rows go in through llh_kv_write_blocks, prefill runs on q / out
    that are 2 bytes off 16-byte alignment when misalign is set (q scaled by
    helpers.magnitude_rows with q_magnitudes).  Returns the output and the oracle's."""
    import torch

    ctxlen = [p + c for p, c in zip(prefix, chunk)]
    batch = workloads.paged_batch(ctxlen, bt, 0.10, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, head_dim), Hkv,
                                      head_dim)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, head_dim), Hkv,
                                    head_dim)
    pool = ctx.pool(fmt, bt, Hkv, head_dim, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    starts = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    n = int(starts[-1]) * Hq * head_dim
    q = oracle.normal_bf16(seed + 3, n)
    if q_magnitudes:
        q = magnitude_rows(q, Hq, head_dim)
    off = 1 if misalign else 0
    qbuf = torch.zeros(n + 8, dtype=torch.int16, device="cuda")
    qbuf[off:off + n] = to_dev(q)
    obuf = torch.full((n + 8,), 0x7FC0, dtype=torch.int16, device="cuda")
    d_starts, d_lens, d_tab = to_dev(starts), to_dev(batch.seq_lens), to_dev(batch.tables)
    desc = ctx.prefill_desc(d_starts, d_lens, d_tab, Hq, max(chunk), window, total_q_rows=int(starts[-1]))
    scale = 1.0 / math.sqrt(head_dim)
    ctx.paged_prefill(pool, desc, qbuf[off:off + n], obuf[off:off + n], scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    opool = oracle.Pool.from_raw(fmt, bt, Hkv, head_dim, batch.n_blocks, pool.raw())
    st, ref = opool.prefill(Hq, starts, batch.seq_lens, batch.tables, window, q, scale, threads=16)
    assert st == oracle.OK
    return from_dev_bf16(obuf[off:off + n]), ref


@pytest.mark.parametrize("head_dim,bt,Hq,Hkv,W,fmt", [
    (256, 32, 8, 4, 0, llm_hip.KV_BF16),       # head_dim 256 on 32-token blocks
    (256, 16, 8, 4, 200, llm_hip.KV_INT8),
    (64, 32, 12, 4, 48, llm_hip.KV_BF16),      # odd group (3), 32-token blocks, window
    (96, 8, 4, 1, 0, llm_hip.KV_FP8_E4M3),     # MQA, 8-token blocks
    (128, 32, 16, 8, 0, llm_hip.KV_INT8),      # tuned head_dim, other block size
    (128, 16, 16, 8, 300, llm_hip.KV_INT8_ROW),  # the reference's int8 layout
])
def test_prefill_generic_shapes_full_oracle(ctx, head_dim, bt, Hq, Hkv, W, fmt):
    """Shapes the MFMA kernel does not take run the element-wise prefill kernel: ragged
    chunks (an empty one included) over cached prefixes, every row against the oracle."""
    before = ctx.metrics()["generic_prefill_calls"]
    out, ref = build_shape(ctx, [100, 0, 37, 5], [37, 70, 0, 130], Hq, Hkv, W, 900 + head_dim + bt, head_dim, bt, fmt)
    assert ctx.metrics()["generic_prefill_calls"] == before + 1
    assert_parity(out, ref, what=f"generic D={head_dim} bt={bt} fmt={fmt} W={W}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_prefill_unaligned_rows_take_the_generic_kernel(ctx, fmt):
    """q and out 2 bytes off 16-byte alignment on the tuned shape: the element-wise kernel
    runs and matches the oracle like the MFMA kernel."""
    before = ctx.metrics()["generic_prefill_calls"]
    out, ref = build_shape(ctx, [300, 0], [129, 64], 16, 8, 0, 77, D, BT, fmt, misalign=True)
    assert ctx.metrics()["generic_prefill_calls"] == before + 1
    assert_parity(out, ref, what=f"unaligned fmt={fmt}")


@pytest.mark.parametrize("W", [0, 300])
def test_prefill_force_generic_matches_mfma_kernel(ctx, opts, W):
    """The same call on the tuned shape through both kernels (the force-generic option):
    each within the bar of the oracle, and of each other."""
    prefix, chunk = [0, 700], [200, 333]
    fast, ref = build_shape(ctx, prefix, chunk, 16, 4, W, 41 + W, D, BT)
    opts(llm_hip.OPT_FORCE_GENERIC, 1)
    before = ctx.metrics()["generic_prefill_calls"]
    gen, ref2 = build_shape(ctx, prefix, chunk, 16, 4, W, 41 + W, D, BT)
    assert ctx.metrics()["generic_prefill_calls"] == before + 1
    assert np.array_equal(ref, ref2)
    assert_parity(fast, ref, what="mfma")
    assert_parity(gen, ref, what="generic")
    assert_parity(gen, oracle.bf16_to_f32(fast), what="generic vs mfma")


def test_prefill_query_magnitudes(ctx):
    """Query rows from bf16 subnormal to 1e30 (scores to ~1e31 in log2 units) on the MFMA
    kernel: tiles whose scaled max passes 2^26 scale their scores before the exponent
    (the fused form's rounding would overflow the weights there); every row at the bar.
    bf16 blocks (fp16 ones in test_gpu_f16.py): int8 / fp8 tiles are dequantised to bf16
    (code x scale rounded, relative error 2^-9), so at these magnitudes, where softmax is
    one-hot, a row can pick a different top key than the oracle's f32 dequantisation."""
    before = ctx.metrics()["generic_prefill_calls"]
    out, ref = build_shape(ctx, [300, 0], [200, 129], 16, 8, 0, 95, D, BT, q_magnitudes=True)
    assert ctx.metrics()["generic_prefill_calls"] == before
    assert_parity(out, ref, what="prefill query magnitudes")


def test_prefill_rejects_head_dim_beyond_generic_bound(ctx):
    import torch

    pool = ctx.pool(llm_hip.KV_BF16, BT, 1, 520, 2)
    z = torch.zeros(2, dtype=torch.int32, device="cuda")
    desc = ctx.prefill_desc(z, z[:1], z.view(1, 2), 1, 1, 0, total_q_rows=1)
    buf = torch.zeros(520, dtype=torch.int16, device="cuda")
    with pytest.raises(llm_hip.LlhError) as e:
        ctx.paged_prefill(pool, desc, buf, buf, 0.1)
    assert e.value.status == llm_hip.ERR_UNSUPPORTED


@pytest.mark.parametrize("W", [0, 300])
def test_prefill_two_heads_per_workgroup_match_one(ctx, W, opts):
    """Two query heads sharing a workgroup's K/V tiles give the same bits as one head
    per workgroup: the per-wavefront arithmetic is identical, only the tile loads are shared."""
    prefix, chunk = [0, 300, 1500], [77, 256, 512]
    opts(llm_hip.OPT_PREFILL_HEADS_PER_WG, 1)
    one = build(ctx, prefix, chunk, 16, 4, W, 60 + W)[4]
    opts(llm_hip.OPT_PREFILL_HEADS_PER_WG, 0)
    two = build(ctx, prefix, chunk, 16, 4, W, 60 + W)[4]
    assert np.array_equal(one, two)


@pytest.mark.parametrize("generic", [0, 1])
def test_prefill_span_beyond_table_row_raises_flag(ctx, opts, generic):
    """Every key from the chunk's first row to its last must be resident at once; a table
    row shorter than that span (rows are read modulo their length) raises the span flag
    instead of attending aliased blocks (both prefill kernels)."""
    import torch

    opts(llm_hip.OPT_FORCE_GENERIC, generic)

    pool = ctx.pool(llm_hip.KV_BF16, BT, 4, D, 16)
    starts = torch.tensor([0, 20], dtype=torch.int32, device="cuda")
    clens = torch.tensor([100], dtype=torch.int32, device="cuda")
    tab = torch.arange(4, dtype=torch.int32, device="cuda").view(1, 4)  # 64 tokens
    q = torch.zeros(20 * 8 * D, dtype=torch.int16, device="cuda")
    out = torch.zeros_like(q)
    ctx.paged_prefill(pool, ctx.prefill_desc(starts, clens, tab, 8, 20, 0, total_q_rows=20), q, out, 0.1)
    torch.cuda.synchronize()
    assert ctx.device_errors() & llm_hip.ERR_FLAG_SPAN
    # a window whose span (first row's window start .. context end) fits the ring is accepted
    ctx.paged_prefill(pool, ctx.prefill_desc(starts, clens, tab, 8, 20, 40, total_q_rows=20), q, out, 0.1)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
