"""Block-table gather and masking of the hot kernels, exactly (the position-coded probe
of tests/attended_set.py): q = 0 gives every attended token weight exactly 1, value
rows are one-hot codes of their absolute position, and the integer counts recovered
from each output row must equal those of the set the reference attends --
[max(0, len - W), len) for decode (native_attention.rs:307-329 with the window of
qwen/ops/cache.rs:116-121), [max(0, pos - W + 1), pos] for a prefill row
(native_attention.rs:400-461).  tests/test_attended_set_probe.py shows on the CPU
oracle that a dropped or duplicated block, the edge block swapped, a window off by
one and a token past the end each fail this comparison.

Covered: both tuned decode kernels on C2 at full size and on window edges (W = 1, 17,
100, 4096), C4 decode, the full C5 launch (int8 and fp8, all 64 sequences), a window
ring of exactly W/16 blocks, the fused append (bf16, both kernels) and the quantised
and fp16 append-then-attend, the allocation-free entry point, C3 and C4 prefill at full
size (bf16, int8, fp8, fp16 blocks), fp16 pools under windows, and the element-wise
decode and prefill kernels.  Slots past
a sequence's end and before its window hold codes of their own positions, so
attending any of them changes a count.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from attended_set import BT, D, check_decode, check_prefill, code
from helpers import from_dev_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu


def stored_one(fmt: int) -> float:
    """The value a 1.0 in a row whose absmax is 1 reads back as from a pool of this format
    (the oracle's own quantisers)."""
    row = np.zeros(D, np.float32)
    row[0] = 1.0
    if fmt == llm_hip.KV_INT8:
        st, codes, s16 = oracle.quantize_int8_head(row)
        assert st == oracle.OK
        return float(codes[0]) * float(np.array([s16], np.uint16).view(np.float16)[0])
    if fmt == llm_hip.KV_FP8_E4M3:
        st, codes, s = oracle.quantize_fp8_block(np.tile(row, BT))
        assert st == oracle.OK
        return float(oracle.fp8_decode_table()[codes[0]]) * s
    return 1.0


def resident_blocks(batch):
    """(logical block index, pool block) of every block the tables hold for the sequences."""
    js, blks = [], []
    for b in range(batch.seq_lens.size):
        L = int(batch.seq_lens[b])
        j = np.arange(int(batch.first_block[b]), (L + BT - 1) // BT)
        js.append(j)
        blks.append(batch.tables[b, j % batch.max_blocks])
    if not js:
        return np.zeros(0, np.int64), np.zeros(0, np.int32)
    return np.concatenate(js).astype(np.int64), np.concatenate(blks).astype(np.int32)


def coded_pool(ctx, batch, Hkv, fmt, seed):
    """A pool whose value rows are the position codes (every slot of every resident block,
    past-the-end slots included); keys N(0,1).  Built on the device."""
    import torch

    pool = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
    J, BLK = resident_blocks(batch)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dJ, dB = torch.from_numpy(J).cuda(), torch.from_numpy(BLK).cuda()
    t = torch.arange(BT, device="cuda")
    for s in range(0, J.size, 4096):
        j = dJ[s:s + 4096]
        n = j.numel()
        pos = j[:, None] * BT + t[None, :]
        v = torch.zeros((n, BT, Hkv, D), dtype=torch.bfloat16, device="cuda")
        ii = torch.arange(n, device="cuda")[:, None].expand(n, BT)
        tt = t[None, :].expand(n, BT)
        for h in range(Hkv):
            v[ii, tt, h, code(pos, h)] = 1.0
        k = torch.randn((n, BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        ctx.write_blocks(pool, dB[s:s + 4096], k, v)
    torch.cuda.synchronize()
    return pool


def decode_q0(ctx, pool, batch, Hq, window, noalloc=False):
    import torch

    B = batch.seq_lens.size
    q = torch.zeros(B * Hq * D, dtype=torch.int16, device="cuda")
    out = torch.full((B * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(batch.seq_lens.max()), window)
    if noalloc:
        ctx.paged_decode_noalloc(pool, desc, q, out, 0.125)
    else:
        ctx.paged_decode(pool, desc, q, out, 0.125)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    return from_dev_bf16(out)


@pytest.fixture(params=["split", "stream"])
def decode_kernel(request, opts):
    opts(llm_hip.OPT_DECODE_KERNEL, request.param)
    return request.param


def test_decode_c2_attended_set(ctx, decode_kernel):
    """configs[1] at full size: every (sequence, head) of the step attends exactly [0, len)."""
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    batch = workloads.paged_batch(lens, BT, 0.10, workloads.SEED_BASE + 1)
    pool = coded_pool(ctx, batch, 8, llm_hip.KV_BF16, 1)
    check_decode(decode_q0(ctx, pool, batch, 16, 0), lens, 0, 16, 8, 1.0, f"C2 {decode_kernel}")


@pytest.mark.parametrize("W", [1, 17, 100, 4096])
def test_decode_window_edges_attended_set(ctx, decode_kernel, W):
    """Windows cutting blocks at every offset: lengths around block edges and the window."""
    lens = np.array([1, 5, 16, 17, 40, 99, 100, 101, 333, 4096, 4097, 4111, 5000], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=W)
    pool = coded_pool(ctx, batch, 8, llm_hip.KV_BF16, W)
    check_decode(decode_q0(ctx, pool, batch, 16, W), lens, W, 16, 8, 1.0, f"W={W} {decode_kernel}")


def test_decode_c4_attended_set(ctx, decode_kernel):
    """configs[3] decode: 4 x 32768 positions, window 4096; blocks before the window are
    absent from the pool (-1), the window's first block is partly masked."""
    L, W = 32768, 4096
    lens = np.array([L, L - 7, L - 16, L - 9], np.int32)
    first = [(int(x) - W) // BT for x in lens]
    batch = workloads.paged_batch(lens, BT, 0.10, workloads.SEED_BASE + 3, resident_from=first)
    pool = coded_pool(ctx, batch, 8, llm_hip.KV_BF16, 3)
    check_decode(decode_q0(ctx, pool, batch, 16, W), lens, W, 16, 8, 1.0, f"C4 {decode_kernel}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_c5_full_launch_attended_set(ctx, opts, fmt):
    """configs[4] as bench.py launches it: 64 x 8192 tokens, Hq32/Hkv8, one stream launch;
    all 64 sequences checked."""
    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    B, L = 64, 8192
    batch = workloads.paged_batch([L] * B, BT, 0.0, workloads.SEED_BASE + 4)
    pool = coded_pool(ctx, batch, 8, fmt, 4)
    before = ctx.metrics()["stream_decode_calls"]
    out = decode_q0(ctx, pool, batch, 32, 0)
    assert ctx.metrics()["stream_decode_calls"] == before + 1
    check_decode(out, batch.seq_lens, 0, 32, 8, stored_one(fmt), f"C5 fmt={fmt}")
    pool.close()


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3, llm_hip.KV_F16])
def test_decode_quantized_windows_attended_set(ctx, decode_kernel, fmt):
    lens = np.array([1, 17, 250, 1025, 3000], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=fmt + 70)
    pool = coded_pool(ctx, batch, 8, fmt, fmt)
    for W in (0, 17, 333):
        check_decode(decode_q0(ctx, pool, batch, 32, W), lens, W, 32, 8, stored_one(fmt),
                     f"fmt={fmt} W={W} {decode_kernel}")


def test_decode_ring_of_exactly_window_blocks_attended_set(ctx, decode_kernel):
    """A window served by a ring of W/16 blocks: position p in table[(p / 16) % (W / 16)].
    The ring holds the window's positions, written by appends in position order (older
    passes round the ring overwritten), and each sequence attends exactly its window."""
    import torch

    W, nb, Hq, Hkv = 64, 4, 16, 8
    lens = np.array([1000, 77, 64, 65, 7, 129], np.int32)
    B = lens.size
    n_pool = 29  # prime: the entries i * 3 + 1 (mod 29) of the B * nb = 24 table slots are distinct
    tables = (np.arange(B * nb, dtype=np.int32).reshape(B, nb) * 3 + 1) % n_pool
    assert np.unique(tables).size == B * nb
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, n_pool)
    # two calls, older positions first: one call must not hold two tokens of one slot
    for older in (True, False):
        slots, ks, vs = [], [], []
        for b in range(B):
            L = int(lens[b])
            rng = range(max(0, L - W - 20), max(0, L - W)) if older else range(max(0, L - W), L)
            for p in rng:
                slots.append(int(tables[b, (p // BT) % nb]) * BT + p % BT)
                ks.append(oracle.normal_bf16(b, Hkv * D, p * Hkv * D).reshape(Hkv, D))
                v = np.zeros((Hkv, D), np.uint16)
                for h in range(Hkv):
                    v[h, code(np.int64(p), h)] = 0x3F80
                vs.append(v)
        ctx.append(pool, to_dev(np.array(slots, np.int64)), to_dev(np.stack(ks)), to_dev(np.stack(vs)))
    torch.cuda.synchronize()
    batch = workloads.PagedBatch(lens, tables, n_pool, BT, np.zeros(B, np.int32))
    check_decode(decode_q0(ctx, pool, batch, Hq, W), lens, W, Hq, Hkv, 1.0, f"ring {decode_kernel}")


def test_decode_noalloc_attended_set(ctx):
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    batch = workloads.paged_batch(lens, BT, 0.10, 5)
    pool = coded_pool(ctx, batch, 8, llm_hip.KV_BF16, 5)
    for W in (0, 1000):
        check_decode(decode_q0(ctx, pool, batch, 16, W, noalloc=True), lens, W, 16, 8, 1.0, f"noalloc W={W}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_F16])
def test_decode_element_wise_kernel_attended_set(ctx, opts, fmt):
    opts(llm_hip.OPT_FORCE_GENERIC, 1)
    lens = np.array([1, 17, 250, 1025], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=90 + fmt)
    pool = coded_pool(ctx, batch, 8, fmt, 90)
    for W in (0, 100):
        check_decode(decode_q0(ctx, pool, batch, 16, W), lens, W, 16, 8, stored_one(fmt), f"generic W={W}")


# ---- the fused append: the new token (position len - 1) comes from the call's rows ----------------

def coded_new_rows(lens, Hkv):
    """The new token of each sequence: its code at position len - 1 (zeros for empty ones)."""
    v = np.zeros((lens.size, Hkv, D), np.uint16)
    for b, L in enumerate(lens):
        if L > 0:
            for h in range(Hkv):
                v[b, h, code(np.int64(L - 1), h)] = 0x3F80
    return v


def decoy_last_slots(ctx, pool, batch, Hkv):
    """Overwrites the pool slot of position len - 1 with a decoy code (its code + 64): a
    kernel attending the stale slot instead of the call's new row is caught."""
    import torch

    lens = batch.seq_lens.astype(np.int64)
    live = lens > 0
    pos = lens[live] - 1
    blk = batch.tables[np.flatnonzero(live), (pos // BT) % batch.max_blocks].astype(np.int64)
    v = np.zeros((pos.size, Hkv, D), np.uint16)
    for i, p in enumerate(pos):
        for h in range(Hkv):
            v[i, h, (code(np.int64(p), h) + 64) % D] = 0x3F80
    k = oracle.normal_bf16(77, pos.size * Hkv * D).reshape(pos.size, Hkv, D)
    ctx.append(pool, to_dev(blk * BT + pos % BT), to_dev(k), to_dev(v))
    torch.cuda.synchronize()


@pytest.mark.parametrize("window", [0, 1000])
@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3, llm_hip.KV_F16])
def test_decode_append_attended_set(ctx, decode_kernel, fmt, window):
    """llh_paged_decode_append: the step attends [lo, len - 1) from the pool plus the new
    token from the call's rows (never the stale slot), and leaves that token in the slot."""
    import torch

    Hq, Hkv = 16, 8
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    lens[:6] = [1, 16, 17, 32, 33, 4096]
    free = 0.10
    batch = workloads.paged_batch(lens, BT, free, 5 + window)
    pool = coded_pool(ctx, batch, Hkv, fmt, 6)
    decoy_last_slots(ctx, pool, batch, Hkv)
    B = lens.size
    kn = oracle.normal_bf16(78, B * Hkv * D).reshape(B, Hkv, D)
    vn = coded_new_rows(lens, Hkv)
    q = torch.zeros(B * Hq * D, dtype=torch.int16, device="cuda")
    out = torch.full((B * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    desc = ctx.decode_desc(to_dev(lens), to_dev(batch.tables), Hq, int(lens.max()), window)
    ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), q, out, 0.125)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    one = stored_one(fmt)
    check_decode(from_dev_bf16(out), lens, window, Hq, Hkv, one, f"fused fmt={fmt} W={window} {decode_kernel}")
    # the slot now holds the new token: a plain decode over the pool attends the same set
    check_decode(decode_q0(ctx, pool, batch, Hq, window), lens, window, Hq, Hkv, one, "decode after the append")


# ---- prefill ------------------------------------------------------------------------------------

def prefill_q0(ctx, pool, batch, chunks, Hq, window):
    import torch

    starts = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    T = int(starts[-1])
    q = torch.zeros(T * Hq * D, dtype=torch.int16, device="cuda")
    out = torch.full((T * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    desc = ctx.prefill_desc(to_dev(starts), to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(max(chunks)), window,
                            total_q_rows=T)
    ctx.paged_prefill(pool, desc, q, out, 0.125)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    return from_dev_bf16(out), starts


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3, llm_hip.KV_F16])
def test_prefill_c3_attended_set(ctx, fmt):
    """configs[2] at full size: 8 x (1536 cached + 512 new), Hq32/Hkv4; every row of every
    sequence attends exactly [0, pos]."""
    B, prefix, chunk = 8, 1536, 512
    batch = workloads.paged_batch([prefix + chunk] * B, BT, 0.10, workloads.SEED_BASE + 2)
    pool = coded_pool(ctx, batch, 4, fmt, 2)
    out, starts = prefill_q0(ctx, pool, batch, [chunk] * B, 32, 0)
    check_prefill(out, starts, batch.seq_lens, 0, 32, 4, stored_one(fmt), f"C3 fmt={fmt}")


def test_prefill_c4_attended_set(ctx):
    """configs[3] prefill: 4 x (31744 + 1024) with window 4096; blocks before the earliest
    row's window are absent (-1); every row attends exactly [pos - 4095, pos]."""
    B, prefix, chunk, W = 4, 31744, 1024, 4096
    res = (prefix - W) // BT
    batch = workloads.paged_batch([prefix + chunk] * B, BT, 0.10, workloads.SEED_BASE + 3, resident_from=[res] * B)
    pool = coded_pool(ctx, batch, 8, llm_hip.KV_BF16, 3)
    out, starts = prefill_q0(ctx, pool, batch, [chunk] * B, 16, W)
    check_prefill(out, starts, batch.seq_lens, W, 16, 8, 1.0, "C4 prefill")


@pytest.mark.parametrize("W", [0, 1, 17, 100])
def test_prefill_ragged_chunks_attended_set(ctx, W):
    """Chunks of 1, 5, 64, 130 and 300 rows at prefixes around block edges."""
    prefix = [0, 15, 16, 100, 333]
    chunks = [1, 5, 64, 130, 300]
    batch = workloads.paged_batch([p + c for p, c in zip(prefix, chunks)], BT, 0.10, seed=W + 200)
    pool = coded_pool(ctx, batch, 4, llm_hip.KV_BF16, W)
    out, starts = prefill_q0(ctx, pool, batch, chunks, 8, W)
    check_prefill(out, starts, batch.seq_lens, W, 8, 4, 1.0, f"ragged W={W}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_prefill_element_wise_kernel_attended_set(ctx, opts, fmt):
    opts(llm_hip.OPT_FORCE_GENERIC, 1)
    prefix = [0, 17, 200]
    chunks = [20, 33, 70]
    batch = workloads.paged_batch([p + c for p, c in zip(prefix, chunks)], BT, 0.10, seed=300 + fmt)
    pool = coded_pool(ctx, batch, 4, fmt, 301)
    for W in (0, 50):
        out, starts = prefill_q0(ctx, pool, batch, chunks, 8, W)
        check_prefill(out, starts, batch.seq_lens, W, 8, 4, stored_one(fmt), f"generic prefill W={W}")
