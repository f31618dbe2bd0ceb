"""Pools past 4 GiB per tensor: every kernel addresses the pool with 64-bit offsets.

A large pool (2^21 block-heads above the small pool's: K alone holds 8 GiB of
bf16, 2^32 + elements, or 4 GiB of int8 / e4m3 codes) holds the same blocks at
the top of its index range as a small pool holds from block 0.  Decode (split-K
and stream), chunked prefill, the per-token append, the fused append+attend,
the allocation-free decode and row export must give bit-identical results on
both pools (only the addresses differ); the small pool's decode and prefill are
checked against the oracle.  A pool of this size is an ordinary slice of the
288 GB of HBM the kernels are laid out for.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, rows_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu

D = 128
BT = 16
HQ, HKV = 16, 8
LENS = [1000, 17, 300, 2049]  # no length is a multiple of 16: the next position's block is in the table
CHUNK = 100


def _tables(batch, off):
    return np.where(batch.tables >= 0, batch.tables + off, -1).astype(np.int32)


def _decode(ctx, pool, lens, tables, q, scale, fused=None, noalloc=False):
    import torch

    d_lens, d_tab = to_dev(np.asarray(lens, np.int32)), to_dev(tables)
    desc = ctx.decode_desc(d_lens, d_tab, HQ, int(max(lens)), 0)
    d_out = torch.full((len(lens) * HQ * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    if fused is not None:
        ctx.paged_decode_append(pool, desc, fused[0], fused[1], to_dev(q), d_out, scale)
    elif noalloc:
        ctx.paged_decode_noalloc(pool, desc, to_dev(q), d_out, scale)
    else:
        ctx.paged_decode(pool, desc, to_dev(q), d_out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    return from_dev_bf16(d_out)


def _prefill(ctx, pool, tables, q, scale):
    import torch

    chunk = [min(CHUNK, L) for L in LENS]
    starts = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    desc = ctx.prefill_desc(to_dev(starts), to_dev(np.asarray(LENS, np.int32)), to_dev(tables), HQ, max(chunk), 0,
                            total_q_rows=int(starts[-1]))
    d_out = torch.full((int(starts[-1]) * HQ * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    ctx.paged_prefill(pool, desc, to_dev(q), d_out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    return from_dev_bf16(d_out), starts


@pytest.mark.parametrize("generic", [False, True], ids=["tuned", "generic"])
@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_pool_beyond_4gib_matches_small_pool(ctx, opts, fmt, generic):
    """generic: the element-wise decode and prefill kernels (force-generic option)."""
    import torch

    if generic:
        opts(llm_hip.OPT_FORCE_GENERIC, 1)
    seed = 910 + fmt
    scale = 1.0 / math.sqrt(D)
    batch = workloads.paged_batch(LENS, BT, 0.10, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, HKV, D), HKV, D)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, HKV, D), HKV, D)
    n_small = batch.n_blocks
    off = (1 << 21) // HKV
    small = ctx.pool(fmt, BT, HKV, D, n_small)
    big = ctx.pool(fmt, BT, HKV, D, off + n_small)
    try:
        ctx.write_blocks(small, to_dev(ids), to_dev(sk), to_dev(sv))
        ctx.write_blocks(big, to_dev(ids + off), to_dev(sk), to_dev(sv))
        tab_s, tab_b = batch.tables.astype(np.int32), _tables(batch, off)
        q = oracle.normal_bf16(seed + 3, len(LENS) * HQ * D)

        # decode through both kernels; the small pool's result against the oracle
        opool = oracle.Pool.from_raw(fmt, BT, HKV, D, n_small, small.raw())
        st, ref = opool.decode(HQ, batch.seq_lens, batch.tables, 0, q, scale, threads=16)
        assert st == oracle.OK
        for kernel in ("split", "stream"):
            opts(llm_hip.OPT_DECODE_KERNEL, kernel)
            out_s = _decode(ctx, small, LENS, tab_s, q, scale)
            out_b = _decode(ctx, big, LENS, tab_b, q, scale)
            assert_parity(out_s, ref, what=f"{kernel} decode, small pool")
            np.testing.assert_array_equal(out_b, out_s, err_msg=f"{kernel} decode: large pool differs")
        opts(llm_hip.OPT_DECODE_KERNEL, 0)

        # chunked prefill over the last CHUNK positions of every sequence
        chunk = [min(CHUNK, L) for L in LENS]
        qp = oracle.normal_bf16(seed + 4, sum(chunk) * HQ * D)
        pre_s, starts = _prefill(ctx, small, tab_s, qp, scale)
        pre_b, _ = _prefill(ctx, big, tab_b, qp, scale)
        st, pref = opool.prefill(HQ, starts, batch.seq_lens, batch.tables, 0, qp, scale, threads=16)
        assert st == oracle.OK
        assert_parity(pre_s, pref, what="prefill, small pool")
        np.testing.assert_array_equal(pre_b, pre_s, err_msg="prefill: large pool differs")

        # append the token at position len, then decode over len + 1 and export the new rows
        B = len(LENS)
        pos = np.asarray(LENS, np.int64)
        blk = batch.tables[np.arange(B), pos // BT].astype(np.int64)
        slots_s = to_dev(blk * BT + pos % BT)
        slots_b = to_dev((blk + off) * BT + pos % BT)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        k_new = torch.randn((B, HKV, D), generator=g, device="cuda").to(torch.bfloat16)
        v_new = torch.randn((B, HKV, D), generator=g, device="cuda").to(torch.bfloat16)
        ctx.append(small, slots_s, k_new, v_new)
        ctx.append(big, slots_b, k_new, v_new)
        lens1 = [L + 1 for L in LENS]
        out_s = _decode(ctx, small, lens1, tab_s, q, scale)
        out_b = _decode(ctx, big, lens1, tab_b, q, scale)
        np.testing.assert_array_equal(out_b, out_s, err_msg="decode after append: large pool differs")
        tab1 = batch.tables.copy()
        opool1 = oracle.Pool.from_raw(fmt, BT, HKV, D, n_small, small.raw())
        st, ref1 = opool1.decode(HQ, np.asarray(lens1, np.int32), tab1, 0, q, scale, threads=16)
        assert st == oracle.OK
        assert_parity(out_s, ref1, what="decode after append, small pool")
        rows = []
        for pool, slots in ((small, slots_s), (big, slots_b)):
            k_out = torch.empty((B, HKV, D), dtype=torch.float32, device="cuda")
            v_out = torch.empty_like(k_out)
            ctx.export_rows_f32(pool, slots, k_out, v_out)
            torch.cuda.synchronize()
            rows.append((k_out.cpu().numpy(), v_out.cpu().numpy()))
        np.testing.assert_array_equal(rows[1][0], rows[0][0], err_msg="exported K rows differ")
        np.testing.assert_array_equal(rows[1][1], rows[0][1], err_msg="exported V rows differ")

        # the fused step re-appends the same token (same slot, same rows) and attends
        fs = _decode(ctx, small, lens1, tab_s, q, scale, fused=(k_new, v_new))
        fb = _decode(ctx, big, lens1, tab_b, q, scale, fused=(k_new, v_new))
        np.testing.assert_array_equal(fb, fs, err_msg="fused append+attend: large pool differs")
        assert_parity(fs, ref1, what="fused append+attend, small pool")

        # the allocation-free entry point on the large pool
        na = _decode(ctx, big, lens1, tab_b, q, scale, noalloc=True)
        np.testing.assert_array_equal(na, out_b, err_msg="allocation-free decode: large pool differs")
    finally:
        big.close()
        small.close()
