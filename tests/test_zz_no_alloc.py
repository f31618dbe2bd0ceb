"""llh_paged_decode_noalloc: the decode step on the library's static scratch.

Called through the C ABI, it must give exactly llh_paged_decode's bits (same
plan, same kernels) on two calls in a row -- a C2-shaped step on the stream
kernel, then a smaller split-K step that reuses the array the first one filled
-- allocate no device memory, and reject a step whose plan exceeds the array.
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


def _case(ctx, lens, Hq, Hkv, seed):
    import torch

    batch = workloads.paged_batch(lens, BT, 0.10, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, D), Hkv, D)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, D), Hkv, D)
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    q = oracle.normal_bf16(seed + 3, batch.seq_lens.size * Hq * D)
    d_lens, d_tab, d_q = to_dev(batch.seq_lens), to_dev(batch.tables), to_dev(q)
    desc = ctx.decode_desc(d_lens, d_tab, Hq, int(batch.seq_lens.max()))
    torch.cuda.synchronize()
    return batch, pool, q, (d_lens, d_tab, d_q), desc


def test_noalloc_decode_matches_paged_decode_on_two_calls(ctx):
    import torch

    cases = [
        ("C2 (stream kernel)", workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1), 16, 8, 900),
        ("smaller, split-K", [512, 37, 300], 16, 8, 901),
    ]
    built = [_case(ctx, lens, Hq, Hkv, seed) for _, lens, Hq, Hkv, seed in cases]
    # llh_paged_decode's results first, on the stream the no-allocation calls use: the HIP
    # runtime sets up a stream's hardware queue and loads a kernel's code object into device
    # memory at their first launch, which is not this library's allocation
    stream = torch.cuda.Stream()
    refs, outs = [], []
    for (name, lens, Hq, Hkv, seed), (batch, pool, q, keep, desc) in zip(cases, built):
        n = batch.seq_lens.size * Hq * D
        ref_out = torch.zeros(n, dtype=torch.int16, device="cuda")
        ctx.paged_decode(pool, desc, keep[2], ref_out, 0.088, stream=stream)
        refs.append(ref_out)
        outs.append(torch.full((n,), 0x7FC0, dtype=torch.int16, device="cuda"))
    torch.cuda.synchronize()
    free_before = torch.cuda.mem_get_info()[0]
    for (name, lens, Hq, Hkv, seed), (batch, pool, q, keep, desc), out in zip(cases, built, outs):
        before = ctx.metrics()
        ctx.paged_decode_noalloc(pool, desc, keep[2], out, 0.088, stream=stream)
        stream.synchronize()
        after = ctx.metrics()
        assert after["decode_calls"] == before["decode_calls"] + 1, name
        if name.startswith("C2"):
            assert after["stream_decode_calls"] == before["stream_decode_calls"] + 1, "C2 did not take the stream kernel"
        else:
            assert after["stream_decode_calls"] == before["stream_decode_calls"], "the small step should be split-K"
    free_after = torch.cuda.mem_get_info()[0]
    assert free_after == free_before, f"free device memory changed by {free_before - free_after} bytes"
    assert ctx.device_errors() == 0, ctx.last_error()
    for (name, lens, Hq, Hkv, seed), (batch, pool, q, keep, desc), out, ref_out in zip(cases, built, outs, refs):
        got = from_dev_bf16(out)
        assert np.array_equal(got, from_dev_bf16(ref_out)), f"{name}: differs from llh_paged_decode"
        opool = oracle.Pool.from_raw(llm_hip.KV_BF16, BT, Hkv, D, batch.n_blocks, pool.raw())
        st, ref = opool.decode(Hq, batch.seq_lens, batch.tables, 0, q, 0.088, threads=16)
        assert st == oracle.OK
        assert_parity(got, ref, what=name)


def test_noalloc_decode_rejects_steps_beyond_its_scratch(ctx, opts):
    """A split-K step of 32 sequences of 2048-4096 tokens with 64 query heads plans 33
    partial rows of 520 bytes per (sequence, head) (35 MB), twice the array: the call is
    refused before any launch; llh_paged_decode takes the same step."""
    import torch

    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    lens = workloads.uniform_lengths(32, 2048, 4096, 902)
    batch, pool, q, keep, desc = _case(ctx, lens, 64, 8, 902)
    out = torch.zeros(batch.seq_lens.size * 64 * D, dtype=torch.int16, device="cuda")
    with pytest.raises(llm_hip.LlhError) as e:
        ctx.paged_decode_noalloc(pool, desc, keep[2], out, 0.088)
    assert e.value.status == llm_hip.ERR_CAPACITY
    assert "scratch" in e.value.message
    ctx.paged_decode(pool, desc, keep[2], out, 0.088)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
