"""kir-ai's decode step in one call (llh_paged_decode_append) vs the two calls it
replaces: llh_kv_append of each sequence's new token at position len - 1, then
llh_paged_decode (crates/llm-backend/src/core/native_attention.rs:307-329).

bf16 pools on the tuned kernels run it as one launch (the new token is attended
from the input rows and written to its slot by the wavefront that computes the
sequence's last block); the pool must end up bit-identical to the two-call
path's and the output within the parity bar of the oracle run on that pool.
Other pool formats take the append kernel, then the decode: bit-identical to
the two calls.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, to_dev
from llm_hip import workloads
from test_gpu_decode import build_case, identity_batch

pytestmark = pytest.mark.gpu

D = 128
BT = 16


def new_rows(seed, B, Hkv):
    k = oracle.normal_bf16(seed + 11, B * Hkv * D).reshape(B, Hkv, D)
    v = oracle.normal_bf16(seed + 12, B * Hkv * D).reshape(B, Hkv, D)
    return k, v


def slots_of(batch):
    lens = batch.seq_lens.astype(np.int64)
    pos = lens - 1
    blk = batch.tables[np.arange(lens.size), (np.maximum(pos, 0) // BT) % batch.tables.shape[1]].astype(np.int64)
    return blk * BT + np.maximum(pos, 0) % BT


def assert_pools_equal(batch, raw_a, raw_b):
    """Every block the tables reference is byte-identical (free blocks hold whatever
    their allocation held)."""
    used = np.unique(batch.tables[batch.tables >= 0])
    for key in raw_a:
        a = raw_a[key].reshape(batch.n_blocks, -1)[used]
        b = raw_b[key].reshape(batch.n_blocks, -1)[used]
        assert np.array_equal(a, b), key


def run_both(ctx, batch, Hq, Hkv, fmt, window, seed):
    """Returns (fused output, two-call output, fused pool raw, two-call pool raw, ref)."""
    import torch

    scale = 1.0 / math.sqrt(D)
    B = batch.seq_lens.size
    kn, vn = new_rows(seed, B, Hkv)
    outs, raws = [], []
    for fused in (True, False):
        pool, q = build_case(ctx, batch, Hq, Hkv, fmt, seed)
        d_lens, d_tab, d_q = to_dev(batch.seq_lens), to_dev(batch.tables), to_dev(q)
        desc = ctx.decode_desc(d_lens, d_tab, Hq, int(batch.seq_lens.max()), window)
        d_out = torch.full((B * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
        if fused:
            ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), d_q, d_out, scale)
        else:
            ctx.append(pool, to_dev(slots_of(batch)), to_dev(kn), to_dev(vn))
            ctx.paged_decode(pool, desc, d_q, d_out, scale)
        torch.cuda.synchronize()
        assert ctx.device_errors() == 0, ctx.last_error()
        outs.append(from_dev_bf16(d_out))
        raws.append(pool.raw())
        if not fused:
            opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
            st, ref = opool.decode(Hq, batch.seq_lens, batch.tables, window, q, scale, threads=16)
            assert st == oracle.OK
    return outs[0], outs[1], raws[0], raws[1], ref


@pytest.mark.parametrize("kernel", ["split", "stream"])
@pytest.mark.parametrize("window", [0, 1000])
def test_decode_append_bf16_one_launch(ctx, opts, kernel, window):
    """C2-shaped ragged batch (lengths at block edges included): one launch, the same
    pool bytes as append-then-decode, the output within the bar of the oracle."""
    opts(llm_hip.OPT_DECODE_KERNEL, kernel)
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    lens[:6] = [1, 16, 17, 32, 33, 4096]
    batch = workloads.paged_batch(lens, BT, 0.10, 5 + window)
    before = ctx.metrics()["fused_append_calls"]
    fused, two, raw_f, raw_t, ref = run_both(ctx, batch, 16, 8, llm_hip.KV_BF16, window, 31 + window)
    assert ctx.metrics()["fused_append_calls"] == before + 1
    assert_pools_equal(batch, raw_f, raw_t)
    assert_parity(fused, ref, what=f"fused {kernel} W={window}")
    assert_parity(two, ref, what=f"two calls {kernel} W={window}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (32, 8), (16, 2), (64, 8)])
def test_decode_append_group_sizes(ctx, Hq, Hkv):
    lens = np.array([5, 300, 1024, 77], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, 9)
    fused, _, raw_f, raw_t, ref = run_both(ctx, batch, Hq, Hkv, llm_hip.KV_BF16, 0, 40 + Hq)
    assert_pools_equal(batch, raw_f, raw_t)
    assert_parity(fused, ref, what=f"Hq{Hq}/Hkv{Hkv}")


def test_decode_append_single_token_is_its_value(ctx):
    """A sequence whose only token is the new one attends it alone: the output is its
    V row exactly; an empty sequence gets zeros and no write."""
    import torch

    Hq, Hkv = 16, 8
    batch = identity_batch([1, 0, 1])
    pool, q = build_case(ctx, batch, Hq, Hkv, llm_hip.KV_BF16, 3)
    kn, vn = new_rows(3, 3, Hkv)
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, 1, 0)
    out = torch.full((3 * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), to_dev(q), out, 0.1)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    got = from_dev_bf16(out).reshape(3, Hq, D)
    for b in (0, 2):
        for h in range(Hq):
            assert np.array_equal(got[b, h], vn[b, h // (Hq // Hkv)])
    assert not got[1].any()
    after = pool.raw()
    k = after["k"].view(np.uint16).reshape(batch.n_blocks, Hkv, BT, D)
    for b, blk in ((0, batch.tables[0, 0]), (2, batch.tables[2, 0])):
        assert np.array_equal(k[blk, :, 0, :], kn[b])


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_append_quantized_pools_equal_two_calls(ctx, fmt):
    """int8 / fp8 pools take the append kernel, then the decode: bit-identical to the
    two calls, pool and output."""
    lens = np.array([40, 1, 500, 16, 1777], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, 21)
    before = ctx.metrics()["fused_append_calls"]
    fused, two, raw_f, raw_t, ref = run_both(ctx, batch, 16, 8, fmt, 0, 50 + fmt)
    assert ctx.metrics()["fused_append_calls"] == before
    assert_pools_equal(batch, raw_f, raw_t)
    assert np.array_equal(fused, two)
    assert_parity(fused, ref, what=f"fmt {fmt}")
