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


def test_fp8_append_over_a_window_ring_needs_one_block_more(ctx):
    """An fp8 block keeps one scale per (block, head) that a token at offset 0 restarts: in a
    window ring of exactly W/16 blocks the new token's block still holds live tokens of the
    previous pass round the ring, so the call is refused; with W/16 + 1 blocks the step runs,
    the appended block equals the oracle's per-token rule (oracle.append_fp8_token) bit for
    bit and the output meets the bar of the oracle run on the pool."""
    import torch

    W, Hq, Hkv = 64, 16, 8
    lens = np.array([1000, 77, 129, 97], np.int32)  # new tokens at offsets 7, 12, 0, 0
    B = lens.size
    for nb, ok in ((W // BT, False), (W // BT + 1, True)):
        n_pool = 23  # prime: the entries i * 5 + 1 (mod 23) of the B * nb <= 20 table slots are distinct
        tables = ((np.arange(B * nb, dtype=np.int32) * 5 + 1) % n_pool).reshape(B, nb)
        assert np.unique(tables).size == B * nb
        pool = ctx.pool(llm_hip.KV_FP8_E4M3, BT, Hkv, D, n_pool)
        slots, ks, vs = [], [], []
        for b in range(B):
            for p in range(max(0, int(lens[b]) - W), int(lens[b]) - 1):  # the window before the new token
                slots.append(int(tables[b, (p // BT) % nb]) * BT + p % BT)
                ks.append(oracle.normal_bf16(600 + b, Hkv * D, p * Hkv * D).reshape(Hkv, D))
                vs.append(oracle.normal_bf16(700 + b, Hkv * D, p * Hkv * D).reshape(Hkv, D))
        ctx.append(pool, to_dev(np.array(slots, np.int64)), to_dev(np.stack(ks)), to_dev(np.stack(vs)))
        torch.cuda.synchronize()
        before = pool.raw()
        kn = oracle.normal_bf16(801, B * Hkv * D).reshape(B, Hkv, D)
        vn = oracle.normal_bf16(802, B * Hkv * D).reshape(B, Hkv, D)
        q = oracle.normal_bf16(803, B * Hq * D)
        out = torch.zeros(B * Hq * D, dtype=torch.int16, device="cuda")
        desc = ctx.decode_desc(to_dev(lens), to_dev(tables), Hq, int(lens.max()), W)
        if not ok:
            with pytest.raises(llm_hip.LlhError) as e:
                ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), to_dev(q), out, 0.09)
            assert e.value.status == llm_hip.ERR_INVALID_SHAPE
            continue
        ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), to_dev(q), out, 0.09)
        torch.cuda.synchronize()
        assert ctx.device_errors() == 0, ctx.last_error()
        after = pool.raw()
        kc0, vc0 = before["k"].reshape(n_pool, Hkv, BT, D), before["v"].reshape(n_pool, Hkv, D, BT)
        ks0 = before["k_scales"].view(np.float32).reshape(n_pool, Hkv)
        vs0 = before["v_scales"].view(np.float32).reshape(n_pool, Hkv)
        kc1, vc1 = after["k"].reshape(n_pool, Hkv, BT, D), after["v"].reshape(n_pool, Hkv, D, BT)
        ks1 = after["k_scales"].view(np.float32).reshape(n_pool, Hkv)
        vs1 = after["v_scales"].view(np.float32).reshape(n_pool, Hkv)
        for b in range(B):
            p = int(lens[b]) - 1
            blk, off = int(tables[b, (p // BT) % nb]), p % BT
            for h in range(Hkv):
                for src, c0, s0, c1, s1 in ((kn, kc0[blk, h], ks0[blk, h], kc1[blk, h], ks1[blk, h]),
                                            (vn, vc0[blk, h].T, vs0[blk, h], vc1[blk, h].T, vs1[blk, h])):
                    codes = np.ascontiguousarray(c0).copy()
                    st, s = oracle.append_fp8_token(codes, float(s0), off, oracle.bf16_to_f32(src[b, h]))
                    assert st == oracle.OK
                    assert np.float32(s) == s1, (b, h)
                    assert np.array_equal(codes[:off + 1], c1[:off + 1]), (b, h)
        opool = oracle.Pool.from_raw(llm_hip.KV_FP8_E4M3, BT, Hkv, D, n_pool, after)
        st, ref = opool.decode(Hq, lens, tables, W, q, 0.09)
        assert st == oracle.OK
        assert_parity(from_dev_bf16(out), ref, what=f"fp8 window ring of {nb} blocks")
