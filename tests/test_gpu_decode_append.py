"""kir-ai's decode step in one call (llh_paged_decode_append) vs the two calls it
replaces: llh_kv_append of each sequence's new token at position len - 1, then
llh_paged_decode (crates/llm-backend/src/core/native_attention.rs:307-329).

Every pool format runs it as one launch on the tuned kernels, except fp8 pools on
the persistent stream kernel, which append through the append kernel first (the
fused fp8 re-encode made that kernel slower than the launch it saves).  bf16: the new
token is attended from the input rows and written to its slot by the wavefront
that computes the sequence's last block; the pool must end up bit-identical to
the two-call path's and the output within the parity bar of the oracle run on
that pool.  int8 / fp8: that wavefront quantises the token into the block it
loaded, exactly as the append kernel would (fp8: re-encoding the block's earlier
tokens when the block scale grows), attends the block as stored and writes it
back: pool and output bit-identical to the two calls.
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


def run_both(ctx, batch, Hq, Hkv, fmt, window, seed, mag=None):
    """Returns (fused output, two-call output, fused pool raw, two-call pool raw, ref).
    mag: optional per-sequence factors for the new rows (> 1 grows an fp8 block's scale)."""
    import torch

    scale = 1.0 / math.sqrt(D)
    B = batch.seq_lens.size
    kn, vn = new_rows(seed, B, Hkv)
    if mag is not None:
        f = np.asarray(mag, np.float32)[:, None, None]
        kn = oracle.f32_to_bf16(oracle.bf16_to_f32(kn.ravel()).reshape(kn.shape) * f).reshape(kn.shape)
        vn = oracle.f32_to_bf16(oracle.bf16_to_f32(vn.ravel()).reshape(vn.shape) * f[::-1]).reshape(vn.shape)
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


@pytest.mark.parametrize("kernel", ["split", "stream"])
@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (32, 8), (8, 8), (64, 8)])
def test_decode_append_quantized_one_launch(ctx, opts, kernel, fmt, Hq, Hkv):
    """int8 / fp8 pools, one launch (fp8 on the stream kernel: two), both kernels, the
    token-lane (G <= 4) and row (G = 8) layouts: pool and output bit-identical to
    llh_kv_append + llh_paged_decode.  New tokens land at every offset class (0,
    mid-block, 15); half of them are 4x larger than the block's rows, so fp8 block scales
    grow and earlier tokens are re-encoded."""
    opts(llm_hip.OPT_DECODE_KERNEL, kernel)
    launches = 0 if (fmt == llm_hip.KV_FP8_E4M3 and kernel == "stream") else 1
    lens = np.array([40, 1, 500, 16, 1777, 17, 33, 2048, 4095, 129, 64, 300], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, 21 + Hq)
    mag = [4.0 if i % 2 else 1.0 for i in range(lens.size)]
    for window in (0, 300):
        before = ctx.metrics()["fused_append_calls"]
        fused, two, raw_f, raw_t, ref = run_both(ctx, batch, Hq, Hkv, fmt, window, 50 + fmt + window, mag)
        assert ctx.metrics()["fused_append_calls"] == before + launches
        assert_pools_equal(batch, raw_f, raw_t)
        assert np.array_equal(fused, two), f"fmt {fmt} {kernel} Hq{Hq} W={window}"
        assert_parity(fused, ref, what=f"fmt {fmt} {kernel} Hq{Hq} W={window}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_append_quantized_c5_full_launch(ctx, opts, fmt):
    """The C5 step (64 x 8192, Hq32/Hkv8) on the stream kernel: one fused launch for
    int8, the append kernel then the decode for fp8."""
    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    batch = workloads.paged_batch(np.full(64, 8192, np.int32), BT, 0.0, 22)
    before = ctx.metrics()["fused_append_calls"]
    fused, two, raw_f, raw_t, ref = run_both(ctx, batch, 32, 8, fmt, 0, 60 + fmt)
    assert ctx.metrics()["fused_append_calls"] == before + (fmt == llm_hip.KV_INT8)
    assert_pools_equal(batch, raw_f, raw_t)
    assert np.array_equal(fused, two)
    assert_parity(fused, ref, what=f"C5 fused fmt {fmt}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_append_quantized_non_finite_row(ctx, fmt):
    """A NaN in one sequence's new row: flagged and not appended (as llh_kv_append), and the
    other sequences' pool bytes and outputs still equal the two calls'."""
    import torch

    Hq, Hkv = 16, 8
    lens = np.array([40, 300, 77], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, 23)
    kn, vn = new_rows(70, lens.size, Hkv)
    kn = kn.copy()
    kn[1, 3, 7] = 0x7FC0
    outs, raws = [], []
    for fused in (True, False):
        pool, q = build_case(ctx, batch, Hq, Hkv, fmt, 71)
        desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(lens.max()))
        out = torch.zeros(lens.size * Hq * D, dtype=torch.int16, device="cuda")
        if fused:
            ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), to_dev(q), out, 0.09)
        else:
            ctx.append(pool, to_dev(slots_of(batch)), to_dev(kn), to_dev(vn))
            ctx.paged_decode(pool, desc, to_dev(q), out, 0.09)
        torch.cuda.synchronize()
        assert ctx.device_errors() & llm_hip.ERR_FLAG_NON_FINITE
        outs.append(from_dev_bf16(out).reshape(lens.size, -1))
        raws.append(pool.raw())
    assert_pools_equal(batch, raws[0], raws[1])
    assert np.array_equal(outs[0][[0, 2]], outs[1][[0, 2]])


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
