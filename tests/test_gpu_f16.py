"""fp16 KV pools (LLH_KV_F16): the element type of the reference's Metal KV mirror
(attention_scores_f16 / attention_weighted_sum_f16,
crates/llm-metal/src/device/shaders/generic.metal:89-118,200-258; KvCacheConfig::f16,
crates/llm-kv-cache/src/format.rs:69-120).

* writes: whole-block writes (bf16 rows) and appends (bf16 or f32 rows) store
  numpy's float16 of each value (round to nearest even, overflow to infinity),
  bit for bit; the gather returns the stored bits (== the oracle's gather).
* decode: both tuned kernels (split-K, persistent stream), every group size,
  windows and ragged lengths, against the oracle run on the pool the GPU holds,
  at the parity bar; query heads of very different magnitude (each head is
  scaled into fp16 by its own power of two) and a NaN head that stays in its head.
* prefill: the MFMA kernel on fp16 operands against the oracle (full and
  sampled rows, windows, groups) and every row against the decode kernel; rows of
  very different magnitude (each row has its own power of two).
* the element-wise kernels take the other shapes; decode-append on fp16 pools at
  head_dim 128 is the append kernel then the decode (no fused launch; at head_dim
  256 the stream kernel fuses it, tests/test_gpu_decode256.py); layer caches refuse
  fp16.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, magnitude_rows, rows_bf16, to_dev
from llm_hip import workloads
from test_gpu_decode import build_case, oracle_decode, run_decode
from test_gpu_decode_append import assert_pools_equal, new_rows, slots_of
from test_gpu_prefill import build, build_shape, decode_every_row, oracle_rows, sample_rows

pytestmark = pytest.mark.gpu

D = 128
BT = 16
F16 = llm_hip.KV_F16


def f16_bits(x) -> np.ndarray:
    """numpy's float32 -> float16 (round to nearest even, overflow to infinity)."""
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    """Equal fp16 bits, any NaN matching any NaN."""
    na, nb = np.isnan(a.view(np.float16)), np.isnan(b.view(np.float16))
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na], b[~nb]))


SPECIAL = np.array([1e5, -7e4, 65504.0, 65520.0, 1e-8, -3e-8, 6e-5, 2.9e-8, 0.0, -0.0, 1.0009765625, 3.14159],
                   np.float32)


def test_f16_block_write_rounds_like_numpy(ctx):
    import torch

    Hkv = 4
    batch = workloads.paged_batch([40, 17, 300], BT, 0.1, 700)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(701, b, lo, hi, Hkv, D), Hkv, D)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(702, b, lo, hi, Hkv, D), Hkv, D)
    sk = sk.copy()
    sk[0, 0, 0, :SPECIAL.size] = oracle.f32_to_bf16(SPECIAL)  # overflow, subnormals, signed zero
    sv = sv.copy()
    sv[1, 3, 2, :SPECIAL.size] = oracle.f32_to_bf16(-SPECIAL)
    pool = ctx.pool(F16, BT, Hkv, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    raw = pool.raw()
    assert set(raw) == {"k", "v"}  # no scales
    k = raw["k"].view(np.uint16).reshape(batch.n_blocks, Hkv, BT, D)
    v = raw["v"].view(np.uint16).reshape(batch.n_blocks, Hkv, D, BT)
    for i, blk in enumerate(ids):
        want_k = f16_bits(oracle.bf16_to_f32(sk[i].ravel())).reshape(BT, Hkv, D).transpose(1, 0, 2)
        want_v = f16_bits(oracle.bf16_to_f32(sv[i].ravel())).reshape(BT, Hkv, D).transpose(1, 2, 0)
        assert same_bits(k[blk], want_k), i
        assert same_bits(v[blk], want_v), i
    assert k[ids[0], 0, 0, 0] == 0x7C00 and k[ids[0], 0, 0, 3] == 0x7C00  # 1e5 and 65520 overflow


@pytest.mark.parametrize("src_f32", [False, True])
def test_f16_append_rounds_like_numpy(ctx, src_f32):
    import torch

    Hkv, n_blocks = 8, 6
    pool = ctx.pool(F16, BT, Hkv, D, n_blocks)
    rng = np.random.default_rng(7 + src_f32)
    slots = rng.permutation(n_blocks * BT)[:50].astype(np.int64)
    kf = (rng.standard_normal((50, Hkv, D)) * 10.0 ** rng.integers(-6, 5, (50, Hkv, 1))).astype(np.float32)
    vf = (rng.standard_normal((50, Hkv, D)) * 10.0 ** rng.integers(-6, 5, (50, Hkv, 1))).astype(np.float32)
    kf[0, 0, :SPECIAL.size] = SPECIAL
    vf[1, 1, :SPECIAL.size] = -SPECIAL
    if src_f32:
        ctx.append_f32(pool, to_dev(slots), torch.from_numpy(kf).cuda(), torch.from_numpy(vf).cuda())
    else:
        kb, vb = oracle.f32_to_bf16(kf.ravel()).reshape(kf.shape), oracle.f32_to_bf16(vf.ravel()).reshape(vf.shape)
        ctx.append(pool, to_dev(slots), to_dev(kb), to_dev(vb))
        kf, vf = oracle.bf16_to_f32(kb.ravel()).reshape(kf.shape), oracle.bf16_to_f32(vb.ravel()).reshape(vf.shape)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    raw = pool.raw()
    k = raw["k"].view(np.uint16).reshape(n_blocks, Hkv, BT, D)
    v = raw["v"].view(np.uint16).reshape(n_blocks, Hkv, D, BT)
    for i, s in enumerate(slots):
        blk, t = divmod(int(s), BT)
        assert same_bits(k[blk, :, t, :], f16_bits(kf[i])), i
        assert same_bits(v[blk, :, :, t], f16_bits(vf[i])), i


def test_f16_gather_is_bit_exact(ctx):
    import torch

    Hkv = 4
    batch = workloads.paged_batch([3, 16, 33, 700], BT, 0.1, 104)
    pool, _ = build_case(ctx, batch, 8, Hkv, F16, 104)
    opool = oracle.Pool.from_raw(F16, BT, Hkv, D, batch.n_blocks, pool.raw())
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hkv, int(batch.seq_lens.max()))
    for b, L in enumerate(batch.seq_lens):
        for lo, hi in ((0, int(L)), (int(L) // 3, int(L))):
            for tensor in (0, 1):
                out = torch.zeros((hi - lo) * Hkv * D, dtype=torch.int16, device="cuda")
                ctx.gather(pool, desc, b, lo, hi, tensor, out)
                torch.cuda.synchronize()
                st, ref = opool.gather_raw(batch.tables[b], lo, hi, tensor)
                assert st == oracle.OK
                assert np.array_equal(out.cpu().numpy().view(np.uint16), ref), (b, lo, hi, tensor)
    assert ctx.device_errors() == 0


@pytest.fixture(params=["split", "stream"])
def decode_kernel(request, opts):
    opts(llm_hip.OPT_DECODE_KERNEL, request.param)
    return request.param


def check_decode(ctx, batch, Hq, Hkv, window, seed, q=None, what=""):
    scale = 1.0 / math.sqrt(D)
    pool, q0 = build_case(ctx, batch, Hq, Hkv, F16, seed)
    q = q0 if q is None else q
    before = ctx.metrics()["generic_decode_calls"]
    out = run_decode(ctx, pool, batch, q, Hq, window, scale)
    assert ctx.metrics()["generic_decode_calls"] == before, "the element-wise kernel ran"
    assert ctx.device_errors() == 0, ctx.last_error()
    ref = oracle_decode(pool, batch, F16, Hq, Hkv, window, q, scale)
    return out, ref


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (16, 2), (64, 8)])
def test_f16_decode_groups_and_windows(ctx, decode_kernel, Hq, Hkv):
    batch = workloads.paged_batch([1, 17, 300, 700, 1200], BT, 0.10, seed=Hq * 10 + Hkv + 4)
    for window in (0, 250):
        out, ref = check_decode(ctx, batch, Hq, Hkv, window, 13 + window)
        assert_parity(out, ref, what=f"f16 Hq={Hq} Hkv={Hkv} W={window} {decode_kernel}")


def test_f16_decode_c2_shape(ctx, decode_kernel):
    """configs[1]'s shape (B=32, L~U[256,4096], Hq16/Hkv8) over an fp16 pool."""
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    batch = workloads.paged_batch(lens, BT, 0.10, workloads.SEED_BASE + 1)
    out, ref = check_decode(ctx, batch, 16, 8, 0, workloads.SEED_BASE + 1)
    assert_parity(out, ref, what=f"f16 C2 {decode_kernel}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (32, 8), (16, 2)])
def test_f16_decode_query_magnitudes(ctx, decode_kernel, Hq, Hkv):
    """Heads from bf16 subnormal to 1e30 side by side, outliers 100x the rest of their
    head, an all-zero head: each head's own power of two keeps its q exact in fp16
    (a shared one would flush the small heads or overflow the large)."""
    lens = [300, 700, 1200]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=Hq + Hkv + 50)
    # one row per sequence: head h of sequence b takes magnitude b + h in turn
    qb = magnitude_rows(oracle.normal_bf16(51, len(lens) * Hq * D), Hq, D)
    scale = 1.0 / math.sqrt(D)
    for window in (0, 250):
        pool, _ = build_case(ctx, batch, Hq, Hkv, F16, 52)
        out = run_decode(ctx, pool, batch, qb, Hq, window, scale)
        assert ctx.device_errors() == 0, ctx.last_error()
        ref = oracle_decode(pool, batch, F16, Hq, Hkv, window, qb, scale)
        assert_parity(out, ref, what=f"Hq={Hq} Hkv={Hkv} W={window}")


def test_f16_decode_nan_query_stays_in_its_head(ctx, decode_kernel):
    Hq, Hkv = 32, 8
    lens = [500, 900]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=43)
    pool, q = build_case(ctx, batch, Hq, Hkv, F16, seed=44)
    qn = q.reshape(len(lens), Hq, D).copy()
    qn[1, 5, 17] = 0x7FC0  # NaN in sequence 1, head 5
    scale = 1.0 / math.sqrt(D)
    out = run_decode(ctx, pool, batch, qn.ravel(), Hq, 0, scale).reshape(len(lens), Hq, D)
    assert ctx.device_errors() == 0, ctx.last_error()
    assert np.all(np.isnan(oracle.bf16_to_f32(out[1, 5])))
    ref = oracle_decode(pool, batch, F16, Hq, Hkv, 0, q, scale).reshape(len(lens), Hq, D)
    keep = np.ones((len(lens), Hq), bool)
    keep[1, 5] = False
    assert_parity(out[keep], ref[keep], what="heads without the NaN")


def test_f16_decode_bad_block_is_masked_and_flagged(ctx, decode_kernel):
    batch = workloads.paged_batch([64, 64], BT, 0.10, seed=19)
    pool, q = build_case(ctx, batch, 16, 8, F16, 19)
    bad = workloads.PagedBatch(batch.seq_lens, batch.tables.copy(), batch.n_blocks, BT, batch.first_block)
    bad.tables[1, 2] = batch.n_blocks + 5
    out = run_decode(ctx, pool, bad, q, 16, 0, 0.1)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK
    assert np.all(np.isfinite(oracle.bf16_to_f32(out)))
    first = workloads.PagedBatch(batch.seq_lens[:1], batch.tables[:1], batch.n_blocks, BT, batch.first_block[:1])
    ref = oracle_decode(pool, first, F16, 16, 8, 0, q[: 16 * D], 0.1)
    assert_parity(out[: 16 * D], ref, what="good sequence beside a bad one")


def test_f16_decode_generic_kernel(ctx, opts):
    """Force-generic on the tuned shape and head_dim 64: the element-wise kernel runs
    and meets the bar against the oracle."""
    batch = workloads.paged_batch([5, 77, 300], BT, 0.10, seed=64)
    opts(llm_hip.OPT_FORCE_GENERIC, 1)
    scale = 1.0 / math.sqrt(D)
    pool, q = build_case(ctx, batch, 16, 8, F16, 65)
    before = ctx.metrics()["generic_decode_calls"]
    out = run_decode(ctx, pool, batch, q, 16, 100, scale)
    assert ctx.metrics()["generic_decode_calls"] == before + 1
    assert ctx.device_errors() == 0, ctx.last_error()
    assert_parity(out, oracle_decode(pool, batch, F16, 16, 8, 100, q, scale), what="generic D=128")
    opts(llm_hip.OPT_FORCE_GENERIC, 0)
    batch = workloads.paged_batch([5, 77, 300], 8, 0.10, seed=66)
    pool, q = build_case(ctx, batch, 8, 2, F16, 67, head_dim=64)
    out = run_decode(ctx, pool, batch, q, 8, 0, 0.125, head_dim=64)
    assert ctx.device_errors() == 0, ctx.last_error()
    assert_parity(out, oracle_decode(pool, batch, F16, 8, 2, 0, q, 0.125, head_dim=64), what="generic D=64")


def test_f16_decode_append_is_append_then_decode(ctx, decode_kernel):
    """No fused launch on fp16 pools: llh_paged_decode_append appends through the append
    kernel, then decodes -- pool and output identical to the two calls."""
    import torch

    Hq, Hkv = 16, 8
    batch = workloads.paged_batch([1, 16, 17, 500, 1000], BT, 0.10, seed=88)
    scale = 1.0 / math.sqrt(D)
    B = batch.seq_lens.size
    kn, vn = new_rows(88, B, Hkv)
    outs, raws = [], []
    before = ctx.metrics()["fused_append_calls"]
    for fused in (True, False):
        pool, q = build_case(ctx, batch, Hq, Hkv, F16, 88)
        desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(batch.seq_lens.max()))
        d_out = torch.full((B * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
        if fused:
            ctx.paged_decode_append(pool, desc, to_dev(kn), to_dev(vn), to_dev(q), d_out, scale)
        else:
            ctx.append(pool, to_dev(slots_of(batch)), to_dev(kn), to_dev(vn))
            ctx.paged_decode(pool, desc, to_dev(q), d_out, scale)
        torch.cuda.synchronize()
        assert ctx.device_errors() == 0, ctx.last_error()
        outs.append(from_dev_bf16(d_out))
        raws.append(pool.raw())
    assert ctx.metrics()["fused_append_calls"] == before
    assert np.array_equal(outs[0], outs[1])
    assert_pools_equal(batch, raws[0], raws[1])
    opool = oracle.Pool.from_raw(F16, BT, Hkv, D, batch.n_blocks, raws[0])
    st, ref = opool.decode(Hq, batch.seq_lens, batch.tables, 0, q, scale, threads=16)
    assert st == oracle.OK
    assert_parity(outs[0], ref, what="decode-append f16")


def test_f16_layer_cache_is_unsupported(ctx):
    """LayerKvCache::new_with_config refuses f16 (layer.rs:399-403)."""
    with pytest.raises(llm_hip.LlhError) as e:
        ctx.layer_cache(64, 2, D, F16)
    assert e.value.status == llm_hip.ERR_UNSUPPORTED


def test_f16_prefill_c3_shape(ctx):
    """configs[2]'s shape over fp16 blocks: sampled rows against the oracle, every row
    against the decode kernel on the same pool."""
    prefix, chunk, Hq, Hkv = [1536] * 8, [512] * 8, 32, 4
    before = ctx.metrics()["generic_prefill_calls"]
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, 0, workloads.SEED_BASE + 12, fmt=F16)
    assert ctx.metrics()["generic_prefill_calls"] == before
    ref, picked = oracle_rows(pool, batch, starts, Hq, Hkv, 0, q, scale, [sample_rows(c) for c in chunk], F16)
    got = out.reshape(-1, Hq * D)
    assert_parity(got[picked], ref[picked], what="f16 C3 sampled rows vs oracle")
    dec = decode_every_row(ctx, batch, pool, starts, prefix, chunk, q, Hq, 0, scale)
    assert_parity(out, oracle.bf16_to_f32(dec), what="f16 C3 all rows vs decode kernel")


@pytest.mark.parametrize("W", [0, 37, 200])
@pytest.mark.parametrize("Hq,Hkv", [(16, 8), (12, 4), (16, 1)])
def test_f16_prefill_ragged_full_oracle(ctx, W, Hq, Hkv):
    prefix = [0, 17, 1000, 3, 64]
    chunk = [1, 5, 130, 300, 64]
    before = ctx.metrics()["generic_prefill_calls"]
    batch, pool, starts, q, out, scale = build(ctx, prefix, chunk, Hq, Hkv, W, 90 + W + Hq, fmt=F16)
    assert ctx.metrics()["generic_prefill_calls"] == before
    opool = oracle.Pool.from_raw(F16, BT, Hkv, D, batch.n_blocks, pool.raw())
    st, ref = opool.prefill(Hq, starts, batch.seq_lens, batch.tables, W, q, scale, threads=16)
    assert st == oracle.OK
    assert_parity(out, ref, what=f"f16 ragged Hq={Hq} Hkv={Hkv} W={W}")


def test_f16_prefill_row_magnitudes(ctx):
    """Query rows from bf16 subnormal to 1e30 in one tile: each row's own power of two
    keeps its q exact in fp16; scores to ~1e31 in log2 units."""
    before = ctx.metrics()["generic_prefill_calls"]
    out, ref = build_shape(ctx, [300, 0], [200, 129], 16, 8, 0, 95, D, BT, F16, q_magnitudes=True)
    assert ctx.metrics()["generic_prefill_calls"] == before
    assert_parity(out, ref, what="f16 prefill row magnitudes")


@pytest.mark.parametrize("misalign", [False, True])
def test_f16_prefill_generic_kernel(ctx, misalign):
    """head_dim 64 on 32-token blocks, and the tuned shape 2 bytes off alignment: the
    element-wise prefill kernel over fp16 blocks, every row against the oracle."""
    before = ctx.metrics()["generic_prefill_calls"]
    if misalign:
        out, ref = build_shape(ctx, [300, 0], [129, 64], 16, 8, 0, 77, D, BT, F16, misalign=True)
    else:
        out, ref = build_shape(ctx, [100, 0, 37, 5], [37, 70, 0, 130], 12, 4, 48, 964, 64, 32, F16)
    assert ctx.metrics()["generic_prefill_calls"] == before + 1
    assert_parity(out, ref, what=f"f16 generic prefill misalign={misalign}")
