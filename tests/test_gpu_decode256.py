"""The head_dim-256 decode kernels (decode256.hip): Qwen3.5 / 3.6 full-attention layers,
16 query heads over 2 kv heads, head_dim 256 (fixtures/qwen36/config.json), bf16 or fp16
blocks of 16 tokens.  Both launch shapes (split-K and the persistent stream kernel, forced in
turn) are checked against the oracle (the per-head loop of crates/llm-backend/src/core/
native_attention.rs:731-771, head_dim taken from the call) at the parity bar, their
attended set bit-exactly with the position-coded probe (tests/attended_set.py), the
output gate (native_attention.rs:765-781), split counts from 1 to the merge's 64, stream
segments cut into 1 to hundreds of pieces, and the entry points that share the plan
(noalloc, decode+append)."""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from attended_set import check_decode, code, coded_rows
from helpers import assert_parity, from_dev_bf16, magnitude_rows, to_dev
from llm_hip import workloads
from test_gpu_decode import build_case, oracle_decode

pytestmark = pytest.mark.gpu

D = 256
BT = 16
HQ, HKV = 16, 2
FMTS = {"bf16": llm_hip.KV_BF16, "f16": llm_hip.KV_F16}


@pytest.fixture(params=["split", "stream"])
def d256_kernel(request, opts):
    """Both head_dim-256 kernels (LLH_OPT_DECODE_KERNEL forces the one the planner
    otherwise picks by the step's size)."""
    opts(llm_hip.OPT_DECODE_KERNEL, request.param)
    return request.param


def run(ctx, pool, batch, q, window, scale, Hq=HQ, gate=None, fn="decode", kv_new=None, expect_d256=True):
    import torch

    B = batch.seq_lens.size
    out = torch.full((B * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(batch.seq_lens.max()), window,
                           gate=to_dev(gate) if gate is not None else None)
    before = ctx.metrics()["d256_decode_calls"]
    streamed0 = ctx.metrics()["stream_decode_calls"]
    if fn == "decode":
        ctx.paged_decode(pool, desc, to_dev(q), out, scale)
    elif fn == "noalloc":
        ctx.paged_decode_noalloc(pool, desc, to_dev(q), out, scale)
    else:
        ctx.paged_decode_append(pool, desc, to_dev(kv_new[0]), to_dev(kv_new[1]), to_dev(q), out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    assert ctx.metrics()["d256_decode_calls"] == before + (1 if expect_d256 else 0)
    forced = ctx.get_option(llm_hip.OPT_DECODE_KERNEL)
    streamed = ctx.metrics()["stream_decode_calls"] - streamed0
    if expect_d256 and fn != "noalloc" and forced == llm_hip.DECODE_KERNELS["stream"]:
        assert streamed == 1, "the stream kernel did not run"
    if forced == llm_hip.DECODE_KERNELS["split"]:
        assert streamed == 0, "the stream kernel ran under the split-K option"
    return from_dev_bf16(out)


def case(ctx, lens, seed, free=0.10, Hq=HQ, fmt=llm_hip.KV_BF16):
    batch = workloads.paged_batch(np.asarray(lens, np.int32), BT, free, seed)
    pool, q = build_case(ctx, batch, Hq, HKV, fmt, seed, head_dim=D)
    return batch, pool, q


@pytest.mark.parametrize("fmt", FMTS)
def test_decode256_qwen36_step(ctx, d256_kernel, fmt):
    """The Qwen3.6-shaped step: 32 sequences, lengths in [256, 4096], edges included."""
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    lens[:6] = [1, 16, 17, 32, 33, 4096]
    batch, pool, q = case(ctx, lens, 101, fmt=FMTS[fmt])
    scale = 1.0 / math.sqrt(D)
    out = run(ctx, pool, batch, q, 0, scale)
    assert_parity(out, oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, 0, q, scale, head_dim=D),
                  what=f"qwen36 step {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
def test_decode256_query_magnitudes(ctx, d256_kernel, fmt):
    """Query heads from bf16 subnormal to 1e30 (helpers.magnitude_rows): over fp16 blocks
    each head's power-of-two scaling keeps q in fp16's range and is undone on the scores."""
    lens = np.array([1, 17, 300, 1000, 4096, 33, 16, 2000], np.int32)
    batch, pool, q = case(ctx, lens, 140, fmt=FMTS[fmt])
    q = magnitude_rows(q, HQ, D)
    out = run(ctx, pool, batch, q, 0, 0.0625)
    assert_parity(out, oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, 0, q, 0.0625, head_dim=D),
                  what=f"query magnitudes {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("window", [1, 17, 100, 4096])
def test_decode256_windows(ctx, d256_kernel, window, fmt):
    lens = np.array([1, 15, 16, 17, 100, 101, 700, 4100, 5000], np.int32)
    batch, pool, q = case(ctx, lens, 102 + window, fmt=FMTS[fmt])
    out = run(ctx, pool, batch, q, window, 0.0625)
    assert_parity(out, oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, window, q, 0.0625, head_dim=D),
                  what=f"W={window} {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("split_blocks", [4, 8, 64, 256])
def test_decode256_split_counts(ctx, opts, split_blocks, fmt):
    """One split (split_blocks 256 over 4096 tokens) up to 64 (4 blocks a split), and the
    planner's growth of the split past 64 partials for a 20000-token context."""
    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    opts(llm_hip.OPT_DECODE_SPLIT_BLOCKS, split_blocks)
    lens = np.array([4096, 20000, 1, 333], np.int32)
    batch, pool, q = case(ctx, lens, 103, fmt=FMTS[fmt])
    out = run(ctx, pool, batch, q, 0, 0.0625)
    assert_parity(out, oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, 0, q, 0.0625, head_dim=D),
                  what=f"split_blocks {split_blocks} {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("wgs", [1, 7, 64, 512])
def test_decode256_stream_pieces(ctx, opts, wgs, fmt):
    """The stream kernel over grids of 4 to 2048 wavefronts: segments whole inside one
    wavefront, and segments cut into up to 16, up to 32 and hundreds of pieces (the
    merge's one-round and 32-piece-round paths), ragged and empty sequences included."""
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    opts(llm_hip.OPT_DECODE_STREAM_WGS, wgs)
    lens = np.array([20000, 1, 0, 333, 4096, 17, 2500], np.int32)
    batch, pool, q = case(ctx, lens, 116 + wgs, fmt=FMTS[fmt])
    out = run(ctx, pool, batch, q, 0, 0.0625)
    assert_parity(out, oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, 0, q, 0.0625, head_dim=D),
                  what=f"stream over {wgs} workgroups {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
def test_decode256_is_deterministic(ctx, d256_kernel, fmt):
    lens = workloads.uniform_lengths(8, 256, 4096, 104)
    batch, pool, q = case(ctx, lens, 104, fmt=FMTS[fmt])
    a = run(ctx, pool, batch, q, 0, 0.0625)
    b = run(ctx, pool, batch, q, 0, 0.0625)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("fmt", FMTS)
def test_decode256_empty_sequence_is_zero(ctx, d256_kernel, fmt):
    lens = np.array([0, 20, 0, 300], np.int32)
    batch, pool, q = case(ctx, lens, 105, fmt=FMTS[fmt])
    out = run(ctx, pool, batch, q, 0, 0.0625).reshape(4, -1)
    assert np.all(oracle.bf16_to_f32(out[0]) == 0.0) and np.all(oracle.bf16_to_f32(out[2]) == 0.0)
    assert_parity(out.ravel(), oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, 0, q, 0.0625, head_dim=D),
                  what=f"empty rows {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
def test_decode256_bad_block_is_masked_and_flagged(ctx, d256_kernel, fmt):
    import torch

    lens = np.array([100, 300], np.int32)
    batch, pool, q = case(ctx, lens, 106, fmt=FMTS[fmt])
    tables = batch.tables.copy()
    tables[1, 3] = batch.n_blocks + 5  # outside the pool
    out = torch.zeros(2 * HQ * D, dtype=torch.int16, device="cuda")
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(tables), HQ, 300, 0)
    ctx.paged_decode(pool, desc, to_dev(q), out, 0.0625)
    torch.cuda.synchronize()
    assert ctx.device_errors(reset=True) & llm_hip.ERR_FLAG_BAD_BLOCK
    # sequence 0 is untouched by the bad entry
    ref = oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, 0, q, 0.0625, head_dim=D)
    assert_parity(from_dev_bf16(out)[: HQ * D], ref[: HQ * D], what=f"sequence beside the bad block {fmt}")


def gate_rows(seed, n):
    return oracle.f32_to_bf16(oracle.bf16_to_f32(oracle.normal_bf16(seed, n)) * np.float32(2.0))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("window", [0, 333])
def test_decode256_gate(ctx, d256_kernel, window, fmt):
    """The Qwen3.6 attention output gate: out * sigmoid(gate), applied before the bf16 rounding."""
    lens = workloads.uniform_lengths(16, 1, 3000, 107)
    batch, pool, q = case(ctx, lens, 107, fmt=FMTS[fmt])
    gate = gate_rows(108, lens.size * HQ * D)
    out = run(ctx, pool, batch, q, window, 0.0625, gate=gate)
    ref = oracle.apply_gate(oracle_decode(pool, batch, FMTS[fmt], HQ, HKV, window, q, 0.0625, head_dim=D),
                            oracle.bf16_to_f32(gate))
    assert_parity(out, ref, what=f"gated W={window} {fmt}")


@pytest.mark.parametrize("fmt", FMTS)
def test_decode256_noalloc_matches_decode(ctx, opts, fmt):
    """llh_paged_decode_noalloc runs split-K at head_dim 256 whatever the option asks: the
    stream kernel's partials (two slots per wavefront) exceed the static scratch.  Its
    output equals the split-K call's bit for bit and the stream call's within the bar."""
    lens = workloads.uniform_lengths(16, 256, 4096, 109)  # split-K partials within the static scratch
    batch, pool, q = case(ctx, lens, 109, fmt=FMTS[fmt])
    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    a = run(ctx, pool, batch, q, 0, 0.0625)
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    b = run(ctx, pool, batch, q, 0, 0.0625, fn="noalloc")
    assert np.array_equal(a, b)
    c = run(ctx, pool, batch, q, 0, 0.0625)
    assert_parity(c, oracle.bf16_to_f32(a), what=f"stream vs split-K {fmt}")


def test_decode256_append_then_attend(ctx, d256_kernel):
    """llh_paged_decode_append at head_dim 256 (split-K: the append kernel, then this kernel;
    stream: one launch): the pool holds the new rows and the output matches the oracle on
    that pool."""
    lens = np.array([1, 17, 256, 999, 4096], np.int32)
    batch, pool, q = case(ctx, lens, 110)
    kn = oracle.normal_bf16(111, lens.size * HKV * D).reshape(lens.size, HKV, D)
    vn = oracle.normal_bf16(112, lens.size * HKV * D).reshape(lens.size, HKV, D)
    out = run(ctx, pool, batch, q, 0, 0.0625, fn="append", kv_new=(kn, vn))
    raw = pool.raw()
    k = raw["k"].view(np.uint16).reshape(batch.n_blocks, HKV, BT, D)
    for b, L in enumerate(lens):
        p = int(L) - 1
        blk = batch.tables[b, p // BT]
        assert np.array_equal(k[blk, :, p % BT, :], kn[b])
    ref = oracle_decode(pool, batch, llm_hip.KV_BF16, HQ, HKV, 0, q, 0.0625, head_dim=D)
    assert_parity(out, ref, what="append + attend")


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("window", [0, 100])
def test_decode256_fused_append_equals_two_calls(ctx, d256_kernel, window, fmt):
    """llh_paged_decode_append at head_dim 256 in one launch (the stream kernel writes the new
    token's rows to their slot -- rounded to fp16 for fp16 pools -- and attends them from the
    registers of the block it loads): the pool and the output are bit-identical to
    llh_kv_append followed by llh_paged_decode on the same kernel; under the split-K option
    the call appends through the append kernel."""
    import torch

    lens = workloads.uniform_lengths(24, 256, 4096, 120)
    lens[:8] = [1, 2, 15, 16, 17, 256, 999, 4096]
    batch, pool_two, q = case(ctx, lens, 121, fmt=FMTS[fmt])
    _, pool_one, _ = case(ctx, lens, 121, fmt=FMTS[fmt])
    kn = oracle.normal_bf16(122, lens.size * HKV * D).reshape(lens.size, HKV, D)
    vn = oracle.normal_bf16(123, lens.size * HKV * D).reshape(lens.size, HKV, D)
    slots = np.array([int(batch.tables[b, (int(L) - 1) // BT]) * BT + (int(L) - 1) % BT for b, L in enumerate(lens)],
                     np.int64)
    ctx.append(pool_two, to_dev(slots), to_dev(kn), to_dev(vn))
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D)
    out_two = run(ctx, pool_two, batch, q, window, scale)
    fused0 = ctx.metrics()["fused_append_calls"]
    out_one = run(ctx, pool_one, batch, q, window, scale, fn="append", kv_new=(kn, vn))
    assert ctx.metrics()["fused_append_calls"] - fused0 == (1 if d256_kernel == "stream" else 0)
    a, b = pool_two.raw(), pool_one.raw()
    for key in a:
        assert np.array_equal(a[key], b[key]), key
    assert np.array_equal(out_one, out_two)
    ref = oracle_decode(pool_one, batch, FMTS[fmt], HQ, HKV, window, q, scale, head_dim=D)
    assert_parity(out_one, ref, what=f"fused append + attend W={window} {fmt}")


def coded_case(ctx, lens, seed, code_base, fmt=llm_hip.KV_BF16):
    """K random, V one-hot codes of the absolute position (attended_set.coded_rows) in
    dims 0..127, zeros above."""
    batch = workloads.paged_batch(np.asarray(lens, np.int32), BT, 0.10, seed)
    ids, src_k = workloads.block_sources(
        batch, lambda b, lo, hi: oracle.normal_bf16(seed + b, (hi - lo) * HKV * D).reshape(hi - lo, HKV, D), HKV, D)
    _, src_v = workloads.block_sources(batch, lambda b, lo, hi: coded_rows(lo, hi, HKV, D, code_base), HKV, D)
    pool = ctx.pool(fmt, BT, HKV, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(src_k), to_dev(src_v))
    return batch, pool


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("code_base", [0, 2])
@pytest.mark.parametrize("window", [0, 1, 17, 100, 4096])
def test_decode256_attended_set(ctx, d256_kernel, code_base, window, fmt):
    """q = 0: every attended token weighs exactly 1 and the output counts the position codes
    of the attended set, compared exactly with the reference's set (V's one-hot 1.0 values
    are exact in fp16 too)."""
    lens = workloads.uniform_lengths(32, 256, 4096, 113)
    lens[:8] = [1, 15, 16, 17, 33, 4096, 5000, 8191]
    batch, pool = coded_case(ctx, lens, 114, code_base, FMTS[fmt])
    q = np.zeros(lens.size * HQ * D, np.uint16)
    out = run(ctx, pool, batch, q, window, 0.0625)
    check_decode(out, lens, window, HQ, HKV, 1.0, f"d256 W={window}", head_dim=D, code_base=code_base)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("window", [0, 17, 1000])
def test_decode256_fused_append_attended_set(ctx, d256_kernel, window, fmt):
    """llh_paged_decode_append at head_dim 256 with q = 0 and position-coded V: the step
    attends the pool's [lo, len - 1) plus the new token from the call's rows -- the stale
    slot holds a decoy code (its code + 64), so attending it instead is caught -- and the
    slot holds the new token afterwards (a plain decode counts the same set)."""
    import torch

    code_base = 2
    lens = workloads.uniform_lengths(32, 256, 4096, 130)
    lens[:8] = [1, 15, 16, 17, 33, 4096, 5000, 8191]
    batch, pool = coded_case(ctx, lens, 131, code_base, FMTS[fmt])
    B = lens.size
    pos = lens.astype(np.int64) - 1
    decoy = np.zeros((B, HKV, D), np.uint16)
    new_v = np.zeros((B, HKV, D), np.uint16)
    for b, p in enumerate(pos):
        for h in range(HKV):
            decoy[b, h, (code(p, code_base + h) + 64) % 128] = 0x3F80
            new_v[b, h, code(p, code_base + h)] = 0x3F80
    slots = np.array([int(batch.tables[b, p // BT]) * BT + p % BT for b, p in enumerate(pos)], np.int64)
    ctx.append(pool, to_dev(slots), to_dev(oracle.normal_bf16(132, B * HKV * D).reshape(B, HKV, D)), to_dev(decoy))
    torch.cuda.synchronize()
    kn = oracle.normal_bf16(133, B * HKV * D).reshape(B, HKV, D)
    q = np.zeros(B * HQ * D, np.uint16)
    out = run(ctx, pool, batch, q, window, 0.0625, fn="append", kv_new=(kn, new_v))
    check_decode(out, lens, window, HQ, HKV, 1.0, f"d256 fused append W={window}", head_dim=D, code_base=code_base)
    out = run(ctx, pool, batch, q, window, 0.0625)
    check_decode(out, lens, window, HQ, HKV, 1.0, f"d256 decode after the append W={window}", head_dim=D,
                 code_base=code_base)


def test_decode256_other_shapes_stay_generic(ctx):
    """head_dim 256 with another group size, and int8 pools, take the reference-order kernel."""
    lens = np.array([5, 77, 300], np.int32)
    for Hq, fmt in ((8, llm_hip.KV_BF16), (HQ, llm_hip.KV_INT8)):
        batch = workloads.paged_batch(lens, BT, 0.10, 115)
        pool, q = build_case(ctx, batch, Hq, HKV, fmt, 115, head_dim=D)
        out = run(ctx, pool, batch, q, 0, 0.0625, Hq=Hq, expect_d256=False)
        assert_parity(out, oracle_decode(pool, batch, fmt, Hq, HKV, 0, q, 0.0625, head_dim=D), what=f"Hq{Hq} fmt{fmt}")
