"""Paged GQA decode on the GPU vs the CPU oracle (2, 4, 5 and edge cases).

Every case runs the HIP kernel through the C ABI (llh_paged_decode) and compares
with the oracle's restatement of the reference per-head loop
(crates/llm-backend/src/core/native_attention.rs:707-773) run on the pool the
GPU actually holds, at the BASELINE bar: bf16 output within max-abs 2e-2 and
mean-abs 2e-3 of the fp32 reference rounded to bf16.  The kernel's sticky error
flags must stay clear (no out-of-pool block touched, no split overflow).
"""
import math
import os

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, rows_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu

D = 128
BT = 16


def build_case(ctx, batch, Hq, Hkv, fmt, seed, head_dim=D):
    bt = batch.block_tokens
    ids, src_k = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, head_dim),
                                         Hkv, head_dim)
    _, src_v = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, head_dim),
                                       Hkv, head_dim)
    pool = ctx.pool(fmt, bt, Hkv, head_dim, batch.n_blocks)
    if ids.size:
        ctx.write_blocks(pool, to_dev(ids), to_dev(src_k), to_dev(src_v))
    q = oracle.normal_bf16(seed + 3, batch.seq_lens.size * Hq * head_dim)
    return pool, q


def run_decode(ctx, pool, batch, q, Hq, window, scale, head_dim=D, max_seq_len=None):
    import torch

    B = batch.seq_lens.size
    d_lens, d_tab, d_q = to_dev(batch.seq_lens), to_dev(batch.tables), to_dev(q)
    d_out = torch.full((B * Hq * head_dim,), 0x7FC0, dtype=torch.int16, device="cuda")  # NaN fill
    msl = int(batch.seq_lens.max()) if max_seq_len is None else max_seq_len
    desc = ctx.decode_desc(d_lens, d_tab, Hq, msl, window)
    before = ctx.metrics()["stream_decode_calls"]
    ctx.paged_decode(pool, desc, d_q, d_out, scale)
    torch.cuda.synchronize()
    streamed = ctx.metrics()["stream_decode_calls"] - before
    forced = ctx.get_option(llm_hip.OPT_DECODE_KERNEL)
    if forced == llm_hip.DECODE_KERNELS["stream"] and head_dim == D and batch.block_tokens == BT:
        assert streamed == 1, "the stream kernel did not run"
    if forced == llm_hip.DECODE_KERNELS["split"]:
        assert streamed == 0, "the stream kernel ran under the split-K option"
    return from_dev_bf16(d_out)


def oracle_decode(pool, batch, fmt, Hq, Hkv, window, q, scale, head_dim=D):
    opool = oracle.Pool.from_raw(fmt, batch.block_tokens, Hkv, head_dim, batch.n_blocks, pool.raw())
    st, ref = opool.decode(Hq, batch.seq_lens, batch.tables, window, q, scale, threads=16)
    assert st == oracle.OK
    return ref


def check(ctx, batch, Hq, Hkv, fmt=llm_hip.KV_BF16, window=0, seed=1, head_dim=D, what=""):
    scale = 1.0 / math.sqrt(head_dim)
    pool, q = build_case(ctx, batch, Hq, Hkv, fmt, seed, head_dim)
    out = run_decode(ctx, pool, batch, q, Hq, window, scale, head_dim)
    assert ctx.device_errors() == 0, ctx.last_error()
    ref = oracle_decode(pool, batch, fmt, Hq, Hkv, window, q, scale, head_dim)
    return assert_parity(out, ref, what=what)


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_decode_unaligned_rows_take_the_generic_kernel(ctx, fmt):
    """q and out 2 bytes off 16-byte alignment: the element-wise generic kernel
    runs (no stream launch) and matches the oracle like the fast path."""
    import torch

    Hq, Hkv = 8, 2
    batch = workloads.paged_batch([37, 300, 1], BT, 0.1, 41)
    scale = 1.0 / math.sqrt(D)
    pool, q = build_case(ctx, batch, Hq, Hkv, fmt, 41)

    def shifted(n):
        flat = torch.zeros(n + 1, dtype=torch.int16, device="cuda")
        view = flat[1:]
        assert view.data_ptr() % 16 != 0
        return view

    B = batch.seq_lens.size
    d_q = shifted(q.size)
    d_q.copy_(to_dev(q).view(-1))
    d_out = shifted(B * Hq * D)
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(batch.seq_lens.max()))
    before = ctx.metrics()["stream_decode_calls"]
    ctx.paged_decode(pool, desc, d_q, d_out, scale)
    torch.cuda.synchronize()
    assert ctx.metrics()["stream_decode_calls"] == before
    assert ctx.device_errors() == 0, ctx.last_error()
    ref = oracle_decode(pool, batch, fmt, Hq, Hkv, 0, q, scale)
    assert_parity(from_dev_bf16(d_out), ref, what="unaligned rows")


def identity_batch(lens, block_tokens=BT):
    lens = np.asarray(lens, dtype=np.int32)
    nblk = (lens + block_tokens - 1) // block_tokens
    mb = max(1, int(nblk.max()))
    tables = np.full((lens.size, mb), -1, dtype=np.int32)
    cur = 0
    for b, n in enumerate(nblk):
        tables[b, :n] = np.arange(cur, cur + n)
        cur += n
    return workloads.PagedBatch(lens, tables, max(cur, 1), block_tokens, np.zeros(lens.size, np.int32))


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16])
def test_decode_c1_identity_table(ctx, fmt):
    """B=1, L=512, Hq16/Hkv8, D128, 16-token blocks, identity table."""
    check(ctx, identity_batch([512]), 16, 8, fmt, seed=workloads.SEED_BASE + 0, what="C1")


@pytest.fixture(params=["split", "stream"])
def decode_kernel(request, opts):
    """Both tuned decode kernels: split-K (one workgroup per split) and the persistent stream
    kernel (LLH_OPT_DECODE_KERNEL forces the choice the library otherwise makes by batch size)."""
    opts(llm_hip.OPT_DECODE_KERNEL, request.param)
    return request.param


def test_decode_c1_matches_golden_fixture(ctx, decode_kernel):
    """configs[0] against the committed fixture tests/golden/c1_decode.json (written by
    tests/golden/make_golden.py): the same seeded rows go into a 32-block pool and the
    device output is held to the parity bar against the fixture's f32 output."""
    import json

    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "c1_decode.json")))
    L, Hq, Hkv = g["row_count"], g["q_heads"], g["kv_heads"]
    assert (L, Hq, Hkv, g["head_dim"]) == (512, 16, 8, D) and g["seed"] == workloads.SEED_BASE
    pool, q = build_case(ctx, identity_batch([L]), Hq, Hkv, llm_hip.KV_BF16, g["seed"])
    assert np.array_equal(q, oracle.normal_bf16(g["seed"] + 3, Hq * D))  # the fixture's q
    out = run_decode(ctx, pool, identity_batch([L]), q, Hq, 0, g["scale"])
    assert ctx.device_errors() == 0, ctx.last_error()
    assert_parity(out, np.array(g["output_f32"], np.float32), what=f"C1 golden kernel={decode_kernel}")


def test_decode_c2_full_size(ctx, decode_kernel):
    """B=32, L~U[256,4096], permuted pool +10% free blocks."""
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    batch = workloads.paged_batch(lens, BT, 0.10, workloads.SEED_BASE + 1)
    assert batch.n_blocks == math.ceil(1.1 * int(np.sum((lens + 15) // 16)))
    check(ctx, batch, 16, 8, seed=workloads.SEED_BASE + 1, what=f"C2 kernel={decode_kernel}")


@pytest.mark.parametrize("split_blocks", [4, 8, 64])
def test_decode_split_sizes(ctx, opts, split_blocks):
    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    opts(llm_hip.OPT_DECODE_SPLIT_BLOCKS, split_blocks)
    lens = workloads.uniform_lengths(12, 1, 5000, 17)
    batch = workloads.paged_batch(lens, BT, 0.10, 17)
    check(ctx, batch, 32, 8, seed=17, what=f"split={split_blocks}")


@pytest.mark.parametrize("n_splits", [2, 8, 9, 17, 33, 64, 65, 97, 128, 129, 130, 200])
def test_decode_merge_split_counts(ctx, opts, n_splits):
    """The merge launch's layouts: every partial in registers with one (<= 64 splits)
    or two (<= 128) (max, sum) pairs per lane, in register sets of 8 / 16 / 32 / 64 /
    128; beyond 128 the pairs reduced through LDS with the first 96 partials loaded up
    front and the rest in chunks of 32.  Two sequences per count (n and n - 1 splits)
    at the boundaries, 4-block splits."""
    opts(llm_hip.OPT_DECODE_SPLIT_BLOCKS, 4)
    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    lens = np.array([BT * 4 * n_splits - 5, BT * 4 * (n_splits - 1) + 1], np.int32)  # n_splits each
    batch = workloads.paged_batch(lens, BT, 0.10, 300 + n_splits)
    check(ctx, batch, 16, 8, seed=300 + n_splits, what=f"merge of {n_splits} splits")


def test_decode_split_k_is_deterministic(ctx, opts):
    """Many splits per sequence and many repeated calls: the merge combines partials in
    split order, so every call must give identical bits."""
    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    opts(llm_hip.OPT_DECODE_SPLIT_BLOCKS, 4)
    lens = workloads.uniform_lengths(32, 256, 4096, 23)
    batch = workloads.paged_batch(lens, BT, 0.10, 23)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 23)
    first = run_decode(ctx, pool, batch, q, 16, 0, 0.088)
    for _ in range(30):
        assert np.array_equal(run_decode(ctx, pool, batch, q, 16, 0, 0.088), first)
    assert ctx.device_errors() == 0
    ref = oracle_decode(pool, batch, llm_hip.KV_BF16, 16, 8, 0, q, 0.088)
    assert_parity(first, ref, what="split-K, split 4")


@pytest.mark.parametrize("lens", [[1], [15, 16, 17], [31, 33, 255, 256, 257], [1000, 4095, 4096, 4097]])
def test_decode_ragged_lengths(ctx, decode_kernel, lens):
    batch = workloads.paged_batch(lens, BT, 0.10, seed=len(lens))
    check(ctx, batch, 16, 8, seed=7, what=f"lens={lens} {decode_kernel}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
def test_decode_gqa_groups(ctx, decode_kernel, Hq, Hkv):
    lens = [300, 700, 1200]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=Hq * 10 + Hkv)
    check(ctx, batch, Hq, Hkv, seed=11, what=f"Hq={Hq} Hkv={Hkv}")


def test_decode_c4_sliding_window_skips_blocks(ctx, decode_kernel):
    """configs[3] decode: 4 x 32768 positions, window 4096, shuffled blocks.
    Blocks wholly before the window are not in the pool (table entry -1): any
    access would raise the bad-block flag, so a clear flag proves they are skipped."""
    L, W = 32768, 4096
    lens = [L] * 4
    first = [(L - W) // BT] * 4
    batch = workloads.paged_batch(lens, BT, 0.10, workloads.SEED_BASE + 3, resident_from=first)
    check(ctx, batch, 16, 8, window=W, seed=workloads.SEED_BASE + 3, what="C4 decode")


@pytest.mark.parametrize("W,lens", [(1, [5, 16, 17]), (17, [16, 17, 40, 100]), (100, [50, 99, 100, 101, 333])])
def test_decode_window_edges(ctx, decode_kernel, W, lens):
    batch = workloads.paged_batch(lens, BT, 0.10, seed=W)
    check(ctx, batch, 16, 8, window=W, seed=W + 1, what=f"W={W}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_c5_quantized(ctx, decode_kernel, fmt):
    """configs[4] shape (Hq32/Hkv8, L=8192) at 16 of the 64 sequences; bench.py runs all 64."""
    lens = [8192] * 16
    batch = workloads.paged_batch(lens, BT, 0.0, workloads.SEED_BASE + 4)
    check(ctx, batch, 32, 8, fmt, seed=workloads.SEED_BASE + 4, what=f"C5 fmt={fmt}")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_quantized_ragged_window(ctx, decode_kernel, fmt):
    lens = [1, 17, 250, 1025, 3000]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=fmt)
    check(ctx, batch, 16, 8, fmt, window=0, seed=21, what=f"fmt={fmt}")
    check(ctx, batch, 16, 8, fmt, window=333, seed=22, what=f"fmt={fmt} W=333")


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
def test_decode_quantized_gqa_groups(ctx, decode_kernel, fmt, Hq, Hkv):
    """Every group size through both lane layouts of the quantized path: G <= 4
    scores one (token, head) per lane (token-lane layout, q words of 32 dims),
    G = 8 keeps the row layout; with and without a window cutting blocks."""
    lens = [300, 700, 1200]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=Hq * 10 + Hkv + fmt)
    check(ctx, batch, Hq, Hkv, fmt, seed=13, what=f"fmt={fmt} Hq={Hq} Hkv={Hkv}")
    check(ctx, batch, Hq, Hkv, fmt, window=250, seed=14, what=f"fmt={fmt} Hq={Hq} Hkv={Hkv} W=250")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (16, 2)])
def test_decode_int8_query_magnitudes(ctx, decode_kernel, Hq, Hkv):
    """int8 pools score q . k on integer dot products against q in 16-bit fixed
    point, one step per query head (2^e from the head's largest |q|).  Heads of
    very different magnitude side by side (so a lane taking another head's step
    would be off by orders of magnitude), outlier elements 100x the rest, bf16
    subnormal and all-zero heads all meet the oracle bar."""
    lens = [300, 700, 1200]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=Hq + Hkv)
    pool, q = build_case(ctx, batch, Hq, Hkv, llm_hip.KV_INT8, seed=31)
    B = len(lens)
    qf = oracle.bf16_to_f32(q).reshape(B, Hq, D).copy()
    mags = [1.0, 1e-30, 6.0, 1e-3, 1e-39, 0.0, 3e4, 0.25]
    for h in range(Hq):
        qf[:, h, :] *= np.float32(mags[h % len(mags)])
        if h % 3 == 1:
            qf[:, h, 5 + h] *= np.float32(100.0)
    qb = oracle.f32_to_bf16(qf.ravel())
    scale = 1.0 / math.sqrt(D)
    for window in (0, 250):
        out = run_decode(ctx, pool, batch, qb, Hq, window, scale)
        assert ctx.device_errors() == 0, ctx.last_error()
        ref = oracle_decode(pool, batch, llm_hip.KV_INT8, Hq, Hkv, window, qb, scale)
        assert_parity(out, ref, what=f"Hq={Hq} Hkv={Hkv} W={window}")


def test_decode_int8_nan_query_stays_in_its_head(ctx, decode_kernel):
    """A NaN in one query head's q makes that head's output NaN (as f32 scores
    would) and leaves every other head of the sequence at the oracle bar."""
    Hq, Hkv = 32, 8
    lens = [500, 900]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=41)
    pool, q = build_case(ctx, batch, Hq, Hkv, llm_hip.KV_INT8, seed=42)
    qn = q.reshape(len(lens), Hq, D).copy()
    qn[1, 5, 17] = 0x7FC0  # NaN in sequence 1, head 5
    scale = 1.0 / math.sqrt(D)
    out = run_decode(ctx, pool, batch, qn.ravel(), Hq, 0, scale).reshape(len(lens), Hq, D)
    assert ctx.device_errors() == 0, ctx.last_error()
    assert np.all(np.isnan(oracle.bf16_to_f32(out[1, 5])))
    ref = oracle_decode(pool, batch, llm_hip.KV_INT8, Hq, Hkv, 0, q, scale).reshape(len(lens), Hq, D)
    keep = np.ones((len(lens), Hq), bool)
    keep[1, 5] = False
    assert_parity(out[keep], ref[keep], what="heads without the NaN")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_bad_block_is_masked_and_flagged(ctx, decode_kernel, fmt):
    """A table entry outside the pool raises the sticky flag, its tokens are
    masked (the output stays finite) and the other sequences are unaffected."""
    batch = workloads.paged_batch([64, 64], BT, 0.10, seed=19)
    pool, q = build_case(ctx, batch, 16, 8, fmt, 19)
    bad = workloads.PagedBatch(batch.seq_lens, batch.tables.copy(), batch.n_blocks, BT, batch.first_block)
    bad.tables[1, 2] = batch.n_blocks + 5
    out = run_decode(ctx, pool, bad, q, 16, 0, 0.1)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK
    assert np.all(np.isfinite(oracle.bf16_to_f32(out)))
    first = workloads.PagedBatch(batch.seq_lens[:1], batch.tables[:1], batch.n_blocks, BT, batch.first_block[:1])
    ref = oracle_decode(pool, first, fmt, 16, 8, 0, q[: 16 * D], 0.1)
    assert_parity(out[: 16 * D], ref, what=f"good sequence beside a bad one, fmt={fmt}")


def test_decode_empty_sequence_is_zero(ctx, decode_kernel):
    """R = 0 gives a zero output (weighted sum of nothing, primitives.rs:1125-1128)."""
    batch = workloads.paged_batch([0, 20], BT, 0.10, seed=3)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 5)
    out = run_decode(ctx, pool, batch, q, 16, 0, 0.125)
    assert ctx.device_errors() == 0
    assert np.all(oracle.bf16_to_f32(out[: 16 * D]) == 0.0)
    ref = oracle_decode(pool, batch, llm_hip.KV_BF16, 16, 8, 0, q, 0.125)
    assert_parity(out, ref, what="empty + 20")


@pytest.mark.parametrize("head_dim,bt,Hq,Hkv", [(64, 8, 8, 2), (32, 16, 6, 3), (128, 32, 16, 8)])
def test_decode_generic_shapes(ctx, head_dim, bt, Hq, Hkv):
    """Shapes outside the tuned kernel run the reference-order kernel."""
    batch = workloads.paged_batch([5, 77, 300], bt, 0.10, seed=head_dim)
    check(ctx, batch, Hq, Hkv, seed=31, head_dim=head_dim, what=f"D={head_dim} BT={bt}")


@pytest.mark.parametrize("window", [0, 100])
def test_decode_int8_row_pool(ctx, window):
    """The reference's own int8 layout (LLH_KV_INT8_ROW: f32 scale per token row over all
    kv heads) runs the reference-order kernel, on the tuned shape too."""
    batch = workloads.paged_batch([5, 77, 300, 1024], BT, 0.10, seed=44)
    check(ctx, batch, 16, 8, llm_hip.KV_INT8_ROW, window=window, seed=45, what=f"int8 row W={window}")


def test_decode_bad_block_raises_flag(ctx, decode_kernel):
    batch = workloads.paged_batch([64, 64], BT, 0.10, seed=9)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 9)
    bad = workloads.PagedBatch(batch.seq_lens, batch.tables.copy(), batch.n_blocks, BT, batch.first_block)
    bad.tables[1, 2] = batch.n_blocks + 5  # outside the pool: the kernel's bounds check turns it into a flag
    run_decode(ctx, pool, bad, q, 16, 0, 0.1)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK


def test_decode_max_seq_len_bound_raises_flag(ctx, decode_kernel):
    batch = workloads.paged_batch([2000], BT, 0.10, seed=10)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 10)
    run_decode(ctx, pool, batch, q, 16, 0, 0.1, max_seq_len=100)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_TOO_MANY_SPLITS


def test_decode_repeated_calls_are_identical(ctx, decode_kernel):
    """Split counters return to zero after every call: repeat calls give identical bits."""
    lens = workloads.uniform_lengths(8, 256, 4096, 99)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=99)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 99)
    outs = [run_decode(ctx, pool, batch, q, 16, 0, 0.09) for _ in range(3)]
    assert ctx.device_errors() == 0
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[1], outs[2])


def test_decode_shape_errors(ctx):
    import torch

    batch = workloads.paged_batch([10], BT, 0.10, seed=1)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 1)
    d_lens, d_tab = to_dev(batch.seq_lens), to_dev(batch.tables)
    d_q, d_out = to_dev(q), torch.empty(16 * D, dtype=torch.int16, device="cuda")
    desc = ctx.decode_desc(d_lens, d_tab, 12, 10)  # 12 q heads is not a multiple of 8 kv heads
    with pytest.raises(llm_hip.LlhError) as e:
        ctx.paged_decode(pool, desc, d_q, d_out, 0.1)
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    desc = ctx.decode_desc(d_lens, d_tab, 16, 10, window=-1)
    with pytest.raises(llm_hip.LlhError):
        ctx.paged_decode(pool, desc, d_q, d_out, 0.1)
    desc = ctx.decode_desc(d_lens, d_tab, 16, 10)
    with pytest.raises(llm_hip.LlhError) as e:
        ctx.paged_decode(pool, desc, d_q, d_out, float("nan"))
    assert e.value.status == llm_hip.ERR_NON_FINITE


# ---- the persistent stream kernel's partition -------------------------------------------------

@pytest.mark.parametrize("wgs", [1, 2, 3, 7, 16, 64])
def test_stream_small_grids_cut_segments_everywhere(ctx, wgs, opts):
    """Small grids put wavefront boundaries at every possible place relative to the
    (kv head, block) segments: ranges that start on a segment's last block, span several
    kv heads, or hold one unit; each cut segment is merged from its partials."""
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    opts(llm_hip.OPT_DECODE_STREAM_WGS, wgs)
    lens = [1, 16, 17, 250, 4096, 33, 1000][: max(1, min(7, 2 * wgs - 1))]
    batch = workloads.paged_batch(lens, BT, 0.10, seed=40 + wgs)
    check(ctx, batch, 16, 8, seed=41 + wgs, what=f"stream wgs={wgs}")


@pytest.mark.parametrize("wgs", [1, 3])
@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_stream_ranges_span_many_sequences(ctx, wgs, fmt, opts):
    """The partition runs over all units of the step, so one wavefront's range crosses
    sequence boundaries: on 4 or 12 wavefronts, 100 short sequences (empty ones among
    them, lengths taken from beyond the first 64 lanes too) give ranges holding dozens of
    sequences, some starting or ending inside one; with and without a window."""
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    opts(llm_hip.OPT_DECODE_STREAM_WGS, wgs)
    lens = workloads.uniform_lengths(100, 0, 40, 48 + wgs)
    lens[::17] = 0
    batch = workloads.paged_batch(lens, BT, 0.10, seed=49 + wgs)
    check(ctx, batch, 16, 8, fmt, seed=50 + wgs, what=f"stream wgs={wgs} fmt={fmt}")
    check(ctx, batch, 16, 8, fmt, window=20, seed=51 + wgs, what=f"stream wgs={wgs} fmt={fmt} W=20")


def test_stream_many_partials_per_segment(ctx, opts):
    """Few long sequences on a large grid: ~64 partials per segment, merged in rounds of 16."""
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    opts(llm_hip.OPT_DECODE_STREAM_WGS, 512)
    batch = workloads.paged_batch([4096] * 4, BT, 0.10, seed=44)
    check(ctx, batch, 16, 8, seed=45, what="stream 4 x 4096")


def test_stream_batch_over_64(ctx, decode_kernel):
    """Batches beyond one wavefront's 64 lanes take the chunked length scan."""
    lens = workloads.uniform_lengths(150, 0, 700, 46)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=46)
    check(ctx, batch, 16, 8, seed=47, what=f"B=150 {decode_kernel}")


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (64, 8), (32, 4)])
def test_stream_group_sizes(ctx, Hq, Hkv, opts):
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    lens = workloads.uniform_lengths(24, 1, 3000, Hq)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=Hq + Hkv)
    check(ctx, batch, Hq, Hkv, seed=48, what=f"stream Hq={Hq} Hkv={Hkv}")


def test_stream_is_the_default_for_large_bf16_batches(ctx, opts):
    """Without an override the library picks the stream kernel for C2 and split-K for C1:
    both give the same result as the forced choice, bit for bit."""
    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    batch = workloads.paged_batch(lens, BT, 0.10, workloads.SEED_BASE + 1)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 50)
    before = ctx.metrics()["stream_decode_calls"]
    auto = run_decode(ctx, pool, batch, q, 16, 0, 0.088)
    assert ctx.metrics()["stream_decode_calls"] == before + 1
    c1 = identity_batch([512])
    c1pool, c1q = build_case(ctx, c1, 16, 8, llm_hip.KV_BF16, 51)
    run_decode(ctx, c1pool, c1, c1q, 16, 0, 0.088)
    assert ctx.metrics()["stream_decode_calls"] == before + 1  # C1 stays on split-K
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    assert np.array_equal(run_decode(ctx, pool, batch, q, 16, 0, 0.088), auto)
    opts(llm_hip.OPT_DECODE_KERNEL, "split")
    split = run_decode(ctx, pool, batch, q, 16, 0, 0.088)
    assert not np.array_equal(split, auto)  # different summation order: proves the choice
    assert ctx.device_errors() == 0


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_stream_is_the_default_for_large_quantized_batches(ctx, fmt, opts):
    """A C5-shaped batch (64 sequences, Hq32/Hkv8) of int8 / fp8 blocks takes the stream
    kernel without an override and meets the bar."""
    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    batch = workloads.paged_batch(np.full(64, 2048, np.int32), BT, 0.10, 61)
    before = ctx.metrics()["stream_decode_calls"]
    check(ctx, batch, 32, 8, fmt=fmt, seed=61, what=f"default kernel fmt={fmt}")
    assert ctx.metrics()["stream_decode_calls"] == before + 1


# ---- block-table span: rows are read modulo their length ---------------------------------------

def test_decode_ring_of_exactly_window_blocks(ctx, decode_kernel):
    """A sliding window served by a ring of W/16 blocks (positions p and p + W share a slot):
    the W attended positions fill the ring exactly, so a misaligned window touches the same
    ring block at both ends with disjoint offsets.  Only in-window rows are written."""
    import torch

    W, nb, Hq, Hkv = 64, 4, 16, 8
    lens = np.array([1000, 77, 64, 65, 7], np.int32)
    B = lens.size
    tables = (np.arange(B * nb, dtype=np.int32).reshape(B, nb) * 3 + 1) % (B * nb + 3)
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, B * nb + 3)
    slots, ks, vs = [], [], []
    for b in range(B):
        lo = max(0, int(lens[b]) - W)
        for p in range(lo, int(lens[b])):
            slots.append(int(tables[b, (p // BT) % nb]) * BT + p % BT)
            ks.append(rows_bf16(71, b, p, p + 1, Hkv, D)[0])
            vs.append(rows_bf16(72, b, p, p + 1, Hkv, D)[0])
    ctx.append(pool, to_dev(np.array(slots, np.int64)), to_dev(np.stack(ks)), to_dev(np.stack(vs)))
    torch.cuda.synchronize()
    batch = workloads.PagedBatch(lens, tables, B * nb + 3, BT, np.zeros(B, np.int32))
    q = oracle.normal_bf16(73, B * Hq * D)
    out = run_decode(ctx, pool, batch, q, Hq, W, 0.09)
    assert ctx.device_errors() == 0, ctx.last_error()
    ref = oracle_decode(pool, batch, llm_hip.KV_BF16, Hq, Hkv, W, q, 0.09)
    assert_parity(out, ref, what=f"ring of {nb} blocks, W={W} {decode_kernel}")


def test_decode_span_beyond_table_row_is_rejected(ctx):
    """A bound that lets a sequence attend more tokens than its table row holds is a shape
    error on the host (two attended positions would share a slot)."""
    import torch

    pool = ctx.pool(llm_hip.KV_BF16, BT, 8, D, 8)
    lens = torch.tensor([60], dtype=torch.int32, device="cuda")
    tab = torch.zeros((1, 4), dtype=torch.int32, device="cuda")  # 4 blocks = 64 tokens
    q = torch.zeros(16 * D, dtype=torch.int16, device="cuda")
    out = torch.zeros_like(q)
    for msl, window in ((65, 0), (100, 65), (1000, 65)):
        with pytest.raises(llm_hip.LlhError) as e:
            ctx.paged_decode(pool, ctx.decode_desc(lens, tab, 16, msl, window), q, out, 0.1)
        assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    for msl, window in ((64, 0), (1000, 64), (64, 100)):  # these fit
        ctx.paged_decode(pool, ctx.decode_desc(lens, tab, 16, msl, window), q, out, 0.1)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0


def test_decode_span_flag_when_lengths_exceed_the_bound(ctx, decode_kernel):
    """Lengths past the host bound reach the kernel: a sequence attending more tokens than its
    table row holds raises the span flag and is not attended (no aliased blocks read)."""
    batch = workloads.paged_batch([70], BT, 0.10, seed=12)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 12)
    short = workloads.PagedBatch(batch.seq_lens, batch.tables[:, :4].copy(), batch.n_blocks, BT, batch.first_block)
    run_decode(ctx, pool, short, q, 16, 0, 0.1, max_seq_len=64)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_SPAN


def test_decode_weights_sum_to_one_exactly(ctx, decode_kernel):
    """The softmax normaliser sums exactly the bf16 weights that multiply V: with V = 1 in
    every row, the output is 1.0 exactly.  Every fourth token scores 0 (the max of each
    4-token group the kernels keep a running max for) and the others score -0.9945 in log2
    units, whose weight 2^-0.9945 = 0.50188 rounds to 0.5 in bf16; a normaliser over the
    unrounded weights would give (1 + 3 * 0.5) / (1 + 3 * 0.50188) = 0.99775 -> bf16 0.99609375."""
    Hq, Hkv = 16, 8
    lens = np.array([256, 1000, 33, 4096], np.int32)
    batch = workloads.paged_batch(lens, BT, 0.10, seed=77)
    neg = oracle.f32_to_bf16(np.array([-0.99609375], np.float32))[0]
    one = oracle.f32_to_bf16(np.array([1.0], np.float32))[0]

    def krows(b, lo, hi):
        r = np.zeros((hi - lo, Hkv, D), np.uint16)
        for i, p in enumerate(range(lo, hi)):
            if p % 4 != 0:
                r[i, :, 0] = neg
        return r

    ids, src_k = workloads.block_sources(batch, krows, Hkv, D)
    _, src_v = workloads.block_sources(batch, lambda b, lo, hi: np.full((hi - lo, Hkv, D), one, np.uint16), Hkv, D)
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(src_k), to_dev(src_v))
    q = np.zeros((lens.size, Hq, D), np.uint16)
    q[:, :, 0] = one
    scale = 0.6921  # score * scale * log2(e) = -0.99609375 * 0.99849 = -0.99459
    for window in (0, 100):
        out = run_decode(ctx, pool, batch, q.ravel(), Hq, window, scale)
        assert ctx.device_errors() == 0, ctx.last_error()
        assert np.all(out == one), np.unique(oracle.bf16_to_f32(out))


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_c5_full_launch_sampled(ctx, opts, fmt):
    """configs[4] exactly as bench.py times it: all 64 sequences of 8192 tokens (Hq32/Hkv8)
    in one launch, so the stream kernel's B=64 partition, cut segments and merges are the
    benchmarked ones; 8 sequences (first and last included) are checked against the oracle."""
    import torch

    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    B, L, Hq, Hkv = 64, 8192, 32, 8
    batch = workloads.paged_batch([L] * B, BT, 0.0, workloads.SEED_BASE + 4)
    pool = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
    g = torch.Generator(device="cuda")
    g.manual_seed(workloads.SEED_BASE + 4 + fmt)
    ids = torch.from_numpy(batch.tables.ravel().copy()).cuda()
    for s in range(0, ids.numel(), 4096):
        idx = ids[s:s + 4096]
        k = torch.randn((idx.numel(), BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((idx.numel(), BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
        ctx.write_blocks(pool, idx, k, v)
    del k, v
    q = oracle.normal_bf16(workloads.SEED_BASE + 40 + fmt, B * Hq * D)
    scale = 1.0 / math.sqrt(D)
    before = ctx.metrics()["stream_decode_calls"]
    out = run_decode(ctx, pool, batch, q, Hq, 0, scale)
    assert ctx.metrics()["stream_decode_calls"] == before + 1, "C5 did not take the stream kernel"
    assert ctx.device_errors() == 0, ctx.last_error()
    sub = [0, 9, 17, 31, 32, 47, 55, 63]
    opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
    st, ref = opool.decode(Hq, batch.seq_lens[sub], batch.tables[sub], 0, q.reshape(B, -1)[sub].ravel(), scale,
                           threads=16)
    assert st == oracle.OK
    assert_parity(out.reshape(B, -1)[sub], ref, what=f"C5 full launch fmt={fmt}")
    pool.close()


def test_stream_and_split_k_steps_alternate_on_one_stream(ctx, opts):
    """Stream steps (per-wavefront partial slots and segment descriptors) and split-K steps
    (per-split partials) alternate on one stream's workspace; each keeps giving the bits it
    gave first, and both meet the oracle bar."""
    import torch

    lens = workloads.uniform_lengths(32, 256, 4096, 61)
    batch = workloads.paged_batch(lens, BT, 0.10, 61)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 61)
    small = workloads.paged_batch([3000, 17, 900], BT, 0.10, 62)
    spool, sq = build_case(ctx, small, 16, 8, llm_hip.KV_BF16, 62)
    first = {}
    for it in range(6):
        for kern, (bt, pl, qq) in (("stream", (batch, pool, q)), ("split", (small, spool, sq))):
            opts(llm_hip.OPT_DECODE_KERNEL, kern)
            out = run_decode(ctx, pl, bt, qq, 16, 0, 0.09)
            if it == 0:
                first[kern] = out
            assert np.array_equal(out, first[kern]), (kern, it)
    assert ctx.device_errors() == 0
    assert_parity(first["stream"], oracle_decode(pool, batch, llm_hip.KV_BF16, 16, 8, 0, q, 0.09), what="stream")
    assert_parity(first["split"], oracle_decode(spool, small, llm_hip.KV_BF16, 16, 8, 0, sq, 0.09), what="split")


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_stream_segment_cut_into_hundreds_of_pieces(ctx, opts, fmt):
    """One 32768-token sequence on the full stream grid: each kv head's segment is cut into
    ~256 pieces, which the merge launch combines in rounds of 32."""
    opts(llm_hip.OPT_DECODE_KERNEL, "stream")
    batch = workloads.paged_batch([32768], BT, 0.0, 63)
    check(ctx, batch, 16, 8, fmt, seed=63, what=f"1 x 32768 stream fmt={fmt}")
