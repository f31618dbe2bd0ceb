"""The attention output gate in the batched descriptors (d_gate): Qwen3.5 / 3.6 multiply the
attention output by sigmoid(gate) element-wise (attn_output_gate; apply_attention_gate,
crates/llm-backend/src/core/native_attention.rs:765-781, sigmoid_f32 math.rs:472-474).
Each decode and prefill kernel applies it in f32 before the output's bf16 rounding; the
result meets the bar against the oracle's attention times oracle.apply_gate, and the
reference's own known answer (a window of two, gate 0: [4, 2] -> [2, 1]) comes out exactly.
"""
import json
import math
import os

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, to_dev
from llm_hip import workloads
from test_gpu_decode import build_case, oracle_decode

pytestmark = pytest.mark.gpu

D = 128
BT = 16
KA = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def gate_rows(seed, n):
    """bf16 gates, N(0, 2^2): sigmoids from near 0 to near 1."""
    g = oracle.bf16_to_f32(oracle.normal_bf16(seed, n)) * np.float32(2.0)
    return oracle.f32_to_bf16(g)


def decode_gated(ctx, pool, batch, q, gate, Hq, window, scale, fn="decode", kv_new=None):
    import torch

    B = batch.seq_lens.size
    out = torch.full((B * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
    d_gate = to_dev(gate) if gate is not None else None
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(batch.seq_lens.max()), window,
                           gate=d_gate)
    if fn == "decode":
        ctx.paged_decode(pool, desc, to_dev(q), out, scale)
    elif fn == "noalloc":
        ctx.paged_decode_noalloc(pool, desc, to_dev(q), out, scale)
    else:
        ctx.paged_decode_append(pool, desc, to_dev(kv_new[0]), to_dev(kv_new[1]), to_dev(q), out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    return from_dev_bf16(out)


@pytest.mark.parametrize("kernel", ["split", "stream", "generic"])
@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_decode_gate(ctx, opts, kernel, fmt):
    if kernel == "generic":
        opts(llm_hip.OPT_FORCE_GENERIC, 1)
    else:
        opts(llm_hip.OPT_DECODE_KERNEL, kernel)
    Hq, Hkv = 16, 8
    lens = workloads.uniform_lengths(24, 1, 3000, 71)
    lens[:3] = [1, 16, 0]
    batch = workloads.paged_batch(lens, BT, 0.10, 72)
    pool, q = build_case(ctx, batch, Hq, Hkv, fmt, 73)
    gate = gate_rows(74, lens.size * Hq * D)
    scale = 1.0 / math.sqrt(D)
    for window in (0, 200):
        out = decode_gated(ctx, pool, batch, q, gate, Hq, window, scale)
        ref = oracle.apply_gate(oracle_decode(pool, batch, fmt, Hq, Hkv, window, q, scale), oracle.bf16_to_f32(gate))
        assert_parity(out, ref, what=f"gated {kernel} fmt={fmt} W={window}")
    # no gate: the plain attention
    plain = decode_gated(ctx, pool, batch, q, None, Hq, 0, scale)
    assert_parity(plain, oracle_decode(pool, batch, fmt, Hq, Hkv, 0, q, scale), what="no gate")


@pytest.mark.parametrize("fn", ["noalloc", "append"])
def test_decode_gate_other_entry_points(ctx, fn):
    """The allocation-free entry point and the fused append+attend take the same gate."""
    Hq, Hkv = 16, 8
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    batch = workloads.paged_batch(lens, BT, 0.10, 75)
    pool, q = build_case(ctx, batch, Hq, Hkv, llm_hip.KV_BF16, 76)
    gate = gate_rows(77, lens.size * Hq * D)
    kn = oracle.normal_bf16(78, lens.size * Hkv * D).reshape(lens.size, Hkv, D)
    vn = oracle.normal_bf16(79, lens.size * Hkv * D).reshape(lens.size, Hkv, D)
    out = decode_gated(ctx, pool, batch, q, gate, Hq, 0, 0.088, fn=fn, kv_new=(kn, vn))
    ref = oracle.apply_gate(oracle_decode(pool, batch, llm_hip.KV_BF16, Hq, Hkv, 0, q, 0.088),
                            oracle.bf16_to_f32(gate))
    assert_parity(out, ref, what=f"gated {fn}")


def test_decode_gate_reference_known_answer(ctx):
    """cpu_ops.rs:638-747: a window of two over values [2, 0], [0, 4], [8, 0] with equal scores
    attends [4, 2]; the zero gate half of the q projection halves it to [2, 1], exactly."""
    import torch

    c = KA["sliding_window_two"]
    pool = ctx.pool(llm_hip.KV_BF16, BT, 1, 2, 1)
    k = np.zeros((1, BT, 1, 2), np.uint16)
    v = np.zeros((1, BT, 1, 2), np.uint16)
    for t, val in enumerate(c["values"]):
        k[0, t, 0] = oracle.f32_to_bf16(np.array([1.0, 0.0], np.float32))
        v[0, t, 0] = oracle.f32_to_bf16(np.array(val, np.float32))
    ctx.write_blocks(pool, to_dev(np.array([0], np.int32)), to_dev(k), to_dev(v))
    batch = workloads.PagedBatch(np.array([3], np.int32), np.zeros((1, 1), np.int32), 1, BT, np.zeros(1, np.int32))
    q = oracle.f32_to_bf16(np.array([math.sqrt(2.0), 0.0], np.float32))
    gate = oracle.f32_to_bf16(np.zeros(2, np.float32))
    out = torch.zeros(2, dtype=torch.int16, device="cuda")
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), 1, 3, c["max_tokens"], gate=to_dev(gate))
    ctx.paged_decode(pool, desc, to_dev(q), out, 1.0 / math.sqrt(2.0))
    torch.cuda.synchronize()
    assert np.array_equal(oracle.bf16_to_f32(from_dev_bf16(out)), np.array(c["expected_after_gate"], np.float32))


@pytest.mark.parametrize("fmt,generic", [(llm_hip.KV_BF16, False), (llm_hip.KV_INT8, False), (llm_hip.KV_BF16, True)])
def test_prefill_gate(ctx, opts, fmt, generic):
    import torch

    if generic:
        opts(llm_hip.OPT_FORCE_GENERIC, 1)
    Hq, Hkv = 8, 4
    prefix, chunks = [0, 100, 333], [70, 130, 64]
    batch = workloads.paged_batch([p + c for p, c in zip(prefix, chunks)], BT, 0.10, 81)
    pool, _ = build_case(ctx, batch, Hq, Hkv, fmt, 82)
    starts = np.concatenate([[0], np.cumsum(chunks)]).astype(np.int32)
    T = int(starts[-1])
    q = oracle.normal_bf16(83, T * Hq * D)
    gate = gate_rows(84, T * Hq * D)
    scale = 1.0 / math.sqrt(D)
    for window in (0, 90):
        out = torch.full((T * Hq * D,), 0x7FC0, dtype=torch.int16, device="cuda")
        desc = ctx.prefill_desc(to_dev(starts), to_dev(batch.seq_lens), to_dev(batch.tables), Hq, max(chunks), window,
                                total_q_rows=T, gate=to_dev(gate))
        ctx.paged_prefill(pool, desc, to_dev(q), out, scale)
        torch.cuda.synchronize()
        assert ctx.device_errors() == 0, ctx.last_error()
        opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
        st, ref = opool.prefill(Hq, starts, batch.seq_lens, batch.tables, window, q, scale, threads=16)
        assert st == oracle.OK
        assert_parity(from_dev_bf16(out), oracle.apply_gate(ref, oracle.bf16_to_f32(gate)),
                      what=f"gated prefill fmt={fmt} generic={generic} W={window}")
