"""The NativeMatvecBackend attention hooks over the device LayerKvCache mirror,
on the reference's own test cases (tests/golden/known_answers.json).

These read like the reference tests they come from: a LayerKvCache is built
with append/append_sliding, then full_attention_cache_mix_f32_in_place runs
on the GPU (the reference-order kernel) and is compared with the closed form
or with reference_attention, at the reference's tolerances (1e-4 for exact
inputs, 1e-2 for the 257-row f16-mirror case, 3e-2 for int8).  K/V are stored
as bf16 (or int8 with fp16 per (token, head) scales), so inputs that are not
exact in bf16 use the reference's mirror tolerances.
"""
import json
import math
import os

import numpy as np
import pytest

import llm_hip
import oracle
from llm_hip import HipNativeMatvecBackend, LayerKvCache

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))


def mix(ctx, cache, query, row_count, hq, hkv, d, scale):
    out = np.zeros(hq * d, np.float32)
    handled = HipNativeMatvecBackend(ctx).full_attention_cache_mix_f32_in_place(cache, query, row_count, hq, hkv, d,
                                                                                scale, out)
    assert handled
    return out


def test_full_attention_cache_mix_matches_reference_values(ctx):
    c = KA["two_head_closed_form"]
    cache = LayerKvCache.new(ctx, 8, 1, 2)
    keys = np.array(c["keys"], np.float32).reshape(2, 2)
    vals = np.array(c["values"], np.float32).reshape(2, 2)
    for k, v in zip(keys, vals):
        cache.append_sliding(k, v)
    out = mix(ctx, cache, c["query"], 2, 2, 1, 2, 1.0)
    assert np.max(np.abs(out - np.array(c["expected"]))) < c["tolerance"]


def test_full_attention_cache_mix_int8_matches_reference_values(ctx):
    """primitives/tests.rs:413-466 with the device int8 layout (fp16 scale per (token, head))."""
    c = KA["int8_closed_form"]
    cache = LayerKvCache.new_with_config(ctx, 8, 1, 2, llm_hip.KV_INT8)
    cache.append_sliding([1.0, 0.0], [10.0, 0.0])
    cache.append_sliding([0.0, 1.0], [0.0, 10.0])
    out = mix(ctx, cache, c["query"], 2, 2, 1, 2, 1.0)
    # |error| <= 10 * (f16 rounding of 10/127) ~ 5e-3; the reference's f32 scales give 1e-4
    assert np.max(np.abs(out - np.array(c["expected"]))) < 1e-2


def test_int8_row_cache_stores_the_reference_codes_and_scales(ctx):
    """primitives/tests.rs:413-466 on LLH_KV_INT8_ROW, the reference's own int8 layout: the
    cache holds exactly the test's key/value codes and f32 scales (keys() / values() return
    code * scale), and the output meets the test's own tolerance."""
    c = KA["int8_closed_form"]
    cache = LayerKvCache.new_with_config(ctx, 8, 1, 2, llm_hip.KV_INT8_ROW)
    cache.append_sliding([1.0, 0.0], [10.0, 0.0])
    cache.append_sliding([0.0, 1.0], [0.0, 10.0])
    kc = np.array(c["key_codes"], np.float32).reshape(2, 2)
    vc = np.array(c["value_codes"], np.float32).reshape(2, 2)
    ks = np.array(c["key_scales"], np.float32)[:, None]
    vs = np.array(c["value_scales"], np.float32)[:, None]
    assert np.array_equal(cache.keys(), (kc * ks).ravel())
    assert np.array_equal(cache.values(), (vc * vs).ravel())
    out = mix(ctx, cache, c["query"], 2, 2, 1, 2, 1.0)
    assert np.max(np.abs(out - np.array(c["expected"]))) < c["tolerance"]


def test_sequence_is_causal(ctx):
    c = KA["causal_sequence"]
    cache = LayerKvCache.new(ctx, 8, 1, 1)
    outs = []
    backend = HipNativeMatvecBackend(ctx)
    for q, k, v in zip(c["queries"], c["keys"], c["values"]):
        backend.append_kv_cache_sliding_f32(cache, k, v)
        outs.append(mix(ctx, cache, q, cache.token_count(), 1, 1, 1, c["scale"])[0])
    assert abs(outs[0] - c["expected_first"]) < 1e-5
    assert outs[1] > c["second_greater_than"] and abs(outs[1] - c["second_closed_form"]) < 1e-4


def test_uses_caller_score_scale(ctx):
    c = KA["score_scale"]
    cache = LayerKvCache.new(ctx, 8, 1, 1)
    for k, v in zip(c["keys"], c["values"]):
        cache.append_sliding(k, v)
    assert abs(mix(ctx, cache, [1.0], 2, 1, 1, 1, 0.0)[0] - c["scale_zero_second"]) < 1e-4
    assert mix(ctx, cache, [1.0], 2, 1, 1, 1, 1.0)[0] > c["scale_one_second_greater_than"]


def test_cache_sequence_reads_first_source_rows(ctx):
    c = KA["source_counts"]
    cache = LayerKvCache.new(ctx, 8, 1, 1)
    for k, v in zip(c["cache_keys"], c["cache_values"]):
        cache.append_sliding(k, v)
    first = mix(ctx, cache, c["queries"][0], c["source_counts"][0], 1, 1, 1, c["scale"])[0]
    second = mix(ctx, cache, c["queries"][1], c["source_counts"][1], 1, 1, 1, c["scale"])[0]
    assert cache.token_count() == 2
    assert abs(first - c["expected_first"]) < 1e-5 and second > c["second_greater_than"]


def test_small_cache_uses_sliding_window(ctx):
    c = KA["sliding_window_two"]
    cache = LayerKvCache.new(ctx, c["max_tokens"], 1, 2)
    out = None
    for v in c["values"]:
        cache.append_sliding([1.0, 0.0], v)
        out = mix(ctx, cache, [math.sqrt(2.0), 0.0], cache.token_count(), 1, 1, 2, 1.0 / math.sqrt(2.0))
    assert cache.token_count() == 2
    assert np.array_equal(cache.values(), np.ravel(c["expected_ring_values"]).astype(np.float32))
    assert np.max(np.abs(out - np.array(c["expected_attention"]))) < 1e-6
    assert np.max(np.abs(out * 0.5 - np.array(c["expected_after_gate"]))) < 1e-6


@pytest.mark.parametrize("fmt,tol", [(llm_hip.KV_BF16, "tolerance_f16_mirror"), (llm_hip.KV_INT8, "tolerance_int8"),
                                     (llm_hip.KV_INT8_ROW, "tolerance_int8")])
def test_block_mirror_attention_matches_cpu_reference_across_blocks(ctx, fmt, tol):
    """native_matvec.rs:2065-2184: 257 rows span two device blocks."""
    c = KA["cross_block_257_rows"]
    n = c["row_count"]
    cache = LayerKvCache.new_with_config(ctx, n, 1, 2, fmt)
    keys = np.array([[t / n, 1.0 - t / (n * 2.0)] for t in range(n)], np.float32)
    vals = np.array([[(t % 7) - 3.0, (t % 11) * 0.25 - 1.0] for t in range(n)], np.float32)
    for k, v in zip(keys, vals):
        cache.append(k, v)
    assert len(cache.active_blocks()) >= 2
    out = mix(ctx, cache, c["query"], n, 1, 1, 2, c["scale"])
    q = np.array(c["query"], np.float32)
    s = (q[0] * keys[:, 0] + q[1] * keys[:, 1]) * np.float32(c["scale"])
    w = np.exp(s - s.max())
    ref = (w[:, None] * vals).sum(0) / w.sum()
    assert np.max(np.abs(out - ref)) < c[tol]


def test_active_blocks_after_sliding_wrap(ctx):
    c = KA["active_blocks_after_wrap"]
    cache = LayerKvCache.new(ctx, c["max_tokens"], 1, 1)
    for k, v in zip(c["keys"], c["values"]):
        cache.append_sliding(k, v)
    assert list(cache.keys()) == c["expected_keys"]
    runs = cache.active_blocks()
    assert [(r["logical_token_start"], r["physical_token_start"], r["token_count"]) for r in runs] == \
           [(e["logical_token_start"], e["physical_token_start"], e["token_count"]) for e in c["expected_runs"]]


@pytest.mark.parametrize("max_tokens", [1, 5, 16, 33, 50])
def test_ring_state_and_runs_follow_the_reference(ctx, max_tokens):
    """Random-length append_sliding sequences: keys(), token_count, next_position,
    window start and active runs equal the oracle's LayerKvCache restatement."""
    rng = np.random.default_rng(max_tokens)
    cache = LayerKvCache.new(ctx, max_tokens, 2, 4)
    ring = oracle.Ring(max_tokens, 8, 16)
    for n in range(int(rng.integers(1, 3 * max_tokens + 4))):
        k = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(8).astype(np.float32)))
        v = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(8).astype(np.float32)))
        cache.append_sliding(k, v)
        ring.append_sliding(k, v)
    s = cache.state()
    assert (s.token_count, s.tokens_seen, s.window_start) == (ring.token_count, ring.tokens_seen, ring.window_start)
    assert np.array_equal(cache.keys(), ring.logical_rows(0))
    assert np.array_equal(cache.values(), ring.logical_rows(1))
    got = [(r["block_index"], r["logical_token_start"], r["physical_token_start"], r["block_token_start"],
            r["token_count"]) for r in cache.active_blocks()]
    assert got == ring.active_runs()
    ids = cache.block_ids()
    assert all(r["block_id"] == ids[r["block_index"]] for r in cache.active_blocks())


def test_clone_write_forks_block_identity(ctx):
    """int8_cache_format.rs:62-135: writing through a clone forks block identity;
    the original's rows are untouched."""
    cache = LayerKvCache.new_with_config(ctx, 2, 1, 2, llm_hip.KV_INT8)
    cache.append_sliding([1.0, 2.0], [0.5, 1.0])
    prefix_id = cache.block_ids()[0]
    cache.append_sliding([3.0, 4.0], [1.5, 2.0])
    cache.append_sliding([5.0, 6.0], [2.5, 3.0])
    assert np.max(np.abs(cache.values() - np.array([1.5, 2.0, 2.5, 3.0], np.float32))) < 0.03
    clone = cache.clone()
    assert clone.id() != cache.id()
    assert np.array_equal(clone.keys(), cache.keys())
    clone.append_sliding([7.0, 8.0], [3.5, 4.0])
    assert clone.block_ids()[0] != cache.block_ids()[0]
    assert clone.block_ids()[0] != prefix_id
    assert np.max(np.abs(cache.keys() - np.array([3.0, 4.0, 5.0, 6.0], np.float32))) < 0.03
    assert np.max(np.abs(clone.keys() - np.array([5.0, 6.0, 7.0, 8.0], np.float32))) < 0.05
    # the original now owns its block alone: writing keeps its identity
    before = cache.block_ids()[0]
    cache.append_sliding([9.0, 9.0], [9.0, 9.0])
    assert cache.block_ids()[0] == before


def test_errors_follow_the_reference(ctx):
    backend = HipNativeMatvecBackend(ctx)
    cache = LayerKvCache.new(ctx, 2, 1, 2)
    with pytest.raises(llm_hip.LlhError) as e:
        cache.append_sliding([1.0], [1.0])  # wrong row length
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    cache.append([1.0, 0.0], [1.0, 1.0])
    cache.append([0.0, 1.0], [2.0, 2.0])
    with pytest.raises(llm_hip.LlhError) as e:
        cache.append([0.0, 1.0], [2.0, 2.0])  # strict append on a full cache
    assert e.value.status == llm_hip.ERR_CAPACITY
    out = np.zeros(2, np.float32)
    with pytest.raises(llm_hip.LlhError) as e:
        backend.full_attention_cache_mix_f32_in_place(cache, [1.0, 0.0], 3, 1, 1, 2, 1.0, out)  # rows > tokens
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    with pytest.raises(llm_hip.LlhError):
        backend.full_attention_cache_mix_f32_in_place(cache, [1.0, 0.0], 2, 1, 1, 2, 1.0, np.zeros(1, np.float32))
    with pytest.raises(llm_hip.LlhError):
        backend.full_attention_cache_mix_f32_in_place(cache, [1.0, 0.0, 1.0, 0.0], 2, 2, 2, 2, 1.0,
                                                      np.zeros(4, np.float32))  # kv heads != cache
    assert np.all(mix(ctx, cache, [1.0, 0.0], 0, 1, 1, 2, 1.0) == 0.0)  # no rows -> zero output
    q8 = LayerKvCache.new_with_config(ctx, 2, 1, 2, llm_hip.KV_INT8)
    with pytest.raises(llm_hip.LlhError) as e:
        q8.append_sliding([float("nan"), 0.0], [1.0, 1.0])
    assert e.value.status == llm_hip.ERR_NON_FINITE
    with pytest.raises(llm_hip.LlhError) as e:
        LayerKvCache.new(ctx, 0, 1, 2)
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    with pytest.raises(llm_hip.LlhError) as e:
        LayerKvCache.new_with_config(ctx, 4, 1, 2, llm_hip.KV_FP8_E4M3)
    assert e.value.status == llm_hip.ERR_UNSUPPORTED


def test_non_finite_scores_are_an_error(ctx):
    """softmax_f32's "scores must be finite" (math.rs:485-489) surfaces as ERR_NON_FINITE."""
    cache = LayerKvCache.new(ctx, 4, 1, 1)
    cache.append_sliding([1e30], [1.0])
    out = np.zeros(1, np.float32)
    with pytest.raises(llm_hip.LlhError) as e:
        HipNativeMatvecBackend(ctx).full_attention_cache_mix_f32_in_place(cache, [1e30], 1, 1, 1, 1, 1.0, out)
    assert e.value.status == llm_hip.ERR_NON_FINITE


def test_select_head_rows_and_revision(ctx):
    cache = LayerKvCache.new(ctx, 3, 2, 2)
    rows = [[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0], [9.0, 10.0, 11.0, 12.0], [13.0, 14.0, 15.0, 16.0]]
    for i, r in enumerate(rows):
        cache.append_sliding(r, [-x for x in r])
        assert cache.revision() == i + 1 and cache.next_position() == i + 1
    sel = HipNativeMatvecBackend(ctx).select_kv_cache_head_rows_f32(cache, 0, 3, 2, 2)
    assert list(sel) == [7.0, 8.0, 11.0, 12.0, 15.0, 16.0]
    sel = HipNativeMatvecBackend(ctx).select_kv_cache_head_rows_f32(cache, 1, 2, 0, 2)
    assert list(sel) == [-5.0, -6.0, -9.0, -10.0]
    cache.clear()
    assert cache.token_count() == 0 and cache.next_position() == 0 and cache.revision() == 5


# ---- the trait hooks on the tuned decode kernels (head_dim 128, whole-block rings) ----------------

def _filled_cache(ctx, fmt, max_tokens, n_append, seed, hkv=8):
    """A Qwen3-0.6B-shaped layer cache (8 kv heads x 128) after n_append sliding appends of
    N(0,1) rows (bf16-exact, so the bf16 store holds them exactly)."""
    rng = np.random.default_rng(seed)
    cache = LayerKvCache.new_with_config(ctx, max_tokens, hkv, 128, fmt)
    backend = HipNativeMatvecBackend(ctx)
    for _ in range(n_append):
        k = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(hkv * 128).astype(np.float32)))
        v = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(hkv * 128).astype(np.float32)))
        backend.append_kv_cache_sliding_f32(cache, k, v)
    return cache, rng


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
@pytest.mark.parametrize("max_tokens,n_append,hq", [(512, 512, 16), (64, 200, 16), (512, 300, 32), (128, 128, 8)])
def test_trait_mix_on_tuned_kernels_matches_reference_loop(ctx, opts, fmt, max_tokens, n_append, hq):
    """full_attention_cache_mix_f32_in_place at head_dim 128 runs the tuned decode kernel
    (a batch of one; q rounded to bf16) over the ring, wrapped or not, for every row count
    asked: the result meets the BASELINE bar against the reference's per-head loop on the
    cache's own rows (dequantised for int8), and the reference-order kernel agrees."""
    opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
    cache, rng = _filled_cache(ctx, fmt, max_tokens, n_append, max_tokens + n_append + hq + fmt)
    backend = HipNativeMatvecBackend(ctx)
    q = rng.standard_normal(hq * 128).astype(np.float32)  # not bf16-exact: the tuned path rounds it
    keys, vals = cache.keys(), cache.values()
    n = cache.token_count()
    for rows in sorted({n, max(1, n // 2), 1, 17}):
        if rows > n:
            continue
        out = np.zeros(hq * 128, np.float32)
        before = ctx.metrics()["trait_tuned_calls"]
        assert backend.full_attention_cache_mix_f32_in_place(cache, q, rows, hq, 8, 128, 0.0883883, out)
        assert ctx.metrics()["trait_tuned_calls"] == before + 1
        st, ref = oracle.attention_mix(q, keys, vals, rows, hq, 8, 128, 0.0883883)
        assert st == oracle.OK
        d = np.abs(out - ref)
        assert d.max() <= 2e-2 and d.mean() <= 2e-3, (rows, d.max(), d.mean())
        opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 1)
        exact = np.zeros_like(out)
        assert backend.full_attention_cache_mix_f32_in_place(cache, q, rows, hq, 8, 128, 0.0883883, exact)
        assert ctx.metrics()["trait_tuned_calls"] == before + 1
        opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
        assert np.max(np.abs(exact - ref)) < 1e-4
    cache.close()


def test_trait_mix_projection_on_tuned_kernels(ctx, opts):
    """The fused o_proj hook on the tuned path: the bf16 attention output stays on the device
    and is projected there; it agrees with the reference-order path within the bar."""
    import torch

    opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
    cache, rng = _filled_cache(ctx, llm_hip.KV_BF16, 512, 400, 91)
    backend = HipNativeMatvecBackend(ctx)
    q = rng.standard_normal(16 * 128).astype(np.float32)
    w = torch.from_numpy(oracle.normal_bf16(92, 1024 * 2048).view(np.int16)).cuda().view(1024, 2048)
    tuned = np.zeros(1024, np.float32)
    before = ctx.metrics()["trait_tuned_calls"]
    assert backend.full_attention_cache_mix_bf16_output_projection_f32_in_place(cache, q, 400, 16, 8, 128, 0.088, w,
                                                                               tuned)
    assert ctx.metrics()["trait_tuned_calls"] == before + 1
    st, attn = oracle.attention_mix(q, cache.keys(), cache.values(), 400, 16, 8, 128, 0.088)
    ref = oracle.matvec_bf16_f32(oracle.normal_bf16(92, 1024 * 2048).reshape(1024, 2048), attn)
    d = np.abs(tuned - ref)
    # |W| rows of 2048 N(0,1) weights times an output within 2e-2: the projected bar scales by sqrt(2048)
    assert d.mean() <= 2e-3 * math.sqrt(2048) and d.max() <= 2e-2 * math.sqrt(2048), (d.max(), d.mean())
    cache.close()


def test_trait_mix_non_finite_scores_still_error_on_the_tuned_shape(ctx, opts):
    """A finite but huge key row makes the scores overflow: the tuned kernel's non-finite
    output sends the call to the reference-order kernel, which reports softmax_f32's error."""
    opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
    cache, rng = _filled_cache(ctx, llm_hip.KV_BF16, 64, 10, 93)
    HipNativeMatvecBackend(ctx).append_kv_cache_sliding_f32(cache, np.full(8 * 128, 1e30, np.float32),
                                                            np.ones(8 * 128, np.float32))
    out = np.zeros(16 * 128, np.float32)
    with pytest.raises(llm_hip.LlhError) as e:
        HipNativeMatvecBackend(ctx).full_attention_cache_mix_f32_in_place(cache, np.full(16 * 128, 1e30, np.float32),
                                                                          11, 16, 8, 128, 1.0, out)
    assert e.value.status == llm_hip.ERR_NON_FINITE
    cache.close()
