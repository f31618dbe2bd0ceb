"""The CPU oracle, pinned before it is trusted (no GPU needed).

1. Every known answer the kir-ai reference's own tests hold for this path
   (tests/golden/known_answers.json, each entry citing its reference test).
2. Independent checks chosen so that a plausible mistake fails one of them:
   float64 brute force, torch's scaled_dot_product_attention on the CPU,
   closed forms (uniform scores -> mean), exhaustive code tables (fp8, f16).
3. The paged/window restatement against the reference's ring semantics
   (crates/llm-kv-cache/src/layer.rs:765-805): attending [len - W, len) through
   a permuted block table is bit-identical to appending every token to a ring
   of capacity W and attending its logical rows.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))


def close(a, b, tol):
    return np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))) <= tol


# ---------------------------------------------------------------------------
# 1. reference known answers
# ---------------------------------------------------------------------------

def test_two_head_closed_form():
    c = KA["two_head_closed_form"]
    st, out = oracle.attention_mix(c["query"], c["keys"], c["values"], c["row_count"], c["q_heads"],
                                   c["kv_heads"], c["head_dim"], c["scale"])
    assert st == oracle.OK
    assert close(out, c["expected"], c["tolerance"])
    assert close(out, c["expected"], 1e-5)


def test_int8_closed_form_dequant_then_attend():
    c = KA["int8_closed_form"]
    keys = oracle.dequantize_int8_rows(np.array(c["key_codes"], np.int8), np.array(c["key_scales"], np.float32), 2)
    vals = oracle.dequantize_int8_rows(np.array(c["value_codes"], np.int8), np.array(c["value_scales"], np.float32),
                                       2)
    st, out = oracle.attention_mix(c["query"], keys, vals, c["row_count"], c["q_heads"], c["kv_heads"],
                                   c["head_dim"], c["scale"])
    assert st == oracle.OK
    assert close(out, c["expected"], c["tolerance"])


def ring_step_outputs(queries, keys, values, q_heads, kv_heads, head_dim, scale, max_tokens=64):
    """The reference sequence path: per token append (sliding) then attend over the cache."""
    r = oracle.Ring(max_tokens, kv_heads * head_dim)
    outs = []
    for q, k, v in zip(queries, keys, values):
        r.append_sliding(k, v)
        st, out = oracle.attention_mix(q, r.logical_rows(0), r.logical_rows(1), r.token_count, q_heads, kv_heads,
                                       head_dim, scale)
        assert st == oracle.OK
        outs.append(out)
    return outs


def test_causal_sequence():
    c = KA["causal_sequence"]
    outs = ring_step_outputs(c["queries"], c["keys"], c["values"], 1, 1, 1, c["scale"])
    assert abs(outs[0][0] - c["expected_first"]) < 1e-5
    assert outs[1][0] > c["second_greater_than"]
    assert abs(outs[1][0] - c["second_closed_form"]) < 1e-4


def test_caller_score_scale():
    c = KA["score_scale"]
    flat = ring_step_outputs(c["queries"], c["keys"], c["values"], 1, 1, 1, 0.0)
    sharp = ring_step_outputs(c["queries"], c["keys"], c["values"], 1, 1, 1, 1.0)
    assert abs(flat[1][0] - c["scale_zero_second"]) < 1e-5
    assert sharp[1][0] > c["scale_one_second_greater_than"]


def test_source_counts_read_first_rows():
    c = KA["source_counts"]
    r = oracle.Ring(8, 1)
    for k, v in zip(c["cache_keys"], c["cache_values"]):
        r.append_sliding(k, v)
    keys, vals = r.logical_rows(0), r.logical_rows(1)
    outs = []
    for q, n in zip(c["queries"], c["source_counts"]):
        st, out = oracle.attention_mix(q, keys[:n], vals[:n], n, 1, 1, 1, c["scale"])
        assert st == oracle.OK
        outs.append(out[0])
    assert r.token_count == 2
    assert abs(outs[0] - c["expected_first"]) < 1e-5 and outs[1] > c["second_greater_than"]


def test_cached_matches_uncached_gqa():
    c = KA["cached_matches_uncached_gqa"]
    cached = ring_step_outputs(c["queries"], c["keys"], c["values"], 2, 1, 1, c["scale"], c["max_tokens"])
    for i, q in enumerate(c["queries"]):
        k = np.array(c["keys"][: i + 1], np.float32)
        v = np.array(c["values"][: i + 1], np.float32)
        st, unc = oracle.attention_mix(q, k, v, i + 1, 2, 1, 1, c["scale"])
        assert st == oracle.OK
        assert np.array_equal(unc, cached[i])


def test_fused_cache_mix_per_head_values():
    c = KA["fused_cache_mix"]
    st, out = oracle.attention_mix(c["query"], c["cache_keys"], c["cache_values"], 2, 2, 1, 1, c["scale"])
    assert st == oracle.OK
    # head h: scores q_h * [1, 2]; weights softmax; output 10 w0 + 20 w1
    for h, qv in enumerate(c["query"]):
        w1 = 1.0 / (1.0 + math.exp(-qv))
        assert abs(out[h] - (10 * (1 - w1) + 20 * w1)) < 1e-5


def test_sliding_window_two():
    c = KA["sliding_window_two"]
    keys = [[1.0, 0.0]] * len(c["values"])
    outs = ring_step_outputs([[1.0, 0.0]] * 3, keys, c["values"], 1, 1, 2, 1.0 / math.sqrt(2), c["max_tokens"])
    assert close(outs[-1], c["expected_attention"], 1e-6)
    # the q projection's gate half is zero in the reference test: attention * sigmoid(0)
    assert close(oracle.apply_gate(outs[-1], np.zeros(2, np.float32)), c["expected_after_gate"], 1e-6)
    r = oracle.Ring(c["max_tokens"], 2)
    for k, v in zip(keys, c["values"]):
        r.append_sliding(k, v)
    assert close(r.logical_rows(1), np.ravel(c["expected_ring_values"]), 0)


def test_active_blocks_after_wrap():
    c = KA["active_blocks_after_wrap"]
    r = oracle.Ring(c["max_tokens"], 1, c["block_tokens"])
    for k, v in zip(c["keys"], c["values"]):
        r.append_sliding(k, v)
    assert list(r.logical_rows(0)) == c["expected_keys"]
    runs = r.active_runs()
    assert len(runs) == len(c["expected_runs"])
    for got, exp in zip(runs, c["expected_runs"]):
        _, logical, physical, _, count = got
        assert (logical, physical, count) == (exp["logical_token_start"], exp["physical_token_start"],
                                              exp["token_count"])


def test_int8_rows_reconstruct_within_reference_tolerance():
    c = KA["int8_rows_metrics"]
    for key in ("key0", "value0", "key1", "value1"):
        x = np.array(c[key], np.float32)
        st, codes, scales = oracle.quantize_int8_rows(x, c["vector_len"])
        assert st == oracle.OK
        assert close(oracle.dequantize_int8_rows(codes, scales, c["vector_len"]), x, c["tolerance"])
    c = KA["int8_sliding"]
    r = oracle.Ring(c["max_tokens"], c["vector_len"])
    for k, v in zip(c["keys"], c["values"]):
        r.append_sliding(k, v)
    assert list(r.logical_rows(0)) == c["expected_keys"] and list(r.logical_rows(1)) == c["expected_values"]
    st, codes, scales = oracle.quantize_int8_rows(r.logical_rows(1), c["vector_len"])
    assert close(oracle.dequantize_int8_rows(codes, scales, c["vector_len"]), c["expected_values"], c["tolerance"])


def cross_block_257():
    c = KA["cross_block_257_rows"]
    n = c["row_count"]
    keys = np.array([[t / n, 1.0 - t / (n * 2.0)] for t in range(n)], np.float32)
    vals = np.array([[(t % 7) - 3.0, (t % 11) * 0.25 - 1.0] for t in range(n)], np.float32)
    return c, keys, vals


def reference_attention_257(query, keys, values, scale):
    """reference_attention of native_matvec.rs:2761-2785, restated in numpy f32."""
    q = np.asarray(query, np.float32)
    scores = (q[0] * keys[:, 0] + q[1] * keys[:, 1]) * np.float32(scale)
    scores = np.exp(scores - scores.max()).astype(np.float32)
    w = scores / scores.sum(dtype=np.float32)
    return (w[:, None] * values).sum(axis=0, dtype=np.float32)


def test_cross_block_257_rows():
    c, keys, vals = cross_block_257()
    st, out = oracle.attention_mix(c["query"], keys, vals, c["row_count"], 1, 1, 2, c["scale"])
    assert st == oracle.OK
    assert close(out, reference_attention_257(c["query"], keys, vals, c["scale"]), 1e-5)
    # int8 storage of the reference layout (one scale per token row) stays within the reference's 3e-2
    _, kc, ks = oracle.quantize_int8_rows(keys, 2)
    _, vc, vs = oracle.quantize_int8_rows(vals, 2)
    st, q8 = oracle.attention_mix(c["query"], oracle.dequantize_int8_rows(kc, ks, 2),
                                  oracle.dequantize_int8_rows(vc, vs, 2), c["row_count"], 1, 1, 2, c["scale"])
    assert close(q8, out, c["tolerance_int8"])


def test_c1_golden_fixture():
    g = json.load(open(os.path.join(HERE, "golden", "c1_decode.json")))
    import hashlib

    seed, L, Hq, Hkv, D = g["seed"], g["row_count"], g["q_heads"], g["kv_heads"], g["head_dim"]
    k = oracle.normal_bf16(seed + 1, L * Hkv * D)
    v = oracle.normal_bf16(seed + 2, L * Hkv * D)
    q = oracle.normal_bf16(seed + 3, Hq * D)
    for name, a in (("k", k), ("v", v), ("q", q)):
        assert hashlib.sha256(a.tobytes()).hexdigest() == g[f"sha256_{name}"], f"PRNG drift in {name}"
    assert np.array_equal(oracle.normal_f32(seed + 1, 8), np.array(g["prng_first8"], np.float32))
    st, out = oracle.attention_mix(oracle.bf16_to_f32(q), oracle.bf16_to_f32(k), oracle.bf16_to_f32(v), L, Hq, Hkv,
                                   D, g["scale"])
    assert st == oracle.OK
    assert np.array_equal(out, np.array(g["output_f32"], np.float32))


# ---------------------------------------------------------------------------
# 2. independent checks
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("R,Hq,Hkv,D,scale", [(1, 1, 1, 1, 1.0), (7, 4, 2, 8, 0.3), (300, 16, 8, 128, 0.0884),
                                               (65, 8, 1, 64, 1.7), (2, 3, 3, 5, 0.0)])
def test_oracle_matches_float64_brute_force(R, Hq, Hkv, D, scale):
    rng = np.random.default_rng(R * 131 + D)
    q = rng.standard_normal(Hq * D).astype(np.float32)
    k = rng.standard_normal(R * Hkv * D).astype(np.float32)
    v = rng.standard_normal(R * Hkv * D).astype(np.float32)
    st, o32 = oracle.attention_mix(q, k, v, R, Hq, Hkv, D, scale)
    st2, o64 = oracle.attention_mix_f64(q, k, v, R, Hq, Hkv, D, scale)
    assert st == st2 == oracle.OK
    assert np.max(np.abs(o32 - o64)) < 2e-5


@pytest.mark.parametrize("R,Hq,Hkv,D", [(33, 16, 8, 128), (100, 32, 4, 64), (5, 2, 1, 16)])
def test_oracle_matches_torch_sdpa(R, Hq, Hkv, D):
    """torch.nn.functional.scaled_dot_product_attention in float64 on the CPU; consecutive
    query heads share a kv head (repeat_interleave), the GQA map kv = h / (Hq/Hkv)."""
    import torch

    rng = np.random.default_rng(R + Hq)
    q = rng.standard_normal((Hq, D)).astype(np.float32)
    k = rng.standard_normal((R, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((R, Hkv, D)).astype(np.float32)
    scale = 1.0 / math.sqrt(D)
    st, out = oracle.attention_mix(q, k, v, R, Hq, Hkv, D, scale)
    assert st == oracle.OK
    kt = torch.from_numpy(k).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, dim=0)
    vt = torch.from_numpy(v).double().permute(1, 0, 2).repeat_interleave(Hq // Hkv, dim=0)
    qt = torch.from_numpy(q).double()[:, None, :]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale)[:, 0, :].numpy()
    assert np.max(np.abs(out.reshape(Hq, D) - ref)) < 2e-5


def test_uniform_scores_give_the_mean():
    rng = np.random.default_rng(5)
    v = rng.standard_normal((40, 2, 16)).astype(np.float32)
    k = np.ones((40, 2, 16), np.float32)
    st, out = oracle.attention_mix(np.ones(4 * 16, np.float32), k, v, 40, 4, 2, 16, 0.25)
    assert st == oracle.OK
    assert np.max(np.abs(out.reshape(4, 16) - v.mean(axis=0).repeat(2, axis=0))) < 1e-5


def test_gqa_head_map_is_consecutive():
    """kv = h / (Hq/Hkv): heads 0,1 read kv head 0 and heads 2,3 read kv head 1."""
    v = np.zeros((3, 2, 1), np.float32)
    v[:, 0, 0], v[:, 1, 0] = 1.0, 2.0
    st, out = oracle.attention_mix(np.zeros(4, np.float32), np.zeros((3, 2, 1), np.float32), v, 3, 4, 2, 1, 1.0)
    assert st == oracle.OK and list(out) == [1.0, 1.0, 2.0, 2.0]


def test_empty_rows_give_zero_output():
    st, out = oracle.attention_mix(np.ones(8, np.float32), np.zeros(0, np.float32), np.zeros(0, np.float32), 0, 2,
                                   1, 4, 1.0)
    assert st == oracle.OK and np.all(out == 0)


def test_non_finite_scores_are_an_error():
    """softmax_f32 rejects non-finite scores (math.rs:485-489) instead of masking them."""
    st, _ = oracle.softmax([0.0, float("inf")])
    assert st == oracle.ERR_NON_FINITE
    st, _ = oracle.attention_mix([1.0], [float("nan")], [1.0], 1, 1, 1, 1, 1.0)
    assert st == oracle.ERR_NON_FINITE


def test_shape_errors():
    st, _ = oracle.attention_mix(np.zeros(3, np.float32), np.zeros(2, np.float32), np.zeros(2, np.float32), 1, 3,
                                 2, 1, 1.0)
    assert st == oracle.ERR_INVALID_SHAPE


def test_softmax_matches_definition():
    s = np.array([0.5, -1.0, 3.0, 2.0], np.float32)
    st, p = oracle.softmax(s)
    e = np.exp(s.astype(np.float64) - s.max())
    assert st == oracle.OK and np.max(np.abs(p - e / e.sum())) < 1e-7


# ---------------------------------------------------------------------------
# conversions and quantisation
# ---------------------------------------------------------------------------

def test_bf16_round_to_nearest_even_matches_torch():
    import torch

    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.0e38, -3.0e38, 1e-40, np.inf, -np.inf], np.float32)])
    x = x.astype(np.float32)
    ours = oracle.f32_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    L = oracle.lib()
    assert all(L.orc_f32_to_bf16(float(v)) == o for v, o in zip(x[:200], ours[:200]))


def test_f16_conversions_exhaustive():
    L = oracle.lib()
    codes = np.arange(65536, dtype=np.uint16)
    ours = np.array([L.orc_f16_to_f32(int(c)) for c in codes], np.float32)
    ref = codes.view(np.float16).astype(np.float32)
    both_nan = np.isnan(ours) & np.isnan(ref)
    assert np.array_equal(ours[~both_nan], ref[~both_nan]) and np.array_equal(np.isnan(ours), np.isnan(ref))
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)).astype(np.float32)
    back = np.array([L.orc_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(back, x.astype(np.float16).view(np.uint16))


def test_fp8_e4m3_decode_table_matches_torch():
    import torch

    ours = oracle.fp8_decode_table()
    ref = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and np.isnan(ours[0x7F])


def test_fp8_e4m3_encode_round_to_nearest_even_matches_torch():
    import torch

    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-448, 448, 20000), rng.standard_normal(20000) * 1e-2,
                        oracle.fp8_decode_table()[:0x7F].astype(np.float64)]).astype(np.float32)
    ours = oracle.fp8_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, ref)
    # saturation (the oracle's rule; torch maps overflow to NaN)
    assert oracle.fp8_encode(np.array([1e6, -500.0], np.float32)).tolist() == [0x7E, 0xFE]


def test_round_half_away_from_zero_like_rust():
    L = oracle.lib()
    assert [L.orc_round_half_away(v) for v in (2.5, -2.5, 0.5, 1.49999, -0.5)] == [3.0, -3.0, 1.0, 1.0, -1.0]


def test_int8_head_quantisation_bounds():
    rng = np.random.default_rng(4)
    for _ in range(200):
        x = (rng.standard_normal(128) * rng.uniform(0.01, 10)).astype(np.float32)
        st, codes, s16 = oracle.quantize_int8_head(x)
        s = oracle.lib().orc_f16_to_f32(s16)
        assert st == oracle.OK and np.all(np.abs(codes.astype(np.int32)) <= 127)
        assert abs(s - np.abs(x).max() / 127) <= abs(np.abs(x).max() / 127) * 2 ** -10
        assert np.max(np.abs(codes * np.float32(s) - x)) <= s * 0.5001 + np.abs(x).max() * 2 ** -9
    st, codes, s16 = oracle.quantize_int8_head(np.zeros(16, np.float32))
    assert st == oracle.OK and s16 == 0 and not codes.any()
    st, _, _ = oracle.quantize_int8_head(np.array([1.0, np.nan], np.float32))
    assert st == oracle.ERR_NON_FINITE


def test_int8_head_codes_are_nearest_codes_of_the_stored_scale():
    """Brute force over every code: the stored scale is numpy's fp16 rounding of absmax/127
    (computed in f32), and each code is the c in [-127, 127] nearest to the f32 quotient
    x / scale (the reference's `(value / scale).round()`, format.rs:711-735), ties going
    away from zero.  Exact .5 ties are planted.  A code from the unrounded scale, ties to
    even, truncation or a clamp error each fails here."""
    rng = np.random.default_rng(41)
    cands = np.arange(-127, 128, dtype=np.float64)
    planted = 0
    for trial in range(300):
        n = 128
        x = (rng.standard_normal(n) * rng.uniform(1e-3, 50)).astype(np.float32)
        amax = np.float32(np.abs(x).max())
        s = np.float32(np.float16(np.float32(amax / np.float32(127.0))))
        # plant exact ties (k + 0.5) * s, below the absmax so the scale is unchanged
        others = np.setdiff1d(np.arange(n), [int(np.argmax(np.abs(x)))])
        for i in rng.choice(others, 8, replace=False):
            k = int(rng.integers(-126, 126))
            t = np.float32((k + 0.5) * s)
            if abs(t) < amax:
                x[i] = t
                planted += 1
        assert np.float32(np.abs(x).max()) == amax
        st, codes, s16 = oracle.quantize_int8_head(x)
        assert st == oracle.OK
        assert s16 == int(np.float16(np.float32(amax / np.float32(127.0))).view(np.uint16))
        quot = (x / s).astype(np.float32).astype(np.float64)
        dist = np.abs(quot[:, None] - cands[None, :])
        best = dist.min(axis=1, keepdims=True)
        # nearest codes; among equals the one farthest from zero
        score = np.where(dist == best, np.abs(cands)[None, :], -1.0)
        expect = cands[np.argmax(score, axis=1)]
        assert np.array_equal(codes.astype(np.float64), expect), trial
    assert planted > 1000
    # all-zero rows: scale 0, codes 0 (format.rs: scale 0 -> code 0)
    st, codes, s16 = oracle.quantize_int8_head(np.zeros(8, np.float32))
    assert st == oracle.OK and s16 == 0 and not codes.any()


def test_fp8_block_quantisation_bounds():
    rng = np.random.default_rng(6)
    table = oracle.fp8_decode_table()
    for _ in range(50):
        x = (rng.standard_normal(16 * 128) * rng.uniform(0.01, 10)).astype(np.float32)
        st, codes, s = oracle.quantize_fp8_block(x)
        assert st == oracle.OK and abs(s - np.abs(x).max() / 448) <= 1e-7 * s
        deq = table[codes] * np.float32(s)
        big = np.abs(x) >= 2.0 ** -6 * s
        assert np.all(np.abs(deq - x)[big] <= np.abs(x)[big] * 2.0 ** -4 + 1e-12)
        assert np.all(np.abs(deq - x)[~big] <= 2.0 ** -10 * s + 1e-12)


def test_fp8_append_equals_block_quantiser_when_the_first_row_holds_the_max():
    """Appending a block's rows one by one (the per-token rule) gives exactly the whole-block
    quantiser's codes and scale when no later row raises the block's absmax: the scale is
    fixed by row 0 and every row is encoded x / scale."""
    rng = np.random.default_rng(12)
    for trial in range(40):
        D, n = 128, int(rng.integers(1, 17))
        x = (rng.standard_normal((n, D)) * rng.uniform(0.01, 5)).astype(np.float32)
        x[0, int(rng.integers(D))] = np.float32(np.abs(x).max() * 1.5)  # row 0 holds the block max
        codes = np.zeros((16, D), np.uint8)
        s = 123.0  # stale scale of a reused block: offset 0 ignores it
        for t in range(n):
            st, s = oracle.append_fp8_token(codes, s, t, x[t])
            assert st == oracle.OK
        st, ref_codes, ref_s = oracle.quantize_fp8_block(x)
        assert st == oracle.OK and s == ref_s
        assert np.array_equal(codes[:n].ravel(), ref_codes), trial


def test_fp8_append_rescales_earlier_tokens_within_the_double_rounding_bound():
    """Rows whose absmax grows: the scale follows the running absmax / 448 and every stored
    value stays within the error of one e4m3 rounding per rescale it went through (a 3-bit
    mantissa: half an ulp = 2^-4 relative, plus the subnormal step 2^-10 * scale)."""
    rng = np.random.default_rng(13)
    table = oracle.fp8_decode_table()
    for trial in range(40):
        D, n = 64, 16
        x = (rng.standard_normal((n, D)) * np.geomspace(0.01, 10, n)[:, None]).astype(np.float32)
        codes = np.zeros((16, D), np.uint8)
        s, rescales = 0.0, np.zeros(n, int)
        for t in range(n):
            prev = s
            st, s = oracle.append_fp8_token(codes, s, t, x[t])
            assert st == oracle.OK
            if t > 0 and s != prev:
                rescales[:t] += 1
            assert s == max(prev if t else 0.0, float(np.float32(np.abs(x[t]).max()) / np.float32(448.0)))
        deq = table[codes[:n]] * np.float32(s)
        for t in range(n):
            k = rescales[t] + 1
            bound = np.abs(x[t]) * ((1 + 2.0 ** -4) ** k - 1) + k * 2.0 ** -10 * s + 1e-12
            assert np.all(np.abs(deq[t] - x[t]) <= bound), (trial, t)
    # all-zero rows keep a zero scale and zero codes; non-finite rows are refused
    codes = np.full((16, 8), 7, np.uint8)
    assert oracle.append_fp8_token(codes, 0.0, 0, np.zeros(8)) == (oracle.OK, 0.0) and not codes[0].any()
    assert oracle.append_fp8_token(codes, 0.0, 1, np.array([np.nan] * 8))[0] == oracle.ERR_NON_FINITE


def test_prng_moments():
    x = oracle.normal_f32(123, 200000)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert np.array_equal(oracle.normal_f32(123, 10, 5), x[5:15])


# ---------------------------------------------------------------------------
# 3. paged pool, window and prefill restatement vs the reference ring
# ---------------------------------------------------------------------------

def _paged_case(lens, Hkv, D, BT, seed, free=0.1):
    import sys

    sys.path.insert(0, os.path.join(os.path.dirname(HERE), "kir-ai_amd"))
    from llm_hip import workloads

    batch = workloads.paged_batch(lens, BT, free, seed)
    rk = [oracle.normal_bf16(seed + 1, L * Hkv * D, b << 24).reshape(L, Hkv, D) for b, L in enumerate(lens)]
    rv = [oracle.normal_bf16(seed + 2, L * Hkv * D, b << 24).reshape(L, Hkv, D) for b, L in enumerate(lens)]
    pool = oracle.build_bf16_pool(rk, rv, batch.tables, lens, BT, Hkv, D, batch.n_blocks)
    return batch, rk, rv, pool


def test_pool_gather_is_bit_exact():
    batch, rk, rv, pool = _paged_case([5, 16, 17, 100], 2, 8, 4, 10)
    for b, L in enumerate(batch.seq_lens):
        st, raw = pool.gather_raw(batch.tables[b], 0, int(L), 0)
        assert st == oracle.OK and np.array_equal(raw, rk[b].ravel())
        st, raw = pool.gather_raw(batch.tables[b], 0, int(L), 1)
        assert st == oracle.OK and np.array_equal(raw, rv[b].ravel())
        st, kf, vf = pool.gather_f32(batch.tables[b], 0, int(L))
        assert np.array_equal(kf, oracle.bf16_to_f32(rk[b].ravel()))


def test_f16_pool_elements_are_the_widened_halves():
    """An f16 pool (KvCacheConfig::f16, format.rs:69-120) holds IEEE binary16 bits:
    the oracle reads element (block, head, token, dim) as numpy's float16 -> float32
    of those bits (subnormals, infinities, signed zeros included), through the same
    K token-row / V dim-row layout as the bf16 pool, and decode over it equals the
    reference attention of the widened rows."""
    from llm_hip import workloads

    Hkv, D, BT, Hq = 2, 8, 4, 4
    lens = [5, 16, 23]
    batch = workloads.paged_batch(lens, BT, 0.2, 61)
    rng = np.random.default_rng(61)
    rk = [rng.integers(0, 65536, size=(L, Hkv, D), dtype=np.uint16) for L in lens]
    rv = [rng.integers(0, 65536, size=(L, Hkv, D), dtype=np.uint16) for L in lens]
    for r in rk + rv:  # finite values only (the decode below needs finite scores)
        r[np.isnan(r.view(np.float16)) | np.isinf(r.view(np.float16))] = 0x3C00
    rk[0][0, 0, :4] = [0x0001, 0x8000, 0x03FF, 0x7BFF]  # smallest subnormal, -0, largest subnormal, 65504
    pool = oracle.build_bf16_pool(rk, rv, batch.tables, lens, BT, Hkv, D, batch.n_blocks, fmt=oracle.KV_F16)
    for b, L in enumerate(lens):
        for tensor, rows in ((0, rk[b]), (1, rv[b])):
            st, raw = pool.gather_raw(batch.tables[b], 0, L, tensor)
            assert st == oracle.OK and np.array_equal(raw, rows.ravel())
        st, kf, vf = pool.gather_f32(batch.tables[b], 0, L)
        assert np.array_equal(kf, rk[b].view(np.float16).astype(np.float32).ravel())
        assert np.array_equal(vf, rv[b].view(np.float16).astype(np.float32).ravel())
    # small-magnitude rows so that softmax stays finite
    sk = [(r.view(np.float16).astype(np.float32) * 1e-4).astype(np.float16).view(np.uint16) for r in rk]
    sv = [(r.view(np.float16).astype(np.float32) * 1e-4).astype(np.float16).view(np.uint16) for r in rv]
    pool = oracle.build_bf16_pool(sk, sv, batch.tables, lens, BT, Hkv, D, batch.n_blocks, fmt=oracle.KV_F16)
    q = oracle.normal_bf16(62, len(lens) * Hq * D)
    st, out = pool.decode(Hq, batch.seq_lens, batch.tables, 0, q, 0.5)
    assert st == oracle.OK
    qf = oracle.bf16_to_f32(q).reshape(len(lens), Hq * D)
    for b, L in enumerate(lens):
        kf = sk[b].view(np.float16).astype(np.float32).reshape(L, -1)
        vf = sv[b].view(np.float16).astype(np.float32).reshape(L, -1)
        st, ref = oracle.attention_mix(qf[b], kf, vf, L, Hq, Hkv, D, 0.5)
        assert st == oracle.OK and np.array_equal(out.reshape(len(lens), -1)[b], ref)


def test_pool_gather_rejects_out_of_pool_blocks():
    batch, rk, rv, pool = _paged_case([20], 1, 4, 4, 11)
    t = batch.tables[0].copy()
    t[2] = pool.n_blocks + 3
    st, _ = pool.gather_raw(t, 0, 20, 0)
    assert st == oracle.ERR_INVALID_SHAPE


@pytest.mark.parametrize("W", [1, 3, 16, 17, 40])
def test_window_equals_reference_ring(W):
    """Attending [len-W, len) through block tables == the reference ring of capacity W."""
    Hq, Hkv, D, BT = 4, 2, 8, 4
    lens = [1, 7, 23, 50]
    batch, rk, rv, pool = _paged_case(lens, Hkv, D, BT, 20 + W)
    q = oracle.normal_bf16(99, len(lens) * Hq * D)
    st, out = pool.decode(Hq, batch.seq_lens, batch.tables, W, q, 0.3)
    assert st == oracle.OK
    qf = oracle.bf16_to_f32(q).reshape(len(lens), Hq * D)
    for b, L in enumerate(lens):
        ring = oracle.Ring(W, Hkv * D, 256)
        for t in range(L):
            ring.append_sliding(oracle.bf16_to_f32(rk[b][t].ravel()), oracle.bf16_to_f32(rv[b][t].ravel()))
        assert ring.token_count == min(W, L)
        st, ref = oracle.attention_mix(qf[b], ring.logical_rows(0), ring.logical_rows(1), ring.token_count, Hq, Hkv,
                                       D, 0.3)
        assert np.array_equal(out.reshape(len(lens), -1)[b], ref)


@pytest.mark.parametrize("W", [0, 5])
def test_prefill_equals_per_token_append_then_attend(W):
    """Prefill rows == the reference sequence loop (append token i, attend the cache)
    (native_attention.rs:400-461), and == decode at each row's position."""
    Hq, Hkv, D, BT = 4, 2, 8, 4
    prefix, chunk = [6, 0, 13], [5, 9, 3]
    lens = [p + c for p, c in zip(prefix, chunk)]
    batch, rk, rv, pool = _paged_case(lens, Hkv, D, BT, 40 + W)
    starts = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    q = oracle.normal_bf16(77, int(starts[-1]) * Hq * D)
    st, out = pool.prefill(Hq, starts, batch.seq_lens, batch.tables, W, q, 0.2)
    assert st == oracle.OK
    out = out.reshape(-1, Hq * D)
    qf = oracle.bf16_to_f32(q).reshape(-1, Hq * D)
    for b in range(len(lens)):
        ring = oracle.Ring(W if W else 64, Hkv * D)
        for t in range(prefix[b]):
            ring.append_sliding(oracle.bf16_to_f32(rk[b][t].ravel()), oracle.bf16_to_f32(rv[b][t].ravel()))
        for i in range(chunk[b]):
            t = prefix[b] + i
            ring.append_sliding(oracle.bf16_to_f32(rk[b][t].ravel()), oracle.bf16_to_f32(rv[b][t].ravel()))
            st, ref = oracle.attention_mix(qf[starts[b] + i], ring.logical_rows(0), ring.logical_rows(1),
                                           ring.token_count, Hq, Hkv, D, 0.2)
            assert np.array_equal(out[starts[b] + i], ref)
            one = np.array([t + 1], np.int32)
            st, dec = pool.decode(Hq, one, batch.tables[b:b + 1], W, q.reshape(-1, Hq * D)[starts[b] + i], 0.2)
            assert np.array_equal(dec, ref)


def test_ring_runs_incremental_equal_closed_form_with_small_blocks():
    """The reference's incremental run bookkeeping (layer.rs:1089-1152) equals the
    closed form the device cache mirror reports, for 16-token blocks and random lengths."""
    rng = np.random.default_rng(8)
    for max_tokens in (1, 3, 16, 17, 40):
        r = oracle.Ring(max_tokens, 1, 16)
        for n in range(int(rng.integers(1, 3 * max_tokens + 3))):
            r.append_sliding([float(n)], [float(n)])
            runs = []
            for i in range(r.token_count):
                phys = (r.window_start + i) % max_tokens
                bi, off = phys // 16, phys % 16
                if runs and runs[-1][0] == bi and runs[-1][1] + runs[-1][4] == i and \
                        runs[-1][2] + runs[-1][4] == phys and runs[-1][3] + runs[-1][4] == off:
                    runs[-1][4] += 1
                else:
                    runs.append([bi, i, phys, off, 1])
            assert [tuple(x) for x in runs] == r.active_runs()


def test_strict_append_capacity_error():
    r = oracle.Ring(2, 1)
    r.append([1.0], [1.0])
    r.append([2.0], [2.0])
    with pytest.raises(OverflowError):
        r.append([3.0], [3.0])


def test_bf16_matvec_known_answer():
    """crates/llm-backend/src/core/tests/safetensors_loader/shard_store.rs:16-51."""
    ka = KA["bf16_matvec"]
    w = oracle.f32_to_bf16(np.array(ka["weight"], np.float32)).reshape(ka["rows"], ka["cols"])
    for x, exp in zip(ka["inputs"], ka["expected"]):
        assert oracle.matvec_bf16_f32(w, np.array(x, np.float32)).tolist() == exp


def test_bf16_matvec_matches_float64():
    rng = np.random.default_rng(11)
    rows, cols = 37, 300
    w = oracle.f32_to_bf16(rng.standard_normal((rows, cols)).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    got = oracle.matvec_bf16_f32(w, x)
    ref = oracle.bf16_to_f32(w.ravel()).reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert np.max(np.abs(got - ref)) < 1e-4
    # a transposed operand or a dropped row fails this
    assert not np.allclose(got[:-1], ref[1:], atol=1e-2)


def test_sigmoid_and_gate():
    """sigmoid_f32 (math.rs:472-474) and apply_attention_gate (native_attention.rs:775-781):
    sigmoid(0) is exactly one half, the f32 result is within 2 ulp of float64 1 / (1 + e^-x)
    over [-30, 30], the symmetry sigmoid(-x) = 1 - sigmoid(x) holds to f32 rounding, the tails
    saturate to 0 and 1 (exp overflow gives 0, not NaN), and the gate multiplies element-wise
    (a gate of a different element must not leak: one planted swap fails)."""
    assert oracle.sigmoid(0.0) == 0.5
    xs = np.linspace(-30.0, 30.0, 6001).astype(np.float32)
    got = np.array([oracle.sigmoid(float(x)) for x in xs], np.float32)
    ref = 1.0 / (1.0 + np.exp(-xs.astype(np.float64)))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2 * ulp)
    mid = np.abs(xs) < 8
    assert np.all(np.abs(got[mid] + got[mid][::-1] - 1.0) <= 2 * np.spacing(np.float32(1.0)))
    assert oracle.sigmoid(200.0) == 1.0 and oracle.sigmoid(-200.0) == 0.0
    att = np.arange(1, 9, dtype=np.float32)
    gate = np.array([0, 0, 1, -1, 30, -30, 2, -2], np.float32)
    out = oracle.apply_gate(att, gate)
    assert np.all(out == np.array([att[i] * oracle.sigmoid(float(gate[i])) for i in range(8)], np.float32))
    swapped = gate.copy()
    swapped[[2, 3]] = swapped[[3, 2]]
    assert not np.array_equal(oracle.apply_gate(att, swapped), out)
