"""Writes the golden fixtures under tests/golden/.

known_answers.json: inputs and expected outputs of the kir-ai reference's own
tests for the attention path, transcribed as data (each entry cites the
reference test it comes from).  Nothing of the reference is imported or run:
the reference is Rust and is not buildable here.

c1_decode.json: BASELINE configs[0] (B=1, L=512, Hq16/Hkv8, D128, identity
table) generated from the seeded PRNG: SHA-256 digests of the inputs and the
oracle's fp32 output, accepted only if it agrees with the float64 brute force
to 1e-5.  It pins the PRNG, the oracle and (in the GPU tests) the kernel.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

E = math.e

KNOWN_ANSWERS = {
    "two_head_closed_form": {
        "source": "crates/llm-metal/src/device/primitives/tests.rs:36-73",
        "row_count": 2, "q_heads": 2, "kv_heads": 1, "head_dim": 2, "scale": 1.0,
        "query": [1.0, 0.0, 0.0, 1.0],
        "keys": [1.0, 0.0, 0.0, 1.0],
        "values": [10.0, 20.0, 30.0, 40.0],
        "expected": [10 * E / (E + 1) + 30 / (E + 1), 20 * E / (E + 1) + 40 / (E + 1),
                     10 / (E + 1) + 30 * E / (E + 1), 20 / (E + 1) + 40 * E / (E + 1)],
        "tolerance": 1e-4,
    },
    "int8_closed_form": {
        "source": "crates/llm-metal/src/device/primitives/tests.rs:413-466",
        "row_count": 2, "q_heads": 2, "kv_heads": 1, "head_dim": 2, "scale": 1.0,
        "query": [1.0, 0.0, 0.0, 1.0],
        "key_codes": [127, 0, 0, 127], "key_scales": [1.0 / 127.0, 1.0 / 127.0],
        "value_codes": [127, 0, 0, 127], "value_scales": [10.0 / 127.0, 10.0 / 127.0],
        "expected": [10 * E / (E + 1), 10 / (E + 1), 10 / (E + 1), 10 * E / (E + 1)],
        "tolerance": 1e-4,
    },
    "causal_sequence": {
        "source": "crates/llm-backend/src/core/native_attention.rs:1178-1207",
        "q_heads": 1, "kv_heads": 1, "head_dim": 1, "scale": 1.0,
        "queries": [[1.0], [1.0]], "keys": [[1.0], [3.0]], "values": [[10.0], [30.0]],
        "expected_first": 10.0, "second_greater_than": 27.0,
        "second_closed_form": 10.0 + 20.0 * E ** 2 / (1.0 + E ** 2),
    },
    "score_scale": {
        "source": "crates/llm-backend/src/core/native_attention.rs:1286-1332",
        "q_heads": 1, "kv_heads": 1, "head_dim": 1,
        "queries": [[1.0], [1.0]], "keys": [[0.0], [10.0]], "values": [[0.0], [100.0]],
        "scale_zero_second": 50.0, "scale_one_second_greater_than": 99.0,
    },
    "source_counts": {
        "source": "crates/llm-backend/src/core/native_attention.rs:1335-1374",
        "q_heads": 1, "kv_heads": 1, "head_dim": 1, "scale": 1.0,
        "cache_keys": [[1.0], [3.0]], "cache_values": [[10.0], [30.0]],
        "queries": [[1.0], [1.0]], "source_counts": [1, 2],
        "expected_first": 10.0, "second_greater_than": 27.0,
    },
    "cached_matches_uncached_gqa": {
        "source": "crates/llm-backend/src/core/native_attention.rs:1242-1283",
        "q_heads": 2, "kv_heads": 1, "head_dim": 1, "scale": 1.0, "max_tokens": 8,
        "queries": [[1.0, 0.5], [0.25, 1.0]], "keys": [[1.0], [0.5]], "values": [[4.0], [8.0]],
    },
    "fused_cache_mix": {
        "source": "crates/llm-backend/src/core/native_attention.rs:1581-1619",
        "q_heads": 2, "kv_heads": 1, "head_dim": 1, "scale": 1.0, "max_tokens": 8,
        "cache_keys": [[1.0], [2.0]], "cache_values": [[10.0], [20.0]],
        "query": [1.0, 2.0],
        "note": "the reference's mock backend returns 11, 22; the per-head path gives softmax-weighted values",
    },
    "sliding_window_two": {
        "source": "crates/llm-backend/src/core/tests/cpu_ops.rs:638-747",
        "max_tokens": 2, "q_heads": 1, "kv_heads": 1, "head_dim": 2,
        "values": [[2.0, 0.0], [0.0, 4.0], [8.0, 0.0]],
        "note": "equal scores, so the output is the mean of the last two values; the reference "
                "multiplies by a sigmoid(0) = 0.5 gate after the attention boundary",
        "expected_attention": [4.0, 2.0], "expected_after_gate": [2.0, 1.0],
        "expected_ring_values": [[0.0, 4.0], [8.0, 0.0]],
    },
    "active_blocks_after_wrap": {
        "source": "crates/llm-kv-cache/tests/layer_cache_active_blocks.rs:3-24",
        "max_tokens": 3, "kv_heads": 1, "head_dim": 1, "block_tokens": 256,
        "keys": [[1.0], [2.0], [3.0], [4.0]], "values": [[10.0], [20.0], [30.0], [40.0]],
        "expected_keys": [2.0, 3.0, 4.0],
        "expected_runs": [{"logical_token_start": 0, "physical_token_start": 1, "token_count": 2},
                          {"logical_token_start": 2, "physical_token_start": 0, "token_count": 1}],
    },
    "int8_rows_metrics": {
        "source": "crates/llm-kv-cache/tests/int8_cache_format.rs:13-60",
        "vector_len": 16,
        "key0": [v / 16.0 for v in range(16)], "value0": [(v - 8.0) / 8.0 for v in range(16)],
        "key1": [v / 16.0 for v in range(16, 32)], "value1": [(v - 24.0) / 8.0 for v in range(16, 32)],
        "tolerance": 0.01,
    },
    "int8_sliding": {
        "source": "crates/llm-kv-cache/tests/int8_cache_format.rs:62-135",
        "max_tokens": 2, "vector_len": 2,
        "keys": [[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]], "values": [[0.5, 1.0], [1.5, 2.0], [2.5, 3.0]],
        "expected_keys": [3.0, 4.0, 5.0, 6.0], "expected_values": [1.5, 2.0, 2.5, 3.0],
        "tolerance": 0.03,
    },
    "cross_block_257_rows": {
        "source": "crates/llm-native-runtime/src/native_matvec.rs:2065-2184,2761-2785",
        "row_count": 257, "q_heads": 1, "kv_heads": 1, "head_dim": 2,
        "query": [0.25, -0.5], "scale": 0.7,
        "keys_rule": "key[t] = [t / 257, 1 - t / (257 * 2)]",
        "values_rule": "value[t] = [(t % 7) - 3, (t % 11) * 0.25 - 1]",
        "tolerance_f16_mirror": 1e-2, "tolerance_int8": 3e-2,
    },
    "bf16_matvec": {
        "source": "crates/llm-backend/src/core/tests/safetensors_loader/shard_store.rs:16-51",
        "rows": 2, "cols": 3, "weight": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0],
        "inputs": [[1.0, 2.0, 3.0], [3.0, 2.0, 1.0]],
        "expected": [[14.0, 32.0], [10.0, 28.0]],
    },
}


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_fixture() -> dict:
    """BASELINE configs[0] from the seeded PRNG (seed 0x6B69722D00)."""
    seed = 0x6B69722D00
    L, Hq, Hkv, D = 512, 16, 8, 128
    k = oracle.normal_bf16(seed + 1, L * Hkv * D)
    v = oracle.normal_bf16(seed + 2, L * Hkv * D)
    q = oracle.normal_bf16(seed + 3, Hq * D)
    scale = 1.0 / math.sqrt(D)
    kf, vf, qf = (oracle.bf16_to_f32(x) for x in (k, v, q))
    st, out = oracle.attention_mix(qf, kf, vf, L, Hq, Hkv, D, scale)
    st2, out64 = oracle.attention_mix_f64(qf, kf, vf, L, Hq, Hkv, D, scale)
    assert st == 0 and st2 == 0
    err = float(np.abs(out - out64).max())
    assert err < 1e-5, err
    return {
        "source": "BASELINE.json configs[0]",
        "seed": seed, "row_count": L, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D, "scale": scale,
        "inputs": "k = normal_bf16(seed+1, L*Hkv*D), v = normal_bf16(seed+2, ...), q = normal_bf16(seed+3, Hq*D); "
                  "rows token-major [L][Hkv][D]",
        "sha256_k": sha(k), "sha256_v": sha(v), "sha256_q": sha(q),
        "prng_first8": [float(x) for x in oracle.normal_f32(seed + 1, 8)],
        "output_f32": [float(x) for x in out],
        "max_abs_vs_f64": err,
    }


def main() -> None:
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(KNOWN_ANSWERS, f, indent=1)
    with open(os.path.join(HERE, "c1_decode.json"), "w") as f:
        json.dump(c1_fixture(), f)
    print("wrote known_answers.json and c1_decode.json")


if __name__ == "__main__":
    main()
