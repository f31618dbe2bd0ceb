"""Output projection after attention on the device (MFMA skinny GEMM), against the
oracle's per-row bf16 dot (crates/llm-backend/src/core/safetensors/math.rs:66-72):

* the reference's known answer (shard_store.rs:16-51), and the "not handled"
  answer for shapes the kernel does not take;
* random shapes with ragged row / input counts, bf16 and f32 inputs;
* the fused decode + projection (llh_paged_decode_output_projection) equals
  decode followed by the projection bit for bit, and the oracle's f32 chain
  within the parity bar;
* the trait hook full_attention_cache_mix_bf16_output_projection_f32_in_place.
"""
import json
import math
import os

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, rows_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KA = json.load(open(os.path.join(HERE, "golden", "known_answers.json")))


def dev_f32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def test_known_answer_and_unsupported_shape(ctx):
    import torch

    ka = KA["bf16_matvec"]
    w = oracle.f32_to_bf16(np.array(ka["weight"], np.float32)).reshape(ka["rows"], ka["cols"])
    x = np.array(ka["inputs"], np.float32)
    out = torch.zeros(2 * ka["rows"], dtype=torch.float32, device="cuda")
    with pytest.raises(llm_hip.LlhError) as e:  # 3 columns: not a multiple of 128
        ctx.matvec_bf16(to_dev(w), ka["rows"], ka["cols"], dev_f32(x), 2, out)
    assert e.value.status == llm_hip.ERR_UNSUPPORTED
    # the same problem zero-padded to 128 columns
    wp = np.zeros((ka["rows"], 128), np.uint16)
    wp[:, :3] = w
    xp = np.zeros((2, 128), np.float32)
    xp[:, :3] = x
    ctx.matvec_bf16(to_dev(wp), ka["rows"], 128, dev_f32(xp), 2, out)
    torch.cuda.synchronize()
    assert out.cpu().numpy().reshape(2, ka["rows"]).tolist() == ka["expected"]


# On 256 compute units K is split over 8 (1024x2048, 1000x2048), 16 (300x512),
# 4 (2048x1024) and 2 (4096x512) workgroups; 77 and 99 rows take the generic sum.
@pytest.mark.parametrize("rows,cols,n", [(1024, 2048, 32), (1000, 2048, 1), (77, 128, 45), (300, 512, 7), (99, 512, 5),
                                         (2048, 1024, 3), (4096, 512, 2)])
@pytest.mark.parametrize("x_f32", [False, True])
def test_matvec_matches_oracle(ctx, rows, cols, n, x_f32):
    import torch

    rng = np.random.default_rng(rows + cols + n)
    w = oracle.f32_to_bf16((rng.standard_normal((rows, cols)) / math.sqrt(cols)).astype(np.float32))
    x = rng.standard_normal((n, cols)).astype(np.float32)
    if not x_f32:
        xb = oracle.f32_to_bf16(x)
        x = oracle.bf16_to_f32(xb.ravel()).reshape(n, cols)
    out = torch.full((n * rows,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matvec_bf16(to_dev(w), rows, cols, dev_f32(x) if x_f32 else to_dev(xb), n, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(n, rows)
    ref = np.stack([oracle.matvec_bf16_f32(w, x[i]) for i in range(n)])
    d = np.abs(got - ref)
    # bf16 inputs: the same products, only the f32 summation order differs;
    # f32 inputs are rounded to bf16 for the MFMA (relative 2^-9 per product)
    assert d.max() <= (2e-2 if x_f32 else 1e-4), d.max()
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("rows,cols,n", [(1024, 2048, 32), (4096, 512, 2), (300, 512, 7)])
def test_matvec_unaligned_output_is_identical(ctx, rows, cols, n):
    """An output one float off 16-byte alignment takes the element-wise stores
    of both launches: the same sums in the same order, bit for bit."""
    import torch

    rng = np.random.default_rng(7 * rows + n)
    w = oracle.f32_to_bf16((rng.standard_normal((rows, cols)) / math.sqrt(cols)).astype(np.float32))
    xb = oracle.f32_to_bf16(rng.standard_normal((n, cols)).astype(np.float32))
    out = torch.zeros(n * rows, dtype=torch.float32, device="cuda")
    ctx.matvec_bf16(to_dev(w), rows, cols, to_dev(xb), n, out)
    flat = torch.zeros(n * rows + 1, dtype=torch.float32, device="cuda")
    shifted = flat[1:]
    assert shifted.data_ptr() % 16 != 0
    ctx.matvec_bf16(to_dev(w), rows, cols, to_dev(xb), n, shifted)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), shifted.cpu().numpy().view(np.uint32))


def test_fused_decode_projection(ctx):
    import torch

    Hq, Hkv, D, rows = 16, 8, 128, 1024
    lens = [300, 4096, 17, 1000, 2048, 1, 777, 3000]
    seed = workloads.SEED_BASE + 9
    batch = workloads.paged_batch(lens, 16, 0.1, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, D), Hkv, D)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, D), Hkv, D)
    pool = ctx.pool(llm_hip.KV_BF16, 16, Hkv, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    B = len(lens)
    q = oracle.normal_bf16(seed + 3, B * Hq * D)
    rng = np.random.default_rng(5)
    w = oracle.f32_to_bf16((rng.standard_normal((rows, Hq * D)) / math.sqrt(Hq * D)).astype(np.float32))
    d_w, d_q = to_dev(w), to_dev(q)
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hq, int(batch.seq_lens.max()))
    scale = 1.0 / math.sqrt(D)
    fused = torch.full((B * rows,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.paged_decode_output_projection(pool, desc, d_q, d_w, rows, fused, scale)
    attn = torch.empty(B * Hq * D, dtype=torch.int16, device="cuda")
    ctx.paged_decode(pool, desc, d_q, attn, scale)
    split = torch.full((B * rows,), float("nan"), dtype=torch.float32, device="cuda")
    ctx.matvec_bf16(d_w, rows, Hq * D, attn, B, split)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    got = fused.cpu().numpy().reshape(B, rows)
    assert np.array_equal(got, split.cpu().numpy().reshape(B, rows))
    # the reference chain: f32 attention (oracle), then the bf16-weight matvec in f32
    opool = oracle.Pool.from_raw(llm_hip.KV_BF16, 16, Hkv, D, batch.n_blocks, pool.raw())
    st, ref_attn = opool.decode(Hq, batch.seq_lens, batch.tables, 0, q, scale, threads=16)
    assert st == oracle.OK
    ref_attn = ref_attn.reshape(B, Hq * D)
    ref = np.stack([oracle.matvec_bf16_f32(w, ref_attn[i]) for i in range(B)])
    d = np.abs(got - ref)
    assert d.max() <= 2e-2 and d.mean() <= 2e-3, (d.max(), d.mean())
    # and the attention it projected passes the attention bar on its own
    assert_parity(from_dev_bf16(attn), ref_attn.ravel(), what="attention under the projection")


def test_trait_hook_projection(ctx):
    Hq, Hkv, D, R, rows = 4, 2, 128, 257, 300
    cache = llm_hip.LayerKvCache.new(ctx, 512, Hkv, D)
    rng = np.random.default_rng(8)
    keys = rng.standard_normal((R, Hkv * D)).astype(np.float32)
    values = rng.standard_normal((R, Hkv * D)).astype(np.float32)
    backend = llm_hip.HipNativeMatvecBackend(ctx)
    for t in range(R):
        backend.append_kv_cache_sliding_f32(cache, keys[t], values[t])
    q = rng.standard_normal(Hq * D).astype(np.float32)
    w = oracle.f32_to_bf16((rng.standard_normal((rows, Hq * D)) / math.sqrt(Hq * D)).astype(np.float32))
    d_w = to_dev(w).view(rows, Hq * D)
    out = np.zeros(rows, np.float32)
    scale = 1.0 / math.sqrt(D)
    assert backend.full_attention_cache_mix_bf16_output_projection_f32_in_place(cache, q, R, Hq, Hkv, D, scale,
                                                                              d_w, out)
    kf = oracle.bf16_to_f32(oracle.f32_to_bf16(keys).ravel())  # the cache stores bf16 rows
    vf = oracle.bf16_to_f32(oracle.f32_to_bf16(values).ravel())
    st, attn = oracle.attention_mix(q, kf, vf, R, Hq, Hkv, D, scale)
    assert st == oracle.OK
    ref = oracle.matvec_bf16_f32(w, attn)
    d = np.abs(out - ref)
    assert d.max() <= 2e-2 and d.mean() <= 2e-3, (d.max(), d.mean())
    # zero rows project zero; shapes the fused path does not take are "not handled"
    zero = np.ones(rows, np.float32)
    assert backend.full_attention_cache_mix_bf16_output_projection_f32_in_place(cache, q, 0, Hq, Hkv, D, scale,
                                                                              d_w, zero)
    assert not zero.any()
    narrow = to_dev(w[:, :256].copy()).view(rows, 256)
    assert not backend.full_attention_cache_mix_bf16_output_projection_f32_in_place(cache, q, R, Hq, Hkv, D, scale,
                                                                                  narrow, out)
    small = np.zeros(rows - 1, np.float32)
    assert not backend.full_attention_cache_mix_bf16_output_projection_f32_in_place(cache, q, R, Hq, Hkv, D, scale,
                                                                                  d_w, small)
