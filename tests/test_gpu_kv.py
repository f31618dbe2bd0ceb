"""KV writes into the paged pool and the block-table gather, bit-exact against the oracle.

* gather: llh_debug_gather through permuted tables == the oracle's gather of the
  same pool bytes (bf16, int8, fp8), including ranges that start mid-block and
  ring-style tables (position p in table[(p / 16) % max_blocks]).
* quantise on write: int8 codes/fp16 scales per (token, head) and fp8 codes/f32
  scales per (block, head) == the oracle's quantisers on the same bf16 input.
* append == whole-block write, bit for bit; fp8 decode table == the OCP table.
"""
import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, rows_bf16, to_dev
from llm_hip import workloads

pytestmark = pytest.mark.gpu

D = 128
BT = 16


def write_case(ctx, fmt, lens, Hkv, seed, head_dim=D, free=0.1):
    batch = workloads.paged_batch(lens, BT, free, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, head_dim), Hkv,
                                      head_dim)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, head_dim), Hkv,
                                    head_dim)
    pool = ctx.pool(fmt, BT, Hkv, head_dim, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    return batch, pool, ids, sk, sv


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3, llm_hip.KV_INT8_ROW,
                                 llm_hip.KV_F16])
def test_gather_is_bit_exact(ctx, fmt):
    import torch

    Hkv = 4
    batch, pool, _, _, _ = write_case(ctx, fmt, [3, 16, 33, 700], Hkv, 100 + fmt)
    opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
    d_lens, d_tab = to_dev(batch.seq_lens), to_dev(batch.tables)
    desc = ctx.decode_desc(d_lens, d_tab, Hkv, int(batch.seq_lens.max()))
    esz = 2 if fmt in (llm_hip.KV_BF16, llm_hip.KV_F16) else 1
    for b, L in enumerate(batch.seq_lens):
        for lo, hi in ((0, int(L)), (int(L) // 3, int(L))):
            for tensor in (0, 1):
                out = torch.zeros((hi - lo) * Hkv * D * esz, dtype=torch.uint8, device="cuda")
                ctx.gather(pool, desc, b, lo, hi, tensor, out)
                torch.cuda.synchronize()
                st, ref = opool.gather_raw(batch.tables[b], lo, hi, tensor)
                assert st == oracle.OK
                assert np.array_equal(out.cpu().numpy(), ref.view(np.uint8)), (fmt, b, lo, hi, tensor)
    assert ctx.device_errors() == 0


def test_gather_bf16_returns_the_written_rows(ctx):
    import torch

    Hkv = 2
    batch, pool, _, _, _ = write_case(ctx, llm_hip.KV_BF16, [77], Hkv, 7)
    desc = ctx.decode_desc(to_dev(batch.seq_lens), to_dev(batch.tables), Hkv, 77)
    out = torch.zeros(77 * Hkv * D, dtype=torch.int16, device="cuda")
    ctx.gather(pool, desc, 0, 0, 77, 0, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), rows_bf16(8, 0, 0, 77, Hkv, D).ravel())


def test_gather_ring_table(ctx):
    """A 3-block ring serving positions 40..87 (table index (p / 16) % 3)."""
    import torch

    Hkv = 1
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, 5)
    ring = np.array([[4, 0, 2]], np.int32)
    rows = rows_bf16(9, 0, 0, 96, Hkv, D)
    ids, src = [], []
    for j in range(3, 6):  # positions 48..95 -> ring slots 0, 1, 2
        ids.append(ring[0, j % 3])
        src.append(rows[j * BT:(j + 1) * BT])
    ctx.write_blocks(pool, to_dev(np.array(ids, np.int32)), to_dev(np.stack(src)), to_dev(np.stack(src)))
    desc = ctx.decode_desc(to_dev(np.array([96], np.int32)), to_dev(ring), 1, 96)
    out = torch.zeros(40 * D, dtype=torch.int16, device="cuda")
    ctx.gather(pool, desc, 0, 50, 90, 0, out)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), rows[50:90].ravel())


def test_int8_row_quantise_on_write_is_the_reference_rule(ctx):
    """LLH_KV_INT8_ROW, the reference's own int8 layout (format.rs:702-737): one f32 scale
    per token row over every kv head.  Whole-block writes store exactly the oracle's
    quantize_int8_rows codes and scales of each token row."""
    Hkv = 4
    batch, pool, ids, sk, sv = write_case(ctx, llm_hip.KV_INT8_ROW, [40, 17], Hkv, 210)
    raw = pool.raw()
    n = batch.n_blocks
    k = raw["k"].view(np.int8).reshape(n, Hkv, BT, D)
    v = raw["v"].view(np.int8).reshape(n, Hkv, D, BT)
    ks = raw["k_scales"].view(np.float32).reshape(n, BT)
    vs = raw["v_scales"].view(np.float32).reshape(n, BT)
    for i, blk in enumerate(ids):
        for src, codes_dev, scales_dev in ((sk, k[blk].transpose(1, 0, 2), ks[blk]),
                                           (sv, v[blk].transpose(2, 0, 1), vs[blk])):
            st, codes, scales = oracle.quantize_int8_rows(oracle.bf16_to_f32(src[i]).reshape(BT, Hkv * D), Hkv * D)
            assert st == oracle.OK
            assert np.array_equal(codes_dev, codes.reshape(BT, Hkv, D)) and np.array_equal(scales_dev, scales)
    assert ctx.device_errors() == 0


@pytest.mark.parametrize("src_f32", [False, True])
def test_int8_row_append_is_the_reference_rule(ctx, src_f32):
    """Per-token appends into an LLH_KV_INT8_ROW pool, from bf16 or f32 rows (the trait
    mirror's f32 rows are quantised as they are, like the reference's), store the oracle's
    quantize_int8_rows codes and scale; the f32 export returns code * scale."""
    import torch

    Hkv, n_tok, n_blocks = 3, 40, 8
    pool = ctx.pool(llm_hip.KV_INT8_ROW, BT, Hkv, D, n_blocks)
    rng = np.random.default_rng(17)
    mag = np.exp(rng.uniform(-4, 3, n_tok)).astype(np.float32)[:, None, None]
    xk = (rng.standard_normal((n_tok, Hkv, D)) * mag).astype(np.float32)
    xv = (rng.standard_normal((n_tok, Hkv, D)) * mag[::-1]).astype(np.float32)
    xk[3] = 0.0  # an all-zero row: scale 0, codes 0
    slots = rng.permutation(n_blocks * BT)[:n_tok].astype(np.int64)
    if src_f32:
        ctx.append_f32(pool, to_dev(slots), to_dev(xk), to_dev(xv))
    else:
        xk, xv = (oracle.bf16_to_f32(oracle.f32_to_bf16(x)).reshape(x.shape) for x in (xk, xv))
        ctx.append(pool, to_dev(slots), to_dev(oracle.f32_to_bf16(xk)), to_dev(oracle.f32_to_bf16(xv)))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    raw = pool.raw()
    k = raw["k"].view(np.int8).reshape(n_blocks, Hkv, BT, D)
    v = raw["v"].view(np.int8).reshape(n_blocks, Hkv, D, BT)
    ks = raw["k_scales"].view(np.float32).reshape(n_blocks, BT)
    vs = raw["v_scales"].view(np.float32).reshape(n_blocks, BT)
    ko = torch.zeros((n_tok, Hkv, D), dtype=torch.float32, device="cuda")
    vo = torch.zeros_like(ko)
    ctx.export_rows_f32(pool, to_dev(slots), ko, vo)
    ko, vo = ko.cpu().numpy(), vo.cpu().numpy()
    for i, sl in enumerate(slots):
        blk, t = divmod(int(sl), BT)
        for x, codes_dev, scale_dev, exported in ((xk, k[blk, :, t, :], ks[blk, t], ko[i]),
                                                  (xv, v[blk, :, :, t], vs[blk, t], vo[i])):
            st, codes, scales = oracle.quantize_int8_rows(x[i].ravel(), Hkv * D)
            assert st == oracle.OK
            assert np.array_equal(codes_dev.ravel(), codes) and scale_dev == scales[0]
            assert np.array_equal(exported.ravel(), oracle.dequantize_int8_rows(codes, scales, Hkv * D))


def test_int8_quantise_on_write_is_bit_exact(ctx):
    Hkv = 4
    batch, pool, ids, sk, sv = write_case(ctx, llm_hip.KV_INT8, [40, 17], Hkv, 200)
    raw = pool.raw()
    k = raw["k"].view(np.int8).reshape(batch.n_blocks, Hkv, BT, D)
    v = raw["v"].view(np.int8).reshape(batch.n_blocks, Hkv, D, BT)
    ks = raw["k_scales"].view(np.uint16).reshape(batch.n_blocks, Hkv, BT)
    vs = raw["v_scales"].view(np.uint16).reshape(batch.n_blocks, Hkv, BT)
    for i, blk in enumerate(ids):
        for h in range(Hkv):
            for t in range(BT):
                st, codes, s16 = oracle.quantize_int8_head(oracle.bf16_to_f32(sk[i, t, h]))
                assert st == oracle.OK
                assert np.array_equal(k[blk, h, t], codes) and ks[blk, h, t] == s16
                st, codes, s16 = oracle.quantize_int8_head(oracle.bf16_to_f32(sv[i, t, h]))
                assert np.array_equal(v[blk, h, :, t], codes) and vs[blk, h, t] == s16


def test_fp8_quantise_on_write_is_bit_exact(ctx):
    Hkv = 4
    batch, pool, ids, sk, sv = write_case(ctx, llm_hip.KV_FP8_E4M3, [40, 17], Hkv, 300)
    raw = pool.raw()
    k = raw["k"].reshape(batch.n_blocks, Hkv, BT, D)
    v = raw["v"].reshape(batch.n_blocks, Hkv, D, BT)
    ks = raw["k_scales"].view(np.float32).reshape(batch.n_blocks, Hkv)
    vs = raw["v_scales"].view(np.float32).reshape(batch.n_blocks, Hkv)
    for i, blk in enumerate(ids):
        for h in range(Hkv):
            st, codes, s = oracle.quantize_fp8_block(oracle.bf16_to_f32(sk[i, :, h, :]))
            assert st == oracle.OK
            assert np.array_equal(k[blk, h], codes.reshape(BT, D)) and ks[blk, h] == np.float32(s)
            st, codes, s = oracle.quantize_fp8_block(oracle.bf16_to_f32(sv[i, :, h, :]))
            assert np.array_equal(v[blk, h], codes.reshape(BT, D).T) and vs[blk, h] == np.float32(s)


@pytest.mark.parametrize("fmt,head_dim", [(llm_hip.KV_BF16, D), (llm_hip.KV_INT8, D), (llm_hip.KV_FP8_E4M3, D),
                                          (llm_hip.KV_F16, D), (llm_hip.KV_BF16, 256), (llm_hip.KV_F16, 256)])
def test_block_write_vector_and_generic_kernels_agree(ctx, fmt, head_dim):
    """16-token blocks from 16-byte aligned rows take the vector kernels (head_dim 128, every
    format; head_dim 256, bf16 and fp16); the same rows 2 bytes off alignment take the
    generic one.  Pools equal."""
    import torch

    Hkv = 4
    batch, pool_fast, ids, sk, sv = write_case(ctx, fmt, [40, 17, 300], Hkv, 500, head_dim=head_dim)
    pool_gen = ctx.pool(fmt, BT, Hkv, head_dim, batch.n_blocks)

    def misaligned(a):
        flat = torch.zeros(a.size + 1, dtype=torch.int16, device="cuda")
        flat[1:] = to_dev(a).reshape(-1)
        view = flat[1:]
        assert view.data_ptr() % 16 != 0
        return view

    ctx.write_blocks(pool_gen, to_dev(ids), misaligned(sk), misaligned(sv))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    rf, rg = pool_fast.raw(), pool_gen.raw()
    written = np.asarray(ids)  # blocks no write touched hold whatever the allocation held
    for key in rf:
        f = rf[key].reshape(batch.n_blocks, -1)[written]
        g = rg[key].reshape(batch.n_blocks, -1)[written]
        assert np.array_equal(f, g), key


def test_int8_quantise_on_write_generic_head_dim(ctx):
    """head_dim 64 goes through the generic kernel: same quantiser, bit for bit."""
    Hkv, hd = 2, 64
    batch, pool, ids, sk, sv = write_case(ctx, llm_hip.KV_INT8, [33], Hkv, 600, head_dim=hd)
    raw = pool.raw()
    k = raw["k"].view(np.int8).reshape(batch.n_blocks, Hkv, BT, hd)
    v = raw["v"].view(np.int8).reshape(batch.n_blocks, Hkv, hd, BT)
    for i, blk in enumerate(ids):
        for h in range(Hkv):
            for t in range(BT):
                _, codes, _ = oracle.quantize_int8_head(oracle.bf16_to_f32(sk[i, t, h]))
                assert np.array_equal(k[blk, h, t], codes)
                _, codes, _ = oracle.quantize_int8_head(oracle.bf16_to_f32(sv[i, t, h]))
                assert np.array_equal(v[blk, h, :, t], codes)


def test_block_write_flags_bad_block(ctx):
    import torch

    pool = ctx.pool(llm_hip.KV_BF16, BT, 2, D, 2)
    z = torch.zeros(BT * 2 * D, dtype=torch.int16, device="cuda")
    ctx.write_blocks(pool, torch.tensor([2], dtype=torch.int32, device="cuda"), z, z)
    torch.cuda.synchronize()
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_F16])
def test_append_equals_block_write(ctx, fmt):
    import torch

    Hkv = 8
    batch, pool_w, ids, sk, sv = write_case(ctx, fmt, [48, 32], Hkv, 400, free=0.0)
    pool_a = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
    slots = []
    rows_k, rows_v = [], []
    for i, blk in enumerate(ids):
        for t in range(BT):
            slots.append(int(blk) * BT + t)
            rows_k.append(sk[i, t])
            rows_v.append(sv[i, t])
    order = np.random.default_rng(1).permutation(len(slots))  # append order does not matter
    ctx.append(pool_a, to_dev(np.array(slots, np.int64)[order]), to_dev(np.stack(rows_k)[order]),
               to_dev(np.stack(rows_v)[order]))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    ra, rw = pool_a.raw(), pool_w.raw()
    for key in rw:
        assert np.array_equal(ra[key], rw[key]), key


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_FP8_E4M3])
def test_append_flags_bad_slots(ctx, fmt):
    import torch

    pool = ctx.pool(fmt, BT, 2, D, 2)
    z = torch.zeros(2 * D, dtype=torch.int16, device="cuda")
    ctx.append(pool, torch.tensor([2 * BT + 1], dtype=torch.int64, device="cuda"), z, z)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK


def test_fp8_append_matches_oracle_token_by_token(ctx):
    """Per-token appends into fp8 blocks (scale per (block, head) and tensor) re-quantise the
    block as the absmax grows: the pool's codes and scales equal the oracle's restatement of
    the rule bit for bit, for calls of one token, calls of several tokens of one block (call
    order), calls spanning two blocks, and a block reused from a stale scale."""
    import torch

    Hkv, n_tok = 2, 44
    table = [3, 5, 1]  # position p lives in block table[p // 16]
    pool = ctx.pool(llm_hip.KV_FP8_E4M3, BT, Hkv, D, 8)
    # stale content in the blocks: a whole-block write with a large scale first
    big = torch.full((8, BT, Hkv, D), 100.0, device="cuda").to(torch.bfloat16)
    ctx.write_blocks(pool, torch.arange(8, dtype=torch.int32, device="cuda"), big, big)
    rng = np.random.default_rng(5)
    mag = np.exp(rng.uniform(-3, 2, n_tok)).astype(np.float32)
    k = oracle.f32_to_bf16(rng.standard_normal((n_tok, Hkv, D)).astype(np.float32) * mag[:, None, None])
    v = oracle.f32_to_bf16(rng.standard_normal((n_tok, Hkv, D)).astype(np.float32) * mag[:, None, None][::-1])
    slots = np.array([table[p // BT] * BT + p % BT for p in range(n_tok)], np.int64)
    calls = [[p] for p in range(0, 20)] + [list(range(20, 28)), list(range(28, 36)), list(range(36, 44))]
    for c in calls:
        ctx.append(pool, to_dev(slots[c]), to_dev(k[c]), to_dev(v[c]))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    raw = pool.raw()
    kc = raw["k"].reshape(8, Hkv, BT, D)
    vc = raw["v"].reshape(8, Hkv, D, BT)
    ks = raw["k_scales"].view(np.float32).reshape(8, Hkv)
    vs = raw["v_scales"].view(np.float32).reshape(8, Hkv)
    kf, vf = oracle.bf16_to_f32(k), oracle.bf16_to_f32(v)
    for bi, blk in enumerate(table):
        n_in = min(BT, n_tok - bi * BT)
        for h in range(Hkv):
            for tensor, src, got, gs in ((0, kf, kc[blk, h], ks[blk, h]), (1, vf, vc[blk, h].T, vs[blk, h])):
                codes = np.zeros((BT, D), np.uint8)
                s = 999.0
                for t in range(n_in):
                    st, s = oracle.append_fp8_token(codes, s, t, src[bi * BT + t, h])
                    assert st == oracle.OK
                assert gs == np.float32(s), (blk, h, tensor)
                assert np.array_equal(got[:n_in], codes[:n_in]), (blk, h, tensor)
    # attention over the appended cache meets the bar against the dequantise-then-attend oracle
    lens = np.array([n_tok], np.int32)
    tab = np.array([table], np.int32)
    q = oracle.normal_bf16(7, 8 * D)
    out = torch.zeros(8 * D, dtype=torch.int16, device="cuda")
    ctx.paged_decode(pool, ctx.decode_desc(to_dev(lens), to_dev(tab), 8, n_tok), to_dev(q), out, 0.09)
    torch.cuda.synchronize()
    opool = oracle.Pool.from_raw(llm_hip.KV_FP8_E4M3, BT, Hkv, D, 8, pool.raw())
    st, ref = opool.decode(8, lens, tab, 0, q, 0.09)
    assert st == oracle.OK
    assert_parity(out.cpu().numpy().view(np.uint16), ref, what="decode over appended fp8 blocks")


@pytest.mark.parametrize("src_f32", [False, True])
def test_fp8_append_one_row_per_block_calls(ctx, src_f32):
    """Calls whose rows each go to a different block (the single-token fp8 kernel for
    16-token, head_dim-128 blocks) from bf16 or f32 rows: 16 calls fill 8 blocks token by
    token over stale codes, with magnitudes that grow the scale at some offsets (earlier
    tokens re-encoded) and not at others; one row holds a NaN in one kv head's V (flagged;
    that (block, head) left as it was, every other head and row of the call written).  Codes and scales equal the oracle's
    restatement of the rule bit for bit."""
    import torch

    Hkv, nb = 2, 8
    blocks = [5, 0, 7, 2, 9, 4, 1, 6]
    pool = ctx.pool(llm_hip.KV_FP8_E4M3, BT, Hkv, D, 10)
    stale = torch.randn((10, BT, Hkv, D), device="cuda").mul(30.0).to(torch.bfloat16)
    ctx.write_blocks(pool, torch.arange(10, dtype=torch.int32, device="cuda"), stale, stale)
    rng = np.random.default_rng(23)
    mag = np.exp(rng.uniform(-3, 3, (BT, nb))).astype(np.float32)
    x = (rng.standard_normal((BT, nb, 2, Hkv, D)) * mag[:, :, None, None, None]).astype(np.float32)
    if not src_f32:
        x = oracle.bf16_to_f32(oracle.f32_to_bf16(x.ravel())).reshape(x.shape)
    nan_at = (6, 3, 1)  # (offset, row of the call, kv head): block 2's token 6, head 1, holds a NaN
    x[nan_at[0], nan_at[1], 1, nan_at[2], 5] = np.nan
    flags = []
    for t in range(BT):
        slots = np.array([b * BT + t for b in blocks], np.int64)
        k, v = np.ascontiguousarray(x[t, :, 0]), np.ascontiguousarray(x[t, :, 1])
        if src_f32:
            ctx.append_f32(pool, to_dev(slots), to_dev(k), to_dev(v))
        else:
            ctx.append(pool, to_dev(slots), to_dev(oracle.f32_to_bf16(k.ravel()).reshape(k.shape)),
                       to_dev(oracle.f32_to_bf16(v.ravel()).reshape(v.shape)))
        torch.cuda.synchronize()
        flags.append(ctx.device_errors())
    assert all((f & llm_hip.ERR_FLAG_NON_FINITE) != 0 for i, f in enumerate(flags) if i == nan_at[0])
    assert all(f == 0 for i, f in enumerate(flags) if i != nan_at[0])
    raw = pool.raw()
    kc = raw["k"].reshape(10, Hkv, BT, D)
    vc = raw["v"].reshape(10, Hkv, D, BT)
    ks = raw["k_scales"].view(np.float32).reshape(10, Hkv)
    vs = raw["v_scales"].view(np.float32).reshape(10, Hkv)
    grew = 0
    for r, blk in enumerate(blocks):
        for h in range(Hkv):
            for tensor, got, gs in ((0, kc[blk, h], ks[blk, h]), (1, vc[blk, h].T, vs[blk, h])):
                codes = np.zeros((BT, D), np.uint8)
                s = 999.0
                for t in range(BT):
                    if (t, r, h) == nan_at:
                        continue  # rejected for both tensors: the block-head keeps what it held
                    s_before = s
                    st, s = oracle.append_fp8_token(codes, s, t, x[t, r, tensor, h])
                    assert st == oracle.OK
                    grew += t > 0 and s != s_before
                assert gs == np.float32(s), (blk, h, tensor)
                keep = np.ones(BT, bool)
                if (r, h) == nan_at[1:]:
                    keep[nan_at[0]] = False  # that slot still holds the stale block's code
                assert np.array_equal(got[keep], codes[keep]), (blk, h, tensor)
    assert grew > 20  # the re-encoding branch ran many times


def test_fp8_decode_table(ctx):
    import torch

    codes = torch.arange(256, dtype=torch.uint8, device="cuda")
    out = torch.zeros(256, dtype=torch.float32, device="cuda")
    ctx.decode_fp8(codes, out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = oracle.fp8_decode_table()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(got[~nan], ref[~nan])


def test_fp8_encoder_equals_reference_rule_on_every_f32(ctx):
    """The kernels encode fp8 with the hardware conversion (v_cvt_pk_fp8_f32 on inputs
    clamped to +-448); on every f32 bit pattern but NaNs its code equals the integer
    round-to-nearest-even rule (encode_e4m3_soft), which the quantise-on-write tests hold
    to the oracle's encoder."""
    assert ctx.fp8_encode_check() == 0


def test_fp8_append_one_call_equals_token_by_token_calls(ctx):
    """A call of 128 tokens whose blocks' tokens are interleaved across the whole call
    (token i goes to block i % 8 at offset i // 8, so each block's tokens sit in both
    64-slot scans of the call) leaves the pool bit-identical to 128 calls of one token
    in the same order: the tokens of one block are appended in call order."""
    import torch

    Hkv, n_tok, nb = 2, 128, 8
    rng = np.random.default_rng(11)
    mag = np.exp(rng.uniform(-3, 2, n_tok)).astype(np.float32)
    k = oracle.f32_to_bf16(rng.standard_normal((n_tok, Hkv, D)).astype(np.float32) * mag[:, None, None])
    v = oracle.f32_to_bf16(rng.standard_normal((n_tok, Hkv, D)).astype(np.float32) * mag[::-1, None, None])
    blocks = [6, 2, 9, 0, 4, 11, 7, 1]
    slots = np.array([blocks[i % nb] * BT + i // nb for i in range(n_tok)], np.int64)
    one = ctx.pool(llm_hip.KV_FP8_E4M3, BT, Hkv, D, 12)
    many = ctx.pool(llm_hip.KV_FP8_E4M3, BT, Hkv, D, 12)
    ctx.append(one, to_dev(slots), to_dev(k), to_dev(v))
    for i in range(n_tok):
        ctx.append(many, to_dev(slots[i:i + 1]), to_dev(k[i:i + 1]), to_dev(v[i:i + 1]))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0, ctx.last_error()
    a, b = one.raw(), many.raw()
    used = np.array(blocks)  # the other blocks were never written (their contents are unspecified)
    for key, shape in (("k", (12, Hkv, BT, D)), ("v", (12, Hkv, D, BT))):
        assert np.array_equal(a[key].reshape(shape)[used], b[key].reshape(shape)[used]), key
    for key in ("k_scales", "v_scales"):
        sa, sb = a[key].view(np.float32).reshape(12, Hkv), b[key].view(np.float32).reshape(12, Hkv)
        assert np.array_equal(sa[used], sb[used]), key


@pytest.mark.parametrize("src_f32", [0, 1])
def test_int8_row_append_flags_non_finite_rows(ctx, src_f32):
    """A NaN or an infinity in a row appended to an LLH_KV_INT8_ROW pool is the reference's
    NonFiniteValue (format.rs:713-716): the flag is raised and the slot keeps what it held;
    finite rows of the same call are written."""
    import torch

    Hkv = 2
    pool = ctx.pool(llm_hip.KV_INT8_ROW, BT, Hkv, D, 4)
    before = pool.raw()
    rows = oracle.normal_bf16(91, 3 * Hkv * D).reshape(3, Hkv, D)
    rf = oracle.bf16_to_f32(rows.ravel()).reshape(3, Hkv, D).copy()
    rf[1, 1, 7] = np.nan if src_f32 else np.inf
    k = rf if src_f32 else oracle.f32_to_bf16(rf.ravel()).reshape(3, Hkv, D)
    slots = np.array([0 * BT + 3, 1 * BT + 4, 2 * BT + 5], np.int64)
    (ctx.append_f32 if src_f32 else ctx.append)(pool, to_dev(slots), to_dev(k), to_dev(k))
    torch.cuda.synchronize()
    assert ctx.device_errors() & llm_hip.ERR_FLAG_NON_FINITE
    after = pool.raw()
    kc0, kc1 = before["k"].reshape(4, Hkv, BT, D), after["k"].reshape(4, Hkv, BT, D)
    assert np.array_equal(kc1[1, :, 4], kc0[1, :, 4])  # the non-finite row's slot untouched
    assert np.array_equal(after["k_scales"].view(np.float32).reshape(4, BT)[1, 4], 0.0)
    st, codes, scales = oracle.quantize_int8_rows(oracle.bf16_to_f32(rows[0].ravel()), Hkv * D)
    assert st == oracle.OK and np.array_equal(kc1[0, :, 3].view(np.int8).ravel(), codes)


@pytest.mark.parametrize("fmt", [llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3, llm_hip.KV_INT8_ROW])
@pytest.mark.parametrize("misalign", [False, True])
def test_quantised_block_write_flags_non_finite_rows(ctx, fmt, misalign):
    """Whole-block writes into quantised pools (the head_dim-128 vector kernel and, with the
    source 2 bytes off alignment, the element-wise kernels): a NaN or an infinity raises the
    non-finite flag, and the (block, head) holding it -- the token row, for the reference's
    row layout -- is left as it was; the other blocks of the call are written as the oracle
    quantises them."""
    import torch

    Hkv, n = 2, 3
    pool = ctx.pool(fmt, BT, Hkv, D, 4)
    before = pool.raw()
    k = oracle.normal_bf16(95, n * BT * Hkv * D).reshape(n, BT, Hkv, D).copy()
    v = oracle.normal_bf16(96, n * BT * Hkv * D).reshape(n, BT, Hkv, D).copy()
    v[1, 9, 1, 100] = 0x7F80  # +inf in block 1's values
    dk, dv = to_dev(k), to_dev(v)
    if misalign:
        def shifted(t):
            flat = torch.zeros(t.numel() + 1, dtype=torch.int16, device="cuda")
            flat[1:].copy_(t.view(-1))
            return flat[1:]
        dk, dv = shifted(dk), shifted(dv)
    ctx.write_blocks(pool, to_dev(np.array([0, 2, 3], np.int32)), dk, dv)
    torch.cuda.synchronize()
    assert ctx.device_errors() & llm_hip.ERR_FLAG_NON_FINITE
    after = pool.raw()
    if fmt == llm_hip.KV_INT8_ROW:
        # the reference's row layout quantises per token row over all heads: only the
        # non-finite token (9 of pool block 2) is skipped
        vc0, vc1 = before["v"].reshape(4, Hkv, D, BT), after["v"].reshape(4, Hkv, D, BT)
        assert np.array_equal(vc1[2, :, :, 9], vc0[2, :, :, 9])
        assert after["v_scales"].view(np.float32).reshape(4, BT)[2, 9] == 0.0
    else:
        # per (block, head) workgroups: head 1 of pool block 2 (codes and scales) is untouched
        for key in after:
            assert np.array_equal(after[key].reshape(4, Hkv, -1)[2, 1], before[key].reshape(4, Hkv, -1)[2, 1]), key
    # block 0 of the call (pool block 0) is written as the oracle quantises it
    opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, 4, after)
    st, kf, _ = opool.gather_f32(np.array([0], np.int32), 0, BT)
    assert st == oracle.OK
    x = oracle.bf16_to_f32(k[0].ravel()).reshape(BT, Hkv, D)
    err = np.abs(kf.reshape(BT, Hkv, D) - x)
    # one e4m3 rounding (3 mantissa bits) or half an int8 step of the row's absmax / 127
    assert np.all(err <= 0.0625 * np.abs(x) + 0.03), err.max()
