"""BlockPool over a device KV pool: payload rows, copy-on-write device copies, and
decode through prefix-shared session tables (the serving flow of
crates/llm-native-runtime/src/native_text/driver.rs:662-835 with the
BlockPool of crates/llm-kv-cache/src/block_pool.rs), checked against the
oracle's per-head attention over the logical rows.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, rows_bf16, to_dev
from llm_hip import BlockPool, LlhError, cache_block_chain_hash

pytestmark = pytest.mark.gpu

BT = 16


def bf16_round(x: np.ndarray) -> np.ndarray:
    return oracle.bf16_to_f32(oracle.f32_to_bf16(np.asarray(x, np.float32)))


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_append_rows_round_trip(ctx, fmt):
    """CacheBlock::append / keys() / values() (block.rs:250-306) on device blocks."""
    Hkv, D = 2, 64
    pool = ctx.pool(fmt, BT, Hkv, D, 4)
    bp = BlockPool.over(ctx, pool)
    s = bp.create_session()
    b = bp.allocate_for_session(s)
    rng = np.random.default_rng(3)
    ks = rng.standard_normal((BT, Hkv * D)).astype(np.float32)
    vs = rng.standard_normal((BT, Hkv * D)).astype(np.float32) * 3
    for t in range(BT):
        bp.append(b, ks[t], vs[t])
    info = bp.block(b)
    assert info.token_count == BT and info.has_content_hash == 0 and info.revision >= BT
    for tensor, src in ((0, ks), (1, vs)):
        got = bp.rows(b, tensor)
        if fmt == llm_hip.KV_BF16:
            assert np.array_equal(got, bf16_round(src))
        else:  # int8 per (token, head): codes * f16(absmax / 127), quantised from the f32 row
            for t in range(BT):
                for h in range(Hkv):
                    st, codes, s16 = oracle.quantize_int8_head(src[t, h * D:(h + 1) * D])
                    assert st == oracle.OK
                    scale = np.array([s16], np.uint16).view(np.float16).astype(np.float32)[0]
                    assert np.array_equal(got[t, h * D:(h + 1) * D], codes.astype(np.float32) * scale), (t, h)
    with pytest.raises(LlhError) as e:
        bp.append(b, ks[0], vs[0])
    assert e.value.status == llm_hip.ERR_CAPACITY
    with pytest.raises(LlhError) as e:
        bp.append(b, ks[0][:5], vs[0][:5])
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    assert ctx.device_errors() == 0


def test_cow_copies_the_device_payload(ctx):
    """paged_blocks.rs: copy_on_write_session_block_clones_shared_prefix_on_first_write, with payload."""
    Hkv, D = 2, 64
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, 3)
    bp = BlockPool.over(ctx, pool)
    reader, writer = bp.create_session(), bp.create_session()
    shared = bp.allocate_for_session(reader)
    rows = np.arange(3 * Hkv * D, dtype=np.float32).reshape(3, Hkv * D) / 64.0
    for r in rows:
        bp.append(shared, r, -r)
    bp.append_block_to_session(writer, shared)
    with pytest.raises(LlhError):
        bp.append(shared, rows[0], rows[0])  # shared: must be copied first
    wb = bp.copy_on_write_session_block(writer, 0)
    assert wb != shared
    assert np.array_equal(bp.keys(wb), bp.keys(shared)) and np.array_equal(bp.values(wb), bp.values(shared))
    bp.append(wb, rows[0] + 100, rows[0] - 100)
    assert bp.block(shared).token_count == 3 and bp.block(wb).token_count == 4
    assert np.array_equal(bp.keys(shared), bf16_round(rows))
    assert np.array_equal(bp.keys(wb)[3], bf16_round(rows[0] + 100))
    assert bp.block(shared).pool_index != bp.block(wb).pool_index


def test_decode_through_prefix_shared_session_tables(ctx):
    """A 40-token prefix (2.5 blocks) registered under its chain hash, attached by 4
    sessions that copy the partial block on write and append their own tokens; the
    batched decode over the sessions' device tables equals the oracle over each
    session's logical rows, and the shared prefix blocks are unchanged."""
    import torch

    Hq, Hkv, D = 16, 8, 128
    prefix_len, suffix = 40, [1, 9, 30, 77]
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, 64)
    bp = BlockPool.over(ctx, pool)
    seed = 0x5EED
    owner = bp.create_session()
    pk = rows_bf16(seed, 0, 0, prefix_len, Hkv, D)
    pv = rows_bf16(seed + 1, 0, 0, prefix_len, Hkv, D)

    def write_rows(block_id, first_tok, k_rows, v_rows):
        base = bp.block(block_id).pool_index * BT + first_tok
        slots = np.arange(base, base + len(k_rows), dtype=np.int64)
        ctx.append(pool, to_dev(slots), to_dev(k_rows), to_dev(v_rows))
        torch.cuda.synchronize()
        bp.commit_tokens(block_id, len(k_rows))

    prefix_ids, prev = [], bytes(32)
    tokens = list(range(1000, 1000 + prefix_len))
    for j in range(0, prefix_len, BT):
        b = bp.allocate_for_session(owner)
        write_rows(b, 0, pk[j:j + BT], pv[j:j + BT])
        prev = cache_block_chain_hash("qwen3-0.6b", "layer-0", prev, tokens[j:j + BT])
        bp.set_content_hash(b, prev)
        prefix_ids.append(b)
    bp.register_prefix(prev, prefix_ids)
    snapshot_k = [bp.keys(b).copy() for b in prefix_ids]

    sessions, logical_k, logical_v = [], [], []
    for r, n in enumerate(suffix):
        s = bp.create_session()
        assert bp.attach_prefix_to_session(s, prev) == prefix_ids
        sk = rows_bf16(seed + 2, r, 0, n, Hkv, D)
        sv = rows_bf16(seed + 3, r, 0, n, Hkv, D)
        last = bp.copy_on_write_session_block(s, len(prefix_ids) - 1)  # the partial block
        assert last != prefix_ids[-1]
        done = 0
        fill = prefix_len % BT
        while done < n:
            take = min(BT - fill, n - done)
            write_rows(last, fill, sk[done:done + take], sv[done:done + take])
            done += take
            if done < n:
                last, fill = bp.allocate_for_session(s), 0
        sessions.append(s)
        logical_k.append(np.concatenate([pk, sk]))
        logical_v.append(np.concatenate([pv, sv]))

    lens = np.array([prefix_len + n for n in suffix], np.int32)
    mb = max(len(bp.session_blocks(s)[1]) for s in sessions)
    tables = np.full((len(sessions), mb), -1, np.int32)
    for i, s in enumerate(sessions):
        idx = bp.session_blocks(s)[1]
        tables[i, :len(idx)] = idx
    q = oracle.normal_bf16(seed + 4, len(sessions) * Hq * D)
    desc = ctx.decode_desc(to_dev(lens), to_dev(tables), Hq, int(lens.max()))
    out = torch.empty(len(sessions) * Hq * D, dtype=torch.int16, device="cuda")
    scale = 1.0 / math.sqrt(D)
    ctx.paged_decode(pool, desc, to_dev(q), out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    got = from_dev_bf16(out).reshape(len(sessions), Hq * D)
    qf = oracle.bf16_to_f32(q).reshape(len(sessions), Hq * D)
    for i in range(len(sessions)):
        kf = oracle.bf16_to_f32(logical_k[i].ravel())
        vf = oracle.bf16_to_f32(logical_v[i].ravel())
        st, ref = oracle.attention_mix(qf[i], kf, vf, int(lens[i]), Hq, Hkv, D, scale)
        assert st == oracle.OK
        assert_parity(got[i], ref, what=f"session {i}")
    for b, k0 in zip(prefix_ids, snapshot_k):
        assert np.array_equal(bp.keys(b), k0)
    assert bp.block(prefix_ids[0]).ref_count == 1 + len(sessions)
    assert bp.block(prefix_ids[-1]).ref_count == 1  # every reader copied it
    assert bp.metrics_snapshot().total_cow_clones == len(sessions)
