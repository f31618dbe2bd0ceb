"""The prefix cache feeding the device path: a cached prompt prefix (its K/V in
BlockPool device blocks) is found by a longer prompt, reused through a new
session's block table, and the new chunk is prefilled over it -- the caller
side of configs[2] (crates/llm-native-runtime/src/native_text/driver.rs:662-835:
lookup_compatible, then prefill_chunk over the hit's caches).  The prefill over
the reused blocks is checked against the oracle over the logical rows, and the
blocks' reference counts follow the cache's and the sessions' ownership.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, rows_bf16, to_dev
from llm_hip import BlockPool, PrefixCache

pytestmark = pytest.mark.gpu

BT = 16


def test_prefix_cache_hit_feeds_chunked_prefill(ctx):
    import torch

    Hq, Hkv, D = 32, 4, 128
    prefix_len, chunk = 200, 100  # the prefix ends inside a block: its tail block is copied on write
    pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, 48)
    bp = BlockPool.over(ctx, pool)
    seed = 0xCAFE
    block_bytes = 2 * BT * Hkv * D * 2
    cache = PrefixCache(1 << 30, retain=lambda s: [bp.retain(int(b)) for b in s],
                        release=lambda s: [bp.release(int(b)) for b in s])
    namespace = "model=qwen3-0.6b;layout=2;cache_tokens=4096"
    prompt = np.arange(5000, 5000 + prefix_len + chunk, dtype=np.uint32)

    def write_rows(block_id, first_tok, k_rows, v_rows):
        base = bp.block(block_id).pool_index * BT + first_tok
        slots = np.arange(base, base + len(k_rows), dtype=np.int64)
        ctx.append(pool, to_dev(slots), to_dev(k_rows), to_dev(v_rows))
        torch.cuda.synchronize()
        bp.commit_tokens(block_id, len(k_rows))

    # request 1 prefilled the prefix: its blocks belong to a session, then to the cache
    pk = rows_bf16(seed, 0, 0, prefix_len, Hkv, D)
    pv = rows_bf16(seed + 1, 0, 0, prefix_len, Hkv, D)
    owner = bp.create_session()
    prefix_ids = []
    for j in range(0, prefix_len, BT):
        b = bp.allocate_for_session(owner)
        n = min(BT, prefix_len - j)
        write_rows(b, 0, pk[j:j + n], pv[j:j + n])
        prefix_ids.append(b)
    hidden = np.linspace(-1, 1, 64, dtype=np.float32)
    assert cache.store(namespace, prompt[:prefix_len], hidden, prefix_ids, len(prefix_ids) * block_bytes)
    assert bp.block(prefix_ids[0]).ref_count == 2  # the session's and the cache's
    assert bp.release_session(owner)
    assert bp.block(prefix_ids[0]).ref_count == 1  # the cache keeps the prefix resident

    # request 2: the longest cached prefix of the longer prompt
    assert cache.lookup("another-namespace", prompt) is None
    hit = cache.lookup(namespace, prompt)
    assert hit.token_count == prefix_len
    assert np.array_equal(hit.hidden, hidden) and list(hit.states) == prefix_ids
    s = bp.create_session()
    for b in hit.states:
        bp.append_block_to_session(s, int(b))
        bp.release(int(b))  # the session now holds the reference the hit gave us
    last = bp.copy_on_write_session_block(s, len(prefix_ids) - 1)
    ck = rows_bf16(seed + 2, 0, 0, chunk, Hkv, D)
    cv = rows_bf16(seed + 3, 0, 0, chunk, Hkv, D)
    fill, done = prefix_len % BT, 0
    while done < chunk:
        take = min(BT - fill, chunk - done)
        write_rows(last, fill, ck[done:done + take], cv[done:done + take])
        done += take
        if done < chunk:
            last, fill = bp.allocate_for_session(s), 0
    assert bp.block(prefix_ids[0]).ref_count == 2  # cache + the new session (shared, not copied)

    # chunked prefill of the new tokens over the reused prefix
    ids, idx = bp.session_blocks(s)
    ctxlen = prefix_len + chunk
    tables = np.asarray(idx, np.int32).reshape(1, -1)
    starts = np.array([0, chunk], np.int32)
    lens = np.array([ctxlen], np.int32)
    q = oracle.normal_bf16(seed + 4, chunk * Hq * D)
    desc = ctx.prefill_desc(to_dev(starts), to_dev(lens), to_dev(tables), Hq, chunk, 0, total_q_rows=chunk)
    out = torch.empty(chunk * Hq * D, dtype=torch.int16, device="cuda")
    scale = 1.0 / math.sqrt(D)
    ctx.paged_prefill(pool, desc, to_dev(q), out, scale)
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    opool = oracle.Pool.from_raw(llm_hip.KV_BF16, BT, Hkv, D, 48, pool.raw())
    st, ref = opool.prefill(Hq, starts, lens, tables, 0, q, scale, threads=16)
    assert st == oracle.OK
    assert_parity(from_dev_bf16(out), ref, what="prefill over the prefix-cache hit")
    # the same attention from the logical rows (prefix from request 1, chunk from request 2)
    kf = oracle.bf16_to_f32(np.concatenate([pk, ck]).ravel())
    vf = oracle.bf16_to_f32(np.concatenate([pv, cv]).ravel())
    qf = oracle.bf16_to_f32(q).reshape(chunk, Hq * D)
    for i in (0, 1, chunk // 2, chunk - 1):  # row i attends positions [0, prefix_len + i]
        st, r = oracle.attention_mix(qf[i], kf, vf, prefix_len + i + 1, Hq, Hkv, D, scale)
        assert st == oracle.OK
        assert_parity(from_dev_bf16(out).reshape(chunk, Hq * D)[i], r, what=f"row {i} vs logical rows")

    # ownership unwinds: session, then the cache
    assert bp.release_session(s)
    assert bp.block(prefix_ids[0]).ref_count == 1
    cache.close()
    assert bp.block(prefix_ids[0]) is None or bp.block(prefix_ids[0]).ref_count == 0
    assert bp.allocated_blocks() == 0
