"""Device mirrors of host caches that already hold rows, and the context's per-stream
bookkeeping.

* llh_layer_cache_create_from_rows = LayerKvCache::from_snapshot
  (crates/llm-kv-cache/src/layer.rs:467-507: rows re-laid from slot 0, revision and
  tokens_seen kept) and from_prefix_cache_state (layer.rs:544-581: the ring's own
  window_start kept), the caches the driver restores on a prefix-cache hit
  (crates/llm-native-runtime/src/native_text/driver.rs:694-703).  The restored
  mirror's state, active runs and rows follow the oracle's LayerKvCache
  restatement; its attention meets the bar against the reference loop, and a mirror
  restored from a prefix state attends bit for bit like the cache it came from.
* destroying a layer cache releases its stream's workspace slot;
* device error flags are kept per stream.
"""
import numpy as np
import pytest

import llm_hip
import oracle
from helpers import to_dev
from llm_hip import HipNativeMatvecBackend, LayerKvCache
from test_gpu_decode import build_case

pytestmark = pytest.mark.gpu

BT = 16


def bf16_exact(rng, n):
    return oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(n).astype(np.float32)))


def filled(ctx, fmt, max_tokens, hkv, d, n_append, seed):
    """A mirror and the oracle ring after n_append sliding appends of the same bf16-exact rows."""
    rng = np.random.default_rng(seed)
    cache = LayerKvCache.new_with_config(ctx, max_tokens, hkv, d, fmt)
    ring = oracle.Ring(max_tokens, hkv * d, BT)
    for _ in range(n_append):
        k, v = bf16_exact(rng, hkv * d), bf16_exact(rng, hkv * d)
        cache.append_sliding(k, v)
        ring.append_sliding(k, v)
    return cache, ring, rng


def runs_of(cache):
    return [(r["block_index"], r["logical_token_start"], r["physical_token_start"], r["block_token_start"],
             r["token_count"]) for r in cache.active_blocks()]


def mix(ctx, cache, q, rows, hq, hkv, d):
    out = np.zeros(hq * d, np.float32)
    assert HipNativeMatvecBackend(ctx).full_attention_cache_mix_f32_in_place(cache, q, rows, hq, hkv, d, 0.0883883,
                                                                            out)
    return out


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_INT8_ROW])
@pytest.mark.parametrize("max_tokens,hkv,d,n_append,hq", [(64, 8, 128, 150, 16), (512, 8, 128, 700, 16),
                                                          (50, 2, 4, 123, 4), (33, 1, 8, 33, 2)])
def test_restore_from_snapshot_and_prefix_state(ctx, opts, fmt, max_tokens, hkv, d, n_append, hq):
    opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
    orig, ring, rng = filled(ctx, fmt, max_tokens, hkv, d, n_append, max_tokens + n_append + fmt)
    keys, vals = ring.logical_rows(0), ring.logical_rows(1)  # the host cache's keys() / values()
    n = ring.token_count
    snap = LayerKvCache.from_rows(ctx, max_tokens, hkv, d, keys, vals, revision=ring.revision,
                                  tokens_seen=ring.tokens_seen, window_start=0, fmt=fmt)
    pref = LayerKvCache.from_rows(ctx, max_tokens, hkv, d, keys, vals, revision=ring.revision,
                                  tokens_seen=ring.tokens_seen, window_start=ring.window_start, fmt=fmt)
    # from_snapshot: the rows re-laid from slot 0 (a fresh ring appended strictly), revision and tokens_seen kept
    fresh = oracle.Ring(max_tokens, hkv * d, BT)
    for i in range(n):
        fresh.append(keys[i * hkv * d:(i + 1) * hkv * d], vals[i * hkv * d:(i + 1) * hkv * d])
    s = snap.state()
    assert (s.token_count, s.tokens_seen, s.window_start, s.revision) == (n, ring.tokens_seen, 0, ring.revision)
    assert runs_of(snap) == fresh.active_runs()
    # from_prefix_cache_state: the very ring state of the cache it came from
    s = pref.state()
    assert (s.token_count, s.tokens_seen, s.window_start, s.revision) == (
        n, ring.tokens_seen, ring.window_start, ring.revision)
    assert runs_of(pref) == ring.active_runs()
    assert len({orig.id(), snap.id(), pref.id()}) == 3
    assert not set(snap.block_ids()) & set(orig.block_ids())
    # rows stored as appending them stores them (bf16 rounding, int8 quantisation), bit for bit
    for c in (snap, pref):
        assert np.array_equal(c.keys(), orig.keys()) and np.array_equal(c.values(), orig.values())
    # attention: the bar against the reference loop on the stored rows; the prefix-state mirror
    # has the original's layout and attends bit for bit like it
    q = rng.standard_normal(hq * d).astype(np.float32)
    for rows in sorted({n, max(1, n // 2), 1}):
        tuned0 = ctx.metrics()["trait_tuned_calls"]
        ref_out = mix(ctx, orig, q, rows, hq, hkv, d)
        got_p = mix(ctx, pref, q, rows, hq, hkv, d)
        got_s = mix(ctx, snap, q, rows, hq, hkv, d)
        if d == 128 and fmt != llm_hip.KV_INT8_ROW:
            assert ctx.metrics()["trait_tuned_calls"] == tuned0 + 3
        assert np.array_equal(got_p, ref_out)
        st, ref = oracle.attention_mix(q, orig.keys(), orig.values(), rows, hq, hkv, d, 0.0883883)
        assert st == oracle.OK
        for got in (got_s, got_p):
            dd = np.abs(got - ref)
            assert dd.max() <= 2e-2 and dd.mean() <= 2e-3, (rows, dd.max(), dd.mean())
    # both keep going as ring caches: further sliding appends follow the reference ring
    for _ in range(max_tokens + 5):
        k, v = bf16_exact(rng, hkv * d), bf16_exact(rng, hkv * d)
        for c in (snap, pref):
            c.append_sliding(k, v)
        ring.append_sliding(k, v)
        fresh.append_sliding(k, v)
    assert runs_of(pref) == ring.active_runs() and runs_of(snap) == fresh.active_runs()
    assert pref.revision() == ring.revision and pref.next_position() == ring.tokens_seen
    assert np.array_equal(pref.keys(), snap.keys())
    st, ref = oracle.attention_mix(q, pref.keys(), pref.values(), max_tokens, hq, hkv, d, 0.0883883)
    dd = np.abs(mix(ctx, snap, q, max_tokens, hq, hkv, d) - ref)
    assert dd.max() <= 2e-2 and dd.mean() <= 2e-3
    for c in (orig, snap, pref):
        c.close()


def test_restore_empty_cache_and_errors(ctx):
    z = np.zeros(0, np.float32)
    c = LayerKvCache.from_rows(ctx, 16, 1, 4, z, z, revision=7, tokens_seen=40, window_start=3)
    s = c.state()
    assert (s.token_count, s.tokens_seen, s.window_start, s.revision) == (0, 40, 3, 7)
    out = np.zeros(4, np.float32)
    assert HipNativeMatvecBackend(ctx).full_attention_cache_mix_f32_in_place(c, [1.0] * 4, 0, 1, 1, 4, 1.0, out)
    assert not out.any()
    c.close()
    rows = np.ones(3 * 4, np.float32)
    bad = [dict(max_tokens=2),                   # token_count > max_tokens
           dict(tokens_seen=2),                  # tokens_seen < token_count
           dict(window_start=16),                # window_start >= max_tokens
           dict(head_dim=0)]                     # zero size
    for kw in bad:
        args = dict(max_tokens=16, key_value_heads=1, head_dim=4, tokens_seen=3, window_start=0)
        args.update(kw)
        with pytest.raises(llm_hip.LlhError) as e:
            LayerKvCache.from_rows(ctx, args["max_tokens"], args["key_value_heads"], args["head_dim"], rows, rows,
                                   tokens_seen=args["tokens_seen"], window_start=args["window_start"])
        assert e.value.status == llm_hip.ERR_INVALID_SHAPE, kw
    with pytest.raises(llm_hip.LlhError) as e:  # rows not a whole number of vectors
        LayerKvCache.from_rows(ctx, 16, 1, 4, np.ones(10, np.float32), np.ones(10, np.float32))
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE
    nan = rows.copy()
    nan[5] = np.nan
    for fmt in (llm_hip.KV_INT8, llm_hip.KV_INT8_ROW):
        with pytest.raises(llm_hip.LlhError) as e:
            LayerKvCache.from_rows(ctx, 16, 1, 4, nan, rows, fmt=fmt)
        assert e.value.status == llm_hip.ERR_NON_FINITE
    with pytest.raises(llm_hip.LlhError) as e:
        LayerKvCache.from_rows(ctx, 16, 1, 4, rows, rows, fmt=llm_hip.KV_FP8_E4M3)
    assert e.value.status == llm_hip.ERR_UNSUPPORTED
    # a bf16 mirror keeps non-finite rows, as the reference's f32 cache does; its attention
    # then reports softmax_f32's error from the reference-order kernel
    c = LayerKvCache.from_rows(ctx, 16, 1, 4, nan, rows)
    with pytest.raises(llm_hip.LlhError) as e:
        HipNativeMatvecBackend(ctx).full_attention_cache_mix_f32_in_place(c, [1.0] * 4, 3, 1, 1, 4, 1.0, out)
    assert e.value.status == llm_hip.ERR_NON_FINITE
    c.close()


def test_large_restore_goes_through_several_chunks(ctx, opts):
    """A 32768-token cache of 8 x 128 rows (128 MiB of f32 rows per tensor) is restored in
    16 MiB chunks; every row lands in its ring slot."""
    opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
    T, hkv, d = 32768, 8, 128
    keys = oracle.bf16_to_f32(oracle.normal_bf16(3, T * hkv * d))
    vals = oracle.bf16_to_f32(oracle.normal_bf16(4, T * hkv * d))
    c = LayerKvCache.from_rows(ctx, T, hkv, d, keys, vals, revision=1, tokens_seen=T + 5000, window_start=5000)
    assert np.array_equal(c.keys(), keys) and np.array_equal(c.values(), vals)
    runs = c.active_blocks()
    assert runs[0]["physical_token_start"] == 5000 and sum(r["token_count"] for r in runs) == T
    q = oracle.bf16_to_f32(oracle.normal_bf16(5, 16 * d))
    st, ref = oracle.attention_mix(q, keys, vals, T, 16, hkv, d, 0.0883883)
    dd = np.abs(mix(ctx, c, q, T, 16, hkv, d) - ref)
    assert dd.max() <= 2e-2 and dd.mean() <= 2e-3
    c.close()


def test_destroying_caches_releases_their_stream_slots(ctx, opts):
    """Each cache's tuned trait calls lease a workspace slot on the cache's own stream; the
    slot (scratch and error word) goes with the cache, so creating and destroying caches
    leaves the context's slots where they were, and a later workspace reservation (which
    touches every slot's stream) still succeeds."""
    opts(llm_hip.OPT_TRAIT_REFERENCE_ORDER, 0)
    m0 = ctx.metrics()
    rng = np.random.default_rng(1)
    for i in range(40):
        c, _, _ = filled(ctx, llm_hip.KV_BF16, 64, 8, 128, 20, i)
        clone = c.clone() if i % 5 == 0 else None
        mix(ctx, c, rng.standard_normal(16 * 128).astype(np.float32), 20, 16, 8, 128)
        if clone is not None:
            mix(ctx, clone, rng.standard_normal(16 * 128).astype(np.float32), 20, 16, 8, 128)
            clone.close()
        c.close()
    m1 = ctx.metrics()
    assert m1["trait_tuned_calls"] >= m0["trait_tuned_calls"] + 48
    assert m1["stream_slots"] == m0["stream_slots"], (m0["stream_slots"], m1["stream_slots"])
    assert m1["workspace_bytes"] == m0["workspace_bytes"]
    ctx.reserve_workspace(8 << 20)
    assert ctx.device_errors() == 0


def test_device_errors_are_kept_per_stream(ctx):
    """A bad block table entry in a call on one stream raises that stream's flags only: another
    stream's word stays clear, and the context-wide read sees the union."""
    import torch
    from llm_hip import workloads

    batch = workloads.paged_batch([64, 64], BT, 0.10, seed=19)
    pool, q = build_case(ctx, batch, 16, 8, llm_hip.KV_BF16, 19)
    bad_tab = batch.tables.copy()
    bad_tab[1, 2] = batch.n_blocks + 5
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    d_q = to_dev(q)
    outs = [torch.zeros(2 * 16 * 128, dtype=torch.int16, device="cuda") for _ in range(2)]
    d_lens = to_dev(batch.seq_lens)
    tabs = [to_dev(bad_tab), to_dev(batch.tables)]
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0
    for s, t, o in ((sa, tabs[0], outs[0]), (sb, tabs[1], outs[1])):
        ctx.paged_decode(pool, ctx.decode_desc(d_lens, t, 16, 64), d_q, o, 0.1, stream=s)
    assert ctx.stream_device_errors(sb) == 0
    assert ctx.stream_device_errors(sa, reset=False) & llm_hip.ERR_FLAG_BAD_BLOCK
    assert ctx.device_errors(reset=False) & llm_hip.ERR_FLAG_BAD_BLOCK
    assert ctx.stream_device_errors(sa) & llm_hip.ERR_FLAG_BAD_BLOCK  # read and cleared
    assert ctx.device_errors() == 0
    # a released stream's flags are not lost: they fold into the context-wide read
    ctx.paged_decode(pool, ctx.decode_desc(d_lens, tabs[0], 16, 64), d_q, outs[0], 0.1, stream=sa)
    torch.cuda.synchronize()
    ctx.release_stream(sa)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK
    assert ctx.device_errors() == 0
