"""The boundary's threading contract on the GPU: one context shared by several
host threads, as the reference shares one backend process-wide and calls its
&self methods concurrently (crates/llm-native-runtime/src/native_matvec.rs:2787-2819).

Batched decodes on distinct streams use distinct workspaces (split partials,
merge descriptors), so concurrent C2-shaped decodes on two streams must each
give exactly the bits they give alone, call after call, while their workspaces
grow; trait-mirror caches wait for their own streams only.
"""
import math
import threading

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import assert_parity, from_dev_bf16, rows_bf16, to_dev
from llm_hip import LayerKvCache, HipNativeMatvecBackend, workloads

pytestmark = pytest.mark.gpu

D = 128
BT = 16


class Case:
    """A paged batch with its own pool, q, output and stream."""

    def __init__(self, ctx, lens, Hq, Hkv, seed, kernel):
        import torch

        self.batch = workloads.paged_batch(lens, BT, 0.10, seed)
        b = self.batch
        ids, src_k = workloads.block_sources(b, lambda s, lo, hi: rows_bf16(seed + 1, s, lo, hi, Hkv, D), Hkv, D)
        _, src_v = workloads.block_sources(b, lambda s, lo, hi: rows_bf16(seed + 2, s, lo, hi, Hkv, D), Hkv, D)
        self.pool = ctx.pool(llm_hip.KV_BF16, BT, Hkv, D, b.n_blocks)
        ctx.write_blocks(self.pool, to_dev(ids), to_dev(src_k), to_dev(src_v))
        self.q = oracle.normal_bf16(seed + 3, b.seq_lens.size * Hq * D)
        self.d_q = to_dev(self.q)
        self.out = torch.zeros(b.seq_lens.size * Hq * D, dtype=torch.int16, device="cuda")
        self.d_lens, self.d_tab = to_dev(b.seq_lens), to_dev(b.tables)
        self.desc = ctx.decode_desc(self.d_lens, self.d_tab, Hq, int(b.seq_lens.max()))
        self.Hq, self.Hkv, self.kernel = Hq, Hkv, kernel
        self.stream = torch.cuda.Stream()
        torch.cuda.synchronize()

    def run(self, ctx):
        ctx.paged_decode(self.pool, self.desc, self.d_q, self.out, 0.088, stream=self.stream)
        self.stream.synchronize()
        return from_dev_bf16(self.out).copy()

    def reference(self):
        b = self.batch
        opool = oracle.Pool.from_raw(llm_hip.KV_BF16, BT, self.Hkv, D, b.n_blocks, self.pool.raw())
        st, ref = opool.decode(self.Hq, b.seq_lens, b.tables, 0, self.q, 0.088, threads=16)
        assert st == oracle.OK
        return ref


def test_concurrent_decodes_on_two_streams_share_one_context(ctx, opts):
    """Two host threads, two streams, two pools, C2-shaped batches (the stream kernel,
    whose cut segments leave partials in the workspace): 40 calls each, run together.
    Every call must equal the call made alone, and that must meet the oracle bar."""
    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    cases = [Case(ctx, lens, 16, 8, 500, "stream"), Case(ctx, lens[::-1].copy(), 16, 8, 600, "stream")]
    alone = [c.run(ctx) for c in cases]
    for c, out in zip(cases, alone):
        assert_parity(out, c.reference(), what="alone")
    errors = []

    def worker(i):
        try:
            for _ in range(40):
                got = cases[i].run(ctx)
                if not np.array_equal(got, alone[i]):
                    errors.append(f"thread {i}: output differs from the same call made alone")
                    return
        except Exception as e:  # pragma: no cover - reported below
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads), "a decode thread did not finish"
    assert not errors, errors
    assert ctx.device_errors() == 0, ctx.last_error()
    for c in cases:
        ctx.release_stream(c.stream)


def test_concurrent_decodes_while_workspaces_grow(ctx, opts):
    """Each thread alternates a small split-K step and a large stream step on its own
    stream, so its workspace grows mid-run while the other thread's kernels are in
    flight; both keep giving their solo results."""
    opts(llm_hip.OPT_DECODE_KERNEL, "auto")
    small = [Case(ctx, [512], 16, 8, 700 + i, "split") for i in range(2)]
    big = [Case(ctx, workloads.uniform_lengths(48, 1000, 4096, 710 + i), 32, 8, 720 + i, "stream") for i in range(2)]
    for i in range(2):  # each thread's cases share one stream: the small one comes first (smaller workspace)
        big[i].stream = small[i].stream
    alone = [[c.run(ctx) for c in (small[i], big[i])] for i in range(2)]
    for i in range(2):  # start the threads with no workspace: the first small call allocates, the big one grows
        ctx.release_stream(small[i].stream)
    errors = []

    def worker(i):
        try:
            for _ in range(15):
                for j, c in enumerate((small[i], big[i])):
                    if not np.array_equal(c.run(ctx), alone[i][j]):
                        errors.append(f"thread {i} case {j} differs")
                        return
        except Exception as e:  # pragma: no cover
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    assert ctx.device_errors() == 0
    for i in range(2):
        assert_parity(alone[i][1], big[i].reference(), what="large case")
        ctx.release_stream(small[i].stream)


def test_trait_caches_on_two_threads(ctx):
    """Two threads each append to and attend over their own LayerKvCache (each cache waits
    for its own stream): the results equal the oracle's reference loop on the same rows."""
    errors = []
    results = {}

    def worker(i):
        try:
            rng = np.random.default_rng(800 + i)
            cache = LayerKvCache.new(ctx, 256, 8, D)
            backend = HipNativeMatvecBackend(ctx)
            for t in range(200):
                k = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(8 * D).astype(np.float32)))
                v = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.standard_normal(8 * D).astype(np.float32)))
                backend.append_kv_cache_sliding_f32(cache, k, v)
            q = rng.standard_normal(16 * D).astype(np.float32)
            out = np.zeros(16 * D, np.float32)
            for _ in range(20):
                assert backend.full_attention_cache_mix_f32_in_place(cache, q, 200, 16, 8, D, 1 / math.sqrt(D), out)
            results[i] = (q, cache.keys().copy(), cache.values().copy(), out.copy())
            cache.close()
        except Exception as e:  # pragma: no cover
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not errors, errors
    for i in range(2):
        q, keys, vals, out = results[i]
        st, ref = oracle.attention_mix(q, keys, vals, 200, 16, 8, D, 1 / math.sqrt(D))
        assert st == oracle.OK
        d = np.abs(out - ref)
        assert d.max() <= 2e-2 and d.mean() <= 2e-3, (d.max(), d.mean())


def test_last_error_is_per_thread(ctx):
    """llh_ctx_last_error returns the calling thread's copy: a message read by one thread
    stays intact while another thread's failures replace the context's message."""
    pool = ctx.pool(llm_hip.KV_BF16, BT, 8, D, 4)
    import torch

    z = torch.zeros(2, dtype=torch.int32, device="cuda")
    bad = ctx.decode_desc(z[:1], z.view(1, 2), 12, 16)  # 12 q heads over 8 kv heads
    with pytest.raises(llm_hip.LlhError):
        ctx.paged_decode(pool, bad, z, z, 0.1)
    raw = ctx.lib.llh_ctx_last_error(ctx.handle)  # bytes copy of this thread's string
    stop = threading.Event()

    def spam():
        d = ctx.decode_desc(z[:1], z.view(1, 2), 16, 16, window=-5)
        while not stop.is_set():
            try:
                ctx.paged_decode(pool, d, z, z, 0.1)
            except llm_hip.LlhError:
                pass

    t = threading.Thread(target=spam)
    t.start()
    try:
        for _ in range(200):
            assert ctx.lib.llh_ctx_last_error(ctx.handle) in (raw, b"window must be >= 0")
    finally:
        stop.set()
        t.join()
    pool.close()
