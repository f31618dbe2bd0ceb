"""The native prefix cache (llh_prefix_cache_*) on the CPU, against the reference's own tests.

Every test restates one test of
crates/llm-native-runtime/src/native_text/tests/prefix_cache.rs (cited per test) or
crates/llm-native-runtime/src/native_text/prefix_cache.rs, with the reference's
TestCache fixture (tests/fixtures.rs:19-38): a payload of one state whose size is
`bytes` and whose identity is `marker`.  Here the state handle is the marker and
the entry size is 4 * len(hidden) + bytes, exactly prefix_cache_entry_bytes.
"""
import threading

import numpy as np
import pytest

import llm_hip

U64_MAX = (1 << 64) - 1


def ns(name):
    return f"namespace:{name}"


def store(cache, namespace, tokens, hidden, bytes_, marker):
    return cache.store(namespace, tokens, hidden, [marker], bytes_)


def marker(hit):
    return int(hit.states[0])


def test_reuses_longest_namespace_compatible_prefix():
    """prefix_cache_reuses_longest_namespace_compatible_prefix (tests/prefix_cache.rs:40-63)"""
    cache = llm_hip.PrefixCache(1024)
    store(cache, ns("base"), [1, 2], [0.5, 1.5], 11, 7)
    hit = cache.lookup(ns("base"), [1, 2, 3])
    assert hit is not None and hit.token_count == 2
    assert list(hit.hidden) == [0.5, 1.5]
    assert marker(hit) == 7
    assert cache.lookup(ns("different"), [1, 2]) is None


def test_lookup_skips_capacity_incompatible_entries():
    """prefix_cache_lookup_skips_capacity_incompatible_entries (tests/prefix_cache.rs:66-91)"""
    cache = llm_hip.PrefixCache(1024)
    store(cache, ns("capacity"), [1, 2], [0.5, 1.5], 11, 7)
    assert cache.lookup(ns("capacity"), [1, 2, 3], compatible=lambda s: all(s != 7)) is None
    hit = cache.lookup(ns("capacity"), [1, 2, 3], compatible=lambda s: all(s == 7))
    assert hit.token_count == 2


def test_reuses_longest_compatible_prefix_across_branching_index_paths():
    """prefix_cache_reuses_longest_compatible_prefix_across_branching_index_paths (tests/prefix_cache.rs:94-144)"""
    cache = llm_hip.PrefixCache(2048)
    hidden = [0.5, 1.5]
    store(cache, ns("branching"), [1, 2], hidden, 8, 2)
    store(cache, ns("branching"), [1, 2, 3], hidden, 8, 3)
    store(cache, ns("branching"), [1, 4, 5], hidden, 8, 45)
    fallback = cache.lookup(ns("branching"), [1, 2, 3, 9], compatible=lambda s: all(s != 3))
    assert fallback.token_count == 2 and marker(fallback) == 2
    branch = cache.lookup(ns("branching"), [1, 4, 5, 6])
    assert branch.token_count == 3 and marker(branch) == 45


def test_lookup_metrics_count_indexed_candidates_not_full_namespace():
    """prefix_cache_lookup_metrics_count_indexed_candidates_not_full_namespace (tests/prefix_cache.rs:147-177)"""
    cache = llm_hip.PrefixCache(1_000_000)
    store(cache, ns("indexed-metrics"), [1, 2, 3], [1.0], 1, 1)
    for i in range(128):
        store(cache, ns("indexed-metrics"), [10_000 + i], [1.0], 1, 1)
    hit = cache.lookup(ns("indexed-metrics"), [1, 2, 3, 4])
    assert hit.token_count == 3
    m = cache.metrics()
    assert m["entries_scanned"] == 1
    assert m["namespace_entries_scanned"] == 1


def test_lookup_skips_same_length_nonmatching_entries():
    """prefix_cache_lookup_skips_same_length_nonmatching_entries (tests/prefix_cache.rs:180-215)"""
    cache = llm_hip.PrefixCache(1_000_000)
    store(cache, ns("same-length"), [1, 2, 3], [1.0], 1, 7)
    for i in range(128):
        store(cache, ns("same-length"), [10_000 + i, 2, 3], [1.0], 1, 7)
    checks = []

    def compatible(states):
        checks.append(1)
        return all(states == 7)

    hit = cache.lookup(ns("same-length"), [1, 2, 3, 4], compatible=compatible)
    assert hit.token_count == 3
    assert len(checks) == 1
    m = cache.metrics()
    assert m["entries_scanned"] == 1 and m["namespace_entries_scanned"] == 1


def test_replacement_keeps_lookup_index_single_candidate():
    """prefix_cache_replacement_keeps_lookup_index_single_candidate (tests/prefix_cache.rs:218-264)"""
    released = []
    cache = llm_hip.PrefixCache(1024, release=lambda s: released.append(int(s[0])))
    store(cache, ns("replace-index"), [1, 2], [1.0], 8, 1)
    store(cache, ns("replace-index"), [1, 2], [1.0], 8, 2)
    assert released == [1]  # the replaced payload is dropped
    assert marker(cache.lookup(ns("replace-index"), [1, 2, 3])) == 2
    checks = []
    assert cache.lookup(ns("replace-index"), [1, 2, 3], compatible=lambda s: checks.append(1) or False) is None
    assert len(checks) == 1
    assert cache.shape(ns("replace-index"))["indexed"] == 1


def test_eviction_removes_lookup_index_candidate():
    """prefix_cache_eviction_removes_lookup_index_candidate (tests/prefix_cache.rs:267-319)"""
    cache = llm_hip.PrefixCache(32)
    hidden = [1.0] * 4
    store(cache, ns("evict-index"), [1, 2], hidden, 8, 12)
    store(cache, ns("evict-index"), [9], hidden, 8, 9)
    before = cache.metrics()["entries_scanned"]
    checks = []
    assert cache.lookup(ns("evict-index"), [1, 2, 3], compatible=lambda s: checks.append(1) or True) is None
    assert len(checks) == 0
    assert cache.metrics()["entries_scanned"] - before == 0
    assert cache.lookup(ns("evict-index"), [9]) is not None


def test_stores_entries_in_namespace_buckets():
    """prefix_cache_stores_entries_in_namespace_buckets (tests/prefix_cache.rs:322-358)"""
    cache = llm_hip.PrefixCache(1024)
    store(cache, ns("bucket"), [1], [1.0], 8, 1)
    store(cache, ns("bucket"), [1, 2], [1.0], 8, 1)
    store(cache, ns("other-bucket"), [9], [1.0], 8, 1)
    assert cache.shape(ns("bucket"))["namespaces"] == 2
    assert cache.shape(ns("bucket"))["entries"] == 2
    assert cache.shape(ns("other-bucket"))["entries"] == 1


def test_prefers_longest_prefix_over_recency_and_updates_lru():
    """prefix_cache_prefers_longest_prefix_over_recency_and_updates_lru (tests/prefix_cache.rs:361-414)"""
    cache = llm_hip.PrefixCache(48)
    hidden = [1.0, 2.0, 3.0, 4.0]
    store(cache, ns("longest-lru"), [1, 2, 3], hidden, 8, 3)
    store(cache, ns("longest-lru"), [1, 2], hidden, 8, 2)
    hit = cache.lookup(ns("longest-lru"), [1, 2, 3, 4])
    assert hit.token_count == 3 and marker(hit) == 3
    store(cache, ns("longest-lru-other"), [9], hidden, 8, 9)
    assert cache.lookup(ns("longest-lru"), [1, 2]) is None
    assert cache.lookup(ns("longest-lru"), [1, 2, 3]) is not None
    assert cache.lookup(ns("longest-lru-other"), [9]) is not None


def test_lru_index_tracks_store_promotion_replacement_namespace_removal_and_multi_eviction():
    """prefix_cache_lru_index_tracks_store_promotion_replacement_namespace_removal_and_multi_eviction
    (tests/prefix_cache.rs:417-556)"""
    cache = llm_hip.PrefixCache(24)
    base, old, resident, large = ns("lru-index-base"), ns("lru-index-old"), ns("lru-index-resident"), ns(
        "lru-index-large")
    hidden = [1.0]
    assert store(cache, base, [1], hidden, 4, 1)
    assert store(cache, base, [2], hidden, 4, 2)
    assert store(cache, old, [9], hidden, 4, 9)
    assert cache.lru_order() == [(base, [1]), (base, [2]), (old, [9])]
    assert cache.lookup(base, [1]) is not None
    assert cache.lru_order() == [(base, [2]), (old, [9]), (base, [1])]
    assert store(cache, base, [2], hidden, 4, 20)
    assert cache.lru_order() == [(old, [9]), (base, [1]), (base, [2])]
    assert marker(cache.lookup(base, [2])) == 20
    assert store(cache, resident, [7], hidden, 4, 7)
    assert cache.lookup(old, [9]) is None
    # evicting a namespace's last entry removes its bucket and its lookup index
    assert cache.shape(old)["entries"] == 0 and cache.shape(old)["indexed"] == 0
    assert cache.lru_order() == [(base, [1]), (base, [2]), (resident, [7])]
    assert store(cache, large, [4], hidden, 12, 4)
    assert cache.lru_order() == [(resident, [7]), (large, [4])]
    assert cache.lookup(base, [1]) is None
    assert cache.lookup(base, [2]) is None
    assert cache.lookup(resident, [7]) is not None
    assert cache.lookup(large, [4]) is not None


def test_hit_payload_is_handed_out_without_the_cache_lock():
    """prefix_cache_clones_payloads_outside_global_lock (tests/prefix_cache.rs:558-583): the retain
    callback (this backend's clone of the hit payload) runs while the cache's lock is free, so it
    can call back into the cache; a held lock would deadlock here."""
    seen = []
    holder = {}

    def retain(states):
        # re-entering the cache from the retain callback needs its lock to be free
        done = threading.Event()

        def probe():
            seen.append(holder["cache"].shape(ns("clone-lock"))["entries"])
            done.set()

        t = threading.Thread(target=probe)
        t.start()
        assert done.wait(5.0), "cache lock held while handing out the hit payload"
        t.join()

    cache = llm_hip.PrefixCache(1024, retain=retain)
    holder["cache"] = cache
    store(cache, ns("clone-lock"), [1, 2], [0.5, 1.5], 8, 3)
    assert seen == [0]  # the store's own reference is taken before the entry is visible
    hit = cache.lookup(ns("clone-lock"), [1, 2, 3])
    assert hit.token_count == 2
    assert seen == [0, 1]


def test_metrics_record_lookup_scans_and_hit_clone_bytes():
    """prefix_cache_metrics_record_lookup_scans_and_hit_clone_bytes (tests/prefix_cache.rs:585-638)"""
    cache = llm_hip.PrefixCache(1024)
    hidden = [1.0, 2.0, 3.0, 4.0]
    store(cache, ns("scan-metrics"), [1], hidden, 5, 1)
    store(cache, ns("scan-metrics"), [1, 2], hidden, 7, 2)
    store(cache, ns("scan-metrics-other"), [9], hidden, 11, 9)
    assert cache.lookup(ns("scan-metrics"), [1, 2, 3]).token_count == 2
    assert cache.lookup(ns("scan-metrics"), [42]) is None
    m = cache.metrics()
    assert m["entries_scanned"] == 1
    assert m["namespace_entries_scanned"] == 1
    assert m["hit_clone_bytes"] == 4 * 4 + 7


def test_uses_value_sizing_for_eviction_budget():
    """prefix_cache_uses_value_sizing_for_eviction_budget (tests/prefix_cache.rs:640-673)"""
    cache = llm_hip.PrefixCache(32)
    hidden = [1.0] * 4
    store(cache, ns("budget"), [1], hidden, 8, 1)
    store(cache, ns("budget"), [2], hidden, 8, 2)
    assert cache.lookup(ns("budget"), [1]) is None
    assert cache.lookup(ns("budget"), [2]) is not None
    m = cache.metrics()
    assert m["evictions"] == 1
    assert m["resident_bytes"] == 24


def test_metrics_saturate_token_counters():
    """native_text_prefix_cache_metrics_saturate_token_counters (prefix_cache.rs:673-700)"""
    cache = llm_hip.PrefixCache(1024)
    cache.record(llm_hip.PREFIX_RECORD_HIT, U64_MAX - 1)
    cache.record(llm_hip.PREFIX_RECORD_HIT, 2)
    cache.record(llm_hip.PREFIX_RECORD_MISS_TOKENS, U64_MAX - 2)
    cache.record(llm_hip.PREFIX_RECORD_MISS_TOKENS, 3)
    cache.record(llm_hip.PREFIX_RECORD_PREFILL_CHUNK, U64_MAX - 3)
    cache.record(llm_hip.PREFIX_RECORD_PREFILL_CHUNK, 4)
    cache.record(llm_hip.PREFIX_RECORD_CHECKPOINT_STORE, U64_MAX - 4)
    cache.record(llm_hip.PREFIX_RECORD_CHECKPOINT_STORE, 5)
    cache.record(llm_hip.PREFIX_RECORD_CHECKPOINT_REUSE, U64_MAX - 5)
    cache.record(llm_hip.PREFIX_RECORD_CHECKPOINT_REUSE, 6)
    cache.record(llm_hip.PREFIX_RECORD_SHARED_PREFIX_REUSE, U64_MAX - 6)
    cache.record(llm_hip.PREFIX_RECORD_SHARED_PREFIX_REUSE, 7)
    m = cache.metrics()
    assert m["reused_tokens"] == U64_MAX
    assert m["hit_tokens"] == U64_MAX
    assert m["avoided_prefill_tokens"] == U64_MAX
    assert m["miss_tokens"] == U64_MAX
    assert m["prefill_tokens"] == U64_MAX
    assert m["checkpoint_stores"] == 2
    assert m["checkpoint_store_tokens"] == U64_MAX
    assert m["checkpoint_reuse_hits"] == 2
    assert m["checkpoint_reused_tokens"] == U64_MAX
    assert m["shared_prefix_hits"] == 2
    assert m["shared_prefix_reused_tokens"] == U64_MAX
    with pytest.raises(llm_hip.LlhError):
        cache.record(99, 1)


def test_empty_and_oversized_entries_are_not_stored():
    """store (prefix_cache.rs:256-270): no empty prefix; an entry over the whole budget is rejected."""
    touched = []
    cache = llm_hip.PrefixCache(16, retain=lambda s: touched.append(("retain", int(s[0]))),
                                release=lambda s: touched.append(("release", int(s[0]))))
    assert not store(cache, ns("x"), [], [1.0], 1, 1)
    assert not store(cache, ns("x"), [1], [1.0] * 4, 1, 2)  # 17 bytes > 16
    assert cache.metrics()["rejected"] == 1
    assert cache.shape(ns("x"))["entries"] == 0
    assert touched == []  # nothing was kept, so no reference was taken or dropped


def test_release_on_eviction_and_destroy_and_retain_on_hit():
    """The payload handles follow the reference's Arc lifetimes: one reference per resident
    entry (dropped on eviction / replacement / destroy) and one per hit."""
    retained, released = [], []
    cache = llm_hip.PrefixCache(40, retain=lambda s: retained.extend(int(x) for x in s),
                                release=lambda s: released.extend(int(x) for x in s))
    cache.store(ns("r"), [1, 2], [0.0] * 2, [10, 11], 8)   # 16 bytes
    cache.store(ns("r"), [5], [0.0] * 2, [50], 8)           # 16 bytes
    assert retained == [10, 11, 50]  # the cache's own references
    assert cache.lookup(ns("r"), [1, 2, 7]).token_count == 2
    assert retained == [10, 11, 50, 10, 11]  # plus the caller's, for the hit
    cache.store(ns("r"), [6], [0.0] * 2, [60], 8)           # evicts the LRU entry: [5]
    assert released == [50]
    cache.close()
    assert sorted(released) == [10, 11, 50, 60]


def test_random_operations_match_a_python_model():
    """A plain-Python restatement of prefix_cache.rs (dicts, a sorted length list, an access
    counter) driven by random stores and lookups: hits, evictions and LRU order agree."""
    rng = np.random.default_rng(5)
    budget = 200
    cache = llm_hip.PrefixCache(budget)
    model = {}  # (ns, tokens) -> [byte_len, last_used, marker]
    access = [0]

    def tick():
        a = access[0]
        access[0] += 1
        return a

    for step in range(600):
        name = ns(f"n{rng.integers(0, 3)}")
        toks = tuple(int(x) for x in rng.integers(0, 3, size=rng.integers(1, 5)))
        if rng.random() < 0.5:
            hidden_len, extra = int(rng.integers(0, 6)), int(rng.integers(0, 40))
            size = 4 * hidden_len + extra
            ok = store(cache, name, list(toks), [1.0] * hidden_len, extra, step)
            if size > budget:
                assert not ok
                continue
            assert ok
            used = sum(v[0] for k, v in model.items())
            if (name, toks) in model:
                used -= model.pop((name, toks))[0]
            while used + size > budget and model:
                oldest = min(model, key=lambda k: model[k][1])
                used -= model.pop(oldest)[0]
            model[(name, toks)] = [size, tick(), step]
        else:
            prompt = tuple(int(x) for x in rng.integers(0, 3, size=rng.integers(1, 6)))
            hit = cache.lookup(name, list(prompt))
            best = None
            for n in sorted({len(k[1]) for k in model if k[0] == name}, reverse=True):
                if n <= len(prompt) and (name, prompt[:n]) in model:
                    best = (name, prompt[:n])
                    break
            if best is None:
                assert hit is None
            else:
                assert hit is not None and hit.token_count == len(best[1])
                assert marker(hit) == model[best][2]
                model[best][1] = tick()
        order = sorted(model, key=lambda k: model[k][1])
        assert cache.lru_order() == [(k[0], list(k[1])) for k in order]
