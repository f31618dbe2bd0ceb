// Longest-prefix cache over token ids: the driver-side lookup that turns a
// prompt into a reusable prefix (its KV state and last hidden row), as
// crates/llm-native-runtime/src/native_text/prefix_cache.rs:20-300 defines it.
//
// Entries live in per-namespace buckets keyed by their exact token sequence.
// Each namespace keeps the sorted set of entry lengths, so a lookup probes
// only the lengths <= the prompt's, longest first, and checks one exact-match
// candidate per length (prefix_cache.rs:223-255, 501-533).  The first
// candidate the caller accepts (compatibility callback) is the hit; the hit's
// access refreshes its LRU position.  Stores replace an existing entry for the
// same tokens, then evict least-recently-used entries across all namespaces
// until the new entry fits the byte budget (prefix_cache.rs:283-336); an entry
// larger than the whole budget is rejected.  Counters saturate
// (prefix_cache.rs:536-664).
//
// The payload is the caller's: a hidden row (f32) and opaque 64-bit state
// handles -- for this backend, the BlockPool block ids that hold the prefix's
// K/V on the device.  A store takes the cache's own reference to the handles
// (retain), each hit takes one for the caller, and the cache's reference is
// released when the entry is evicted, replaced or the cache destroyed; the
// callbacks run outside the cache's lock, as the reference drops payloads
// after unlocking.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "llm_hip.h"

namespace {

struct Payload {
  std::vector<float> hidden;
  std::vector<uint64_t> states;
  llh_prefix_release_fn release = nullptr;
  void *user = nullptr;
  ~Payload() {
    if (release) release(user, states.data(), states.size());
  }
};

struct TokensHash {
  size_t operator()(const std::vector<uint32_t> &t) const {
    uint64_t h = 1469598103934665603ull;  // FNV-1a over the ids
    for (uint32_t v : t) {
      h ^= v;
      h *= 1099511628211ull;
    }
    return (size_t)h;
  }
};

struct Entry {
  std::shared_ptr<Payload> payload;
  uint64_t byte_len = 0;
  uint64_t last_used = 0;
};

// Sorted distinct entry lengths of one namespace, with multiplicities.
struct LengthIndex {
  std::vector<size_t> lengths;
  std::unordered_map<size_t, size_t> counts;

  void insert(size_t n) {
    size_t &c = counts[n];
    if (c == 0) lengths.insert(std::lower_bound(lengths.begin(), lengths.end(), n), n);
    c++;
  }
  void remove(size_t n) {
    auto it = counts.find(n);
    if (it == counts.end()) return;
    if (it->second > 1) {
      it->second--;
      return;
    }
    counts.erase(it);
    auto pos = std::lower_bound(lengths.begin(), lengths.end(), n);
    if (pos != lengths.end() && *pos == n) lengths.erase(pos);
  }
  bool empty() const { return counts.empty(); }
};

struct LruKey {
  uint64_t access;
  std::string ns;
  std::vector<uint32_t> tokens;
  bool operator<(const LruKey &o) const {
    if (access != o.access) return access < o.access;
    if (ns != o.ns) return ns < o.ns;
    return tokens < o.tokens;
  }
};

uint64_t sat_add(uint64_t a, uint64_t b) { return a > UINT64_MAX - b ? UINT64_MAX : a + b; }

}  // namespace

struct llh_prefix_cache {
  uint64_t max_bytes = 0;
  llh_prefix_retain_fn retain = nullptr;
  llh_prefix_release_fn release = nullptr;
  void *user = nullptr;
  std::mutex mu;
  std::map<std::string, std::unordered_map<std::vector<uint32_t>, Entry, TokensHash>> entries;
  std::map<std::string, LengthIndex> indexes;
  std::set<LruKey> lru;
  uint64_t used_bytes = 0;
  uint64_t next_access = 0;
  std::mutex metrics_mu;
  llh_prefix_cache_counters counters{};

  uint64_t take_access() {
    const uint64_t a = next_access;
    next_access = sat_add(next_access, 1);
    return a;
  }

  // Removes an entry and its index/LRU keys; returns its payload (dropped by the caller outside the lock).
  bool remove_entry(const std::string &ns, const std::vector<uint32_t> &tokens, Entry *out) {
    auto b = entries.find(ns);
    if (b == entries.end()) return false;
    auto e = b->second.find(tokens);
    if (e == b->second.end()) return false;
    *out = std::move(e->second);
    b->second.erase(e);
    lru.erase(LruKey{out->last_used, ns, tokens});
    auto ix = indexes.find(ns);
    if (ix != indexes.end()) {
      ix->second.remove(tokens.size());
      if (ix->second.empty()) indexes.erase(ix);
    }
    if (b->second.empty()) entries.erase(b);
    return true;
  }

  template <class F>
  void update(F f) {
    std::lock_guard<std::mutex> g(metrics_mu);
    f(counters);
  }
};

extern "C" {

int llh_prefix_cache_create(uint64_t max_bytes, llh_prefix_retain_fn retain, llh_prefix_release_fn release, void *user,
                            llh_prefix_cache **out) {
  if (!out) return LLH_ERR_NULL;
  auto *pc = new llh_prefix_cache();
  pc->max_bytes = max_bytes;
  pc->retain = retain;
  pc->release = release;
  pc->user = user;
  *out = pc;
  return LLH_OK;
}

int llh_prefix_cache_destroy(llh_prefix_cache *pc) {
  if (!pc) return LLH_ERR_NULL;
  decltype(pc->entries) doomed;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    doomed.swap(pc->entries);
    pc->indexes.clear();
    pc->lru.clear();
  }
  doomed.clear();  // payloads release their handles here, outside the lock
  delete pc;
  return LLH_OK;
}

int llh_prefix_cache_store(llh_prefix_cache *pc, const char *ns, size_t ns_len, const uint32_t *tokens,
                           size_t n_tokens, const float *hidden, size_t n_hidden, const uint64_t *states,
                           size_t n_states, uint64_t state_bytes, int32_t *stored) {
  if (!pc || !stored || (!ns && ns_len) || (!tokens && n_tokens) || (!hidden && n_hidden) || (!states && n_states))
    return LLH_ERR_NULL;
  *stored = 0;
  if (n_tokens == 0) return LLH_OK;  // an empty prefix is never stored (prefix_cache.rs:262-264)
  // bytes of an entry: the hidden row plus the caller's accounting of its state
  const uint64_t byte_len = sat_add((uint64_t)n_hidden * sizeof(float), state_bytes);
  if (byte_len > pc->max_bytes) {
    pc->update([](llh_prefix_cache_counters &c) { c.rejected = sat_add(c.rejected, 1); });
    return LLH_OK;
  }
  auto payload = std::make_shared<Payload>();
  payload->hidden.assign(hidden, hidden + n_hidden);
  payload->states.assign(states, states + n_states);
  // the cache takes its own reference before the entry becomes visible (the
  // reference clones the caller's caches into the payload)
  if (pc->retain) pc->retain(pc->user, payload->states.data(), payload->states.size());
  std::vector<Entry> dropped;  // released after the lock
  std::vector<uint64_t> evicted_bytes;
  uint64_t resident_bytes, resident_entries;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    const std::string key(ns, ns_len);
    std::vector<uint32_t> toks(tokens, tokens + n_tokens);
    Entry old;
    if (pc->remove_entry(key, toks, &old)) {
      pc->used_bytes = pc->used_bytes > old.byte_len ? pc->used_bytes - old.byte_len : 0;
      dropped.push_back(std::move(old));
    }
    while (sat_add(pc->used_bytes, byte_len) > pc->max_bytes && !pc->lru.empty()) {
      const LruKey oldest = *pc->lru.begin();
      Entry ev;
      if (!pc->remove_entry(oldest.ns, oldest.tokens, &ev)) {
        pc->lru.erase(pc->lru.begin());
        continue;
      }
      pc->used_bytes = pc->used_bytes > ev.byte_len ? pc->used_bytes - ev.byte_len : 0;
      evicted_bytes.push_back(ev.byte_len);
      dropped.push_back(std::move(ev));
    }
    // the payload releases its handles once nothing references it any more
    payload->release = pc->release;
    payload->user = pc->user;
    const uint64_t access = pc->take_access();
    Entry e;
    e.payload = payload;
    e.byte_len = byte_len;
    e.last_used = access;
    pc->entries[key][toks] = std::move(e);
    pc->lru.insert(LruKey{access, key, toks});
    pc->indexes[key].insert(n_tokens);
    pc->used_bytes = sat_add(pc->used_bytes, byte_len);
    resident_bytes = pc->used_bytes;
    resident_entries = pc->lru.size();
  }
  dropped.clear();
  pc->update([&](llh_prefix_cache_counters &c) {
    for (uint64_t b : evicted_bytes) {
      c.evictions = sat_add(c.evictions, 1);
      c.bytes_evicted = sat_add(c.bytes_evicted, b);
    }
    c.stores = sat_add(c.stores, 1);
    c.bytes_stored = sat_add(c.bytes_stored, byte_len);
    c.resident_bytes = resident_bytes;
    c.resident_entries = resident_entries;
  });
  *stored = 1;
  return LLH_OK;
}

int llh_prefix_cache_lookup(llh_prefix_cache *pc, const char *ns, size_t ns_len, const uint32_t *tokens,
                            size_t n_tokens, llh_prefix_compatible_fn compatible, void *compat_user,
                            llh_prefix_hit *hit, float *hidden_out, size_t hidden_cap, uint64_t *states_out,
                            size_t states_cap) {
  if (!pc || !hit || (!ns && ns_len) || (!tokens && n_tokens)) return LLH_ERR_NULL;
  std::memset(hit, 0, sizeof(*hit));
  std::shared_ptr<Payload> found;
  size_t best = 0;
  uint64_t clone_bytes = 0, scanned = 0;
  {
    std::lock_guard<std::mutex> g(pc->mu);
    const std::string key(ns, ns_len);
    auto ix = pc->indexes.find(key);
    auto bucket = pc->entries.find(key);
    if (ix != pc->indexes.end() && bucket != pc->entries.end()) {
      // candidate lengths <= the prompt, longest first
      const auto &L = ix->second.lengths;
      const size_t upper = std::upper_bound(L.begin(), L.end(), n_tokens) - L.begin();
      std::vector<uint32_t> probe;
      for (size_t i = upper; i-- > 0;) {
        const size_t len = L[i];
        probe.assign(tokens, tokens + len);
        auto e = bucket->second.find(probe);
        if (e == bucket->second.end()) continue;
        scanned++;
        const auto &st = e->second.payload->states;
        if (compatible && !compatible(compat_user, st.data(), st.size())) continue;
        const uint64_t access = pc->take_access();
        pc->lru.erase(LruKey{e->second.last_used, key, probe});
        e->second.last_used = access;
        pc->lru.insert(LruKey{access, key, probe});
        found = e->second.payload;
        clone_bytes = e->second.byte_len;
        best = len;
        break;
      }
    }
  }
  pc->update([&](llh_prefix_cache_counters &c) {
    c.entries_scanned = sat_add(c.entries_scanned, scanned);
    c.namespace_entries_scanned = sat_add(c.namespace_entries_scanned, scanned);
  });
  if (!found) {
    pc->update([&](llh_prefix_cache_counters &c) {
      c.misses = sat_add(c.misses, 1);
      c.miss_tokens = sat_add(c.miss_tokens, n_tokens);
    });
    return LLH_OK;
  }
  // copy the payload out (the shared reference keeps it alive without the lock)
  hit->token_count = best;
  hit->n_hidden = found->hidden.size();
  hit->n_states = found->states.size();
  hit->byte_len = clone_bytes;
  if (hidden_out) std::memcpy(hidden_out, found->hidden.data(), std::min(hidden_cap, found->hidden.size()) * 4);
  if (states_out) std::memcpy(states_out, found->states.data(), std::min(states_cap, found->states.size()) * 8);
  if (pc->retain) pc->retain(pc->user, found->states.data(), found->states.size());
  pc->update([&](llh_prefix_cache_counters &c) {
    c.hits = sat_add(c.hits, 1);
    c.reused_tokens = sat_add(c.reused_tokens, best);
    c.hit_tokens = sat_add(c.hit_tokens, best);
    c.avoided_prefill_tokens = sat_add(c.avoided_prefill_tokens, best);
    c.miss_tokens = sat_add(c.miss_tokens, n_tokens - best);
    c.hit_clone_bytes = sat_add(c.hit_clone_bytes, clone_bytes);
  });
  return LLH_OK;
}

int llh_prefix_cache_record(llh_prefix_cache *pc, int32_t kind, uint64_t tokens) {
  if (!pc) return LLH_ERR_NULL;
  switch (kind) {
    case LLH_PREFIX_RECORD_PREFILL_CHUNK:
      pc->update([&](llh_prefix_cache_counters &c) {
        c.prefill_chunks = sat_add(c.prefill_chunks, 1);
        c.prefill_tokens = sat_add(c.prefill_tokens, tokens);
      });
      return LLH_OK;
    case LLH_PREFIX_RECORD_CHECKPOINT_STORE:
      pc->update([&](llh_prefix_cache_counters &c) {
        c.checkpoint_stores = sat_add(c.checkpoint_stores, 1);
        c.checkpoint_store_tokens = sat_add(c.checkpoint_store_tokens, tokens);
      });
      return LLH_OK;
    case LLH_PREFIX_RECORD_CHECKPOINT_REUSE:
      pc->update([&](llh_prefix_cache_counters &c) {
        c.checkpoint_reuse_hits = sat_add(c.checkpoint_reuse_hits, 1);
        c.checkpoint_reused_tokens = sat_add(c.checkpoint_reused_tokens, tokens);
      });
      return LLH_OK;
    case LLH_PREFIX_RECORD_SHARED_PREFIX_REUSE:
      pc->update([&](llh_prefix_cache_counters &c) {
        c.shared_prefix_hits = sat_add(c.shared_prefix_hits, 1);
        c.shared_prefix_reused_tokens = sat_add(c.shared_prefix_reused_tokens, tokens);
      });
      return LLH_OK;
    case LLH_PREFIX_RECORD_HIT:  // a hit served outside this cache (e.g. the disk tier)
      pc->update([&](llh_prefix_cache_counters &c) {
        c.hits = sat_add(c.hits, 1);
        c.reused_tokens = sat_add(c.reused_tokens, tokens);
        c.hit_tokens = sat_add(c.hit_tokens, tokens);
        c.avoided_prefill_tokens = sat_add(c.avoided_prefill_tokens, tokens);
      });
      return LLH_OK;
    case LLH_PREFIX_RECORD_MISS_TOKENS:
      pc->update([&](llh_prefix_cache_counters &c) { c.miss_tokens = sat_add(c.miss_tokens, tokens); });
      return LLH_OK;
  }
  return LLH_ERR_INVALID_SHAPE;
}

int llh_prefix_cache_metrics(llh_prefix_cache *pc, llh_prefix_cache_counters *out) {
  if (!pc || !out) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(pc->metrics_mu);
  *out = pc->counters;
  return LLH_OK;
}

int llh_prefix_cache_shape(llh_prefix_cache *pc, const char *ns, size_t ns_len, uint64_t *namespaces,
                           uint64_t *entries_in_ns, uint64_t *indexed_in_ns, uint64_t *used_bytes) {
  if (!pc || (!ns && ns_len)) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(pc->mu);
  const std::string key(ns, ns_len);
  if (namespaces) *namespaces = pc->entries.size();
  if (entries_in_ns) {
    auto b = pc->entries.find(key);
    *entries_in_ns = b == pc->entries.end() ? 0 : b->second.size();
  }
  if (indexed_in_ns) {
    auto ix = pc->indexes.find(key);
    uint64_t n = 0;
    if (ix != pc->indexes.end())
      for (auto &kv : ix->second.counts) n += kv.second;
    *indexed_in_ns = n;
  }
  if (used_bytes) *used_bytes = pc->used_bytes;
  return LLH_OK;
}

int llh_prefix_cache_lru_entry(llh_prefix_cache *pc, size_t index, char *ns_out, size_t ns_cap, size_t *ns_len,
                               uint32_t *tokens_out, size_t tokens_cap, size_t *n_tokens) {
  if (!pc || !ns_len || !n_tokens) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(pc->mu);
  if (index >= pc->lru.size()) return LLH_ERR_INVALID_SHAPE;
  auto it = pc->lru.begin();
  std::advance(it, index);
  *ns_len = it->ns.size();
  *n_tokens = it->tokens.size();
  if (ns_out) std::memcpy(ns_out, it->ns.data(), std::min(ns_cap, it->ns.size()));
  if (tokens_out) std::memcpy(tokens_out, it->tokens.data(), std::min(tokens_cap, it->tokens.size()) * 4);
  return LLH_OK;
}

}  // extern "C"
