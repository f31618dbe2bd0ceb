// Paged KV block allocator: kir-ai's BlockPool (crates/llm-kv-cache/src/block_pool.rs)
// re-stated over the blocks of a device KV pool, plus the SHA-256 block chain
// hash (crates/llm-kv-cache/src/block.rs:8-33).
//
// The reference keeps each block's f32 payload on the host inside CacheBlock.
// Here block i of the allocator *is* block i of an llh_kv_pool in HBM: the
// allocator hands out pool indices (with their typed BlockIds) that go
// straight into the int32 block tables of llh_paged_decode / llh_paged_prefill,
// a copy-on-write clone is a device block copy, and payload rows are written
// and read through the pool's kernels.  Everything else (free list, refcounts,
// session block tables, prefix registry keyed by chain hash, LRU session
// eviction, metrics) is host bookkeeping under one mutex, as in the reference.
#include <array>
#include <cmath>
#include <cstring>
#include <map>
#include <unordered_map>
#include <unordered_set>

#include "host_state.h"
#include "sha256.h"

using namespace llh;

namespace {

using Hash = std::array<uint8_t, 32>;

// CacheBlock metadata (crates/llm-kv-cache/src/block.rs:36-53); the payload is
// the device pool block of the same index.
struct BlockMeta {
  uint64_t id = 0;
  uint64_t revision = 0;
  size_t token_count = 0;
  size_t ref_count = 0;
  bool has_hash = false;
  Hash hash{};
  uint64_t last_access = 0;

  // CacheBlock::clear (block.rs:322-336)
  void clear() {
    token_count = 0;
    ref_count = 0;
    has_hash = false;
    last_access = 0;
    revision += 1;
  }
};

// SessionBlockTable (crates/llm-kv-cache/src/block_table.rs:78-168)
struct Session {
  uint64_t id = 0;
  uint64_t created_at = 0;
  uint64_t last_access = 0;
  std::vector<uint64_t> table;
  std::unordered_set<uint64_t> owned;
};

struct PrefixBlock {
  uint64_t id;
  Hash hash;
};

// PagedKvCacheMetrics (block_pool.rs:54-97)
struct Metrics {
  uint64_t total_refcount_increments = 0;
  uint64_t total_cow_clones = 0;
  uint64_t cow_bytes_saved = 0;
  uint64_t blocks_evicted_lru = 0;
  uint64_t sessions_evicted_lru = 0;
  uint64_t eviction_high_water_mark = 0;
  uint64_t pool_high_water_blocks = 0;
  uint64_t max_refcount_seen = 0;
};

}  // namespace

struct llh_block_pool {
  llh_ctx *ctx = nullptr;       // null for a host-only pool
  llh_kv_pool *pool = nullptr;  // device payload (null for a host-only pool)
  size_t capacity_tokens = 0;
  size_t vector_len = 0;
  uint64_t payload_bytes = 0;  // bytes of one block's K and V payload
  std::vector<BlockMeta> blocks;              // index = device pool block index
  std::unordered_map<uint64_t, int64_t> index_of;  // BlockId -> index
  std::vector<int64_t> free_list;             // LIFO, like the reference's Vec
  std::map<Hash, std::vector<PrefixBlock>> prefixes;
  std::map<uint64_t, Session> sessions;
  uint64_t next_session_id = 1;
  uint64_t access_clock = 0;
  Metrics metrics;
  void *scratch = nullptr;  // device staging for host rows
  size_t scratch_bytes = 0;
  mutable std::mutex mu;
  mutable std::mutex err_mu;
  std::string last_error;

  ~llh_block_pool() {
    if (scratch) {
      if (ctx) (void)hipSetDevice(ctx->device);
      (void)hipFree(scratch);
    }
  }

  int fail(int status, const std::string &msg) {
    {
      std::lock_guard<std::mutex> g(err_mu);
      last_error = msg;
    }
    if (ctx) return ctx->fail(status, msg);
    return status;
  }

  BlockMeta *find(uint64_t id) {
    auto it = index_of.find(id);
    return it == index_of.end() ? nullptr : &blocks[(size_t)it->second];
  }
  const BlockMeta *find(uint64_t id) const {
    auto it = index_of.find(id);
    return it == index_of.end() ? nullptr : &blocks[(size_t)it->second];
  }
  int64_t index(uint64_t id) const {
    auto it = index_of.find(id);
    return it == index_of.end() ? -1 : it->second;
  }

  uint64_t next_access() { return ++access_clock; }
  size_t resident_from_free_list() const { return blocks.size() - free_list.size(); }

  void record_refcount(size_t rc) { metrics.max_refcount_seen = std::max<uint64_t>(metrics.max_refcount_seen, rc); }
  void record_shared_increment(size_t rc) {
    metrics.total_refcount_increments += 1;
    metrics.cow_bytes_saved += payload_bytes;
    record_refcount(rc);
  }

  // BlockPoolInner::allocate (block_pool.rs:669-678)
  uint64_t allocate() {
    if (free_list.empty()) return 0;
    const int64_t i = free_list.back();
    free_list.pop_back();
    const uint64_t access = next_access();
    BlockMeta &b = blocks[(size_t)i];
    b.clear();  // reset_for_allocation (block.rs:338-342)
    b.ref_count = 1;
    b.last_access = access;
    record_refcount(b.ref_count);
    metrics.pool_high_water_blocks = std::max<uint64_t>(metrics.pool_high_water_blocks, resident_from_free_list());
    return b.id;
  }

  // BlockPoolInner::release (block_pool.rs:698-710)
  bool release(uint64_t id) {
    BlockMeta *b = find(id);
    if (!b || b->ref_count == 0) return false;
    if (--b->ref_count == 0) {
      b->clear();
      free_list.push_back(index(id));
    }
    return true;
  }

  // BlockPoolInner::retain (block_pool.rs:684-696)
  bool retain(uint64_t id) {
    BlockMeta *b = find(id);
    if (!b || b->ref_count == 0) return false;
    b->ref_count += 1;
    record_shared_increment(b->ref_count);
    return true;
  }

  // append_block_to_session_inner (block_pool.rs:738-771); 0 = ok, else an LLH error
  int append_to_session(uint64_t sid, uint64_t id, bool retain_new_owner) {
    BlockMeta *b = find(id);
    if (!b || b->ref_count == 0) return LLH_ERR_INVALID_SHAPE;
    const uint64_t access = next_access();
    auto it = sessions.find(sid);
    if (it == sessions.end() || id == 0) return LLH_ERR_INVALID_SHAPE;
    Session &s = it->second;
    s.table.push_back(id);
    const bool newly_owned = s.owned.insert(id).second;
    s.last_access = access;
    if (retain_new_owner && newly_owned) {
      b->ref_count += 1;
      record_shared_increment(b->ref_count);
    }
    b->last_access = access;
    return LLH_OK;
  }

  // release_session_inner (block_pool.rs:773-793): blocks this released to the free list, or -1
  long release_session(uint64_t sid) {
    auto it = sessions.find(sid);
    if (it == sessions.end()) return -1;
    const std::vector<uint64_t> owned(it->second.owned.begin(), it->second.owned.end());
    sessions.erase(it);
    long freed = 0;
    for (uint64_t id : owned) {
      const BlockMeta *b = find(id);
      const bool was_resident = b && b->ref_count > 0;
      if (release(id) && was_resident && find(id)->ref_count == 0) freed++;
    }
    return freed;
  }

  // lru_session_except (block_pool.rs:856-872): oldest (last_access, created_at, id), non-empty
  uint64_t lru_session_except(uint64_t excluded) const {
    const Session *best = nullptr;
    for (const auto &kv : sessions) {
      const Session &s = kv.second;
      if (s.id == excluded || s.table.empty()) continue;
      if (!best || std::tie(s.last_access, s.created_at, s.id) < std::tie(best->last_access, best->created_at, best->id))
        best = &s;
    }
    return best ? best->id : 0;
  }

  // evict_sessions_until_free (block_pool.rs:841-854)
  void evict_until_free(uint64_t excluded) {
    while (free_list.empty()) {
      const uint64_t sid = lru_session_except(excluded);
      if (sid == 0) break;
      const size_t high_water = resident_from_free_list();
      const long freed = release_session(sid);
      if (freed < 0) break;
      metrics.sessions_evicted_lru += 1;
      metrics.blocks_evicted_lru += (uint64_t)freed;
      metrics.eviction_high_water_mark = std::max<uint64_t>(metrics.eviction_high_water_mark, high_water);
    }
  }

  // prefix_entry_for (block_pool.rs:813-827)
  bool prefix_entry_for(const uint64_t *ids, size_t n, std::vector<PrefixBlock> &out) const {
    out.clear();
    for (size_t i = 0; i < n; i++) {
      const BlockMeta *b = find(ids[i]);
      if (!b || b->ref_count == 0 || !b->has_hash) return false;
      out.push_back(PrefixBlock{ids[i], b->hash});
    }
    return true;
  }

  // prefix_blocks_match (block_pool.rs:829-839)
  bool prefix_matches(const Hash &h, const std::vector<PrefixBlock> &entry) const {
    if (entry.empty() || entry.back().hash != h) return false;
    for (const PrefixBlock &pb : entry) {
      const BlockMeta *b = find(pb.id);
      if (!b || b->ref_count == 0 || !b->has_hash || b->hash != pb.hash) return false;
    }
    return true;
  }

  const std::vector<PrefixBlock> *lookup(const Hash &h) const {
    auto it = prefixes.find(h);
    if (it == prefixes.end() || !prefix_matches(h, it->second)) return nullptr;
    return &it->second;
  }

  hipError_t ensure_scratch(size_t n) {
    if (n <= scratch_bytes) return hipSuccess;
    if (scratch) (void)hipFree(scratch);
    scratch = nullptr;
    scratch_bytes = 0;
    hipError_t e = hipMalloc(&scratch, align_up(n));
    if (e == hipSuccess) scratch_bytes = align_up(n);
    return e;
  }

  // Device copy of block src's payload (K, V and their scales) into block dst,
  // complete on return: null-stream copies are asynchronous to the host and
  // unordered with non-blocking streams, so the device is drained (which also
  // orders the copy after any earlier writes of src).
  hipError_t copy_payload(int64_t src, int64_t dst) {
    const PoolView &v = pool->view;
    const size_t kb = (size_t)v.kv_heads * v.block_tokens * v.head_dim * elem_bytes(v.format);
    const size_t sb = scale_bytes_per_block(v.format, v.kv_heads, v.block_tokens);
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess)
      e = hipMemcpy((char *)pool->k + kb * dst, (char *)pool->k + kb * src, kb, hipMemcpyDeviceToDevice);
    if (e == hipSuccess)
      e = hipMemcpy((char *)pool->v + kb * dst, (char *)pool->v + kb * src, kb, hipMemcpyDeviceToDevice);
    const size_t ksb = scales_interleaved(v.format) ? 2 * sb : sb;  // int8, fp8: K and V scale pairs in one run
    if (e == hipSuccess && sb)
      e = hipMemcpy((char *)pool->ks + ksb * dst, (char *)pool->ks + ksb * src, ksb, hipMemcpyDeviceToDevice);
    if (e == hipSuccess && sb && !scales_interleaved(v.format))
      e = hipMemcpy((char *)pool->vs + sb * dst, (char *)pool->vs + sb * src, sb, hipMemcpyDeviceToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return e;
  }
};

namespace {

Hash to_hash(const uint8_t *p) {
  Hash h;
  std::memcpy(h.data(), p, 32);
  return h;
}

int copy_ids(const std::vector<uint64_t> &ids, uint64_t *h_out, size_t capacity, size_t *count) {
  *count = ids.size();
  if (h_out) std::memcpy(h_out, ids.data(), std::min(capacity, ids.size()) * sizeof(uint64_t));
  return (!h_out || capacity >= ids.size()) ? LLH_OK : LLH_ERR_CAPACITY;
}

llh_block_pool *new_pool(size_t block_count, size_t capacity, size_t vector_len) {
  auto *bp = new llh_block_pool();
  bp->capacity_tokens = capacity;
  bp->vector_len = vector_len;
  bp->blocks.resize(block_count);
  bp->free_list.reserve(block_count);
  for (size_t i = 0; i < block_count; i++) {
    bp->blocks[i].id = next_block_id();
    bp->index_of[bp->blocks[i].id] = (int64_t)i;
    bp->free_list.push_back((int64_t)i);
  }
  return bp;
}

}  // namespace

extern "C" {

int llh_sha256(const void *data, size_t len, uint8_t out[32]) {
  if ((!data && len) || !out) return LLH_ERR_NULL;
  Sha256 h;
  h.update(data, len);
  h.finish(out);
  return LLH_OK;
}

int llh_cache_block_chain_hash(const char *model_id, size_t model_len, const char *cache_context,
                               size_t context_len, const uint8_t previous_hash[32], const uint32_t *token_ids,
                               size_t n, uint8_t out[32]) {
  if ((!model_id && model_len) || (!cache_context && context_len) || !previous_hash || (!token_ids && n) || !out)
    return LLH_ERR_NULL;
  static const char kDomain[] = "kir-ai-kv-block-chain/v1";
  Sha256 h;
  h.update(kDomain, sizeof(kDomain) - 1);
  h.update_u64_le(model_len);
  h.update(model_id, model_len);
  h.update_u64_le(context_len);
  h.update(cache_context, context_len);
  h.update(previous_hash, 32);
  h.update_u64_le(n);
  for (size_t i = 0; i < n; i++) h.update_u32_le(token_ids[i]);
  h.finish(out);
  return LLH_OK;
}

int llh_block_pool_create_host(size_t block_count, size_t block_capacity_tokens, size_t vector_len,
                               llh_block_pool **out) {
  if (!out) return LLH_ERR_NULL;
  *out = nullptr;
  // BlockPoolInner::new and CacheBlock::new (block_pool.rs:345-360, block.rs:96-101)
  if (block_count == 0 || block_capacity_tokens == 0 || vector_len == 0 ||
      block_capacity_tokens > SIZE_MAX / vector_len)
    return LLH_ERR_INVALID_SHAPE;
  llh_block_pool *bp = new_pool(block_count, block_capacity_tokens, vector_len);
  bp->payload_bytes = 2ull * block_capacity_tokens * vector_len * sizeof(float);  // the reference's f32 K and V
  *out = bp;
  return LLH_OK;
}

int llh_block_pool_create(llh_ctx *ctx, llh_kv_pool *pool, llh_block_pool **out) {
  if (!ctx || !pool || !out) return LLH_ERR_NULL;
  *out = nullptr;
  const PoolView &v = pool->view;
  if (v.n_blocks <= 0) return ctx->fail(LLH_ERR_INVALID_SHAPE, "block pool over an empty KV pool");
  llh_block_pool *bp = new_pool((size_t)v.n_blocks, (size_t)v.block_tokens, (size_t)v.kv_heads * v.head_dim);
  bp->ctx = ctx;
  bp->pool = pool;
  bp->payload_bytes = 2ull * ((size_t)v.kv_heads * v.block_tokens * v.head_dim * elem_bytes(v.format) +
                              scale_bytes_per_block(v.format, v.kv_heads, v.block_tokens));
  *out = bp;
  return LLH_OK;
}

int llh_block_pool_destroy(llh_block_pool *bp) {
  if (!bp) return LLH_ERR_NULL;
  delete bp;
  return LLH_OK;
}

const char *llh_block_pool_last_error(const llh_block_pool *bp) {
  if (!bp) return "null block pool";
  std::lock_guard<std::mutex> g(bp->err_mu);
  return bp->last_error.c_str();
}

int llh_block_pool_get_counts(const llh_block_pool *bp, llh_block_pool_counts *out) {
  if (!bp || !out) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  out->total_blocks = bp->blocks.size();
  out->free_blocks = bp->free_list.size();
  uint64_t allocated = 0;
  for (const BlockMeta &b : bp->blocks) allocated += b.ref_count > 0;
  out->allocated_blocks = allocated;
  out->sessions = bp->sessions.size();
  return LLH_OK;
}

// BlockPoolInner::metrics_snapshot (block_pool.rs:381-431)
int llh_block_pool_metrics(const llh_block_pool *bp, llh_paged_kv_metrics *out) {
  if (!bp || !out) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  uint64_t resident = 0, shared = 0, total_rc = 0, max_rc = 0;
  for (const BlockMeta &b : bp->blocks) {
    if (b.ref_count == 0) continue;
    resident++;
    total_rc += b.ref_count;
    max_rc = std::max<uint64_t>(max_rc, b.ref_count);
    if (b.ref_count > 1) shared++;
  }
  uint64_t active = 0;
  for (const auto &kv : bp->sessions) active += kv.second.table.size();
  const uint64_t total = bp->blocks.size();
  out->total_blocks = total;
  out->resident_blocks = resident;
  out->active_blocks = active;
  out->blocks_in_use = resident;
  out->free_blocks = bp->free_list.size();
  out->free_list_blocks = bp->free_list.size();
  out->pool_utilization_pct = total == 0 ? 0.0 : (double)resident / (double)total * 100.0;
  out->sessions = bp->sessions.size();
  out->session_block_tables = bp->sessions.size();
  out->shared_blocks = shared;
  out->refcount_total = total_rc;
  out->avg_refcount = resident == 0 ? 0.0 : (double)total_rc / (double)resident;
  out->max_refcount = max_rc;
  out->max_refcount_seen = std::max(bp->metrics.max_refcount_seen, max_rc);
  out->total_refcount_increments = bp->metrics.total_refcount_increments;
  out->total_cow_clones = bp->metrics.total_cow_clones;
  out->cow_bytes_saved = bp->metrics.cow_bytes_saved;
  out->blocks_evicted_lru = bp->metrics.blocks_evicted_lru;
  out->sessions_evicted_lru = bp->metrics.sessions_evicted_lru;
  out->eviction_high_water_mark = bp->metrics.eviction_high_water_mark;
  out->pool_high_water_blocks = bp->metrics.pool_high_water_blocks;
  return LLH_OK;
}

int llh_block_pool_block_info(const llh_block_pool *bp, uint64_t block_id, llh_cache_block_info *out) {
  if (!bp || !out) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  const BlockMeta *b = bp->find(block_id);
  if (!b) return LLH_ERR_STALE;
  out->block_id = b->id;
  out->pool_index = bp->index(block_id);
  out->revision = b->revision;
  out->capacity_tokens = bp->capacity_tokens;
  out->vector_len = bp->vector_len;
  out->token_count = b->token_count;
  out->ref_count = b->ref_count;
  out->last_access = b->last_access;
  out->payload_bytes = bp->payload_bytes;
  out->has_content_hash = b->has_hash ? 1 : 0;
  std::memcpy(out->content_hash, b->hash.data(), 32);
  return LLH_OK;
}

int llh_block_pool_allocate(llh_block_pool *bp, uint64_t *block_id) {
  if (!bp || !block_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *block_id = bp->allocate();
  return LLH_OK;
}

int llh_block_pool_release(llh_block_pool *bp, uint64_t block_id, int32_t *released) {
  if (!bp || !released) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *released = bp->release(block_id) ? 1 : 0;
  return LLH_OK;
}

int llh_block_pool_retain(llh_block_pool *bp, uint64_t block_id, int32_t *retained) {
  if (!bp || !retained) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *retained = bp->retain(block_id) ? 1 : 0;
  return LLH_OK;
}

// BlockPoolInner::touch (block_pool.rs:712-720): the access clock advances even on a miss
int llh_block_pool_touch(llh_block_pool *bp, uint64_t block_id, int32_t *touched) {
  if (!bp || !touched) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  const uint64_t access = bp->next_access();
  BlockMeta *b = bp->find(block_id);
  *touched = 0;
  if (b && b->ref_count > 0) {
    b->last_access = access;
    *touched = 1;
  }
  return LLH_OK;
}

// BlockPoolInner::lru_block (block_pool.rs:722-728)
int llh_block_pool_lru_block(const llh_block_pool *bp, uint64_t *block_id) {
  if (!bp || !block_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  const BlockMeta *best = nullptr;
  for (const BlockMeta &b : bp->blocks)
    if (b.ref_count > 0 && (!best || b.last_access < best->last_access)) best = &b;
  *block_id = best ? best->id : 0;
  return LLH_OK;
}

// CacheBlock::set_content_hash through block_mut (block_pool.rs:730-737): exclusive blocks only
int llh_block_pool_set_content_hash(llh_block_pool *bp, uint64_t block_id, const uint8_t *hash) {
  if (!bp) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  BlockMeta *b = bp->find(block_id);
  if (!b || b->ref_count != 1)
    return bp->fail(LLH_ERR_INVALID_SHAPE, "block is not exclusively owned (copy it on write first)");
  b->has_hash = hash != nullptr;
  if (hash) b->hash = to_hash(hash);
  return LLH_OK;
}

int llh_block_pool_create_session(llh_block_pool *bp, uint64_t *session_id) {
  if (!bp || !session_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *session_id = 0;
  const uint64_t sid = bp->next_session_id;
  if (sid == UINT64_MAX) return bp->fail(LLH_ERR_INVALID_SHAPE, "session ids exhausted");
  bp->next_session_id += 1;
  const uint64_t access = bp->next_access();
  Session s;
  s.id = sid;
  s.created_at = access;
  s.last_access = access;
  bp->sessions.emplace(sid, std::move(s));
  *session_id = sid;
  return LLH_OK;
}

int llh_block_pool_release_session(llh_block_pool *bp, uint64_t session_id, int32_t *released) {
  if (!bp || !released) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *released = bp->release_session(session_id) >= 0 ? 1 : 0;
  return LLH_OK;
}

// BlockPoolInner::allocate_for_session (block_pool.rs:445-457)
int llh_block_pool_allocate_for_session(llh_block_pool *bp, uint64_t session_id, uint64_t *block_id) {
  if (!bp || !block_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *block_id = 0;
  if (!bp->sessions.count(session_id)) return LLH_OK;
  if (bp->free_list.empty()) bp->evict_until_free(session_id);
  const uint64_t id = bp->allocate();
  if (id == 0) return LLH_OK;
  if (bp->append_to_session(session_id, id, false) == LLH_OK) *block_id = id;
  return LLH_OK;
}

int llh_block_pool_append_block_to_session(llh_block_pool *bp, uint64_t session_id, uint64_t block_id) {
  if (!bp) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  const int st = bp->append_to_session(session_id, block_id, true);
  if (st != LLH_OK) return bp->fail(st, "block or session not live");
  return LLH_OK;
}

// BlockPoolInner::read_session_block (block_pool.rs:467-481)
int llh_block_pool_read_session_block(llh_block_pool *bp, uint64_t session_id, size_t index, uint64_t *block_id) {
  if (!bp || !block_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *block_id = 0;
  const uint64_t access = bp->next_access();
  auto it = bp->sessions.find(session_id);
  if (it == bp->sessions.end() || index >= it->second.table.size()) return LLH_OK;
  const uint64_t id = it->second.table[index];
  it->second.last_access = access;
  BlockMeta *b = bp->find(id);
  if (!b || b->ref_count == 0) return LLH_OK;
  b->last_access = access;
  *block_id = id;
  return LLH_OK;
}

int llh_block_pool_session_info(const llh_block_pool *bp, uint64_t session_id, llh_session_info *out) {
  if (!bp || !out) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  auto it = bp->sessions.find(session_id);
  if (it == bp->sessions.end()) return LLH_ERR_STALE;
  const Session &s = it->second;
  out->session_id = s.id;
  out->created_at = s.created_at;
  out->last_access = s.last_access;
  out->block_count = s.table.size();
  out->owned_block_count = s.owned.size();
  return LLH_OK;
}

// The session's block table as BlockIds and as device pool indices: the row a
// llh_decode_desc / llh_prefill_desc takes (after an upload to the device).
int llh_block_pool_session_blocks(const llh_block_pool *bp, uint64_t session_id, uint64_t *h_ids,
                                  int32_t *h_pool_indices, size_t capacity, size_t *count) {
  if (!bp || !count) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  auto it = bp->sessions.find(session_id);
  if (it == bp->sessions.end()) return LLH_ERR_STALE;
  const std::vector<uint64_t> &t = it->second.table;
  *count = t.size();
  const size_t n = std::min(capacity, t.size());
  for (size_t i = 0; i < n; i++) {
    if (h_ids) h_ids[i] = t[i];
    if (h_pool_indices) h_pool_indices[i] = (int32_t)bp->index(t[i]);
  }
  return (capacity >= t.size() || (!h_ids && !h_pool_indices)) ? LLH_OK : LLH_ERR_CAPACITY;
}

int llh_block_pool_lru_session(const llh_block_pool *bp, uint64_t *session_id) {
  if (!bp || !session_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *session_id = bp->lru_session_except(0);
  return LLH_OK;
}

// BlockPoolInner::register_prefix (block_pool.rs:483-492)
int llh_block_pool_register_prefix(llh_block_pool *bp, const uint8_t prefix_hash[32], const uint64_t *block_ids,
                                   size_t n) {
  if (!bp || !prefix_hash || (!block_ids && n)) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  const Hash h = to_hash(prefix_hash);
  std::vector<PrefixBlock> entry;
  if (bp->prefix_entry_for(block_ids, n, entry) && !entry.empty() && entry.back().hash == h)
    bp->prefixes[h] = std::move(entry);
  else
    bp->prefixes.erase(h);
  return LLH_OK;
}

int llh_block_pool_lookup_prefix(const llh_block_pool *bp, const uint8_t prefix_hash[32], uint64_t *h_ids,
                                 size_t capacity, size_t *count, int32_t *found) {
  if (!bp || !prefix_hash || !count || !found) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  const std::vector<PrefixBlock> *e = bp->lookup(to_hash(prefix_hash));
  *found = e ? 1 : 0;
  std::vector<uint64_t> ids;
  if (e)
    for (const PrefixBlock &pb : *e) ids.push_back(pb.id);
  return copy_ids(ids, h_ids, capacity, count);
}

// BlockPoolInner::attach_prefix_to_session (block_pool.rs:503-519)
int llh_block_pool_attach_prefix_to_session(llh_block_pool *bp, uint64_t session_id, const uint8_t prefix_hash[32],
                                            uint64_t *h_ids, size_t capacity, size_t *count, int32_t *found) {
  if (!bp || !prefix_hash || !count || !found) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *found = 0;
  *count = 0;
  if (!bp->sessions.count(session_id)) return LLH_OK;
  const std::vector<PrefixBlock> *e = bp->lookup(to_hash(prefix_hash));
  if (!e) return LLH_OK;
  std::vector<uint64_t> ids;
  for (const PrefixBlock &pb : *e) ids.push_back(pb.id);
  for (uint64_t id : ids)
    if (bp->append_to_session(session_id, id, true) != LLH_OK) return LLH_OK;
  *found = 1;
  return copy_ids(ids, h_ids, capacity, count);
}

// BlockPoolInner::copy_on_write_session_block (block_pool.rs:521-603).  A
// shared block is cloned into a fresh block (device payload copy) that
// replaces it in this session's table only.
int llh_block_pool_copy_on_write_session_block(llh_block_pool *bp, uint64_t session_id, size_t index,
                                               uint64_t *block_id) {
  if (!bp || !block_id) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  *block_id = 0;
  auto sit = bp->sessions.find(session_id);
  if (sit == bp->sessions.end() || index >= sit->second.table.size())
    return bp->fail(LLH_ERR_INVALID_SHAPE, "no such session block");
  const uint64_t id = sit->second.table[index];
  auto touch_session_block = [&](uint64_t bid) -> int {
    const uint64_t access = bp->next_access();
    bp->sessions[session_id].last_access = access;
    BlockMeta *b = bp->find(bid);
    if (!b || b->ref_count == 0) return bp->fail(LLH_ERR_INVALID_SHAPE, "block is not live");
    b->last_access = access;
    *block_id = bid;
    return LLH_OK;
  };
  BlockMeta *src = bp->find(id);
  if (!src || src->ref_count == 0) return bp->fail(LLH_ERR_INVALID_SHAPE, "block is not live");
  if (src->ref_count == 1) return touch_session_block(id);
  if (bp->free_list.empty()) bp->evict_until_free(session_id);
  src = bp->find(id);
  if (!src || src->ref_count == 0) return bp->fail(LLH_ERR_INVALID_SHAPE, "block is not live");
  if (src->ref_count == 1) return touch_session_block(id);
  const uint64_t fresh = bp->allocate();
  if (fresh == 0) return bp->fail(LLH_ERR_CAPACITY, "KV block pool exhausted: no block for copy-on-write");
  const uint64_t access = bp->next_access();
  if (bp->pool) {
    const hipError_t e = bp->copy_payload(bp->index(id), bp->index(fresh));
    if (e != hipSuccess) {
      bp->release(fresh);
      return bp->fail(LLH_ERR_DEVICE, std::string("copy-on-write block copy: ") + hipGetErrorString(e));
    }
  }
  // CacheBlock::copy_contents_from (block.rs:344-363)
  BlockMeta *dst = bp->find(fresh);
  src = bp->find(id);
  dst->token_count = src->token_count;
  dst->ref_count = 1;
  dst->has_hash = src->has_hash;
  dst->hash = src->hash;
  dst->last_access = access;
  dst->revision += 1;
  // SessionBlockTable::replace_owned_block (block_table.rs:150-163)
  Session &s = bp->sessions[session_id];
  s.table[index] = fresh;
  s.owned.insert(fresh);
  const bool release_previous = std::find(s.table.begin(), s.table.end(), id) == s.table.end();
  if (release_previous) s.owned.erase(id);
  s.last_access = access;
  if (release_previous) bp->release(id);
  bp->metrics.total_cow_clones += 1;
  *block_id = fresh;
  return LLH_OK;
}

// ---- payload (device pools) ----

// CacheBlock::append (block.rs:250-272) through block_mut: the row goes to the
// block's next token slot in the device pool (quantised on write for int8).
int llh_block_pool_append_f32(llh_block_pool *bp, uint64_t block_id, const float *h_key, const float *h_value,
                              size_t len) {
  if (!bp || !h_key || !h_value) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  if (!bp->pool) return bp->fail(LLH_ERR_UNSUPPORTED, "host-only block pool has no payload");
  if (bp->pool->view.format == LLH_KV_FP8_E4M3)
    return bp->fail(LLH_ERR_UNSUPPORTED, "fp8 blocks are written whole (per-block scale): use llh_kv_write_blocks");
  BlockMeta *b = bp->find(block_id);
  if (!b || b->ref_count != 1)
    return bp->fail(LLH_ERR_INVALID_SHAPE, "block is not exclusively owned (copy it on write first)");
  if (len != bp->vector_len) return bp->fail(LLH_ERR_INVALID_SHAPE, "KV row length does not match the block");
  if (b->token_count == bp->capacity_tokens) return bp->fail(LLH_ERR_CAPACITY, "KV block is full");
  if (bp->pool->view.format == LLH_KV_INT8 || bp->pool->view.format == LLH_KV_INT8_ROW)
    for (size_t i = 0; i < len; i++)
      if (!std::isfinite(h_key[i]) || !std::isfinite(h_value[i]))
        return bp->fail(LLH_ERR_NON_FINITE, "int8 KV rows must be finite");
  llh_ctx *ctx = bp->ctx;
  hipError_t e = hipSetDevice(ctx->device);
  const size_t row_bytes = len * sizeof(float);
  if (e == hipSuccess) e = bp->ensure_scratch(kAlign + 2 * align_up(row_bytes));
  if (e != hipSuccess) return bp->fail(LLH_ERR_DEVICE, std::string("staging buffer: ") + hipGetErrorString(e));
  char *sb = static_cast<char *>(bp->scratch);
  int64_t *d_slot = reinterpret_cast<int64_t *>(sb);
  float *d_k = reinterpret_cast<float *>(sb + kAlign);
  float *d_v = reinterpret_cast<float *>(sb + kAlign + align_up(row_bytes));
  const int64_t slot = bp->index(block_id) * (int64_t)bp->capacity_tokens + (int64_t)b->token_count;
  e = hipMemcpy(d_slot, &slot, sizeof(slot), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d_k, h_key, row_bytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d_v, h_value, row_bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) return bp->fail(LLH_ERR_DEVICE, std::string("row upload: ") + hipGetErrorString(e));
  AppendArgs a{};
  a.pool = bp->pool->view;
  a.k_dst = bp->pool->k;
  a.v_dst = bp->pool->v;
  a.ks_dst = bp->pool->ks;
  a.vs_dst = bp->pool->vs;
  a.slots = d_slot;
  a.k = d_k;
  a.v = d_v;
  a.n = 1;
  a.src_f32 = 1;
  a.err = ctx->d_err;
  e = launch_append(a, nullptr);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return bp->fail(LLH_ERR_DEVICE, std::string("append: ") + hipGetErrorString(e));
  ctx->append_calls++;
  b->token_count += 1;
  b->has_hash = false;
  b->revision += 1;
  return LLH_OK;
}

// Bookkeeping for rows a caller wrote itself with llh_kv_append at slots
// pool_index * block_tokens + token_count + i (the batched path).
int llh_block_pool_commit_tokens(llh_block_pool *bp, uint64_t block_id, size_t n) {
  if (!bp) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  BlockMeta *b = bp->find(block_id);
  if (!b || b->ref_count != 1)
    return bp->fail(LLH_ERR_INVALID_SHAPE, "block is not exclusively owned (copy it on write first)");
  if (n > bp->capacity_tokens - b->token_count) return bp->fail(LLH_ERR_CAPACITY, "KV block is full");
  if (n == 0) return LLH_OK;
  b->token_count += n;
  b->has_hash = false;
  b->revision += 1;
  return LLH_OK;
}

// CacheBlock::keys() / values() (block.rs:300-306): the block's token rows as
// f32 ([token_count][vector_len], dequantised for int8 / fp8).
int llh_block_pool_read_rows_f32(llh_block_pool *bp, uint64_t block_id, int32_t tensor, float *h_out,
                                 size_t capacity, size_t *count) {
  if (!bp || !count) return LLH_ERR_NULL;
  std::lock_guard<std::mutex> g(bp->mu);
  if (!bp->pool) return bp->fail(LLH_ERR_UNSUPPORTED, "host-only block pool has no payload");
  if (tensor != 0 && tensor != 1) return bp->fail(LLH_ERR_INVALID_SHAPE, "tensor must be 0 (K) or 1 (V)");
  const BlockMeta *b = bp->find(block_id);
  if (!b || b->ref_count == 0) return bp->fail(LLH_ERR_STALE, "block is not live");
  const size_t n = b->token_count * bp->vector_len;
  *count = n;
  if (!h_out || n == 0) return LLH_OK;
  if (capacity < n) return LLH_ERR_CAPACITY;
  llh_ctx *ctx = bp->ctx;
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = bp->ensure_scratch(kAlign + n * sizeof(float));
  if (e != hipSuccess) return bp->fail(LLH_ERR_DEVICE, std::string("staging buffer: ") + hipGetErrorString(e));
  char *sb = static_cast<char *>(bp->scratch);
  const int32_t idx = (int32_t)bp->index(block_id);
  e = hipMemcpy(sb, &idx, sizeof(idx), hipMemcpyHostToDevice);
  if (e != hipSuccess) return bp->fail(LLH_ERR_DEVICE, std::string("table upload: ") + hipGetErrorString(e));
  GatherArgs a{};
  a.pool = bp->pool->view;
  a.table = reinterpret_cast<const int32_t *>(sb);
  a.max_blocks = 1;
  a.lo = 0;
  a.hi = (int32_t)b->token_count;
  a.tensor = tensor;
  a.ring_tokens = 0;
  a.out_f32 = 1;
  a.out = sb + kAlign;
  a.err = ctx->d_err;
  e = launch_gather(a, nullptr);
  if (e == hipSuccess) e = hipMemcpy(h_out, sb + kAlign, n * sizeof(float), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return bp->fail(LLH_ERR_DEVICE, std::string("gather: ") + hipGetErrorString(e));
  return LLH_OK;
}

}  // extern "C"
