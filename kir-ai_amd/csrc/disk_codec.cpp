// On-disk prefix KV blocks: the hashes that name them and the safetensors
// container that holds them, as kir-ai's disk tier defines both
// (crates/llm-native-runtime/src/native_text/disk_cache/hashing.rs:1-202,
// io.rs:1-479, codec.rs:1-250, disk_cache.rs:160-240).
//
// A block file is a safetensors archive: an 8-byte little-endian header
// length, a JSON header whose first key "__metadata__" holds {"kir_ai": the
// block metadata as a JSON string}, then one F32 tensor per entry in name
// order ("hidden", "layers.<i>.full.keys", ...), raw little-endian f32.  The
// metadata names the codec, layout version, model / snapshot / namespace
// hashes, the block's chain hash and position, and one layout record per
// layer (kind tag first, then the fields in the reference's declaration
// order).  JSON is written compactly with keys in insertion order (serde_json
// with preserve_order), so a block encoded here has the bytes the reference
// writes for the same content.
//
// The device side of persistence is llh_kv_export_rows_f32 (pool rows through
// a block table, dequantised to f32, the only disk format) and llh_kv_append
// (f32 rows back into a pool, quantised on write).
#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "llm_hip.h"
#include "sha256.h"

namespace {

const char kCodec[] = "kir-ai-native-text-prefix-block";
constexpr uint32_t kLayoutVersion = 2;
constexpr uint64_t kMaxHeaderLen = 64ull * 1024 * 1024;
const char kRootHash[] = "0000000000000000000000000000000000000000000000000000000000000000";

thread_local std::string g_disk_error;

int integrity(const std::string &msg) {
  g_disk_error = msg;
  return LLH_ERR_INTEGRITY;
}

std::string hex(const uint8_t d[32]) {
  static const char *k = "0123456789abcdef";
  std::string s(64, '0');
  for (int i = 0; i < 32; i++) {
    s[2 * i] = k[d[i] >> 4];
    s[2 * i + 1] = k[d[i] & 15];
  }
  return s;
}

// update_hash_value (hashing.rs:192-201): 1, u64le(len), bytes -- or a single 0 for None
void update_value(llh::Sha256 &h, const char *v) {
  if (!v) {
    const uint8_t z = 0;
    h.update(&z, 1);
    return;
  }
  const uint8_t one = 1;
  h.update(&one, 1);
  const size_t n = std::strlen(v);
  h.update_u64_le(n);
  h.update(v, n);
}

std::string block_hash(const char *model, const char *ns, const char *prev, uint64_t start, const uint64_t *tokens,
                       size_t n) {
  llh::Sha256 h;
  update_value(h, "kir-ai-native-text-disk-block/v2");
  update_value(h, model);
  update_value(h, ns);
  update_value(h, prev);
  h.update_u64_le(start);
  h.update_u64_le(n);
  for (size_t i = 0; i < n; i++) h.update_u64_le(tokens[i]);
  uint8_t d[32];
  h.finish(d);
  return hex(d);
}

void copy_str(char *dst, size_t cap, const std::string &s) {
  const size_t n = std::min(cap - 1, s.size());
  std::memcpy(dst, s.data(), n);
  dst[n] = 0;
}

// ---- JSON (compact writer; a reader for the subset safetensors headers use) ----

void json_string(std::string &o, const std::string &s) {
  static const char *k = "0123456789abcdef";
  o.push_back('"');
  for (unsigned char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\r': o += "\\r"; break;
      case '\t': o += "\\t"; break;
      case '\b': o += "\\b"; break;
      case '\f': o += "\\f"; break;
      default:
        if (c < 0x20) {
          o += "\\u00";
          o.push_back(k[c >> 4]);
          o.push_back(k[c & 15]);
        } else {
          o.push_back((char)c);
        }
    }
  }
  o.push_back('"');
}

struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  bool integral = false;
  uint64_t u = 0;  // non-negative integers only (all this format uses)
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;  // insertion order
  // a repeated key keeps its last value, as serde_json's map does
  const JVal *get(const std::string &k) const {
    const JVal *v = nullptr;
    for (auto &kv : obj)
      if (kv.first == k) v = &kv.second;
    return v;
  }
};

struct JParser {
  const char *p, *e;
  std::string err;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  bool str(std::string &out) {
    if (p >= e || *p != '"') return fail("expected string");
    p++;
    while (p < e && *p != '"') {
      char c = *p++;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (p >= e) return fail("bad escape");
      c = *p++;
      switch (c) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          if (e - p < 4) return fail("bad \\u escape");
          unsigned cp = 0;
          for (int i = 0; i < 4; i++) {
            const char h = *p++;
            cp = cp * 16 + (h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                            : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 99);
            if (cp >= 0x10000 * 16) return fail("bad \\u escape");
          }
          if (cp >= 0xD800 && cp <= 0xDBFF) {  // surrogate pair
            if (e - p < 6 || p[0] != '\\' || p[1] != 'u') return fail("bad surrogate");
            p += 2;
            unsigned lo = 0;
            for (int i = 0; i < 4; i++) {
              const char h = *p++;
              lo = lo * 16 + (h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
                              : h >= 'A' && h <= 'F' ? h - 'A' + 10 : 0);
            }
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          // UTF-8 encode
          if (cp < 0x80) {
            out.push_back((char)cp);
          } else if (cp < 0x800) {
            out.push_back((char)(0xC0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          } else if (cp < 0x10000) {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          } else {
            out.push_back((char)(0xF0 | (cp >> 18)));
            out.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          }
          break;
        }
        default:
          return fail("bad escape");
      }
    }
    if (p >= e) return fail("unterminated string");
    p++;
    return true;
  }
  bool value(JVal &v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end");
    if (*p == '{') {
      p++;
      v.kind = JVal::Obj;
      ws();
      if (p < e && *p == '}') {
        p++;
        return true;
      }
      while (true) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= e || *p != ':') return fail("expected ':'");
        p++;
        JVal x;
        if (!value(x, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(x));
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == '}') {
          p++;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      p++;
      v.kind = JVal::Arr;
      ws();
      if (p < e && *p == ']') {
        p++;
        return true;
      }
      while (true) {
        JVal x;
        if (!value(x, depth + 1)) return false;
        v.arr.push_back(std::move(x));
        ws();
        if (p < e && *p == ',') {
          p++;
          continue;
        }
        if (p < e && *p == ']') {
          p++;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (*p == '"') {
      v.kind = JVal::Str;
      return str(v.s);
    }
    if (e - p >= 4 && std::strncmp(p, "null", 4) == 0) {
      p += 4;
      v.kind = JVal::Null;
      return true;
    }
    if (e - p >= 4 && std::strncmp(p, "true", 4) == 0) {
      p += 4;
      v.kind = JVal::Bool;
      v.b = true;
      return true;
    }
    if (e - p >= 5 && std::strncmp(p, "false", 5) == 0) {
      p += 5;
      v.kind = JVal::Bool;
      return true;
    }
    if (*p == '-' || (*p >= '0' && *p <= '9')) {
      v.kind = JVal::Num;
      const char *s = p;
      if (*p == '-') p++;
      bool digits_only = *s != '-';
      uint64_t u = 0;
      bool overflow = false;
      while (p < e && *p >= '0' && *p <= '9') {
        const uint64_t d = (uint64_t)(*p - '0');
        if (u > (UINT64_MAX - d) / 10) overflow = true;
        u = u * 10 + d;
        p++;
      }
      while (p < e && (*p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-' || (*p >= '0' && *p <= '9'))) {
        digits_only = false;
        p++;
      }
      v.integral = digits_only && !overflow;
      v.u = u;
      return true;
    }
    return fail("unexpected character");
  }
};

bool as_u64(const JVal *v, uint64_t &out) {
  if (!v || v->kind != JVal::Num || !v->integral) return false;
  out = v->u;
  return true;
}
bool as_str(const JVal *v, std::string &out) {
  if (!v || v->kind != JVal::Str) return false;
  out = v->s;
  return true;
}
bool as_u64_array(const JVal *v, std::vector<uint64_t> &out) {
  if (!v || v->kind != JVal::Arr) return false;
  out.clear();
  for (auto &x : v->arr) {
    uint64_t u;
    if (!as_u64(&x, u)) return false;
    out.push_back(u);
  }
  return true;
}

const char *layer_kind_name(int32_t kind) {
  return kind == LLH_DISK_LAYER_QWEN_FULL ? "qwen_full_attention" : kind == LLH_DISK_LAYER_GEMMA ? "gemma_attention"
                                                                                               : nullptr;
}
const char *layer_tensor_stem(int32_t kind) { return kind == LLH_DISK_LAYER_QWEN_FULL ? "full" : "attention"; }

struct LayerMeta {
  int32_t kind = -1;
  uint64_t revision = 0, max_tokens = 0, kv_heads = 0, head_dim = 0, token_count = 0, tokens_seen = 0;
  std::string cache_format, key_tensor, value_tensor;
  std::vector<uint64_t> shape;
};

struct Metadata {
  std::string codec, model_family, model_hash, snapshot_hash, namespace_hash, previous_block_hash, block_hash;
  uint64_t layout_version = 0, cache_layout_version = 0, block_start = 0, token_count = 0;
  std::vector<uint64_t> hidden_shape;
  std::vector<LayerMeta> layers;
};

// validate_metadata_codec_and_layout (io.rs:263-277)
int check_codec_and_layout(const Metadata &M) {
  if (M.codec != kCodec) return integrity("unsupported disk cache codec");
  if (M.layout_version != kLayoutVersion) return integrity("unsupported disk cache layout version");
  return LLH_OK;
}

struct Tensor {
  std::vector<uint64_t> shape;
  const uint8_t *data = nullptr;
  size_t n = 0;  // f32 values
};

std::string metadata_json(const llh_disk_block_descriptor &d, size_t n_hidden, const llh_disk_layer *layers,
                          size_t n_layers) {
  std::string o = "{";
  auto key = [&](const char *k) {
    if (o.size() > 1) o.push_back(',');
    json_string(o, k);
    o.push_back(':');
  };
  auto num = [&](const char *k, uint64_t v) {
    key(k);
    o += std::to_string(v);
  };
  auto str = [&](const char *k, const std::string &v) {
    key(k);
    json_string(o, v);
  };
  // NativeTextDiskCacheBlockMetadata, fields in declaration order (io.rs:11-26)
  str("codec", kCodec);
  num("layout_version", kLayoutVersion);
  num("cache_layout_version", d.cache_layout_version);
  str("model_family", d.model_family);
  str("model_hash", d.model_hash);
  str("snapshot_hash", d.snapshot_hash);
  str("namespace_hash", d.namespace_hash);
  str("previous_block_hash", d.previous_block_hash);
  str("block_hash", d.block_hash);
  num("block_start", d.block_start);
  num("token_count", d.token_count);
  key("hidden_shape");
  o += "[" + std::to_string(n_hidden) + "]";
  key("layers");
  o.push_back('[');
  for (size_t i = 0; i < n_layers; i++) {
    const llh_disk_layer &L = layers[i];
    const std::string stem = "layers." + std::to_string(i) + "." + layer_tensor_stem(L.kind);
    if (i) o.push_back(',');
    // internally tagged enum: "kind" first, then NativeTextDiskFullAttentionLayout (codec.rs:44-56)
    std::string r = "{";
    json_string(r, "kind");
    r.push_back(':');
    json_string(r, layer_kind_name(L.kind));
    auto rnum = [&](const char *k, uint64_t v) {
      r.push_back(',');
      json_string(r, k);
      r += ":" + std::to_string(v);
    };
    auto rstr = [&](const char *k, const std::string &v) {
      r.push_back(',');
      json_string(r, k);
      r.push_back(':');
      json_string(r, v);
    };
    rnum("revision", L.revision);
    rnum("max_tokens", L.max_tokens);
    rnum("key_value_heads", L.key_value_heads);
    rnum("head_dim", L.head_dim);
    rnum("token_count", L.token_count);
    rnum("tokens_seen", L.tokens_seen);
    rstr("cache_format", "f32");
    rstr("key_tensor", stem + ".keys");
    rstr("value_tensor", stem + ".values");
    r += ",\"shape\":[" + std::to_string(L.token_count) + "," + std::to_string(L.key_value_heads) + "," +
         std::to_string(L.head_dim) + "]}";
    o += r;
  }
  o += "]}";
  return o;
}

}  // namespace

struct llh_disk_block {
  std::vector<uint8_t> bytes;  // owned copy of the file
  Metadata meta;
  std::map<std::string, Tensor> tensors;
};

extern "C" {

const char *llh_disk_last_error(void) { return g_disk_error.c_str(); }

int llh_disk_hash_components(const char *label, size_t n, const char *const *names, const char *const *values,
                             char out_hex[65]) {
  if (!label || (n && !names) || !out_hex) return LLH_ERR_NULL;
  llh::Sha256 h;
  update_value(h, label);
  for (size_t i = 0; i < n; i++) {
    if (!names[i]) return LLH_ERR_NULL;
    update_value(h, names[i]);
    update_value(h, values ? values[i] : nullptr);
  }
  uint8_t d[32];
  h.finish(d);
  copy_str(out_hex, 65, hex(d));
  return LLH_OK;
}

int llh_disk_block_hash(const char *model_hash, const char *namespace_hash, const char *previous_block_hash,
                        uint64_t block_start, const uint64_t *tokens, size_t n_tokens, char out_hex[65]) {
  if (!model_hash || !namespace_hash || !previous_block_hash || (n_tokens && !tokens) || !out_hex)
    return LLH_ERR_NULL;
  copy_str(out_hex, 65, block_hash(model_hash, namespace_hash, previous_block_hash, block_start, tokens, n_tokens));
  return LLH_OK;
}

int llh_disk_previous_block_hash(const char *model_hash, const char *namespace_hash, uint64_t block_start,
                                 uint64_t block_token_count, const uint64_t *prefix_tokens, size_t n_prefix,
                                 char out_hex[65]) {
  if (!model_hash || !namespace_hash || (n_prefix && !prefix_tokens) || !out_hex) return LLH_ERR_NULL;
  if (block_token_count == 0) return integrity("disk cache block token count is zero");
  if (block_start > n_prefix) return integrity("disk cache block start exceeds prefix tokens");
  if (block_start % block_token_count != 0) return integrity("disk cache block start is not block aligned");
  std::string prev = kRootHash;
  for (uint64_t cur = 0; cur < block_start; cur += block_token_count) {
    if (cur + block_token_count > n_prefix) return integrity("disk cache previous block exceeds prefix tokens");
    prev = block_hash(model_hash, namespace_hash, prev.c_str(), cur, prefix_tokens + cur, block_token_count);
  }
  copy_str(out_hex, 65, prev);
  return LLH_OK;
}

int llh_disk_block_descriptor_new(const llh_disk_identity *identity, const char *namespace_hash,
                                  uint32_t cache_layout_version, uint64_t block_start, const uint64_t *prefix_tokens,
                                  size_t n_prefix, llh_disk_block_descriptor *out) {
  if (!identity || !namespace_hash || (n_prefix && !prefix_tokens) || !out) return LLH_ERR_NULL;
  if (block_start > n_prefix) return integrity("disk cache block start exceeds prefix tokens");
  const uint64_t count = n_prefix - block_start;
  if (count == 0) return integrity("disk cache block has no tokens");
  char prev[65];
  const int st = llh_disk_previous_block_hash(identity->model_hash, namespace_hash, block_start, count, prefix_tokens,
                                              n_prefix, prev);
  if (st != LLH_OK) return st;
  std::memset(out, 0, sizeof(*out));
  copy_str(out->model_hash, sizeof(out->model_hash), identity->model_hash);
  copy_str(out->snapshot_hash, sizeof(out->snapshot_hash), identity->snapshot_hash);
  copy_str(out->model_family, sizeof(out->model_family), identity->model_family);
  copy_str(out->namespace_hash, sizeof(out->namespace_hash), namespace_hash);
  copy_str(out->previous_block_hash, sizeof(out->previous_block_hash), prev);
  copy_str(out->block_hash, sizeof(out->block_hash),
           block_hash(identity->model_hash, namespace_hash, prev, block_start, prefix_tokens + block_start, count));
  out->block_start = block_start;
  out->token_count = count;
  out->cache_layout_version = cache_layout_version;
  return LLH_OK;
}

int llh_disk_block_path(const llh_disk_block_descriptor *d, char *out, size_t capacity, size_t *length) {
  if (!d || !length) return LLH_ERR_NULL;
  // path_for_descriptor (disk_cache.rs:527-534), relative to the cache root
  const std::string bh = d->block_hash;
  const std::string p = std::string(d->model_hash) + "/" + d->namespace_hash + "/" +
                        (bh.size() >= 2 ? bh.substr(0, 2) : std::string("00")) + "/" + bh + ".safetensors";
  *length = p.size();
  if (!out) return LLH_OK;
  if (capacity < p.size() + 1) return LLH_ERR_CAPACITY;
  std::memcpy(out, p.c_str(), p.size() + 1);
  return LLH_OK;
}

int llh_disk_block_encode(const llh_disk_block_descriptor *d, const float *hidden, size_t n_hidden,
                          const llh_disk_layer *layers, size_t n_layers, uint8_t *out, size_t capacity,
                          size_t *length) {
  if (!d || (n_hidden && !hidden) || (n_layers && !layers) || !length) return LLH_ERR_NULL;
  for (size_t i = 0; i < n_layers; i++) {
    const llh_disk_layer &L = layers[i];
    if (!layer_kind_name(L.kind)) return integrity("unsupported layer layout kind");
    const uint64_t n = L.token_count * L.key_value_heads * L.head_dim;
    if (L.key_value_heads && L.head_dim && n / L.key_value_heads / L.head_dim != L.token_count)
      return integrity("tensor shape overflow");
    if (n && (!L.keys || !L.values)) return LLH_ERR_NULL;
  }
  // tensors, sorted by name (io.rs:291-293)
  struct Src {
    std::string name;
    std::vector<uint64_t> shape;
    const float *v;
    size_t n;
  };
  std::vector<Src> ts;
  ts.push_back({"hidden", {n_hidden}, hidden, n_hidden});
  for (size_t i = 0; i < n_layers; i++) {
    const llh_disk_layer &L = layers[i];
    const std::string stem = "layers." + std::to_string(i) + "." + layer_tensor_stem(L.kind);
    const size_t n = (size_t)(L.token_count * L.key_value_heads * L.head_dim);
    ts.push_back({stem + ".keys", {L.token_count, L.key_value_heads, L.head_dim}, L.keys, n});
    ts.push_back({stem + ".values", {L.token_count, L.key_value_heads, L.head_dim}, L.values, n});
  }
  std::sort(ts.begin(), ts.end(), [](const Src &a, const Src &b) { return a.name < b.name; });
  std::string header = "{";
  json_string(header, "__metadata__");
  header += ":{";
  json_string(header, "kir_ai");
  header.push_back(':');
  json_string(header, metadata_json(*d, n_hidden, layers, n_layers));
  header.push_back('}');
  uint64_t off = 0;
  for (const Src &t : ts) {
    header.push_back(',');
    json_string(header, t.name);
    header += ":{\"dtype\":\"F32\",\"shape\":[";
    for (size_t k = 0; k < t.shape.size(); k++) header += (k ? "," : "") + std::to_string(t.shape[k]);
    header += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + 4 * t.n) + "]}";
    off += 4 * t.n;
  }
  header.push_back('}');
  const size_t total = 8 + header.size() + (size_t)off;
  *length = total;
  if (!out) return LLH_OK;
  if (capacity < total) return LLH_ERR_CAPACITY;
  const uint64_t hl = header.size();
  for (int i = 0; i < 8; i++) out[i] = (uint8_t)(hl >> (8 * i));  // little-endian u64
  std::memcpy(out + 8, header.data(), header.size());
  uint8_t *p = out + 8 + header.size();
  for (const Src &t : ts) {
    if (t.n) std::memcpy(p, t.v, 4 * t.n);  // little-endian host
    p += 4 * t.n;
  }
  return LLH_OK;
}

int llh_disk_block_open(const uint8_t *bytes, size_t length, llh_disk_block **out) {
  if (!bytes || !out) return LLH_ERR_NULL;
  *out = nullptr;
  if (length < 8) return integrity("safetensors file is missing header length");
  uint64_t hl = 0;
  for (int i = 0; i < 8; i++) hl |= (uint64_t)bytes[i] << (8 * i);
  if (hl > kMaxHeaderLen) return integrity("safetensors header exceeds limit");
  if (hl > length - 8) return integrity("safetensors header is truncated");
  auto blk = std::make_unique<llh_disk_block>();
  blk->bytes.assign(bytes, bytes + length);
  const char *h = reinterpret_cast<const char *>(blk->bytes.data()) + 8;
  JParser jp{h, h + hl, {}};
  JVal root;
  if (!jp.value(root, 0)) return integrity("invalid safetensors header json: " + jp.err);
  if (root.kind != JVal::Obj) return integrity("safetensors header is not an object");
  // metadata (io.rs:359-372)
  const JVal *md = root.get("__metadata__");
  const JVal *ka = md && md->kind == JVal::Obj ? md->get("kir_ai") : nullptr;
  std::string mtext;
  if (!as_str(ka, mtext)) return integrity("missing disk cache metadata");
  JParser mp{mtext.data(), mtext.data() + mtext.size(), {}};
  JVal m;
  if (!mp.value(m, 0) || m.kind != JVal::Obj) return integrity("invalid disk cache metadata: " + mp.err);
  Metadata &M = blk->meta;
  if (!as_str(m.get("codec"), M.codec) || !as_u64(m.get("layout_version"), M.layout_version) ||
      !as_u64(m.get("cache_layout_version"), M.cache_layout_version) ||
      !as_str(m.get("model_family"), M.model_family) || !as_str(m.get("model_hash"), M.model_hash) ||
      !as_str(m.get("snapshot_hash"), M.snapshot_hash) || !as_str(m.get("namespace_hash"), M.namespace_hash) ||
      !as_str(m.get("previous_block_hash"), M.previous_block_hash) ||
      !as_str(m.get("block_hash"), M.block_hash) || !as_u64(m.get("block_start"), M.block_start) ||
      !as_u64(m.get("token_count"), M.token_count) || !as_u64_array(m.get("hidden_shape"), M.hidden_shape))
    return integrity("invalid disk cache metadata: missing or mistyped field");
  if (M.layout_version > UINT32_MAX || M.cache_layout_version > UINT32_MAX)
    return integrity("invalid disk cache metadata: version out of range");
  const JVal *lay = m.get("layers");
  if (!lay || lay->kind != JVal::Arr) return integrity("invalid disk cache metadata: layers");
  for (const JVal &l : lay->arr) {
    LayerMeta L;
    std::string kind;
    if (l.kind != JVal::Obj || !as_str(l.get("kind"), kind)) return integrity("invalid disk cache layer layout");
    if (kind == "qwen_full_attention") {
      L.kind = LLH_DISK_LAYER_QWEN_FULL;
    } else if (kind == "gemma_attention") {
      L.kind = LLH_DISK_LAYER_GEMMA;
    } else if (kind == "qwen_linear_attention") {
      // recurrent state (NativeTextDiskLinearAttentionLayout, codec.rs:57-70), not paged KV:
      // its fields are checked so the block parses as the reference parses it
      L.kind = LLH_DISK_LAYER_OTHER;
      uint64_t u;
      std::string t;
      std::vector<uint64_t> sh;
      for (const char *f : {"revision", "conv_kernel_size", "conv_dim", "num_value_heads", "key_head_dim",
                            "value_head_dim", "token_count"})
        if (!as_u64(l.get(f), u)) return integrity("invalid disk cache metadata: layer field");
      for (const char *f : {"conv_window_tensor", "recurrent_state_tensor"})
        if (!as_str(l.get(f), t)) return integrity("invalid disk cache metadata: layer field");
      for (const char *f : {"conv_window_shape", "recurrent_state_shape"})
        if (!as_u64_array(l.get(f), sh)) return integrity("invalid disk cache metadata: layer field");
    } else {
      return integrity("invalid disk cache metadata: unknown layer kind `" + kind + "`");
    }
    if (L.kind != LLH_DISK_LAYER_OTHER &&
        (!as_u64(l.get("revision"), L.revision) || !as_u64(l.get("max_tokens"), L.max_tokens) ||
         !as_u64(l.get("key_value_heads"), L.kv_heads) || !as_u64(l.get("head_dim"), L.head_dim) ||
         !as_u64(l.get("token_count"), L.token_count) || !as_u64(l.get("tokens_seen"), L.tokens_seen) ||
         !as_str(l.get("cache_format"), L.cache_format) || !as_str(l.get("key_tensor"), L.key_tensor) ||
         !as_str(l.get("value_tensor"), L.value_tensor) || !as_u64_array(l.get("shape"), L.shape)))
      return integrity("invalid disk cache metadata: layer field");
    M.layers.push_back(std::move(L));
  }
  // tensors (io.rs:374-470)
  const uint64_t data_start = 8 + hl;
  for (const auto &kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const JVal &t = kv.second;
    if (t.kind != JVal::Obj) return integrity("tensor `" + kv.first + "` header is not an object");
    std::string dtype;
    if (!as_str(t.get("dtype"), dtype) || dtype != "F32") return integrity("tensor `" + kv.first + "` is not F32");
    Tensor T;
    if (!as_u64_array(t.get("shape"), T.shape)) return integrity("tensor `" + kv.first + "` is missing shape");
    std::vector<uint64_t> offs;
    if (!as_u64_array(t.get("data_offsets"), offs) || offs.size() != 2)
      return integrity("tensor `" + kv.first + "` data offsets are invalid");
    if (offs[1] < offs[0] || (offs[1] - offs[0]) % 4 != 0)
      return integrity("tensor `" + kv.first + "` byte range is invalid");
    if (offs[1] > length - data_start) return integrity("tensor `" + kv.first + "` payload is truncated");
    T.data = blk->bytes.data() + data_start + offs[0];
    T.n = (size_t)((offs[1] - offs[0]) / 4);
    blk->tensors[kv.first] = T;
  }
  if (blk->tensors.empty()) return integrity("disk cache block has no tensors");
  *out = blk.release();
  return LLH_OK;
}

int llh_disk_block_close(llh_disk_block *blk) {
  if (!blk) return LLH_ERR_NULL;
  delete blk;
  return LLH_OK;
}

int llh_disk_block_read_descriptor(const llh_disk_block *blk, llh_disk_block_descriptor *out) {
  if (!blk || !out) return LLH_ERR_NULL;
  const Metadata &M = blk->meta;
  // decode_descriptor (io.rs:105-121): the index rebuild reads only this
  const int st = check_codec_and_layout(M);
  if (st != LLH_OK) return st;
  std::memset(out, 0, sizeof(*out));
  copy_str(out->model_hash, sizeof(out->model_hash), M.model_hash);
  copy_str(out->snapshot_hash, sizeof(out->snapshot_hash), M.snapshot_hash);
  copy_str(out->model_family, sizeof(out->model_family), M.model_family);
  copy_str(out->namespace_hash, sizeof(out->namespace_hash), M.namespace_hash);
  copy_str(out->previous_block_hash, sizeof(out->previous_block_hash), M.previous_block_hash);
  copy_str(out->block_hash, sizeof(out->block_hash), M.block_hash);
  out->block_start = M.block_start;
  out->token_count = M.token_count;
  out->cache_layout_version = (uint32_t)M.cache_layout_version;
  out->n_layers = (uint32_t)M.layers.size();
  return LLH_OK;
}

int llh_disk_block_validate(const llh_disk_block *blk, const llh_disk_block_descriptor *expected,
                            const llh_disk_identity *identity) {
  if (!blk || !expected || !identity) return LLH_ERR_NULL;
  const Metadata &M = blk->meta;
  // NativeTextDiskCacheBlock::decode (io.rs:71-103)
  if (M.namespace_hash != expected->namespace_hash || M.previous_block_hash != expected->previous_block_hash ||
      M.block_hash != expected->block_hash || M.block_start != expected->block_start ||
      M.token_count != expected->token_count)
    return integrity("disk cache block descriptor mismatch");
  // descriptor.validate_for_identity (disk_cache.rs:219-240)
  if (std::strcmp(expected->model_hash, identity->model_hash) != 0) return integrity("model hash mismatch");
  if (std::strcmp(expected->snapshot_hash, identity->snapshot_hash) != 0) return integrity("snapshot hash mismatch");
  if (std::strcmp(expected->model_family, identity->model_family) != 0) return integrity("model family mismatch");
  if (identity->allowed_namespace_hash && std::strcmp(expected->namespace_hash, identity->allowed_namespace_hash))
    return integrity("namespace hash mismatch");
  // validate_metadata_for_identity (io.rs:238-261)
  const int st = check_codec_and_layout(M);
  if (st != LLH_OK) return st;
  if (M.model_hash != identity->model_hash) return integrity("model hash mismatch");
  if (M.snapshot_hash != identity->snapshot_hash) return integrity("snapshot hash mismatch");
  if (M.model_family != identity->model_family) return integrity("model family mismatch");
  if (identity->allowed_namespace_hash && M.namespace_hash != identity->allowed_namespace_hash)
    return integrity("namespace hash mismatch");
  if (M.cache_layout_version != expected->cache_layout_version) return integrity("cache layout version mismatch");
  auto h = blk->tensors.find("hidden");
  if (h == blk->tensors.end()) return integrity("tensor `hidden` not found");
  if (M.hidden_shape.size() != 1 || M.hidden_shape[0] != h->second.n)
    return integrity("hidden tensor shape does not match metadata");
  return LLH_OK;
}

int llh_disk_block_hidden(const llh_disk_block *blk, float *out, size_t capacity, size_t *count) {
  if (!blk || !count) return LLH_ERR_NULL;
  auto h = blk->tensors.find("hidden");
  if (h == blk->tensors.end()) return integrity("tensor `hidden` not found");
  *count = h->second.n;
  if (out) std::memcpy(out, h->second.data, 4 * std::min(capacity, h->second.n));
  return LLH_OK;
}

int llh_disk_block_layer(const llh_disk_block *blk, size_t index, llh_disk_layer_info *info, float *keys,
                         float *values, size_t capacity) {
  if (!blk || !info) return LLH_ERR_NULL;
  if (index >= blk->meta.layers.size()) return LLH_ERR_INVALID_SHAPE;
  const LayerMeta &L = blk->meta.layers[index];
  std::memset(info, 0, sizeof(*info));
  info->kind = L.kind;
  if (L.kind == LLH_DISK_LAYER_OTHER) return LLH_ERR_UNSUPPORTED;
  // decode_layer_kv_snapshot (codec.rs:101-130)
  if (L.cache_format != "f32") return integrity("unsupported KV cache disk format");
  auto kt = blk->tensors.find(L.key_tensor);
  auto vt = blk->tensors.find(L.value_tensor);
  if (kt == blk->tensors.end()) return integrity("tensor `" + L.key_tensor + "` not found");
  if (vt == blk->tensors.end()) return integrity("tensor `" + L.value_tensor + "` not found");
  if (kt->second.shape != L.shape) return integrity("tensor `" + L.key_tensor + "` shape mismatch");
  if (vt->second.shape != L.shape) return integrity("tensor `" + L.value_tensor + "` shape mismatch");
  uint64_t prod = 1;
  for (uint64_t s : L.shape) prod *= s;
  if (prod != kt->second.n || prod != vt->second.n) return integrity("tensor shape does not match value count");
  // LayerKvCache::from_snapshot's checks (crates/llm-kv-cache/src/layer.rs): the rows are
  // token_count x key_value_heads x head_dim and fit the cache
  if (L.shape.size() != 3 || L.shape[0] != L.token_count || L.shape[1] != L.kv_heads || L.shape[2] != L.head_dim)
    return integrity("KV snapshot shape does not match its layout");
  if (L.token_count > L.max_tokens || L.token_count > L.tokens_seen)
    return integrity("KV snapshot token count exceeds its cache");
  info->revision = L.revision;
  info->max_tokens = L.max_tokens;
  info->key_value_heads = L.kv_heads;
  info->head_dim = L.head_dim;
  info->token_count = L.token_count;
  info->tokens_seen = L.tokens_seen;
  info->n_values = kt->second.n;
  if (keys) std::memcpy(keys, kt->second.data, 4 * std::min(capacity, kt->second.n));
  if (values) std::memcpy(values, vt->second.data, 4 * std::min(capacity, vt->second.n));
  return LLH_OK;
}

int llh_disk_blocks_assemble_check(const llh_disk_block *const *blocks, size_t n, uint64_t *total_tokens) {
  if ((n && !blocks) || !total_tokens) return LLH_ERR_NULL;
  *total_tokens = 0;
  // validate_contiguous_disk_blocks (codec.rs:305-322)
  uint64_t expect = 0;
  for (size_t b = 0; b < n; b++) {
    if (!blocks[b]) return LLH_ERR_NULL;
    if (blocks[b]->meta.block_start != expect) return integrity("disk cache blocks are not contiguous");
    expect += blocks[b]->meta.token_count;
  }
  if (n == 0) return LLH_OK;
  // assemble_*_disk_block_states / assemble_layer_kv_prefix_state_blocks (codec.rs:252-303, 396-450)
  const auto &first = blocks[0]->meta.layers;
  for (size_t b = 1; b < n; b++) {
    const auto &ls = blocks[b]->meta.layers;
    if (ls.size() != first.size()) return integrity("inconsistent disk block layer count");
    for (size_t i = 0; i < ls.size(); i++) {
      if (ls[i].kind != first[i].kind) return integrity("inconsistent disk block layer kinds");
      if (ls[i].kind == LLH_DISK_LAYER_OTHER) continue;
      if (ls[i].max_tokens != first[i].max_tokens || ls[i].kv_heads != first[i].kv_heads ||
          ls[i].head_dim != first[i].head_dim)
        return integrity("incompatible KV block shapes");
    }
  }
  for (size_t i = 0; i < first.size(); i++) {
    if (first[i].kind == LLH_DISK_LAYER_OTHER) continue;
    uint64_t tokens = 0;
    for (size_t b = 0; b < n; b++) tokens += blocks[b]->meta.layers[i].token_count;
    if (tokens > first[i].max_tokens) return integrity("assembled KV prefix exceeds cache capacity");
  }
  *total_tokens = expect;
  return LLH_OK;
}

}  // extern "C"
