// SHA-256 (FIPS 180-4), incremental.  Used for kir-ai's KV block chain hash
// (crates/llm-kv-cache/src/block.rs:8-33), which the reference computes with
// the `sha2` crate (0.10.9).
#pragma once

#include <cstddef>
#include <cstdint>

namespace llh {

class Sha256 {
 public:
  Sha256();
  void update(const void *data, size_t len);
  void update_u64_le(uint64_t v);
  void update_u32_le(uint32_t v);
  void finish(uint8_t out[32]);

 private:
  void compress(const uint8_t block[64]);
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t fill_ = 0;
  uint64_t total_ = 0;  // bytes
};

}  // namespace llh
