"""On-disk prefix KV block format and hashes, restated in Python.

TEST INFRASTRUCTURE ONLY: the checker for libllm_hip's disk codec.  Only
tests/ import this module; the product library never does.

Restates crates/llm-native-runtime/src/native_text/disk_cache/:
  hashing.rs:178-201  hash_components / update_hash_value (SHA-256 from hashlib)
  hashing.rs:130-176  block hash and the previous-block chain
  io.rs:11-26         NativeTextDiskCacheBlockMetadata (field order)
  io.rs:279-320       encode_safetensors (header map in insertion order, tensors
                      sorted by name, compact JSON as serde_json writes it)
  codec.rs:43-99      full-attention layer layout and tensor names
JSON is produced by Python's json module (compact separators, non-ASCII kept
as UTF-8, control characters escaped with lowercase \\u00XX), which is how
serde_json's compact writer formats the same values.
"""
from __future__ import annotations

import hashlib
import json
import struct

import numpy as np

ROOT_BLOCK_HASH = "0" * 64
CODEC = "kir-ai-native-text-prefix-block"
LAYOUT_VERSION = 2


def update_hash_value(h, value) -> None:
    """hashing.rs:192-201: Some(v) -> 0x01, u64-LE byte length, bytes; None -> 0x00."""
    if value is None:
        h.update(b"\x00")
        return
    b = value.encode()
    h.update(b"\x01" + struct.pack("<Q", len(b)) + b)


def hash_components(label: str, components) -> str:
    h = hashlib.sha256()
    update_hash_value(h, label)
    for name, value in components:
        update_hash_value(h, name)
        update_hash_value(h, value)
    return h.hexdigest()


def block_hash(model_hash: str, namespace_hash: str, previous_block_hash: str, block_start: int, tokens) -> str:
    h = hashlib.sha256()
    for v in ("kir-ai-native-text-disk-block/v2", model_hash, namespace_hash, previous_block_hash):
        update_hash_value(h, v)
    h.update(struct.pack("<Q", block_start))
    h.update(struct.pack("<Q", len(tokens)))
    for t in tokens:
        h.update(struct.pack("<Q", int(t)))
    return h.hexdigest()


def previous_block_hash(model_hash: str, namespace_hash: str, block_start: int, block_token_count: int,
                        prefix_tokens) -> str:
    """hashing.rs:152-176 (raises ValueError where the reference returns Integrity)."""
    if block_token_count == 0:
        raise ValueError("disk cache block token count is zero")
    if block_start > len(prefix_tokens):
        raise ValueError("disk cache block start exceeds prefix tokens")
    if block_start % block_token_count:
        raise ValueError("disk cache block start is not block aligned")
    prev = ROOT_BLOCK_HASH
    for cur in range(0, block_start, block_token_count):
        if cur + block_token_count > len(prefix_tokens):
            raise ValueError("disk cache previous block exceeds prefix tokens")
        prev = block_hash(model_hash, namespace_hash, prev, cur, prefix_tokens[cur:cur + block_token_count])
    return prev


def layer_layout(kind: str, index: int, revision: int, max_tokens: int, kv_heads: int, head_dim: int,
                 token_count: int, tokens_seen: int) -> dict:
    """codec.rs:43-55 / 72-99: the internally tagged layout record, fields in declaration order."""
    stem = f"layers.{index}.{'full' if kind == 'qwen_full_attention' else 'attention'}"
    return {"kind": kind, "revision": revision, "max_tokens": max_tokens, "key_value_heads": kv_heads,
            "head_dim": head_dim, "token_count": token_count, "tokens_seen": tokens_seen, "cache_format": "f32",
            "key_tensor": f"{stem}.keys", "value_tensor": f"{stem}.values",
            "shape": [token_count, kv_heads, head_dim]}


def metadata(desc: dict, n_hidden: int, layouts: list) -> dict:
    """io.rs:11-26 / 53-67 in field order; desc holds the descriptor's fields."""
    return {"codec": CODEC, "layout_version": LAYOUT_VERSION,
            "cache_layout_version": desc["cache_layout_version"], "model_family": desc["model_family"],
            "model_hash": desc["model_hash"], "snapshot_hash": desc["snapshot_hash"],
            "namespace_hash": desc["namespace_hash"], "previous_block_hash": desc["previous_block_hash"],
            "block_hash": desc["block_hash"], "block_start": desc["block_start"],
            "token_count": desc["token_count"], "hidden_shape": [n_hidden], "layers": layouts}


def _dumps(v) -> str:
    return json.dumps(v, separators=(",", ":"), ensure_ascii=False)


def encode_safetensors(meta: dict, tensors: list) -> bytes:
    """io.rs:279-320: tensors = [(name, shape, f32 array)]."""
    header = {"__metadata__": {"kir_ai": _dumps(meta)}}
    payload = bytearray()
    for name, shape, values in sorted(tensors, key=lambda t: t[0].encode()):
        start = len(payload)
        payload += np.ascontiguousarray(values, dtype="<f4").tobytes()
        header[name] = {"dtype": "F32", "shape": list(shape), "data_offsets": [start, len(payload)]}
    hb = _dumps(header).encode()
    return struct.pack("<Q", len(hb)) + hb + bytes(payload)


def encode_block(desc: dict, hidden, layers: list) -> bytes:
    """NativeTextDiskCacheBlock::encode (io.rs:40-69).  layers = [dict(kind, revision,
    max_tokens, kv_heads, head_dim, tokens_seen, keys[token_count][kv_heads][head_dim], values)]."""
    hidden = np.asarray(hidden, np.float32)
    tensors = [("hidden", [hidden.size], hidden)]
    layouts = []
    for i, L in enumerate(layers):
        k = np.asarray(L["keys"], np.float32)
        lay = layer_layout(L["kind"], i, L["revision"], L["max_tokens"], L["kv_heads"], L["head_dim"], k.shape[0],
                           L["tokens_seen"])
        tensors.append((lay["key_tensor"], lay["shape"], k))
        tensors.append((lay["value_tensor"], lay["shape"], np.asarray(L["values"], np.float32)))
        layouts.append(lay)
    return encode_safetensors(metadata(desc, hidden.size, layouts), tensors)


def read_header(data: bytes) -> tuple[dict, dict, bytes]:
    """(header map, metadata, payload) of a block file."""
    (n,) = struct.unpack("<Q", data[:8])
    header = json.loads(data[8:8 + n])
    return header, json.loads(header["__metadata__"]["kir_ai"]), data[8 + n:]


def rewrite_metadata(data: bytes, **changes) -> bytes:
    """The rewrite_*_for_test helpers of io.rs:123-147: decode, change metadata fields,
    re-encode with the same tensors."""
    header, meta, payload = read_header(data)
    meta.update(changes)
    tensors = []
    for name, t in header.items():
        if name == "__metadata__":
            continue
        s, e = t["data_offsets"]
        tensors.append((name, t["shape"], np.frombuffer(payload[s:e], "<f4")))
    return encode_safetensors(meta, tensors)
