"""Python binding of libllm_hip (the C ABI in include/llm_hip.h).

Two layers, both thin:

* ``Context`` / ``KvPool``: the batched paged-attention hot path.  Device
  buffers are torch tensors (torch is used for device memory and streams only);
  calls are asynchronous on the current torch stream.
* ``LayerKvCache`` / ``HipNativeMatvecBackend``: a mirror of kir-ai's
  ``LayerKvCache`` (crates/llm-kv-cache/src/layer.rs) and of the attention
  hooks of ``NativeMatvecBackend`` (crates/llm-backend/src/core/native_matvec.rs:619-668),
  with the same method names, argument meaning and error behaviour, so tests
  read like the reference's own.

The shared library must exist: there is no fallback path.  Build it with
``python kir-ai_amd/build.py``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
import os
from typing import Optional, Sequence

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libllm_hip.so")

OK = 0
NOT_HANDLED = 1
ERR_INVALID_SHAPE = -1
ERR_CAPACITY = -2
ERR_NON_FINITE = -3
ERR_UNSUPPORTED = -4
ERR_DEVICE = -5
ERR_STALE = -6
ERR_NULL = -7
ERR_INTEGRITY = -8

KV_BF16 = 0
KV_INT8 = 1
KV_FP8_E4M3 = 2
KV_INT8_ROW = 3  # the reference's int8 layout: f32 scale per token row over all kv heads
KV_F16 = 4  # IEEE fp16 elements (no scales)

ERR_FLAG_BAD_BLOCK = 1
ERR_FLAG_TOO_MANY_SPLITS = 2
ERR_FLAG_NON_FINITE = 4
ERR_FLAG_SPAN = 8

# llh_option
OPT_DECODE_KERNEL = 0           # 0 = by step size, 1 = split-K, 2 = stream
OPT_DECODE_SPLIT_BLOCKS = 1
OPT_DECODE_STREAM_WGS = 2
OPT_FORCE_GENERIC = 3
OPT_PREFILL_HEADS_PER_WG = 4
OPT_TRAIT_REFERENCE_ORDER = 5
DECODE_KERNELS = {"auto": 0, "split": 1, "stream": 2}

_STATUS_NAMES = {
    NOT_HANDLED: "not handled",
    ERR_INVALID_SHAPE: "invalid shape",
    ERR_CAPACITY: "capacity exceeded",
    ERR_NON_FINITE: "non-finite value",
    ERR_UNSUPPORTED: "unsupported format",
    ERR_DEVICE: "device error",
    ERR_STALE: "stale block table",
    ERR_NULL: "null pointer",
    ERR_INTEGRITY: "disk cache integrity",
}


class LlhError(RuntimeError):
    """A non-OK status from the C ABI (MathError / KvCacheError in the reference)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


class DecodeDesc(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("max_seq_len", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("total_tokens_hint", ctypes.c_int32),
        ("d_seq_lens", ctypes.c_void_p),
        ("d_block_tables", ctypes.c_void_p),
        ("d_gate", ctypes.c_void_p),
    ]


class PrefillDesc(ctypes.Structure):
    _fields_ = [
        ("num_seqs", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("total_q_rows", ctypes.c_int32),
        ("max_chunk_len", ctypes.c_int32),
        ("d_chunk_starts", ctypes.c_void_p),
        ("d_context_lens", ctypes.c_void_p),
        ("d_block_tables", ctypes.c_void_p),
        ("d_gate", ctypes.c_void_p),
    ]


class PoolInfo(ctypes.Structure):
    _fields_ = [
        ("format", ctypes.c_int32),
        ("block_tokens", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("n_blocks", ctypes.c_int64),
        ("d_k", ctypes.c_void_p),
        ("d_v", ctypes.c_void_p),
        ("d_k_scales", ctypes.c_void_p),
        ("d_v_scales", ctypes.c_void_p),
        ("k_bytes", ctypes.c_size_t),
        ("scale_bytes", ctypes.c_size_t),
    ]


class Metrics(ctypes.Structure):
    _fields_ = [
        ("decode_calls", ctypes.c_uint64),
        ("prefill_calls", ctypes.c_uint64),
        ("append_calls", ctypes.c_uint64),
        ("not_handled", ctypes.c_uint64),
        ("device_errors", ctypes.c_uint64),
        ("shape_errors", ctypes.c_uint64),
        ("stream_decode_calls", ctypes.c_uint64),
        ("trait_tuned_calls", ctypes.c_uint64),
        ("generic_prefill_calls", ctypes.c_uint64),
        ("fused_append_calls", ctypes.c_uint64),
        ("stream_slots", ctypes.c_uint64),
        ("workspace_bytes", ctypes.c_uint64),
        ("d256_decode_calls", ctypes.c_uint64),
        ("generic_decode_calls", ctypes.c_uint64),
    ]


class LayerCacheState(ctypes.Structure):
    _fields_ = [
        ("id", ctypes.c_uint64),
        ("revision", ctypes.c_uint64),
        ("max_tokens", ctypes.c_uint64),
        ("kv_heads", ctypes.c_uint64),
        ("head_dim", ctypes.c_uint64),
        ("token_count", ctypes.c_uint64),
        ("tokens_seen", ctypes.c_uint64),
        ("window_start", ctypes.c_uint64),
        ("block_count", ctypes.c_uint64),
        ("format", ctypes.c_int32),
        ("block_tokens", ctypes.c_int32),
    ]


class LayerCacheRows(ctypes.Structure):
    _fields_ = [
        ("max_tokens", ctypes.c_uint64),
        ("kv_heads", ctypes.c_uint64),
        ("head_dim", ctypes.c_uint64),
        ("format", ctypes.c_int32),
        ("revision", ctypes.c_uint64),
        ("token_count", ctypes.c_uint64),
        ("tokens_seen", ctypes.c_uint64),
        ("window_start", ctypes.c_uint64),
        ("h_keys", ctypes.POINTER(ctypes.c_float)),
        ("h_values", ctypes.POINTER(ctypes.c_float)),
        ("keys_len", ctypes.c_size_t),
    ]


class BlockRun(ctypes.Structure):
    _fields_ = [
        ("block_id", ctypes.c_uint64),
        ("block_index", ctypes.c_uint64),
        ("logical_token_start", ctypes.c_uint64),
        ("physical_token_start", ctypes.c_uint64),
        ("block_token_start", ctypes.c_uint64),
        ("token_count", ctypes.c_uint64),
    ]


class BlockPoolCounts(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("total_blocks", "free_blocks", "allocated_blocks", "sessions")]


class PagedKvMetrics(ctypes.Structure):
    """PagedKvCacheMetricsSnapshot (crates/llm-kv-cache/src/block_pool.rs:99-122)."""
    _fields_ = (
        [(n, ctypes.c_uint64) for n in ("total_blocks", "resident_blocks", "active_blocks", "blocks_in_use",
                                         "free_blocks", "free_list_blocks")]
        + [("pool_utilization_pct", ctypes.c_double)]
        + [(n, ctypes.c_uint64) for n in ("sessions", "session_block_tables", "shared_blocks", "refcount_total")]
        + [("avg_refcount", ctypes.c_double)]
        + [(n, ctypes.c_uint64) for n in ("max_refcount", "max_refcount_seen", "total_refcount_increments",
                                         "total_cow_clones", "cow_bytes_saved", "blocks_evicted_lru",
                                         "sessions_evicted_lru", "eviction_high_water_mark",
                                         "pool_high_water_blocks")]
    )


class CacheBlockInfo(ctypes.Structure):
    _fields_ = [
        ("block_id", ctypes.c_uint64),
        ("pool_index", ctypes.c_int64),
        ("revision", ctypes.c_uint64),
        ("capacity_tokens", ctypes.c_uint64),
        ("vector_len", ctypes.c_uint64),
        ("token_count", ctypes.c_uint64),
        ("ref_count", ctypes.c_uint64),
        ("last_access", ctypes.c_uint64),
        ("payload_bytes", ctypes.c_uint64),
        ("has_content_hash", ctypes.c_int32),
        ("content_hash", ctypes.c_uint8 * 32),
    ]

    def content_hash_bytes(self) -> Optional[bytes]:
        return bytes(self.content_hash) if self.has_content_hash else None


class SessionInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("session_id", "created_at", "last_access", "block_count",
                                              "owned_block_count")]


class PrefixHit(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("token_count", "n_hidden", "n_states", "byte_len")]


PREFIX_COUNTER_FIELDS = (
    "hits", "misses", "stores", "evictions", "rejected", "reused_tokens", "prefill_chunks", "prefill_tokens",
    "checkpoint_stores", "checkpoint_store_tokens", "checkpoint_reuse_hits", "checkpoint_reused_tokens",
    "shared_prefix_hits", "shared_prefix_reused_tokens", "hit_tokens", "miss_tokens", "avoided_prefill_tokens",
    "entries_scanned", "namespace_entries_scanned", "hit_clone_bytes", "bytes_stored", "bytes_evicted",
    "resident_bytes", "resident_entries")


class PrefixCacheCounters(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in PREFIX_COUNTER_FIELDS]


PREFIX_HANDLES_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64), ctypes.c_size_t)
PREFIX_COMPATIBLE_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64),
                                        ctypes.c_size_t)
PREFIX_RECORD_PREFILL_CHUNK = 0
PREFIX_RECORD_CHECKPOINT_STORE = 1
PREFIX_RECORD_CHECKPOINT_REUSE = 2
PREFIX_RECORD_SHARED_PREFIX_REUSE = 3
PREFIX_RECORD_HIT = 4
PREFIX_RECORD_MISS_TOKENS = 5

DISK_LAYER_QWEN_FULL = 0
DISK_LAYER_GEMMA = 1
DISK_LAYER_OTHER = 2


class DiskBlockDescriptor(ctypes.Structure):
    _fields_ = [("model_hash", ctypes.c_char * 65), ("snapshot_hash", ctypes.c_char * 65),
                ("model_family", ctypes.c_char * 64), ("namespace_hash", ctypes.c_char * 65),
                ("previous_block_hash", ctypes.c_char * 65), ("block_hash", ctypes.c_char * 65),
                ("block_start", ctypes.c_uint64), ("token_count", ctypes.c_uint64),
                ("cache_layout_version", ctypes.c_uint32), ("n_layers", ctypes.c_uint32)]


class DiskIdentity(ctypes.Structure):
    _fields_ = [("model_hash", ctypes.c_char_p), ("snapshot_hash", ctypes.c_char_p),
                ("model_family", ctypes.c_char_p), ("allowed_namespace_hash", ctypes.c_char_p)]


class DiskLayer(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32)] + [(n, ctypes.c_uint64) for n in (
        "revision", "max_tokens", "key_value_heads", "head_dim", "token_count", "tokens_seen")] + [
        ("keys", ctypes.POINTER(ctypes.c_float)), ("values", ctypes.POINTER(ctypes.c_float))]


class DiskLayerInfo(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32)] + [(n, ctypes.c_uint64) for n in (
        "revision", "max_tokens", "key_value_heads", "head_dim", "token_count", "tokens_seen", "n_values")]


_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_SZ = ctypes.c_size_t
_FP = ctypes.POINTER(ctypes.c_float)
_U64 = ctypes.c_uint64

# name -> (restype, argtypes); this is the full exported surface of include/llm_hip.h
SIGNATURES = {
    "llh_ctx_create": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(_P)]),
    "llh_ctx_destroy": (ctypes.c_int, [_P]),
    "llh_ctx_last_error": (ctypes.c_char_p, [_P]),
    "llh_ctx_reserve_workspace": (ctypes.c_int, [_P, _SZ]),
    "llh_ctx_reserve_stream_workspace": (ctypes.c_int, [_P, _P, _SZ]),
    "llh_ctx_release_stream": (ctypes.c_int, [_P, _P]),
    "llh_ctx_set_option": (ctypes.c_int, [_P, _I32, _I32]),
    "llh_ctx_get_option": (ctypes.c_int, [_P, _I32, ctypes.POINTER(_I32)]),
    "llh_decode_workspace_bytes": (_SZ, [_I32, _I32, _I32]),
    "llh_ctx_metrics": (ctypes.c_int, [_P, ctypes.POINTER(Metrics)]),
    "llh_ctx_device_errors": (ctypes.c_int, [_P, ctypes.POINTER(_I32), _I32]),
    "llh_ctx_stream_device_errors": (ctypes.c_int, [_P, _P, ctypes.POINTER(_I32), _I32]),
    "llh_ctx_set_kernel_timing": (ctypes.c_int, [_P, _I32]),
    "llh_ctx_kernel_time": (ctypes.c_int, [_P, _I32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64),
                                           _I32]),
    "llh_kv_pool_create": (ctypes.c_int, [_P, _I32, _I32, _I32, _I32, ctypes.c_int64, ctypes.POINTER(_P)]),
    "llh_kv_pool_destroy": (ctypes.c_int, [_P]),
    "llh_kv_pool_get_info": (ctypes.c_int, [_P, ctypes.POINTER(PoolInfo)]),
    "llh_kv_write_blocks": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _P]),
    "llh_kv_append": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _P]),
    "llh_kv_append_f32": (ctypes.c_int, [_P, _P, _P, _P, _P, _I32, _P]),
    "llh_kv_export_rows_f32": (ctypes.c_int, [_P, _P, _P, ctypes.c_int64, _P, _P, _P]),
    "llh_paged_decode": (ctypes.c_int, [_P, _P, ctypes.POINTER(DecodeDesc), _P, _P, ctypes.c_float, _P]),
    "llh_paged_decode_noalloc": (ctypes.c_int, [_P, _P, ctypes.POINTER(DecodeDesc), _P, _P, ctypes.c_float, _P]),
    "llh_paged_decode_append": (ctypes.c_int, [_P, _P, ctypes.POINTER(DecodeDesc), _P, _P, _P, _P, ctypes.c_float,
                                               _P]),
    "llh_paged_prefill": (ctypes.c_int, [_P, _P, ctypes.POINTER(PrefillDesc), _P, _P, ctypes.c_float, _P]),
    "llh_debug_gather": (ctypes.c_int, [_P, _P, ctypes.POINTER(DecodeDesc), _I32, _I32, _I32, _I32, _P, _P]),
    "llh_debug_decode_fp8": (ctypes.c_int, [_P, _P, _P, _I32, _P]),
    "llh_debug_fp8_encode_check": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "llh_layer_cache_create": (ctypes.c_int, [_P, _SZ, _SZ, _SZ, _I32, ctypes.POINTER(_P)]),
    "llh_layer_cache_destroy": (ctypes.c_int, [_P]),
    "llh_layer_cache_create_from_rows": (ctypes.c_int, [_P, ctypes.POINTER(LayerCacheRows), ctypes.POINTER(_P)]),
    "llh_layer_cache_clone": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "llh_layer_cache_clear": (ctypes.c_int, [_P]),
    "llh_layer_cache_get_state": (ctypes.c_int, [_P, ctypes.POINTER(LayerCacheState)]),
    "llh_layer_cache_active_blocks": (ctypes.c_int, [_P, ctypes.POINTER(BlockRun), _SZ, ctypes.POINTER(_SZ)]),
    "llh_layer_cache_block_ids": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_uint64), _SZ, ctypes.POINTER(_SZ)]),
    "llh_append_kv_cache_sliding_f32": (ctypes.c_int, [_P, _P, _FP, _FP, _SZ]),
    "llh_append_kv_cache_f32": (ctypes.c_int, [_P, _P, _FP, _FP, _SZ]),
    "llh_full_attention_cache_mix_f32_in_place": (
        ctypes.c_int,
        [_P, _P, _FP, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _FP, _SZ],
    ),
    "llh_select_kv_cache_head_rows_f32_in_place": (ctypes.c_int, [_P, _P, _I32, _SZ, _SZ, _SZ, _FP, _SZ]),
    "llh_matvec_bf16_f32": (ctypes.c_int, [_P, _P, _I32, _I32, _P, _I32, _I32, _P, _P]),
    "llh_paged_decode_output_projection": (ctypes.c_int, [_P, _P, ctypes.POINTER(DecodeDesc), _P, _P, _I32, _P,
                                                          ctypes.c_float, _P]),
    "llh_full_attention_cache_mix_bf16_output_projection_f32_in_place": (
        ctypes.c_int, [_P, _P, _FP, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P, _I32, _I32, _FP, _SZ]),
    "llh_sha256": (ctypes.c_int, [_P, _SZ, _P]),
    "llh_cache_block_chain_hash": (ctypes.c_int, [ctypes.c_char_p, _SZ, ctypes.c_char_p, _SZ, _P, _P, _SZ, _P]),
    "llh_block_pool_create_host": (ctypes.c_int, [_SZ, _SZ, _SZ, ctypes.POINTER(_P)]),
    "llh_block_pool_create": (ctypes.c_int, [_P, _P, ctypes.POINTER(_P)]),
    "llh_block_pool_destroy": (ctypes.c_int, [_P]),
    "llh_block_pool_last_error": (ctypes.c_char_p, [_P]),
    "llh_block_pool_get_counts": (ctypes.c_int, [_P, ctypes.POINTER(BlockPoolCounts)]),
    "llh_block_pool_metrics": (ctypes.c_int, [_P, ctypes.POINTER(PagedKvMetrics)]),
    "llh_block_pool_block_info": (ctypes.c_int, [_P, _U64, ctypes.POINTER(CacheBlockInfo)]),
    "llh_block_pool_allocate": (ctypes.c_int, [_P, ctypes.POINTER(_U64)]),
    "llh_block_pool_release": (ctypes.c_int, [_P, _U64, ctypes.POINTER(_I32)]),
    "llh_block_pool_retain": (ctypes.c_int, [_P, _U64, ctypes.POINTER(_I32)]),
    "llh_block_pool_touch": (ctypes.c_int, [_P, _U64, ctypes.POINTER(_I32)]),
    "llh_block_pool_lru_block": (ctypes.c_int, [_P, ctypes.POINTER(_U64)]),
    "llh_block_pool_set_content_hash": (ctypes.c_int, [_P, _U64, _P]),
    "llh_block_pool_create_session": (ctypes.c_int, [_P, ctypes.POINTER(_U64)]),
    "llh_block_pool_release_session": (ctypes.c_int, [_P, _U64, ctypes.POINTER(_I32)]),
    "llh_block_pool_allocate_for_session": (ctypes.c_int, [_P, _U64, ctypes.POINTER(_U64)]),
    "llh_block_pool_append_block_to_session": (ctypes.c_int, [_P, _U64, _U64]),
    "llh_block_pool_read_session_block": (ctypes.c_int, [_P, _U64, _SZ, ctypes.POINTER(_U64)]),
    "llh_block_pool_session_info": (ctypes.c_int, [_P, _U64, ctypes.POINTER(SessionInfo)]),
    "llh_block_pool_session_blocks": (ctypes.c_int, [_P, _U64, _P, _P, _SZ, ctypes.POINTER(_SZ)]),
    "llh_block_pool_lru_session": (ctypes.c_int, [_P, ctypes.POINTER(_U64)]),
    "llh_block_pool_register_prefix": (ctypes.c_int, [_P, _P, _P, _SZ]),
    "llh_block_pool_lookup_prefix": (ctypes.c_int, [_P, _P, _P, _SZ, ctypes.POINTER(_SZ), ctypes.POINTER(_I32)]),
    "llh_block_pool_attach_prefix_to_session": (
        ctypes.c_int, [_P, _U64, _P, _P, _SZ, ctypes.POINTER(_SZ), ctypes.POINTER(_I32)]),
    "llh_block_pool_copy_on_write_session_block": (ctypes.c_int, [_P, _U64, _SZ, ctypes.POINTER(_U64)]),
    "llh_block_pool_append_f32": (ctypes.c_int, [_P, _U64, _FP, _FP, _SZ]),
    "llh_block_pool_commit_tokens": (ctypes.c_int, [_P, _U64, _SZ]),
    "llh_block_pool_read_rows_f32": (ctypes.c_int, [_P, _U64, _I32, _FP, _SZ, ctypes.POINTER(_SZ)]),
    "llh_prefix_cache_create": (ctypes.c_int, [_U64, PREFIX_HANDLES_FN, PREFIX_HANDLES_FN, _P, ctypes.POINTER(_P)]),
    "llh_prefix_cache_destroy": (ctypes.c_int, [_P]),
    "llh_prefix_cache_store": (ctypes.c_int, [_P, ctypes.c_char_p, _SZ, _P, _SZ, _P, _SZ, _P, _SZ, _U64,
                                              ctypes.POINTER(_I32)]),
    "llh_prefix_cache_lookup": (ctypes.c_int, [_P, ctypes.c_char_p, _SZ, _P, _SZ, PREFIX_COMPATIBLE_FN, _P,
                                               ctypes.POINTER(PrefixHit), _P, _SZ, _P, _SZ]),
    "llh_prefix_cache_record": (ctypes.c_int, [_P, _I32, _U64]),
    "llh_prefix_cache_metrics": (ctypes.c_int, [_P, ctypes.POINTER(PrefixCacheCounters)]),
    "llh_prefix_cache_shape": (ctypes.c_int, [_P, ctypes.c_char_p, _SZ, ctypes.POINTER(_U64), ctypes.POINTER(_U64),
                                              ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "llh_prefix_cache_lru_entry": (ctypes.c_int, [_P, _SZ, _P, _SZ, ctypes.POINTER(_SZ), _P, _SZ,
                                                  ctypes.POINTER(_SZ)]),
    "llh_disk_last_error": (ctypes.c_char_p, []),
    "llh_disk_hash_components": (ctypes.c_int, [ctypes.c_char_p, _SZ, _P, _P, _P]),
    "llh_disk_block_hash": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _U64, _P, _SZ, _P]),
    "llh_disk_previous_block_hash": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, _U64, _U64, _P, _SZ, _P]),
    "llh_disk_block_descriptor_new": (ctypes.c_int, [ctypes.POINTER(DiskIdentity), ctypes.c_char_p, ctypes.c_uint32,
                                                     _U64, _P, _SZ, ctypes.POINTER(DiskBlockDescriptor)]),
    "llh_disk_block_path": (ctypes.c_int, [ctypes.POINTER(DiskBlockDescriptor), _P, _SZ, ctypes.POINTER(_SZ)]),
    "llh_disk_block_encode": (ctypes.c_int, [ctypes.POINTER(DiskBlockDescriptor), _P, _SZ, ctypes.POINTER(DiskLayer),
                                             _SZ, _P, _SZ, ctypes.POINTER(_SZ)]),
    "llh_disk_block_open": (ctypes.c_int, [_P, _SZ, ctypes.POINTER(_P)]),
    "llh_disk_block_close": (ctypes.c_int, [_P]),
    "llh_disk_block_read_descriptor": (ctypes.c_int, [_P, ctypes.POINTER(DiskBlockDescriptor)]),
    "llh_disk_block_validate": (ctypes.c_int, [_P, ctypes.POINTER(DiskBlockDescriptor),
                                               ctypes.POINTER(DiskIdentity)]),
    "llh_disk_block_hidden": (ctypes.c_int, [_P, _P, _SZ, ctypes.POINTER(_SZ)]),
    "llh_disk_block_layer": (ctypes.c_int, [_P, _SZ, ctypes.POINTER(DiskLayerInfo), _P, _P, _SZ]),
    "llh_disk_blocks_assemble_check": (ctypes.c_int, [_P, _SZ, ctypes.POINTER(_U64)]),
}

_lib: Optional[ctypes.CDLL] = None


def load_library() -> ctypes.CDLL:
    """Loads libllm_hip.so; raises if it was not built (no silent fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with `python kir-ai_amd/build.py`")
    # torch ships its own libamdhip64.so.7; loading torch first makes this library
    # bind to that same runtime (same soname), so the process has one HIP runtime.
    import torch  # noqa: F401

    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _f32_ptr(a: np.ndarray):
    return a.ctypes.data_as(_FP)


def _ptr(t) -> int:
    """Device pointer of a torch tensor (or None)."""
    if t is None:
        return None
    return t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


class Context:
    """An llh_ctx on one HIP device."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _P()
        st = self.lib.llh_ctx_create(device, ctypes.byref(h))
        if st != OK:
            raise LlhError(st, f"llh_ctx_create({device}) failed")
        self.handle = h
        self.device = device

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.llh_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter teardown order
        try:
            self.close()
        except Exception:
            pass

    def check(self, st: int) -> int:
        if st < 0:
            raise LlhError(st, self.lib.llh_ctx_last_error(self.handle).decode())
        return st

    def last_error(self) -> str:
        return self.lib.llh_ctx_last_error(self.handle).decode()

    def metrics(self) -> dict:
        m = Metrics()
        self.check(self.lib.llh_ctx_metrics(self.handle, ctypes.byref(m)))
        return {f: getattr(m, f) for f, _ in Metrics._fields_}

    def device_errors(self, reset: bool = True) -> int:
        """OR of every stream's sticky device flags (waits for the device)."""
        flags = _I32()
        self.check(self.lib.llh_ctx_device_errors(self.handle, ctypes.byref(flags), 1 if reset else 0))
        return flags.value

    def stream_device_errors(self, stream=None, reset: bool = True) -> int:
        """The flags raised by the calls made on one stream (waits for that stream only)."""
        flags = _I32()
        self.check(self.lib.llh_ctx_stream_device_errors(self.handle, _stream(stream), ctypes.byref(flags),
                                                         1 if reset else 0))
        return flags.value

    def set_kernel_timing(self, enable: bool) -> None:
        self.check(self.lib.llh_ctx_set_kernel_timing(self.handle, 1 if enable else 0))

    def kernel_time(self, kind: str, reset: bool = True) -> tuple[float, int]:
        """(summed ms, count) of the timed main kernels: kind 'decode' or 'prefill'."""
        ms, n = ctypes.c_double(), ctypes.c_int64()
        self.check(self.lib.llh_ctx_kernel_time(self.handle, {"decode": 0, "prefill": 1}[kind], ctypes.byref(ms),
                                                ctypes.byref(n), 1 if reset else 0))
        return ms.value, n.value

    def reserve_workspace(self, nbytes: int) -> None:
        self.check(self.lib.llh_ctx_reserve_workspace(self.handle, nbytes))

    def reserve_stream_workspace(self, nbytes: int, stream=None) -> None:
        self.check(self.lib.llh_ctx_reserve_stream_workspace(self.handle, _stream(stream), nbytes))

    def release_stream(self, stream) -> None:
        self.check(self.lib.llh_ctx_release_stream(self.handle, _stream(stream)))

    def set_option(self, option: int, value: int) -> None:
        self.check(self.lib.llh_ctx_set_option(self.handle, option, int(value)))

    def get_option(self, option: int) -> int:
        v = _I32()
        self.check(self.lib.llh_ctx_get_option(self.handle, option, ctypes.byref(v)))
        return v.value

    def pool(self, fmt: int, block_tokens: int, kv_heads: int, head_dim: int, n_blocks: int) -> "KvPool":
        return KvPool(self, fmt, block_tokens, kv_heads, head_dim, n_blocks)

    # ---- batched hot path ----
    @staticmethod
    def decode_desc(seq_lens, block_tables, num_q_heads: int, max_seq_len: int, window: int = 0,
                    total_tokens_hint: int = 0, gate=None) -> DecodeDesc:
        """Descriptor over device int32 tensors; it keeps them alive (it stores raw pointers).
        total_tokens_hint: the sum of attended tokens if the caller knows it (sizes split-K);
        gate: None, or a bf16 [num_seqs][num_q_heads][head_dim] tensor (out *= sigmoid(gate))."""
        d = DecodeDesc(
            num_seqs=seq_lens.shape[0],
            num_q_heads=num_q_heads,
            max_blocks_per_seq=block_tables.shape[1],
            max_seq_len=max_seq_len,
            window=window,
            total_tokens_hint=total_tokens_hint,
            d_seq_lens=_ptr(seq_lens),
            d_block_tables=_ptr(block_tables),
            d_gate=_ptr(gate),
        )
        d._keep = (seq_lens, block_tables, gate)
        return d

    @staticmethod
    def prefill_desc(chunk_starts, context_lens, block_tables, num_q_heads: int, max_chunk_len: int,
                     window: int = 0, total_q_rows: Optional[int] = None, gate=None) -> PrefillDesc:
        """Descriptor over device int32 tensors; it keeps them alive (it stores raw pointers).
        gate: None, or a bf16 [total_q_rows][num_q_heads][head_dim] tensor (out *= sigmoid(gate))."""
        if total_q_rows is None:
            total_q_rows = int(chunk_starts[-1].item())
        d = PrefillDesc(
            num_seqs=context_lens.shape[0],
            num_q_heads=num_q_heads,
            max_blocks_per_seq=block_tables.shape[1],
            window=window,
            total_q_rows=total_q_rows,
            max_chunk_len=max_chunk_len,
            d_chunk_starts=_ptr(chunk_starts),
            d_context_lens=_ptr(context_lens),
            d_block_tables=_ptr(block_tables),
            d_gate=_ptr(gate),
        )
        d._keep = (chunk_starts, context_lens, block_tables, gate)
        return d

    def paged_decode(self, pool: "KvPool", desc: DecodeDesc, q, out, score_scale: float, stream=None) -> None:
        self.check(
            self.lib.llh_paged_decode(
                self.handle, pool.handle, ctypes.byref(desc), _ptr(q), _ptr(out), score_scale, _stream(stream)
            )
        )

    def bind(self, name: str, *args):
        """A zero-argument call of the C entry point `name` with the context handle and the
        given arguments converted to ctypes values once (device tensors become their
        pointers, DecodeDesc / PrefillDesc are passed by reference, streams by handle), for
        loops that issue the same call many times: the per-call Python work is one C call and
        the status check.  The tensors and descriptors must outlive the returned call."""
        fn = getattr(self.lib, name)
        conv = [self.handle]
        for a in args:
            if isinstance(a, (DecodeDesc, PrefillDesc)):
                conv.append(ctypes.byref(a))
            elif isinstance(a, (KvPool, LayerKvCache)):
                conv.append(a.handle)
            elif isinstance(a, float):
                conv.append(ctypes.c_float(a))
            elif hasattr(a, "data_ptr"):
                conv.append(_P(a.data_ptr()))
            elif hasattr(a, "cuda_stream"):
                conv.append(_P(a.cuda_stream))
            else:
                conv.append(a)
        conv = tuple(conv)
        keep = args

        def call():
            st = fn(*conv)
            if st < 0:
                raise LlhError(st, self.lib.llh_ctx_last_error(self.handle).decode() + f" ({len(keep)} args)")

        return call

    def paged_decode_append(self, pool: "KvPool", desc: DecodeDesc, k_new, v_new, q, out, score_scale: float,
                            stream=None) -> None:
        """llh_paged_decode_append: append each sequence's new token (position len - 1), then attend."""
        self.check(self.lib.llh_paged_decode_append(self.handle, pool.handle, ctypes.byref(desc), _ptr(k_new),
                                                    _ptr(v_new), _ptr(q), _ptr(out), ctypes.c_float(score_scale),
                                                    _stream(stream)))

    def paged_decode_noalloc(self, pool: "KvPool", desc: DecodeDesc, q, out, score_scale: float,
                             stream=None) -> None:
        """llh_paged_decode_noalloc: the same step on the library's static scratch (allocates nothing)."""
        self.check(self.lib.llh_paged_decode_noalloc(self.handle, pool.handle, ctypes.byref(desc), _ptr(q), _ptr(out),
                                                     ctypes.c_float(score_scale), _stream(stream)))

    def matvec_bf16(self, w, rows: int, cols: int, x, n: int, out, stream=None) -> None:
        """out[n][rows] f32 = x[n][cols] (bf16 or f32 tensor) times W[rows][cols]^T (bf16)."""
        import torch

        self.check(self.lib.llh_matvec_bf16_f32(self.handle, _ptr(w), rows, cols, _ptr(x),
                                                1 if x.dtype == torch.float32 else 0, n, _ptr(out),
                                                _stream(stream)))

    def paged_decode_output_projection(self, pool: "KvPool", desc: DecodeDesc, q, w_o, rows: int, out,
                                       score_scale: float, stream=None) -> None:
        self.check(self.lib.llh_paged_decode_output_projection(
            self.handle, pool.handle, ctypes.byref(desc), _ptr(q), _ptr(w_o), rows, _ptr(out), score_scale,
            _stream(stream)))

    def paged_prefill(self, pool: "KvPool", desc: PrefillDesc, q, out, score_scale: float, stream=None) -> None:
        self.check(
            self.lib.llh_paged_prefill(
                self.handle, pool.handle, ctypes.byref(desc), _ptr(q), _ptr(out), score_scale, _stream(stream)
            )
        )

    def write_blocks(self, pool: "KvPool", blocks, k, v, stream=None) -> None:
        self.check(
            self.lib.llh_kv_write_blocks(
                self.handle, pool.handle, _ptr(blocks), _ptr(k), _ptr(v), blocks.shape[0], _stream(stream)
            )
        )

    def append(self, pool: "KvPool", slots, k, v, stream=None) -> None:
        self.check(
            self.lib.llh_kv_append(self.handle, pool.handle, _ptr(slots), _ptr(k), _ptr(v), slots.shape[0],
                                   _stream(stream))
        )

    def append_f32(self, pool: "KvPool", slots, k, v, stream=None) -> None:
        """llh_kv_append_f32: f32 token rows (a restored disk block) into pool slots."""
        self.check(
            self.lib.llh_kv_append_f32(self.handle, pool.handle, _ptr(slots), _ptr(k), _ptr(v), slots.shape[0],
                                       _stream(stream))
        )

    def export_rows_f32(self, pool: "KvPool", slots, k_out, v_out, stream=None) -> None:
        """llh_kv_export_rows_f32: K/V of pool slots as dequantised f32 rows."""
        self.check(
            self.lib.llh_kv_export_rows_f32(self.handle, pool.handle, _ptr(slots), slots.shape[0], _ptr(k_out),
                                            _ptr(v_out), _stream(stream))
        )

    def gather(self, pool: "KvPool", desc: DecodeDesc, seq: int, lo: int, hi: int, tensor: int, out,
               stream=None) -> None:
        self.check(
            self.lib.llh_debug_gather(self.handle, pool.handle, ctypes.byref(desc), seq, lo, hi, tensor, _ptr(out),
                                      _stream(stream))
        )

    def decode_fp8(self, codes, out, stream=None) -> None:
        self.check(self.lib.llh_debug_decode_fp8(self.handle, _ptr(codes), _ptr(out), codes.numel(), _stream(stream)))

    def fp8_encode_check(self) -> int:
        """llh_debug_fp8_encode_check: f32 values (NaNs excepted) whose fp8 code from the
        kernels' encoder differs from the integer reference rule."""
        n = ctypes.c_uint64(0)
        self.check(self.lib.llh_debug_fp8_encode_check(self.handle, ctypes.byref(n)))
        return int(n.value)

    def layer_cache(self, max_tokens: int, kv_heads: int, head_dim: int, fmt: int = KV_BF16) -> "LayerKvCache":
        return LayerKvCache.new_with_config(self, max_tokens, kv_heads, head_dim, fmt)


class KvPool:
    """A device-resident paged KV pool (llh_kv_pool)."""

    def __init__(self, ctx: Context, fmt: int, block_tokens: int, kv_heads: int, head_dim: int, n_blocks: int):
        self.ctx = ctx
        h = _P()
        ctx.check(ctx.lib.llh_kv_pool_create(ctx.handle, fmt, block_tokens, kv_heads, head_dim, n_blocks,
                                             ctypes.byref(h)))
        self.handle = h
        info = PoolInfo()
        ctx.check(ctx.lib.llh_kv_pool_get_info(h, ctypes.byref(info)))
        self.info = info

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx.lib.llh_kv_pool_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def raw(self) -> dict:
        """Copies K, V (and scales) to host numpy arrays of raw storage bytes."""
        import torch

        i = self.info
        torch.cuda.synchronize()

        def dl(ptr: int, nbytes: int) -> np.ndarray:
            buf = torch.empty(nbytes, dtype=torch.uint8, device=f"cuda:{self.ctx.device}")
            _memcpy_d2d(buf.data_ptr(), ptr, nbytes)
            return buf.cpu().numpy()

        out = {"k": dl(i.d_k, i.k_bytes), "v": dl(i.d_v, i.k_bytes)}
        if i.scale_bytes and i.format in (KV_INT8, KV_FP8_E4M3):
            # one allocation of (K scale, V scale) pairs: fp16 per (block, head, token)
            # for int8, f32 per (block, head) for fp8
            esz = 2 if i.format == KV_INT8 else 4
            both = dl(i.d_k_scales, 2 * i.scale_bytes).reshape(-1, 2, esz)
            out["k_scales"] = np.ascontiguousarray(both[:, 0]).ravel()
            out["v_scales"] = np.ascontiguousarray(both[:, 1]).ravel()
        elif i.scale_bytes:
            out["k_scales"] = dl(i.d_k_scales, i.scale_bytes)
            out["v_scales"] = dl(i.d_v_scales, i.scale_bytes)
        return out


def _memcpy_d2d(dst: int, src: int, nbytes: int) -> None:
    """hipMemcpy device-to-device of raw pointers (used to read a pool back)."""
    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime torch already loaded
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipMemcpy.argtypes = [_P, _P, _SZ, ctypes.c_int]
    st = hip.hipMemcpy(dst, src, nbytes, 3)  # hipMemcpyDeviceToDevice
    if st != 0:
        raise LlhError(ERR_DEVICE, f"hipMemcpy failed with {st}")


class LayerKvCache:
    """Mirror of kir-ai's LayerKvCache over device blocks (crates/llm-kv-cache/src/layer.rs)."""

    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self.handle = handle

    @classmethod
    def new(cls, ctx: Context, max_tokens: int, key_value_heads: int, head_dim: int) -> "LayerKvCache":
        return cls.new_with_config(ctx, max_tokens, key_value_heads, head_dim, KV_BF16)

    @classmethod
    def new_with_config(cls, ctx: Context, max_tokens: int, key_value_heads: int, head_dim: int,
                        fmt: int) -> "LayerKvCache":
        h = _P()
        ctx.check(ctx.lib.llh_layer_cache_create(ctx.handle, max_tokens, key_value_heads, head_dim, fmt,
                                                 ctypes.byref(h)))
        return cls(ctx, h)

    @classmethod
    def from_rows(cls, ctx: Context, max_tokens: int, key_value_heads: int, head_dim: int, keys, values,
                  revision: int = 0, tokens_seen: Optional[int] = None, window_start: int = 0,
                  fmt: int = KV_BF16) -> "LayerKvCache":
        """A cache that already holds rows: LayerKvCache::from_snapshot (window_start 0) and
        from_prefix_cache_state (layer.rs:467-507, 544-581).  keys / values: the logical rows
        (keys() / values()), token_count x (key_value_heads * head_dim) f32."""
        k = np.ascontiguousarray(keys, dtype=np.float32).ravel()
        v = np.ascontiguousarray(values, dtype=np.float32).ravel()
        vl = key_value_heads * head_dim
        n = k.size // vl if vl else 0
        r = LayerCacheRows(max_tokens=max_tokens, kv_heads=key_value_heads, head_dim=head_dim, format=fmt,
                           revision=revision, token_count=n, tokens_seen=n if tokens_seen is None else tokens_seen,
                           window_start=window_start, h_keys=_f32_ptr(k), h_values=_f32_ptr(v), keys_len=k.size)
        if v.size != k.size:
            raise LlhError(ERR_INVALID_SHAPE, "key and value lengths differ")
        h = _P()
        ctx.check(ctx.lib.llh_layer_cache_create_from_rows(ctx.handle, ctypes.byref(r), ctypes.byref(h)))
        return cls(ctx, h)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx.lib.llh_layer_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def clone(self) -> "LayerKvCache":
        h = _P()
        self.ctx.check(self.ctx.lib.llh_layer_cache_clone(self.handle, ctypes.byref(h)))
        return LayerKvCache(self.ctx, h)

    def clear(self) -> None:
        self.ctx.check(self.ctx.lib.llh_layer_cache_clear(self.handle))

    def state(self) -> LayerCacheState:
        s = LayerCacheState()
        self.ctx.check(self.ctx.lib.llh_layer_cache_get_state(self.handle, ctypes.byref(s)))
        return s

    def id(self) -> int:
        return self.state().id

    def revision(self) -> int:
        return self.state().revision

    def token_count(self) -> int:
        return self.state().token_count

    def next_position(self) -> int:
        return self.state().tokens_seen

    def max_tokens(self) -> int:
        return self.state().max_tokens

    def vector_len(self) -> int:
        s = self.state()
        return s.kv_heads * s.head_dim

    def append_sliding(self, key: Sequence[float], value: Sequence[float]) -> None:
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        if k.size != v.size:
            raise LlhError(ERR_INVALID_SHAPE, "key and value lengths differ")
        self.ctx.check(self.ctx.lib.llh_append_kv_cache_sliding_f32(self.ctx.handle, self.handle, _f32_ptr(k),
                                                                    _f32_ptr(v), k.size))

    def append(self, key: Sequence[float], value: Sequence[float]) -> None:
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        if k.size != v.size:
            raise LlhError(ERR_INVALID_SHAPE, "key and value lengths differ")
        self.ctx.check(self.ctx.lib.llh_append_kv_cache_f32(self.ctx.handle, self.handle, _f32_ptr(k), _f32_ptr(v),
                                                            k.size))

    def block_ids(self) -> list:
        n = _SZ()
        self.ctx.check(self.ctx.lib.llh_layer_cache_block_ids(self.handle, None, 0, ctypes.byref(n)))
        arr = (ctypes.c_uint64 * max(1, n.value))()
        self.ctx.check(self.ctx.lib.llh_layer_cache_block_ids(self.handle, arr, n.value, ctypes.byref(n)))
        return list(arr[: n.value])

    def active_blocks(self) -> list:
        n = _SZ()
        self.ctx.check(self.ctx.lib.llh_layer_cache_active_blocks(self.handle, None, 0, ctypes.byref(n)))
        arr = (BlockRun * max(1, n.value))()
        self.ctx.check(self.ctx.lib.llh_layer_cache_active_blocks(self.handle, arr, n.value, ctypes.byref(n)))
        return [{f: getattr(r, f) for f, _ in BlockRun._fields_} for r in arr[: n.value]]

    def keys(self) -> np.ndarray:
        return HipNativeMatvecBackend(self.ctx).select_kv_cache_head_rows_f32(
            self, 0, self.token_count(), 0, self.vector_len())

    def values(self) -> np.ndarray:
        return HipNativeMatvecBackend(self.ctx).select_kv_cache_head_rows_f32(
            self, 1, self.token_count(), 0, self.vector_len())


class HipNativeMatvecBackend:
    """The attention hooks of NativeMatvecBackend (native_matvec.rs:619-668) on the device."""

    KEY = 0
    VALUE = 1

    def __init__(self, ctx: Context):
        self.ctx = ctx

    def append_kv_cache_sliding_f32(self, cache: LayerKvCache, key, value) -> None:
        cache.append_sliding(key, value)

    def full_attention_cache_mix_f32_in_place(self, cache: LayerKvCache, query, row_count: int,
                                              num_attention_heads: int, num_key_value_heads: int, head_dim: int,
                                              score_scale: float, output: np.ndarray) -> bool:
        q = np.ascontiguousarray(query, dtype=np.float32)
        if output.dtype != np.float32 or not output.flags["C_CONTIGUOUS"]:
            raise LlhError(ERR_INVALID_SHAPE, "output must be a contiguous float32 array")
        st = self.ctx.lib.llh_full_attention_cache_mix_f32_in_place(
            self.ctx.handle, cache.handle, _f32_ptr(q), q.size, row_count, num_attention_heads,
            num_key_value_heads, head_dim, float(score_scale), _f32_ptr(output), output.size)
        if st == NOT_HANDLED:
            return False
        self.ctx.check(st)
        return True

    def full_attention_cache_mix_bf16_output_projection_f32_in_place(
            self, cache: LayerKvCache, query, row_count: int, num_attention_heads: int, num_key_value_heads: int,
            head_dim: int, score_scale: float, weight, output: np.ndarray) -> bool:
        """``weight``: device bf16 tensor [rows][cols] (the o_proj tensor, already resident)."""
        q = np.ascontiguousarray(query, dtype=np.float32)
        if output.dtype != np.float32 or not output.flags["C_CONTIGUOUS"]:
            raise LlhError(ERR_INVALID_SHAPE, "output must be a contiguous float32 array")
        rows, cols = weight.shape
        st = self.ctx.lib.llh_full_attention_cache_mix_bf16_output_projection_f32_in_place(
            self.ctx.handle, cache.handle, _f32_ptr(q), q.size, row_count, num_attention_heads,
            num_key_value_heads, head_dim, float(score_scale), _ptr(weight), rows, cols, _f32_ptr(output),
            output.size)
        if st == NOT_HANDLED:
            return False
        self.ctx.check(st)
        return True

    def select_kv_cache_head_rows_f32(self, cache: LayerKvCache, tensor: int, row_count: int, head_start: int,
                                      head_len: int) -> np.ndarray:
        out = np.zeros(row_count * head_len, dtype=np.float32)
        self.select_kv_cache_head_rows_f32_in_place(cache, tensor, row_count, head_start, head_len, out)
        return out

    def select_kv_cache_head_rows_f32_in_place(self, cache: LayerKvCache, tensor: int, row_count: int,
                                               head_start: int, head_len: int, output: np.ndarray) -> None:
        self.ctx.check(self.ctx.lib.llh_select_kv_cache_head_rows_f32_in_place(
            self.ctx.handle, cache.handle, tensor, row_count, head_start, head_len, _f32_ptr(output), output.size))


# ---------------------------------------------------------------------------
# BlockPool mirror (crates/llm-kv-cache/src/block_pool.rs, block.rs:8-33)
# ---------------------------------------------------------------------------

def sha256(data: bytes) -> bytes:
    """SHA-256 computed by the library (FIPS 180-4)."""
    lib = load_library()
    out = (ctypes.c_uint8 * 32)()
    buf = ctypes.create_string_buffer(bytes(data), len(data) or 1)
    st = lib.llh_sha256(ctypes.cast(buf, _P), len(data), out)
    if st != OK:
        raise LlhError(st, "sha256")
    return bytes(out)


def cache_block_chain_hash(model_id: str, cache_context: str, previous_hash: bytes, token_ids) -> bytes:
    """cache_block_chain_hash (crates/llm-kv-cache/src/block.rs:8-28)."""
    lib = load_library()
    m, c = model_id.encode(), cache_context.encode()
    prev = (ctypes.c_uint8 * 32).from_buffer_copy(bytes(previous_hash))
    toks = np.ascontiguousarray(np.asarray(token_ids, dtype=np.uint32))
    out = (ctypes.c_uint8 * 32)()
    st = lib.llh_cache_block_chain_hash(m, len(m), c, len(c), prev, toks.ctypes.data_as(_P) if toks.size else None,
                                        toks.size, out)
    if st != OK:
        raise LlhError(st, "chain hash")
    return bytes(out)


class BlockPool:
    """kir-ai's BlockPool with the reference's method names.  ``new`` makes a
    bookkeeping-only pool (BlockPool::new(block_count, capacity, vector_len));
    ``over`` makes one over a device KvPool whose blocks carry the payload.
    Option results are None, bool results are bool, errors raise LlhError."""

    def __init__(self, handle, ctx: Optional[Context] = None, kv_pool: Optional["KvPool"] = None):
        self._lib = load_library()
        self._h = handle
        self._ctx = ctx
        self._kv_pool = kv_pool  # keeps the device pool alive

    @classmethod
    def new(cls, block_count: int, block_capacity_tokens: int, vector_len: int) -> "BlockPool":
        lib = load_library()
        h = _P()
        st = lib.llh_block_pool_create_host(block_count, block_capacity_tokens, vector_len, ctypes.byref(h))
        if st != OK:
            raise LlhError(st, "BlockPool::new")
        return cls(h)

    @classmethod
    def over(cls, ctx: Context, kv_pool: "KvPool") -> "BlockPool":
        h = _P()
        ctx.check(ctx.lib.llh_block_pool_create(ctx.handle, kv_pool.handle, ctypes.byref(h)))
        return cls(h, ctx, kv_pool)

    def close(self) -> None:
        if self._h:
            self._lib.llh_block_pool_destroy(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int) -> None:
        if st != OK:
            raise LlhError(st, (self._lib.llh_block_pool_last_error(self._h) or b"").decode())

    def _u64_out(self, fn, *args) -> Optional[int]:
        v = _U64()
        self._check(fn(self._h, *args, ctypes.byref(v)))
        return v.value or None

    def _flag(self, fn, *args) -> bool:
        v = _I32()
        self._check(fn(self._h, *args, ctypes.byref(v)))
        return bool(v.value)

    def _counts(self) -> BlockPoolCounts:
        c = BlockPoolCounts()
        self._check(self._lib.llh_block_pool_get_counts(self._h, ctypes.byref(c)))
        return c

    def total_blocks(self) -> int:
        return self._counts().total_blocks

    def free_blocks(self) -> int:
        return self._counts().free_blocks

    def allocated_blocks(self) -> int:
        return self._counts().allocated_blocks

    def session_count(self) -> int:
        return self._counts().sessions

    def metrics_snapshot(self) -> PagedKvMetrics:
        m = PagedKvMetrics()
        self._check(self._lib.llh_block_pool_metrics(self._h, ctypes.byref(m)))
        return m

    def block(self, block_id: int) -> Optional[CacheBlockInfo]:
        info = CacheBlockInfo()
        st = self._lib.llh_block_pool_block_info(self._h, block_id, ctypes.byref(info))
        if st == ERR_STALE:
            return None
        self._check(st)
        return info

    def allocate(self) -> Optional[int]:
        return self._u64_out(self._lib.llh_block_pool_allocate)

    def deallocate(self, block_id: int) -> bool:
        return self.release(block_id)

    def release(self, block_id: int) -> bool:
        return self._flag(self._lib.llh_block_pool_release, block_id)

    def retain(self, block_id: int) -> bool:
        return self._flag(self._lib.llh_block_pool_retain, block_id)

    def touch(self, block_id: int) -> Optional[bool]:
        return True if self._flag(self._lib.llh_block_pool_touch, block_id) else None

    def lru_block(self) -> Optional[int]:
        return self._u64_out(self._lib.llh_block_pool_lru_block)

    def set_content_hash(self, block_id: int, content_hash: Optional[bytes]) -> None:
        buf = None if content_hash is None else (ctypes.c_uint8 * 32).from_buffer_copy(bytes(content_hash))
        self._check(self._lib.llh_block_pool_set_content_hash(self._h, block_id, buf))

    def create_session(self) -> int:
        return self._u64_out(self._lib.llh_block_pool_create_session)

    def release_session(self, session_id: int) -> bool:
        return self._flag(self._lib.llh_block_pool_release_session, session_id)

    def allocate_for_session(self, session_id: int) -> Optional[int]:
        return self._u64_out(self._lib.llh_block_pool_allocate_for_session, session_id)

    def append_block_to_session(self, session_id: int, block_id: int) -> None:
        self._check(self._lib.llh_block_pool_append_block_to_session(self._h, session_id, block_id))

    def read_session_block(self, session_id: int, index: int) -> Optional[int]:
        return self._u64_out(self._lib.llh_block_pool_read_session_block, session_id, index)

    def session(self, session_id: int) -> Optional[SessionInfo]:
        info = SessionInfo()
        st = self._lib.llh_block_pool_session_info(self._h, session_id, ctypes.byref(info))
        if st == ERR_STALE:
            return None
        self._check(st)
        return info

    def session_blocks(self, session_id: int) -> tuple[list, np.ndarray]:
        """(BlockIds, int32 device pool indices) of the session's table, in order."""
        n = _SZ()
        self._check(self._lib.llh_block_pool_session_blocks(self._h, session_id, None, None, 0, ctypes.byref(n)))
        ids = (_U64 * max(1, n.value))()
        idx = np.zeros(n.value, np.int32)
        self._check(self._lib.llh_block_pool_session_blocks(self._h, session_id, ids,
                                                            idx.ctypes.data_as(_P) if n.value else None,
                                                            n.value, ctypes.byref(n)))
        return list(ids)[: n.value], idx

    def lru_session(self) -> Optional[int]:
        return self._u64_out(self._lib.llh_block_pool_lru_session)

    def register_prefix(self, prefix_hash: bytes, block_ids) -> None:
        h = (ctypes.c_uint8 * 32).from_buffer_copy(bytes(prefix_hash))
        ids = (_U64 * max(1, len(block_ids)))(*block_ids)
        self._check(self._lib.llh_block_pool_register_prefix(self._h, h, ids, len(block_ids)))

    def _ids_query(self, fn, *args) -> Optional[list]:
        n, found = _SZ(), _I32()
        cap = self.total_blocks()
        ids = (_U64 * max(1, cap))()
        self._check(fn(self._h, *args, ids, cap, ctypes.byref(n), ctypes.byref(found)))
        return list(ids)[: n.value] if found.value else None

    def lookup_prefix(self, prefix_hash: bytes) -> Optional[list]:
        h = (ctypes.c_uint8 * 32).from_buffer_copy(bytes(prefix_hash))
        return self._ids_query(self._lib.llh_block_pool_lookup_prefix, h)

    def attach_prefix_to_session(self, session_id: int, prefix_hash: bytes) -> Optional[list]:
        h = (ctypes.c_uint8 * 32).from_buffer_copy(bytes(prefix_hash))
        n, found = _SZ(), _I32()
        cap = self.total_blocks()
        ids = (_U64 * max(1, cap))()
        self._check(self._lib.llh_block_pool_attach_prefix_to_session(self._h, session_id, h, ids, cap,
                                                                      ctypes.byref(n), ctypes.byref(found)))
        return list(ids)[: n.value] if found.value else None

    def copy_on_write_session_block(self, session_id: int, index: int) -> int:
        return self._u64_out(self._lib.llh_block_pool_copy_on_write_session_block, session_id, index)

    # payload (device pools)
    def append(self, block_id: int, key, value) -> None:
        """CacheBlock::append through block_mut (exclusive blocks only)."""
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        if k.size != v.size:
            raise LlhError(ERR_INVALID_SHAPE, "key and value rows differ in length")
        self._check(self._lib.llh_block_pool_append_f32(self._h, block_id, _f32_ptr(k), _f32_ptr(v), k.size))

    def commit_tokens(self, block_id: int, n: int) -> None:
        self._check(self._lib.llh_block_pool_commit_tokens(self._h, block_id, n))

    def rows(self, block_id: int, tensor: int) -> np.ndarray:
        """CacheBlock::keys() (tensor 0) / values() (tensor 1): [token_count, vector_len] f32."""
        n = _SZ()
        self._check(self._lib.llh_block_pool_read_rows_f32(self._h, block_id, tensor, None, 0, ctypes.byref(n)))
        out = np.zeros(max(1, n.value), np.float32)
        self._check(self._lib.llh_block_pool_read_rows_f32(self._h, block_id, tensor, _f32_ptr(out), n.value,
                                                          ctypes.byref(n)))
        info = self.block(block_id)
        return out[: n.value].reshape(info.token_count, info.vector_len)

    def keys(self, block_id: int) -> np.ndarray:
        return self.rows(block_id, 0)

    def values(self, block_id: int) -> np.ndarray:
        return self.rows(block_id, 1)


@dataclass
class PrefixCacheHitResult:
    """NativeTextPrefixCacheHit (prefix_cache.rs:162-167): the reused token count, the cached
    hidden row and the state handles (the caller now holds a reference to them)."""
    token_count: int
    hidden: np.ndarray
    states: np.ndarray
    byte_len: int


class PrefixCache:
    """ctypes mirror of the native prefix cache (NativeTextPrefixCache,
    crates/llm-native-runtime/src/native_text/prefix_cache.rs:20-336).

    `retain` / `release` receive the payload's state handles (a numpy uint64 array):
    release when the cache drops a payload, retain for each hit."""

    def __init__(self, max_bytes: int, retain=None, release=None):
        self._lib = load_library()
        h = ctypes.c_void_p()

        def wrap(fn):
            if fn is None:
                return PREFIX_HANDLES_FN()
            return PREFIX_HANDLES_FN(lambda _u, p, n: fn(np.ctypeslib.as_array(p, (n,)).copy() if n else
                                                          np.zeros(0, np.uint64)))

        self._retain = wrap(retain)
        self._release = wrap(release)
        st = self._lib.llh_prefix_cache_create(max_bytes, self._retain, self._release, None, ctypes.byref(h))
        if st != OK:
            raise LlhError(st, "llh_prefix_cache_create")
        self._h = h

    def close(self):
        if self._h:
            self._lib.llh_prefix_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _ns(namespace) -> bytes:
        return namespace if isinstance(namespace, bytes) else str(namespace).encode()

    def _check(self, st: int, what: str):
        if st != OK:
            raise LlhError(st, what)

    def store(self, namespace, tokens, hidden, states, state_bytes: int) -> bool:
        ns = self._ns(namespace)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        hd = np.ascontiguousarray(hidden, dtype=np.float32)
        sv = np.ascontiguousarray(states, dtype=np.uint64)
        out = _I32()
        self._check(self._lib.llh_prefix_cache_store(self._h, ns, len(ns), t.ctypes.data, t.size, hd.ctypes.data,
                                                     hd.size, sv.ctypes.data, sv.size, int(state_bytes),
                                                     ctypes.byref(out)), "llh_prefix_cache_store")
        return bool(out.value)

    def lookup(self, namespace, tokens, compatible=None, max_hidden: int = 1 << 16, max_states: int = 1 << 16):
        """lookup / lookup_compatible: the longest stored prefix of `tokens` that `compatible`
        (a function of the state handles) accepts, or None."""
        ns = self._ns(namespace)
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        hit = PrefixHit()
        hidden = np.zeros(max_hidden, np.float32)
        states = np.zeros(max_states, np.uint64)
        cb = PREFIX_COMPATIBLE_FN() if compatible is None else PREFIX_COMPATIBLE_FN(
            lambda _u, p, n: 1 if compatible(np.ctypeslib.as_array(p, (n,)).copy() if n else np.zeros(0, np.uint64))
            else 0)
        self._check(self._lib.llh_prefix_cache_lookup(self._h, ns, len(ns), t.ctypes.data, t.size, cb, None,
                                                      ctypes.byref(hit), hidden.ctypes.data, hidden.size,
                                                      states.ctypes.data, states.size), "llh_prefix_cache_lookup")
        if hit.token_count == 0:
            return None
        return PrefixCacheHitResult(int(hit.token_count), hidden[: hit.n_hidden].copy(),
                                    states[: hit.n_states].copy(), int(hit.byte_len))

    def record(self, kind: int, tokens: int):
        self._check(self._lib.llh_prefix_cache_record(self._h, kind, int(tokens)), "llh_prefix_cache_record")

    def metrics(self) -> dict:
        c = PrefixCacheCounters()
        self._check(self._lib.llh_prefix_cache_metrics(self._h, ctypes.byref(c)), "llh_prefix_cache_metrics")
        return {f: int(getattr(c, f)) for f in PREFIX_COUNTER_FIELDS}

    def shape(self, namespace=b"") -> dict:
        ns = self._ns(namespace)
        a, b, c, d = _U64(), _U64(), _U64(), _U64()
        self._check(self._lib.llh_prefix_cache_shape(self._h, ns, len(ns), ctypes.byref(a), ctypes.byref(b),
                                                     ctypes.byref(c), ctypes.byref(d)), "llh_prefix_cache_shape")
        return {"namespaces": a.value, "entries": b.value, "indexed": c.value, "used_bytes": d.value}

    def lru_order(self) -> list:
        """(namespace, tokens) of every resident entry, least recently used first."""
        out = []
        i = 0
        while True:
            nl, nt = _SZ(), _SZ()
            st = self._lib.llh_prefix_cache_lru_entry(self._h, i, None, 0, ctypes.byref(nl), None, 0, ctypes.byref(nt))
            if st != OK:
                break
            nsb = ctypes.create_string_buffer(max(1, nl.value))
            toks = np.zeros(max(1, nt.value), np.uint32)
            self._check(self._lib.llh_prefix_cache_lru_entry(self._h, i, nsb, nl.value, ctypes.byref(nl),
                                                             toks.ctypes.data, nt.value, ctypes.byref(nt)),
                        "llh_prefix_cache_lru_entry")
            out.append((nsb.raw[: nl.value].decode(), [int(x) for x in toks[: nt.value]]))
            i += 1
        return out


# ---------------------------------------------------------------------------
# On-disk prefix KV blocks (native_text/disk_cache.rs, disk_cache/{io,codec,hashing}.rs)
# ---------------------------------------------------------------------------

NATIVE_TEXT_DISK_CACHE_ROOT_BLOCK_HASH = "0" * 64


class DiskCacheIntegrityError(LlhError):
    """NativeTextDiskCacheError::Integrity (native_text/disk_cache.rs:262-270)."""


def _disk_check(st: int, what: str) -> None:
    if st == OK:
        return
    lib = load_library()
    if st == ERR_INTEGRITY:
        raise DiskCacheIntegrityError(st, lib.llh_disk_last_error().decode())
    raise LlhError(st, what)


def _b(s: Optional[str]) -> Optional[bytes]:
    return None if s is None else s.encode()


def disk_hash_components(label: str, components) -> str:
    """hash_components (hashing.rs:178-190): `components` is a sequence of
    (name, value-or-None) pairs."""
    lib = load_library()
    comps = list(components)
    names = (ctypes.c_char_p * max(1, len(comps)))(*[_b(n) for n, _ in comps])
    values = (ctypes.c_char_p * max(1, len(comps)))(*[_b(v) for _, v in comps])
    out = ctypes.create_string_buffer(65)
    _disk_check(lib.llh_disk_hash_components(label.encode(), len(comps), names, values, out),
                "llh_disk_hash_components")
    return out.value.decode()


def native_text_disk_snapshot_hash(snapshot_identity: Optional[str]) -> str:
    """hashing.rs:32-37"""
    return disk_hash_components("kir-ai-native-text-disk-snapshot/v1", [("snapshot_identity", snapshot_identity)])


def native_text_disk_model_hash(model_id: str, backend: str, snapshot_hash: str, family: Optional[str] = None,
                                quantization: Optional[str] = None, repo_id: Optional[str] = None,
                                resolved_commit: Optional[str] = None, profile: Optional[str] = None) -> str:
    """hashing.rs:50-64"""
    return disk_hash_components("kir-ai-native-text-disk-model/v1", [
        ("model_id", model_id), ("backend", backend), ("family", family), ("quantization", quantization),
        ("repo_id", repo_id), ("resolved_commit", resolved_commit), ("profile", profile),
        ("snapshot_hash", snapshot_hash)])


# NativeTextPrefixCacheNamespace fields in the order the namespace hash takes them (hashing.rs:66-128);
# a value is a string, an int (the three counters are decimal strings there) or None for an absent option
DISK_NAMESPACE_FIELDS = (
    "model_id", "backend", "family", "quantization", "repo_id", "resolved_commit", "profile", "tokenizer_kind",
    "tokenizer_hash", "tokenizer_normalization", "cache_template_id", "chat_template_kwargs_hash",
    "adapter_settings", "cache_key", "tool_schema", "request_mode", "cache_layout_version", "cache_tokens",
    "max_prefill_tokens")


def native_text_disk_namespace_hash(namespace: dict) -> str:
    comps = []
    for f in DISK_NAMESPACE_FIELDS:
        v = namespace.get(f)
        comps.append((f, None if v is None else str(v)))
    return disk_hash_components("kir-ai-native-text-disk-namespace/v1", comps)


def native_text_disk_block_hash(model_hash: str, namespace_hash: str, previous_block_hash: str, block_start: int,
                                tokens) -> str:
    """hashing.rs:130-150"""
    lib = load_library()
    t = np.ascontiguousarray(tokens, dtype=np.uint64)
    out = ctypes.create_string_buffer(65)
    _disk_check(lib.llh_disk_block_hash(model_hash.encode(), namespace_hash.encode(), previous_block_hash.encode(),
                                        block_start, t.ctypes.data, t.size, out), "llh_disk_block_hash")
    return out.value.decode()


def native_text_disk_previous_block_hash(model_hash: str, namespace_hash: str, block_start: int,
                                         block_token_count: int, prefix_tokens) -> str:
    """hashing.rs:152-176"""
    lib = load_library()
    t = np.ascontiguousarray(prefix_tokens, dtype=np.uint64)
    out = ctypes.create_string_buffer(65)
    _disk_check(lib.llh_disk_previous_block_hash(model_hash.encode(), namespace_hash.encode(), block_start,
                                                 block_token_count, t.ctypes.data, t.size, out),
                "llh_disk_previous_block_hash")
    return out.value.decode()


@dataclass
class DiskIdentityInfo:
    """NativeTextDiskCacheIdentity (disk_cache.rs:93-147)."""
    model_hash: str
    snapshot_hash: str
    model_family: str
    allowed_namespace_hash: Optional[str] = None

    def c(self) -> DiskIdentity:
        return DiskIdentity(_b(self.model_hash), _b(self.snapshot_hash), _b(self.model_family),
                            _b(self.allowed_namespace_hash))


def disk_block_descriptor(identity: DiskIdentityInfo, namespace_hash: str, cache_layout_version: int,
                          block_start: int, prefix_tokens) -> DiskBlockDescriptor:
    """NativeTextDiskCacheBlockDescriptor::new (disk_cache.rs:176-217)."""
    lib = load_library()
    t = np.ascontiguousarray(prefix_tokens, dtype=np.uint64)
    d = DiskBlockDescriptor()
    ident = identity.c()
    _disk_check(lib.llh_disk_block_descriptor_new(ctypes.byref(ident), namespace_hash.encode(), cache_layout_version,
                                                  block_start, t.ctypes.data, t.size, ctypes.byref(d)),
                "llh_disk_block_descriptor_new")
    return d


def disk_block_path(desc: DiskBlockDescriptor) -> str:
    """path_for_descriptor (disk_cache.rs:527-534), relative to the cache root."""
    lib = load_library()
    n = _SZ()
    _disk_check(lib.llh_disk_block_path(ctypes.byref(desc), None, 0, ctypes.byref(n)), "llh_disk_block_path")
    buf = ctypes.create_string_buffer(n.value + 1)
    _disk_check(lib.llh_disk_block_path(ctypes.byref(desc), buf, n.value + 1, ctypes.byref(n)),
                "llh_disk_block_path")
    return buf.value.decode()


@dataclass
class DiskLayerRows:
    """One full-attention layer of a block: keys / values [token_count][kv_heads][head_dim] f32."""
    kind: int
    revision: int
    max_tokens: int
    key_value_heads: int
    head_dim: int
    token_count: int
    tokens_seen: int
    keys: np.ndarray
    values: np.ndarray


def encode_disk_block(desc: DiskBlockDescriptor, hidden, layers: Sequence[DiskLayerRows]) -> bytes:
    """NativeTextDiskCacheBlock::encode (io.rs:40-69)."""
    lib = load_library()
    h = np.ascontiguousarray(hidden, dtype=np.float32)
    keep = []
    arr = (DiskLayer * max(1, len(layers)))()
    for i, L in enumerate(layers):
        k = np.ascontiguousarray(L.keys, dtype=np.float32)
        v = np.ascontiguousarray(L.values, dtype=np.float32)
        keep += [k, v]
        arr[i] = DiskLayer(L.kind, L.revision, L.max_tokens, L.key_value_heads, L.head_dim, L.token_count,
                           L.tokens_seen, _f32_ptr(k), _f32_ptr(v))
    n = _SZ()
    _disk_check(lib.llh_disk_block_encode(ctypes.byref(desc), h.ctypes.data, h.size, arr, len(layers), None, 0,
                                          ctypes.byref(n)), "llh_disk_block_encode")
    out = (ctypes.c_uint8 * n.value)()
    _disk_check(lib.llh_disk_block_encode(ctypes.byref(desc), h.ctypes.data, h.size, arr, len(layers), out, n.value,
                                          ctypes.byref(n)), "llh_disk_block_encode")
    return bytes(out)


class DiskBlock:
    """A parsed block file (llh_disk_block): metadata, hidden row and layer tensors."""

    def __init__(self, data: bytes):
        self._lib = load_library()
        h = _P()
        buf = (ctypes.c_uint8 * max(1, len(data))).from_buffer_copy(data if data else b"\0")
        _disk_check(self._lib.llh_disk_block_open(buf, len(data), ctypes.byref(h)), "llh_disk_block_open")
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.llh_disk_block_close(self._h)
            self._h = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass

    def descriptor(self) -> DiskBlockDescriptor:
        """decode_descriptor (io.rs:105-121)."""
        d = DiskBlockDescriptor()
        _disk_check(self._lib.llh_disk_block_read_descriptor(self._h, ctypes.byref(d)),
                    "llh_disk_block_read_descriptor")
        return d

    def validate(self, expected: DiskBlockDescriptor, identity: DiskIdentityInfo) -> None:
        """The checks of NativeTextDiskCacheBlock::decode (io.rs:71-103)."""
        ident = identity.c()
        _disk_check(self._lib.llh_disk_block_validate(self._h, ctypes.byref(expected), ctypes.byref(ident)),
                    "llh_disk_block_validate")

    def hidden(self) -> np.ndarray:
        n = _SZ()
        _disk_check(self._lib.llh_disk_block_hidden(self._h, None, 0, ctypes.byref(n)), "llh_disk_block_hidden")
        out = np.zeros(n.value, np.float32)
        _disk_check(self._lib.llh_disk_block_hidden(self._h, out.ctypes.data, out.size, ctypes.byref(n)),
                    "llh_disk_block_hidden")
        return out

    def layer(self, index: int) -> DiskLayerRows:
        """decode_layer_kv_snapshot (codec.rs:101-130) for one layer."""
        info = DiskLayerInfo()
        _disk_check(self._lib.llh_disk_block_layer(self._h, index, ctypes.byref(info), None, None, 0),
                    "llh_disk_block_layer")
        k = np.zeros(info.n_values, np.float32)
        v = np.zeros(info.n_values, np.float32)
        _disk_check(self._lib.llh_disk_block_layer(self._h, index, ctypes.byref(info), k.ctypes.data, v.ctypes.data,
                                                   k.size), "llh_disk_block_layer")
        shape = (int(info.token_count), int(info.key_value_heads), int(info.head_dim))
        return DiskLayerRows(int(info.kind), int(info.revision), int(info.max_tokens), int(info.key_value_heads),
                             int(info.head_dim), int(info.token_count), int(info.tokens_seen), k.reshape(shape),
                             v.reshape(shape))


def disk_blocks_assemble_check(blocks: Sequence[DiskBlock]) -> int:
    """The joins of consecutive blocks of one prefix (codec.rs:252-322); returns the prefix length."""
    lib = load_library()
    arr = (_P * max(1, len(blocks)))(*[b._h.value for b in blocks])
    total = _U64()
    _disk_check(lib.llh_disk_blocks_assemble_check(arr, len(blocks), ctypes.byref(total)),
                "llh_disk_blocks_assemble_check")
    return int(total.value)


def decode_disk_block(data: bytes, identity: DiskIdentityInfo, expected: DiskBlockDescriptor):
    """NativeTextDiskCacheBlock::decode (io.rs:71-103): (hidden, [layers]) or DiskCacheIntegrityError."""
    blk = DiskBlock(data)
    try:
        blk.validate(expected, identity)
        d = blk.descriptor()
        return blk.hidden(), [blk.layer(i) for i in range(d.n_layers)]
    finally:
        blk.close()
