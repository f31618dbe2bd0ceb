"""ctypes wrapper of the C oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module;
the product library never does.  Function-level citations of the kir-ai
reference are in oracle.h / oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")

OK = 0
ERR_INVALID_SHAPE = -1
ERR_CAPACITY = -2
ERR_NON_FINITE = -3

KV_BF16 = 0
KV_INT8 = 1
KV_FP8_E4M3 = 2
KV_INT8_ROW = 3
KV_F16 = 4

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return LIB_PATH


class _Run(ctypes.Structure):
    _fields_ = [
        ("block_index", ctypes.c_int64),
        ("logical_token_start", ctypes.c_int64),
        ("physical_token_start", ctypes.c_int64),
        ("block_token_start", ctypes.c_int64),
        ("token_count", ctypes.c_int64),
    ]


class _Ring(ctypes.Structure):
    _fields_ = [
        ("max_tokens", ctypes.c_int64),
        ("vector_len", ctypes.c_int64),
        ("block_tokens", ctypes.c_int64),
        ("token_count", ctypes.c_int64),
        ("tokens_seen", ctypes.c_int64),
        ("window_start", ctypes.c_int64),
        ("revision", ctypes.c_uint64),
        ("keys", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("runs", ctypes.c_void_p),
        ("run_cap", ctypes.c_int64),
        ("run_count", ctypes.c_int64),
    ]


class _Pool(ctypes.Structure):
    _fields_ = [
        ("format", ctypes.c_int32),
        ("block_tokens", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("n_blocks", ctypes.c_int64),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("k_scales", ctypes.c_void_p),
        ("v_scales", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_U64 = ctypes.c_uint64
_F = ctypes.c_float

_SIGS = {
    "orc_f32_to_bf16": (ctypes.c_uint16, [_F]),
    "orc_bf16_to_f32": (_F, [ctypes.c_uint16]),
    "orc_f32_to_f16": (ctypes.c_uint16, [_F]),
    "orc_f16_to_f32": (_F, [ctypes.c_uint16]),
    "orc_f32_to_fp8e4m3": (ctypes.c_uint8, [_F]),
    "orc_fp8e4m3_to_f32": (_F, [ctypes.c_uint8]),
    "orc_round_half_away": (_F, [_F]),
    "orc_mix64": (_U64, [_U64]),
    "orc_normal": (_F, [_U64, _U64]),
    "orc_fill_normal_f32": (None, [_U64, _U64, _SZ, _P]),
    "orc_fill_normal_bf16": (None, [_U64, _U64, _SZ, _P]),
    "orc_uniform_int": (_I64, [_U64, _U64, _I64, _I64]),
    "orc_permutation": (None, [_U64, _I32, _P]),
    "orc_matvec_row_major": (None, [_P, _P, _SZ, _SZ, _P]),
    "orc_matvec_bf16_f32": (None, [_P, _SZ, _SZ, _P, _P]),
    "orc_softmax": (ctypes.c_int, [_P, _SZ, _P]),
    "orc_weighted_sum": (None, [_P, _P, _SZ, _SZ, _P]),
    "orc_select_head_rows": (None, [_P, _SZ, _SZ, _SZ, _SZ, _P]),
    "orc_attention_mix": (ctypes.c_int, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, _F, _P]),
    "orc_sigmoid": (_F, [_F]),
    "orc_apply_gate": (None, [_P, _P, _SZ]),
    "orc_attention_mix_f64": (ctypes.c_int, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, ctypes.c_double, _P]),
    "orc_ring_init": (ctypes.c_int, [ctypes.POINTER(_Ring), _I64, _I64, _I64, _P, _P, _P, _I64]),
    "orc_ring_append_sliding": (ctypes.c_int, [ctypes.POINTER(_Ring), _P, _P, _P, _P]),
    "orc_ring_append": (ctypes.c_int, [ctypes.POINTER(_Ring), _P, _P, _P]),
    "orc_ring_logical_rows": (None, [ctypes.POINTER(_Ring), ctypes.c_int, _P]),
    "orc_pool_elem": (_F, [ctypes.POINTER(_Pool), ctypes.c_int, _I64, _I32, _I32, _I32]),
    "orc_pool_gather_f32": (ctypes.c_int, [ctypes.POINTER(_Pool), _P, _I32, _I32, _I32, _P, _P]),
    "orc_pool_gather_raw": (ctypes.c_int, [ctypes.POINTER(_Pool), _P, _I32, _I32, _I32, ctypes.c_int, _P]),
    "orc_paged_decode": (ctypes.c_int, [ctypes.POINTER(_Pool), _I32, _I32, _P, _P, _I32, _I32, _P, _F, _P,
                                        ctypes.c_int]),
    "orc_paged_prefill": (ctypes.c_int, [ctypes.POINTER(_Pool), _I32, _I32, _P, _P, _P, _I32, _I32, _P, _F, _P,
                                         ctypes.c_int]),
    "orc_paged_prefill_rows": (ctypes.c_int, [ctypes.POINTER(_Pool), _I32, _I32, _P, _P, _P, _I32, _I32, _P, _F,
                                              _P, _I32, _I32, ctypes.c_int]),
    "orc_quantize_int8_rows": (ctypes.c_int, [_P, _SZ, _SZ, _P, _P]),
    "orc_dequantize_int8_rows": (None, [_P, _P, _SZ, _SZ, _P]),
    "orc_quantize_int8_head": (ctypes.c_int, [_P, _I32, _P, _P]),
    "orc_quantize_fp8_block": (ctypes.c_int, [_P, _I32, _P, _P]),
    "orc_append_fp8_token": (ctypes.c_int, [_P, _I32, _P, _I32, _P]),
}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ---------------- conversions (numpy, same algorithms as the C functions) ----------------

def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def fp8_decode_table() -> np.ndarray:
    L = lib()
    return np.array([L.orc_fp8e4m3_to_f32(c) for c in range(256)], dtype=np.float32)


def fp8_encode(x: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.orc_f32_to_fp8e4m3(float(v)) for v in np.ravel(x)], dtype=np.uint8).reshape(np.shape(x))


# ---------------- PRNG ----------------

def normal_f32(seed: int, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal_f32(seed, offset, n, _p(out))
    return out


def normal_bf16(seed: int, n: int, offset: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().orc_fill_normal_bf16(seed, offset, n, _p(out))
    return out


def uniform_int(seed: int, index: int, lo: int, hi: int) -> int:
    return lib().orc_uniform_int(seed, index, lo, hi)


def permutation(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().orc_permutation(seed, n, _p(out))
    return out


# ---------------- reference math ----------------

def softmax(scores) -> tuple[int, np.ndarray]:
    s = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros_like(s)
    st = lib().orc_softmax(_p(s), s.size, _p(out))
    return st, out


def sigmoid(x: float) -> float:
    """sigmoid_f32 (math.rs:472-474)."""
    return lib().orc_sigmoid(float(x))


def apply_gate(attended, gate) -> np.ndarray:
    """apply_attention_gate (native_attention.rs:775-781): attended * sigmoid(gate), element-wise,
    on a copy (f32)."""
    out = np.ascontiguousarray(attended, dtype=np.float32).ravel().copy()
    g = np.ascontiguousarray(gate, dtype=np.float32).ravel()
    assert g.size == out.size
    lib().orc_apply_gate(_p(out), _p(g), out.size)
    return out


def attention_mix(query, keys, values, row_count, q_heads, kv_heads, head_dim, scale) -> tuple[int, np.ndarray]:
    """native_full_attention_mix_from_cache per-head loop over logical rows."""
    q = np.ascontiguousarray(query, dtype=np.float32).ravel()
    k = np.ascontiguousarray(keys, dtype=np.float32).ravel()
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.zeros(q_heads * head_dim, dtype=np.float32)
    st = lib().orc_attention_mix(_p(q), _p(k), _p(v), row_count, q_heads, kv_heads, head_dim, scale, _p(out))
    return st, out


def attention_mix_f64(query, keys, values, row_count, q_heads, kv_heads, head_dim, scale) -> tuple[int, np.ndarray]:
    q = np.ascontiguousarray(query, dtype=np.float32).ravel()
    k = np.ascontiguousarray(keys, dtype=np.float32).ravel()
    v = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.zeros(q_heads * head_dim, dtype=np.float64)
    st = lib().orc_attention_mix_f64(_p(q), _p(k), _p(v), row_count, q_heads, kv_heads, head_dim, scale, _p(out))
    return st, out


# ---------------- ring cache ----------------

class Ring:
    """LayerKvCache ring semantics (layer.rs) with a configurable block size."""

    def __init__(self, max_tokens: int, vector_len: int, block_tokens: int = 256):
        self.keys = np.zeros(max_tokens * vector_len, dtype=np.float32)
        self.values = np.zeros(max_tokens * vector_len, dtype=np.float32)
        cap = max_tokens // block_tokens + 4 + max_tokens
        self.runs = (_Run * cap)()
        self.r = _Ring()
        st = lib().orc_ring_init(ctypes.byref(self.r), max_tokens, vector_len, block_tokens, _p(self.keys),
                                 _p(self.values), ctypes.cast(self.runs, _P), cap)
        if st != OK:
            raise ValueError(f"ring init failed: {st}")
        self.vector_len = vector_len

    def append_sliding(self, key, value) -> tuple[int, int]:
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        ti, pi = ctypes.c_int64(), ctypes.c_int64()
        st = lib().orc_ring_append_sliding(ctypes.byref(self.r), _p(k), _p(v), ctypes.addressof(ti),
                                           ctypes.addressof(pi))
        if st != OK:
            raise ValueError(f"append failed: {st}")
        return ti.value, pi.value

    def append(self, key, value) -> int:
        k = np.ascontiguousarray(key, dtype=np.float32)
        v = np.ascontiguousarray(value, dtype=np.float32)
        ti = ctypes.c_int64()
        st = lib().orc_ring_append(ctypes.byref(self.r), _p(k), _p(v), ctypes.addressof(ti))
        if st != OK:
            raise OverflowError(f"append failed: {st}")
        return ti.value

    @property
    def token_count(self) -> int:
        return self.r.token_count

    @property
    def tokens_seen(self) -> int:
        return self.r.tokens_seen

    @property
    def window_start(self) -> int:
        return self.r.window_start

    @property
    def revision(self) -> int:
        return self.r.revision

    def logical_rows(self, tensor: int) -> np.ndarray:
        out = np.zeros(self.r.token_count * self.vector_len, dtype=np.float32)
        lib().orc_ring_logical_rows(ctypes.byref(self.r), tensor, _p(out))
        return out

    def active_runs(self) -> list[tuple[int, int, int, int, int]]:
        return [
            (x.block_index, x.logical_token_start, x.physical_token_start, x.block_token_start, x.token_count)
            for x in self.runs[: self.r.run_count]
        ]


# ---------------- paged pool ----------------

class Pool:
    """Host view of a paged pool in the device layout (see oracle.h)."""

    def __init__(self, fmt: int, block_tokens: int, kv_heads: int, head_dim: int, n_blocks: int, k: np.ndarray,
                 v: np.ndarray, k_scales: np.ndarray | None = None, v_scales: np.ndarray | None = None):
        self.k = np.ascontiguousarray(k)
        self.v = np.ascontiguousarray(v)
        self.k_scales = None if k_scales is None else np.ascontiguousarray(k_scales)
        self.v_scales = None if v_scales is None else np.ascontiguousarray(v_scales)
        self.c = _Pool(fmt, block_tokens, kv_heads, head_dim, n_blocks, _p(self.k), _p(self.v),
                       None if self.k_scales is None else _p(self.k_scales),
                       None if self.v_scales is None else _p(self.v_scales))
        self.fmt, self.bt, self.hkv, self.d, self.n_blocks = fmt, block_tokens, kv_heads, head_dim, n_blocks

    @classmethod
    def from_raw(cls, fmt: int, block_tokens: int, kv_heads: int, head_dim: int, n_blocks: int, raw: dict) -> "Pool":
        """From the raw byte arrays of llm_hip.KvPool.raw()."""
        if fmt in (KV_BF16, KV_F16):
            k, v = raw["k"].view(np.uint16), raw["v"].view(np.uint16)
            ks = vs = None
        elif fmt == KV_INT8:
            k, v = raw["k"].view(np.int8), raw["v"].view(np.int8)
            ks, vs = raw["k_scales"].view(np.uint16), raw["v_scales"].view(np.uint16)
        elif fmt == KV_INT8_ROW:
            k, v = raw["k"].view(np.int8), raw["v"].view(np.int8)
            ks, vs = raw["k_scales"].view(np.float32), raw["v_scales"].view(np.float32)
        else:
            k, v = raw["k"].view(np.uint8), raw["v"].view(np.uint8)
            ks, vs = raw["k_scales"].view(np.float32), raw["v_scales"].view(np.float32)
        return cls(fmt, block_tokens, kv_heads, head_dim, n_blocks, k, v, ks, vs)

    def gather_f32(self, table: np.ndarray, lo: int, hi: int) -> tuple[int, np.ndarray, np.ndarray]:
        t = np.ascontiguousarray(table, dtype=np.int32)
        n = max(0, hi - lo) * self.hkv * self.d
        ko = np.zeros(n, dtype=np.float32)
        vo = np.zeros(n, dtype=np.float32)
        st = lib().orc_pool_gather_f32(ctypes.byref(self.c), _p(t), t.size, lo, hi, _p(ko), _p(vo))
        return st, ko, vo

    def gather_raw(self, table: np.ndarray, lo: int, hi: int, tensor: int) -> tuple[int, np.ndarray]:
        t = np.ascontiguousarray(table, dtype=np.int32)
        n = max(0, hi - lo) * self.hkv * self.d
        out = np.zeros(n, dtype=np.uint16 if self.fmt in (KV_BF16, KV_F16) else np.uint8)
        st = lib().orc_pool_gather_raw(ctypes.byref(self.c), _p(t), t.size, lo, hi, tensor, _p(out))
        return st, out

    def decode(self, q_heads: int, seq_lens, tables, window: int, q_bf16, scale: float,
               threads: int = 1) -> tuple[int, np.ndarray]:
        sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
        tb = np.ascontiguousarray(tables, dtype=np.int32)
        q = np.ascontiguousarray(q_bf16, dtype=np.uint16)
        out = np.zeros(sl.size * q_heads * self.d, dtype=np.float32)
        st = lib().orc_paged_decode(ctypes.byref(self.c), sl.size, q_heads, _p(sl), _p(tb), tb.shape[1], window,
                                    _p(q), scale, _p(out), threads)
        return st, out

    def prefill(self, q_heads: int, chunk_starts, context_lens, tables, window: int, q_bf16, scale: float,
                threads: int = 1) -> tuple[int, np.ndarray]:
        cs = np.ascontiguousarray(chunk_starts, dtype=np.int32)
        cl = np.ascontiguousarray(context_lens, dtype=np.int32)
        tb = np.ascontiguousarray(tables, dtype=np.int32)
        q = np.ascontiguousarray(q_bf16, dtype=np.uint16)
        out = np.zeros(int(cs[-1]) * q_heads * self.d, dtype=np.float32)
        st = lib().orc_paged_prefill(ctypes.byref(self.c), cl.size, q_heads, _p(cs), _p(cl), _p(tb), tb.shape[1],
                                     window, _p(q), scale, _p(out), threads)
        return st, out

    def prefill_rows(self, b: int, q_heads: int, chunk_starts, context_lens, tables, window: int, q_bf16,
                     scale: float, row_lo: int, row_hi: int, out: np.ndarray, threads: int = 1) -> int:
        cs = np.ascontiguousarray(chunk_starts, dtype=np.int32)
        cl = np.ascontiguousarray(context_lens, dtype=np.int32)
        tb = np.ascontiguousarray(tables, dtype=np.int32)
        q = np.ascontiguousarray(q_bf16, dtype=np.uint16)
        return lib().orc_paged_prefill_rows(ctypes.byref(self.c), b, q_heads, _p(cs), _p(cl), _p(tb), tb.shape[1],
                                            window, _p(q), scale, _p(out), row_lo, row_hi, threads)


def build_bf16_pool(rows_k: np.ndarray, rows_v: np.ndarray, tables: np.ndarray, seq_lens, block_tokens: int,
                    kv_heads: int, head_dim: int, n_blocks: int, fmt: int = KV_BF16) -> Pool:
    """Host-side pool (bf16, or f16 with fmt=KV_F16) in the device layout from
    per-sequence token rows.

    rows_k[b] / rows_v[b]: uint16 arrays [len_b][kv_heads][head_dim] of the
    format's element bits."""
    k = np.zeros((n_blocks, kv_heads, block_tokens, head_dim), dtype=np.uint16)
    v = np.zeros((n_blocks, kv_heads, head_dim, block_tokens), dtype=np.uint16)
    for b, L in enumerate(seq_lens):
        for pos in range(L):
            blk = tables[b][(pos // block_tokens) % tables.shape[1]]
            t = pos % block_tokens
            k[blk, :, t, :] = rows_k[b][pos]
            v[blk, :, :, t] = rows_v[b][pos]
    return Pool(fmt, block_tokens, kv_heads, head_dim, n_blocks, k, v)


# ---------------- quantisation ----------------

def quantize_int8_rows(x: np.ndarray, vector_len: int) -> tuple[int, np.ndarray, np.ndarray]:
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    rows = a.size // vector_len
    codes = np.zeros(a.size, dtype=np.int8)
    scales = np.zeros(rows, dtype=np.float32)
    st = lib().orc_quantize_int8_rows(_p(a), rows, vector_len, _p(codes), _p(scales))
    return st, codes, scales


def dequantize_int8_rows(codes: np.ndarray, scales: np.ndarray, vector_len: int) -> np.ndarray:
    c = np.ascontiguousarray(codes, dtype=np.int8).ravel()
    s = np.ascontiguousarray(scales, dtype=np.float32).ravel()
    out = np.zeros(c.size, dtype=np.float32)
    lib().orc_dequantize_int8_rows(_p(c), _p(s), s.size, vector_len, _p(out))
    return out


def quantize_int8_head(x: np.ndarray) -> tuple[int, np.ndarray, int]:
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    codes = np.zeros(a.size, dtype=np.int8)
    s = ctypes.c_uint16()
    st = lib().orc_quantize_int8_head(_p(a), a.size, _p(codes), ctypes.addressof(s))
    return st, codes, s.value


def quantize_fp8_block(x: np.ndarray) -> tuple[int, np.ndarray, float]:
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    codes = np.zeros(a.size, dtype=np.uint8)
    s = ctypes.c_float()
    st = lib().orc_quantize_fp8_block(_p(a), a.size, _p(codes), ctypes.addressof(s))
    return st, codes, s.value


def append_fp8_token(codes: np.ndarray, scale: float, off: int, x: np.ndarray) -> tuple[int, float]:
    """orc_append_fp8_token on codes [block_tokens][dim] uint8 (updated in place); returns (status, scale)."""
    assert codes.dtype == np.uint8 and codes.flags["C_CONTIGUOUS"]
    xx = np.ascontiguousarray(x, dtype=np.float32).ravel()
    s = ctypes.c_float(scale)
    st = lib().orc_append_fp8_token(codes.ctypes.data_as(ctypes.c_void_p), xx.size, ctypes.addressof(s), off, _p(xx))
    return st, s.value


def chain_hash(model_id: str, cache_context: str, previous_hash: bytes, token_ids) -> bytes:
    """cache_block_chain_hash restated (crates/llm-kv-cache/src/block.rs:8-33): SHA-256
    (Python's hashlib, an independent implementation) over the domain tag
    "kir-ai-kv-block-chain/v1", the u64-LE length-prefixed model id and cache
    context, the 32-byte previous hash, the u64-LE token count and the u32-LE ids."""
    import hashlib
    import struct

    m, c = model_id.encode(), cache_context.encode()
    h = hashlib.sha256()
    h.update(b"kir-ai-kv-block-chain/v1")
    h.update(struct.pack("<Q", len(m)) + m)
    h.update(struct.pack("<Q", len(c)) + c)
    h.update(bytes(previous_hash))
    h.update(struct.pack("<Q", len(token_ids)))
    for t in token_ids:
        h.update(struct.pack("<I", int(t)))
    return h.digest()


def matvec_bf16_f32(w_bf16: np.ndarray, x: np.ndarray) -> np.ndarray:
    """bf16_matvec_row_major_f32: w [rows][cols] bf16 bits, x [cols] f32 -> [rows] f32."""
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    rows, cols = w.shape
    xx = np.ascontiguousarray(x, dtype=np.float32).ravel()
    assert xx.size == cols
    out = np.zeros(rows, np.float32)
    lib().orc_matvec_bf16_f32(w.ctypes.data_as(ctypes.c_void_p), rows, cols, _p(xx), _p(out))
    return out
