"""The on-disk prefix KV block codec (host side, no GPU).

Ports the reference's codec tests
(crates/llm-native-runtime/src/native_text/disk_cache/tests/codec_reindex.rs,
fixtures.rs) and checks the native encoder against two independent readings
of the format: the Python restatement in oracle/disk_block.py (hashlib and
Python's json writer) must produce the same bytes, and the `safetensors`
library must read the container, its metadata and every tensor.  Hashes are
further pinned by properties of the tagged encoding (root chain start, chain
step, None versus empty string, length-prefix boundaries).
"""
import hashlib
import json
import struct

import numpy as np
import pytest

import llm_hip
from llm_hip import (DISK_LAYER_GEMMA, DISK_LAYER_QWEN_FULL, DiskBlock, DiskCacheIntegrityError, DiskIdentityInfo,
                     DiskLayerRows)
from oracle import disk_block as ref


def namespace(label: str, family: str) -> dict:
    """fixtures.rs:16-38"""
    return {
        "model_id": f"model-{label}", "backend": "native-test", "family": family, "quantization": "bf16",
        "repo_id": "org/model", "resolved_commit": "abc123", "profile": label,
        "tokenizer_kind": "huggingface-tokenizer-json", "tokenizer_hash": f"sha256:tokenizer-{label}",
        "tokenizer_normalization": "llm-tokenizer/hf-json/v1", "cache_template_id": f"template-{label}/v1",
        "chat_template_kwargs_hash": None, "adapter_settings": f"native-test-adapter-{label}/v1",
        "cache_key": f"cache-key-{label}", "tool_schema": None,
        "request_mode": "chat,json_object=false,required_tool=None", "cache_layout_version": 1,
        "cache_tokens": 16, "max_prefill_tokens": 4,
    }


def identity_from_namespace(ns: dict, family: str) -> DiskIdentityInfo:
    """NativeTextDiskCacheIdentity::from_namespace (disk_cache.rs:103-114)."""
    ns_hash = llm_hip.native_text_disk_namespace_hash(ns)
    snap = llm_hip.native_text_disk_snapshot_hash(ns_hash)
    model = llm_hip.native_text_disk_model_hash(
        ns["model_id"], ns["backend"], snap, family=ns["family"], quantization=ns["quantization"],
        repo_id=ns["repo_id"], resolved_commit=ns["resolved_commit"], profile=ns["profile"])
    return DiskIdentityInfo(model, snap, family, ns_hash)


def filled_layer(kind: int = DISK_LAYER_QWEN_FULL, max_tokens: int = 4) -> DiskLayerRows:
    """fixtures.rs:39-54: two tokens of a 2-head, head_dim 3 cache."""
    k = np.array([[1, 2, 3, 4, 5, 6], [7, 8, 9, 10, 11, 12]], np.float32).reshape(2, 2, 3)
    v = np.array([[10, 20, 30, 40, 50, 60], [70, 80, 90, 100, 110, 120]], np.float32).reshape(2, 2, 3)
    return DiskLayerRows(kind, 2, max_tokens, 2, 3, 2, 2, k, v)


def descriptor(identity: DiskIdentityInfo, ns: dict, block_start: int, prefix_tokens):
    return llm_hip.disk_block_descriptor(identity, llm_hip.native_text_disk_namespace_hash(ns),
                                         ns["cache_layout_version"], block_start, prefix_tokens)


def desc_dict(d) -> dict:
    return {f: (getattr(d, f).decode() if isinstance(getattr(d, f), bytes) else getattr(d, f))
            for f in ("model_hash", "snapshot_hash", "model_family", "namespace_hash", "previous_block_hash",
                      "block_hash", "block_start", "token_count", "cache_layout_version")}


def ref_layers(layers):
    kinds = {DISK_LAYER_QWEN_FULL: "qwen_full_attention", DISK_LAYER_GEMMA: "gemma_attention"}
    return [{"kind": kinds[L.kind], "revision": L.revision, "max_tokens": L.max_tokens,
             "kv_heads": L.key_value_heads, "head_dim": L.head_dim, "tokens_seen": L.tokens_seen,
             "keys": L.keys, "values": L.values} for L in layers]


def integrity(fn, match: str):
    with pytest.raises(DiskCacheIntegrityError, match=match):
        fn()


# ---- hashes ------------------------------------------------------------------


def test_hash_components_matches_restatement_and_tagging_properties():
    cases = [("label", []), ("kir-ai-native-text-disk-snapshot/v1", [("snapshot_identity", None)]),
             ("kir-ai-native-text-disk-snapshot/v1", [("snapshot_identity", "manifest:sha256:abc")]),
             ("l", [("a", "é中"), ("b", ""), ("c", None)])]
    for label, comps in cases:
        assert llm_hip.disk_hash_components(label, comps) == ref.hash_components(label, comps)
    # None is a single 0 tag, "" is tag 1 + zero length: distinct
    assert (llm_hip.disk_hash_components("l", [("a", None)]) != llm_hip.disk_hash_components("l", [("a", "")]))
    # the u64 length prefix keeps component boundaries: ("ab","c") != ("a","bc")
    assert (llm_hip.disk_hash_components("l", [("ab", "c")]) != llm_hip.disk_hash_components("l", [("a", "bc")]))
    # spelled out once: label "x", no components = sha256(01 || u64le(1) || "x")
    assert llm_hip.disk_hash_components("x", []) == hashlib.sha256(b"\x01" + struct.pack("<Q", 1) + b"x").hexdigest()


def test_block_hash_chain():
    m, n = "m" * 64, "n" * 64
    toks = list(range(100, 124))
    # the chain starts at the all-zero root and each step hashes the previous link
    assert llm_hip.native_text_disk_previous_block_hash(m, n, 0, 8, toks) == llm_hip.NATIVE_TEXT_DISK_CACHE_ROOT_BLOCK_HASH
    h0 = llm_hip.native_text_disk_block_hash(m, n, "0" * 64, 0, toks[:8])
    h1 = llm_hip.native_text_disk_block_hash(m, n, h0, 8, toks[8:16])
    assert llm_hip.native_text_disk_previous_block_hash(m, n, 8, 8, toks) == h0
    assert llm_hip.native_text_disk_previous_block_hash(m, n, 16, 8, toks) == h1
    assert h0 == ref.block_hash(m, n, "0" * 64, 0, toks[:8])
    assert h1 == ref.previous_block_hash(m, n, 16, 8, toks)
    # tokens are u64 (usize) values
    big = [2 ** 40 + 5, 7]
    assert llm_hip.native_text_disk_block_hash(m, n, h0, 3, big) == ref.block_hash(m, n, h0, 3, big)
    # position and token count are bound into the hash
    assert llm_hip.native_text_disk_block_hash(m, n, h0, 9, toks[8:16]) != h1
    assert llm_hip.native_text_disk_block_hash(m, n, h0, 8, toks[8:15]) != h1


def test_previous_block_hash_errors():
    m, n = "m", "n"
    integrity(lambda: llm_hip.native_text_disk_previous_block_hash(m, n, 0, 0, [1]), "token count is zero")
    integrity(lambda: llm_hip.native_text_disk_previous_block_hash(m, n, 3, 1, [1, 2]), "exceeds prefix tokens")
    integrity(lambda: llm_hip.native_text_disk_previous_block_hash(m, n, 3, 2, [1, 2, 3, 4]), "not block aligned")
    # aligned start whose earlier block runs past the prefix (block_token_count > start)
    integrity(lambda: llm_hip.native_text_disk_previous_block_hash(m, n, 4, 4, [1, 2, 3]), "exceeds prefix tokens")


def test_identity_snapshot_hash_is_derived_from_namespace_fixture_context():
    """codec_reindex.rs:14-27"""
    a = identity_from_namespace(namespace("first-snapshot", "qwen"), "qwen")
    b = identity_from_namespace(namespace("second-snapshot", "qwen"), "qwen")
    assert a.snapshot_hash != b.snapshot_hash
    assert a.model_hash != b.model_hash


def test_namespace_and_model_hashes_match_restatement():
    ns = namespace("x", "gemma")
    comps = [(f, None if ns[f] is None else str(ns[f])) for f in llm_hip.DISK_NAMESPACE_FIELDS]
    assert llm_hip.native_text_disk_namespace_hash(ns) == ref.hash_components(
        "kir-ai-native-text-disk-namespace/v1", comps)
    # from_model_metadata (disk_cache.rs:116-137) with manifest snapshot identities
    snap1 = llm_hip.native_text_disk_snapshot_hash("manifest:sha256:first")
    snap2 = llm_hip.native_text_disk_snapshot_hash("manifest:sha256:second")
    m1 = llm_hip.native_text_disk_model_hash("model-shared", "native-test", snap1, family="qwen",
                                             repo_id="org/model", resolved_commit="abc123", profile="default")
    m2 = llm_hip.native_text_disk_model_hash("model-shared", "native-test", snap2, family="qwen",
                                             repo_id="org/model", resolved_commit="abc123", profile="default")
    assert snap1 != snap2 and m1 != m2
    assert m1 == ref.hash_components("kir-ai-native-text-disk-model/v1", [
        ("model_id", "model-shared"), ("backend", "native-test"), ("family", "qwen"), ("quantization", None),
        ("repo_id", "org/model"), ("resolved_commit", "abc123"), ("profile", "default"), ("snapshot_hash", snap1)])


def test_descriptor_new():
    ns = namespace("d", "qwen")
    ident = identity_from_namespace(ns, "qwen")
    toks = [11, 12, 13, 14]
    d = descriptor(ident, ns, 2, toks)
    assert (d.block_start, d.token_count, d.cache_layout_version) == (2, 2, 1)
    nsh = llm_hip.native_text_disk_namespace_hash(ns)
    prev = ref.previous_block_hash(ident.model_hash, nsh, 2, 2, toks)
    assert d.previous_block_hash.decode() == prev
    assert d.block_hash.decode() == ref.block_hash(ident.model_hash, nsh, prev, 2, toks[2:])
    assert d.model_family == b"qwen" and d.namespace_hash.decode() == nsh
    integrity(lambda: descriptor(ident, ns, 5, toks), "exceeds prefix tokens")
    integrity(lambda: descriptor(ident, ns, 4, toks), "has no tokens")
    integrity(lambda: descriptor(ident, ns, 1, [1, 2, 3]), "not block aligned")  # 2-token block at 1
    h = d.block_hash.decode()
    assert llm_hip.disk_block_path(d) == f"{ident.model_hash}/{nsh}/{h[:2]}/{h}.safetensors"


# ---- container ------------------------------------------------------------------


def encode_both(ns, family, layers, hidden, toks=(11, 12), start=0):
    ident = identity_from_namespace(ns, family)
    d = descriptor(ident, ns, start, list(toks))
    ours = llm_hip.encode_disk_block(d, hidden, layers)
    theirs = ref.encode_block(desc_dict(d), hidden, ref_layers(layers))
    return ident, d, ours, theirs


@pytest.mark.parametrize("family,kind", [("qwen", DISK_LAYER_QWEN_FULL), ("gemma", DISK_LAYER_GEMMA)])
def test_snapshot_codec_round_trips_full_attention_blocks(family, kind):
    """codec_reindex.rs:3-12 (full-attention layers) and fixtures.rs:163-196"""
    ns = namespace("round-trip", family)
    layers = [filled_layer(kind), filled_layer(kind)]
    hidden = np.array([0.25, 0.5, 0.75], np.float32)
    ident, d, enc, theirs = encode_both(ns, family, layers, hidden)
    assert enc == theirs  # byte for byte
    h, out = llm_hip.decode_disk_block(enc, ident, d)
    assert np.array_equal(h, hidden)
    assert len(out) == 2
    for got, want in zip(out, layers):
        assert (got.kind, got.revision, got.max_tokens, got.key_value_heads, got.head_dim, got.token_count,
                got.tokens_seen) == (want.kind, want.revision, want.max_tokens, 2, 3, 2, 2)
        assert np.array_equal(got.keys, want.keys) and np.array_equal(got.values, want.values)
    blk = DiskBlock(enc)
    rd = blk.descriptor()
    assert desc_dict(rd) == desc_dict(d) and rd.n_layers == 2
    # blocks for another cache layout must not decode
    wrong = ref.rewrite_metadata(enc, cache_layout_version=d.cache_layout_version + 1)
    integrity(lambda: llm_hip.decode_disk_block(wrong, ident, d), "cache layout version mismatch")


def test_container_reads_with_safetensors_library(tmp_path):
    from safetensors import safe_open
    from safetensors.numpy import load

    rng = np.random.default_rng(7)
    layers = [DiskLayerRows(DISK_LAYER_QWEN_FULL, 9, 64, 4, 8, 5, 20, rng.standard_normal((5, 4, 8), np.float32),
                            rng.standard_normal((5, 4, 8), np.float32)) for _ in range(12)]
    hidden = rng.standard_normal(16, np.float32)
    ident, d, enc, theirs = encode_both(namespace("st", "qwen"), "qwen", layers, hidden,
                                        toks=list(range(20)), start=15)
    assert enc == theirs
    tensors = load(enc)
    assert set(tensors) == {"hidden"} | {f"layers.{i}.full.{t}" for i in range(12) for t in ("keys", "values")}
    assert np.array_equal(tensors["hidden"], hidden)
    for i, L in enumerate(layers):
        assert np.array_equal(tensors[f"layers.{i}.full.keys"], L.keys)
        assert np.array_equal(tensors[f"layers.{i}.full.values"], L.values)
    p = tmp_path / "b.safetensors"
    p.write_bytes(enc)
    with safe_open(str(p), framework="numpy") as f:
        meta = json.loads(f.metadata()["kir_ai"])
    assert list(meta) == ["codec", "layout_version", "cache_layout_version", "model_family", "model_hash",
                          "snapshot_hash", "namespace_hash", "previous_block_hash", "block_hash", "block_start",
                          "token_count", "hidden_shape", "layers"]
    assert meta["codec"] == "kir-ai-native-text-prefix-block" and meta["layout_version"] == 2
    assert (meta["block_start"], meta["token_count"], meta["hidden_shape"]) == (15, 5, [16])
    assert meta["layers"][10]["key_tensor"] == "layers.10.full.keys"
    assert list(meta["layers"][0]) == ["kind", "revision", "max_tokens", "key_value_heads", "head_dim",
                                       "token_count", "tokens_seen", "cache_format", "key_tensor", "value_tensor",
                                       "shape"]
    # tensors are laid out in name order ("layers.10" sorts before "layers.2")
    header, _, _ = ref.read_header(enc)
    names = [k for k in header if k != "__metadata__"]
    assert names == sorted(names)
    assert names.index("layers.10.full.keys") < names.index("layers.2.full.keys")


def test_json_escaping_matches_restatement():
    ns = namespace("esc", "qwen")
    ident = identity_from_namespace(ns, "qwen")
    ident.model_family = 'q"w\\e\n\t\x01é'  # quotes, backslash, control characters, non-ASCII
    d = descriptor(ident, ns, 0, [1])
    enc = llm_hip.encode_disk_block(d, [1.0], [])
    assert enc == ref.encode_block(desc_dict(d), [1.0], [])
    assert DiskBlock(enc).descriptor().model_family.decode() == ident.model_family


def test_startup_reindex_ignores_wrong_namespace_model_layout_version_and_corrupt_files():
    """codec_reindex.rs:29-103: of the files under a cache root only the valid block
    survives the descriptor read + identity check that the index rebuild applies."""
    valid_ns = namespace("valid", "qwen")
    ident = identity_from_namespace(valid_ns, "qwen")
    hidden = [0.25, 0.5]
    layers = [filled_layer()]
    valid_d = descriptor(ident, valid_ns, 0, [11, 12])
    valid = llm_hip.encode_disk_block(valid_d, hidden, layers)
    wrong_ns_d = descriptor(ident, namespace("wrong", "qwen"), 0, [11, 12])
    wrong_ns = llm_hip.encode_disk_block(wrong_ns_d, hidden, layers)
    wm = dict(valid_ns, model_id="wrong-model")
    wrong_model_d = descriptor(identity_from_namespace(wm, "qwen"), valid_ns, 0, [11, 12])
    wrong_model = llm_hip.encode_disk_block(wrong_model_d, hidden, layers)
    wrong_version = ref.rewrite_metadata(valid, layout_version=99)
    corrupt = b"not a safetensors file"

    def indexable(data: bytes) -> bool:
        try:
            blk = DiskBlock(data)
            d = blk.descriptor()
        except DiskCacheIntegrityError:
            return False
        return (d.model_hash.decode() == ident.model_hash and d.snapshot_hash.decode() == ident.snapshot_hash
                and d.model_family.decode() == ident.model_family
                and d.namespace_hash.decode() == ident.allowed_namespace_hash)

    files = [valid, wrong_ns, wrong_model, wrong_version, corrupt]
    assert [indexable(f) for f in files] == [True, False, False, False, False]
    integrity(lambda: DiskBlock(wrong_version).descriptor(), "unsupported disk cache layout version")
    integrity(lambda: llm_hip.decode_disk_block(wrong_ns, ident, wrong_ns_d), "namespace hash mismatch")
    integrity(lambda: llm_hip.decode_disk_block(wrong_model, ident, wrong_model_d), "model hash mismatch")


def test_snapshot_identity_rejects_wrong_snapshot_metadata():
    """codec_reindex.rs:105-178: a block written under one snapshot does not decode
    under another snapshot of the same model."""
    snap1 = llm_hip.native_text_disk_snapshot_hash("manifest:sha256:first")
    snap2 = llm_hip.native_text_disk_snapshot_hash("manifest:sha256:second")
    mk = lambda s: DiskIdentityInfo(llm_hip.native_text_disk_model_hash(  # noqa: E731
        "model-shared", "native-test", s, family="qwen", repo_id="org/model", resolved_commit="abc123",
        profile="default"), s, "qwen")
    first, second = mk(snap1), mk(snap2)
    ns = namespace("snapshot", "qwen")
    d1 = descriptor(first, ns, 0, [11, 12])
    d2 = descriptor(second, ns, 0, [11, 12])
    wrong = llm_hip.encode_disk_block(d1, [0.25, 0.5], [filled_layer()])
    # filed under the second snapshot's descriptor: descriptor check fails first (different block hash)
    integrity(lambda: llm_hip.decode_disk_block(wrong, second, d2), "descriptor mismatch")
    # with its own descriptor, the identity check rejects it
    integrity(lambda: llm_hip.decode_disk_block(wrong, second, d1), "model hash mismatch")
    # same model hash but another snapshot / family
    integrity(lambda: llm_hip.decode_disk_block(wrong, DiskIdentityInfo(first.model_hash, snap2, "qwen"), d1),
              "snapshot hash mismatch")
    integrity(lambda: llm_hip.decode_disk_block(wrong, DiskIdentityInfo(first.model_hash, snap1, "gemma"), d1),
              "model family mismatch")
    llm_hip.decode_disk_block(wrong, first, d1)


def test_decode_validation_failures():
    ns = namespace("v", "qwen")
    ident, d, enc, _ = encode_both(ns, "qwen", [filled_layer()], np.array([1.0, 2.0], np.float32))
    # descriptor fields
    for field, value in (("block_start", 2), ("token_count", 3)):
        e = llm_hip.DiskBlockDescriptor.from_buffer_copy(d)
        setattr(e, field, value)
        integrity(lambda: llm_hip.decode_disk_block(enc, ident, e), "descriptor mismatch")
    for field in ("namespace_hash", "previous_block_hash", "block_hash"):
        e = llm_hip.DiskBlockDescriptor.from_buffer_copy(d)
        setattr(e, field, b"f" * 64)
        integrity(lambda: llm_hip.decode_disk_block(enc, ident, e), "descriptor mismatch")
    # metadata rewrites
    integrity(lambda: llm_hip.decode_disk_block(ref.rewrite_metadata(enc, codec="other"), ident, d),
              "unsupported disk cache codec")
    integrity(lambda: llm_hip.decode_disk_block(ref.rewrite_metadata(enc, hidden_shape=[3]), ident, d),
              "hidden tensor shape does not match metadata")
    header, meta, payload = ref.read_header(enc)
    lay = dict(meta["layers"][0], cache_format="f16")
    integrity(lambda: llm_hip.decode_disk_block(ref.rewrite_metadata(enc, layers=[lay]), ident, d),
              "unsupported KV cache disk format")
    lay = dict(meta["layers"][0], shape=[2, 3, 2])
    integrity(lambda: llm_hip.decode_disk_block(ref.rewrite_metadata(enc, layers=[lay]), ident, d),
              "shape mismatch")
    lay = dict(meta["layers"][0], key_tensor="layers.0.full.missing")
    integrity(lambda: llm_hip.decode_disk_block(ref.rewrite_metadata(enc, layers=[lay]), ident, d), "not found")
    lay = dict(meta["layers"][0], kind="unknown_kind")
    integrity(lambda: DiskBlock(ref.rewrite_metadata(enc, layers=[lay])), "unknown layer kind")
    lay = {k: v for k, v in meta["layers"][0].items() if k != "revision"}
    integrity(lambda: DiskBlock(ref.rewrite_metadata(enc, layers=[lay])), "layer field")
    integrity(lambda: DiskBlock(ref.rewrite_metadata(enc, block_start=-1)), "invalid disk cache metadata")
    integrity(lambda: DiskBlock(ref.rewrite_metadata(enc, token_count=1.5)), "invalid disk cache metadata")


def raw_container(header: dict, payload: bytes = b"") -> bytes:
    hb = json.dumps(header, separators=(",", ":")).encode()
    return struct.pack("<Q", len(hb)) + hb + payload


def test_container_errors():
    ns = namespace("c", "qwen")
    _, _, enc, _ = encode_both(ns, "qwen", [filled_layer()], np.array([1.0], np.float32))
    (n,) = struct.unpack("<Q", enc[:8])
    integrity(lambda: DiskBlock(enc[:7]), "missing header length")
    integrity(lambda: DiskBlock(struct.pack("<Q", 64 * 1024 * 1024 + 1) + b"{}"), "exceeds limit")
    integrity(lambda: DiskBlock(enc[:8 + n - 1]), "header is truncated")
    integrity(lambda: DiskBlock(enc[:-1]), "payload is truncated")
    integrity(lambda: DiskBlock(b"\x02\x00\x00\x00\x00\x00\x00\x00[]"), "not an object")
    integrity(lambda: DiskBlock(b"\x03\x00\x00\x00\x00\x00\x00\x00{x}"), "invalid safetensors header json")
    integrity(lambda: DiskBlock(raw_container({"t": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}},
                                              b"\0" * 4)), "missing disk cache metadata")
    integrity(lambda: DiskBlock(raw_container({"__metadata__": {"kir_ai": "{"}})), "invalid disk cache metadata")
    header, meta, payload = ref.read_header(enc)
    mdata = header["__metadata__"]
    integrity(lambda: DiskBlock(raw_container({"__metadata__": mdata})), "has no tensors")
    bad = {"__metadata__": mdata, "hidden": {"dtype": "F16", "shape": [1], "data_offsets": [0, 4]}}
    integrity(lambda: DiskBlock(raw_container(bad, b"\0" * 4)), "is not F32")
    bad = {"__metadata__": mdata, "hidden": {"dtype": "F32", "shape": [1], "data_offsets": [4, 0]}}
    integrity(lambda: DiskBlock(raw_container(bad, b"\0" * 4)), "byte range is invalid")
    bad = {"__metadata__": mdata, "hidden": {"dtype": "F32", "shape": [1], "data_offsets": [0, 3]}}
    integrity(lambda: DiskBlock(raw_container(bad, b"\0" * 4)), "byte range is invalid")
    bad = {"__metadata__": mdata, "hidden": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}
    integrity(lambda: DiskBlock(raw_container(bad, b"\0" * 4)), "data offsets are invalid")
    bad = {"__metadata__": mdata, "hidden": {"dtype": "F32", "data_offsets": [0, 4]}}
    integrity(lambda: DiskBlock(raw_container(bad, b"\0" * 4)), "missing shape")


def test_linear_attention_layers_parse_but_do_not_restore_as_kv():
    """A Qwen hybrid block (codec.rs:329-369): layer 1 is linear attention; its
    record parses, the full-attention layers around it restore."""
    ns = namespace("hybrid", "qwen")
    ident, d, enc, _ = encode_both(ns, "qwen", [filled_layer()], np.array([1.0], np.float32))
    header, meta, payload = ref.read_header(enc)
    lin = {"kind": "qwen_linear_attention", "revision": 3, "conv_kernel_size": 2, "conv_dim": 3,
           "num_value_heads": 2, "key_head_dim": 2, "value_head_dim": 3, "token_count": 2,
           "conv_window_tensor": "layers.1.linear.conv_window",
           "recurrent_state_tensor": "layers.1.linear.recurrent_state", "conv_window_shape": [2, 3],
           "recurrent_state_shape": [2, 2, 3]}
    full2 = dict(meta["layers"][0])
    tensors = []
    for name, t in header.items():
        if name != "__metadata__":
            s, e = t["data_offsets"]
            arr = np.frombuffer(payload[s:e], "<f4")
            tensors.append((name, t["shape"], arr))
            if name.startswith("layers.0."):
                tensors.append((name.replace("layers.0.", "layers.2."), t["shape"], arr))
    tensors += [("layers.1.linear.conv_window", [2, 3], np.arange(6, dtype=np.float32)),
                ("layers.1.linear.recurrent_state", [2, 2, 3], np.arange(12, dtype=np.float32))]
    full2.update(key_tensor="layers.2.full.keys", value_tensor="layers.2.full.values")
    meta["layers"] = [meta["layers"][0], lin, full2]
    data = ref.encode_safetensors(meta, tensors)
    blk = DiskBlock(data)
    blk.validate(d, ident)
    assert blk.descriptor().n_layers == 3
    with pytest.raises(llm_hip.LlhError) as e:
        blk.layer(1)
    assert e.value.status == llm_hip.ERR_UNSUPPORTED
    assert np.array_equal(blk.layer(2).keys, filled_layer().keys)
    with pytest.raises(llm_hip.LlhError) as e:
        blk.layer(3)
    assert e.value.status == llm_hip.ERR_INVALID_SHAPE


def test_assemble_consecutive_blocks():
    """assemble_layer_kv_prefix_state_blocks / validate_contiguous_disk_blocks (codec.rs:252-322)"""
    ns = namespace("asm", "qwen")
    ident = identity_from_namespace(ns, "qwen")
    toks = list(range(1, 9))

    def block(start, n, max_tokens=8, kvh=2):
        d = descriptor(ident, ns, start, toks[:start + n])
        k = np.full((n, kvh, 3), start, np.float32)
        return DiskBlock(llm_hip.encode_disk_block(
            d, [0.0], [DiskLayerRows(DISK_LAYER_QWEN_FULL, 1, max_tokens, kvh, 3, n, start + n, k, k)]))

    b0, b1, b2 = block(0, 2), block(2, 2), block(4, 2)
    assert llm_hip.disk_blocks_assemble_check([b0, b1, b2]) == 6
    assert llm_hip.disk_blocks_assemble_check([]) == 0
    integrity(lambda: llm_hip.disk_blocks_assemble_check([b0, b2]), "not contiguous")
    integrity(lambda: llm_hip.disk_blocks_assemble_check([b1]), "not contiguous")
    integrity(lambda: llm_hip.disk_blocks_assemble_check([b0, block(2, 2, kvh=1)]), "incompatible KV block shapes")
    integrity(lambda: llm_hip.disk_blocks_assemble_check([block(0, 2, 3), block(2, 2, 3)]), "exceeds cache capacity")


def test_null_arguments():
    lib = llm_hip.load_library()
    assert lib.llh_disk_block_open(None, 0, None) == llm_hip.ERR_NULL
    assert lib.llh_disk_block_close(None) == llm_hip.ERR_NULL
    assert lib.llh_disk_hash_components(None, 0, None, None, None) == llm_hip.ERR_NULL
    assert lib.llh_kv_export_rows_f32(None, None, None, 0, None, None, None) == llm_hip.ERR_NULL
