"""The C-ABI library on the CPU: it loads, exports every function include/llm_hip.h
declares, the Python binding's struct layouts match the header, and host-only
entry points behave (no GPU compute is issued here)."""
import ctypes
import os
import re
import subprocess
import tempfile

import pytest

import llm_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "llm_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(llh_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = llm_hip.load_library()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(llm_hip.SIGNATURES), set(names) ^ set(llm_hip.SIGNATURES)


def test_library_is_built_for_gfx950():
    """The fat binary carries a gfx950 code object (and no other GPU target)."""
    data = open(llm_hip.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    others = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-f]+)", data)) - {b"gfx950"}
    assert not others, others


STRUCTS = {
    "llh_decode_desc": llm_hip.DecodeDesc,
    "llh_prefill_desc": llm_hip.PrefillDesc,
    "llh_kv_pool_info": llm_hip.PoolInfo,
    "llh_metrics": llm_hip.Metrics,
    "llh_layer_cache_state": llm_hip.LayerCacheState,
    "llh_layer_cache_rows": llm_hip.LayerCacheRows,
    "llh_block_run": llm_hip.BlockRun,
    "llh_block_pool_counts": llm_hip.BlockPoolCounts,
    "llh_paged_kv_metrics": llm_hip.PagedKvMetrics,
    "llh_cache_block_info": llm_hip.CacheBlockInfo,
    "llh_session_info": llm_hip.SessionInfo,
    "llh_prefix_hit": llm_hip.PrefixHit,
    "llh_prefix_cache_counters": llm_hip.PrefixCacheCounters,
    "llh_disk_block_descriptor": llm_hip.DiskBlockDescriptor,
    "llh_disk_identity": llm_hip.DiskIdentity,
    "llh_disk_layer": llm_hip.DiskLayer,
    "llh_disk_layer_info": llm_hip.DiskLayerInfo,
}


def test_struct_layouts_match_header():
    src = ['#include <stdio.h>', '#include <stddef.h>', '#include "llm_hip.h"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        src.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            src.append(f'  printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    src.append("  return 0; }")
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "probe.c")
        exe = os.path.join(d, "probe")
        open(c, "w").write("\n".join(src))
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    got = {}
    for line in out.splitlines():
        cname, field, val = line.split()
        got[(cname, field)] = int(val)
    for cname, py in STRUCTS.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert got[(cname, field)] == getattr(py, field).offset, (cname, field)


def test_status_codes_match_header():
    text = open(HEADER).read()
    for name, val in re.findall(r"LLH_(OK|NOT_HANDLED|ERR_[A-Z_]+)\s*=\s*(-?\d+)", text):
        assert getattr(llm_hip, name) == int(val), name
    for name, val in re.findall(r"LLH_(KV_[A-Z0-9_]+)\s*=\s*(\d+)", text):
        assert getattr(llm_hip, name) == int(val), name


def test_host_only_entry_points():
    lib = llm_hip.load_library()
    assert lib.llh_ctx_destroy(None) == llm_hip.ERR_NULL
    assert lib.llh_ctx_last_error(None) == b"null context"
    assert lib.llh_kv_pool_destroy(None) == llm_hip.ERR_NULL
    assert lib.llh_layer_cache_destroy(None) == llm_hip.ERR_NULL
    assert lib.llh_paged_decode(None, None, None, None, None, 0.0, None) == llm_hip.ERR_NULL
    assert lib.llh_block_pool_destroy(None) == llm_hip.ERR_NULL
    assert lib.llh_block_pool_create(None, None, None) == llm_hip.ERR_NULL
    out = ctypes.c_void_p()
    assert lib.llh_ctx_create(0, None) == llm_hip.ERR_NULL
    # workspace sizing is host arithmetic
    assert lib.llh_decode_workspace_bytes(0, 16, 100) == 0
    n = lib.llh_decode_workspace_bytes(32, 16, 4096)
    splits = ((4096 + 15) // 16 + 1 + 3) // 4
    assert n >= 32 * 16 * splits * (128 * 4 + 8)
    del out


def test_context_creation_without_gpu_fails_cleanly():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(llm_hip.LlhError) as e:
        llm_hip.Context(0)
    assert e.value.status == llm_hip.ERR_DEVICE


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(llm_hip, "LIB_PATH", str(tmp_path / "libllm_hip.so"))
    monkeypatch.setattr(llm_hip, "_lib", None)
    with pytest.raises(ImportError):
        llm_hip.load_library()
