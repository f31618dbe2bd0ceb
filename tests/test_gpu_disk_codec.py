"""Persisting device KV to the on-disk block format and restoring it.

* llh_kv_export_rows_f32: the f32 rows a disk block holds, read from bf16,
  int8 and fp8 pools through permuted block tables, bit for bit equal to the
  oracle's dequantising gather of the same pool bytes.
* write -> read -> restore: a 300-token sequence in two layer pools is written
  as 128-token disk blocks (the reference persists whole blocks only,
  native_text/disk_cache.rs:356-418), the files are read back, validated,
  joined and appended into fresh pools under a different block permutation
  (llh_kv_append_f32).  The restored rows equal the originals bit for bit
  (bf16 rows are exact in f32; int8 rows requantise to the same codes and
  scales, since every row's largest code is 127) and paged decode over the
  restored pools returns the same bits as over the originals.
"""
import math

import numpy as np
import pytest

import llm_hip
import oracle
from helpers import rows_bf16, to_dev
from llm_hip import DISK_LAYER_QWEN_FULL, DiskBlock, DiskIdentityInfo, DiskLayerRows, workloads

pytestmark = pytest.mark.gpu

BT = 16


def slots_of(table: np.ndarray, lo: int, hi: int) -> np.ndarray:
    p = np.arange(lo, hi, dtype=np.int64)
    return table[p // BT].astype(np.int64) * BT + p % BT


def export(ctx, pool, slots: np.ndarray, Hkv: int, D: int):
    import torch

    k = torch.empty(slots.size * Hkv * D, dtype=torch.float32, device="cuda")
    v = torch.empty_like(k)
    ctx.export_rows_f32(pool, to_dev(slots), k, v)
    torch.cuda.synchronize()
    return k.cpu().numpy(), v.cpu().numpy()


def fill(ctx, fmt, lens, Hkv, D, seed):
    batch = workloads.paged_batch(lens, BT, 0.1, seed)
    ids, sk = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 1, b, lo, hi, Hkv, D), Hkv, D)
    _, sv = workloads.block_sources(batch, lambda b, lo, hi: rows_bf16(seed + 2, b, lo, hi, Hkv, D), Hkv, D)
    pool = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
    ctx.write_blocks(pool, to_dev(ids), to_dev(sk), to_dev(sv))
    return batch, pool


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8, llm_hip.KV_FP8_E4M3])
def test_export_rows_match_oracle_gather(ctx, fmt):
    Hkv, D = 4, 128
    batch, pool = fill(ctx, fmt, [3, 16, 33, 700], Hkv, D, 300 + fmt)
    opool = oracle.Pool.from_raw(fmt, BT, Hkv, D, batch.n_blocks, pool.raw())
    for b, L in enumerate(batch.seq_lens):
        for lo, hi in ((0, int(L)), (int(L) // 3, int(L))):
            k, v = export(ctx, pool, slots_of(batch.tables[b], lo, hi), Hkv, D)
            st, rk, rv = opool.gather_f32(batch.tables[b], lo, hi)
            assert st == oracle.OK
            assert np.array_equal(k.view(np.uint32), rk.view(np.uint32)), (fmt, b, lo, hi)
            assert np.array_equal(v.view(np.uint32), rv.view(np.uint32)), (fmt, b, lo, hi)
    assert ctx.device_errors() == 0


def test_export_flags_bad_slots(ctx):
    Hkv, D = 2, 64
    batch, pool = fill(ctx, llm_hip.KV_BF16, [40], Hkv, D, 7)
    export(ctx, pool, np.array([0, batch.n_blocks * BT], np.int64), Hkv, D)
    assert ctx.device_errors() & llm_hip.ERR_FLAG_BAD_BLOCK


@pytest.mark.parametrize("fmt", [llm_hip.KV_BF16, llm_hip.KV_INT8])
def test_device_kv_round_trips_through_disk_blocks(ctx, tmp_path, fmt):
    import torch

    Hkv, D, Hq = 8, 128, 16
    L, disk_bt, n_layers = 300, 128, 2
    persisted = (L // disk_bt) * disk_bt
    tokens = list(range(9000, 9000 + L))
    src = [fill(ctx, fmt, [L], Hkv, D, 500 + 10 * i) for i in range(n_layers)]
    ns_hash = llm_hip.disk_hash_components("kir-ai-native-text-disk-namespace/v1", [("cache_key", "device-test")])
    snap = llm_hip.native_text_disk_snapshot_hash("manifest:sha256:device-test")
    ident = DiskIdentityInfo(llm_hip.native_text_disk_model_hash("m", "hip", snap), snap, "qwen", ns_hash)
    hidden = np.linspace(-1, 1, 32, dtype=np.float32)

    # write: one file per disk block, every layer's rows exported from its pool
    paths = []
    for start in range(0, persisted, disk_bt):
        d = llm_hip.disk_block_descriptor(ident, ns_hash, 1, start, tokens[:start + disk_bt])
        layers = []
        for batch, pool in src:
            k, v = export(ctx, pool, slots_of(batch.tables[0], start, start + disk_bt), Hkv, D)
            layers.append(DiskLayerRows(DISK_LAYER_QWEN_FULL, start + disk_bt, 4096, Hkv, D, disk_bt,
                                        start + disk_bt, k.reshape(disk_bt, Hkv, D), v.reshape(disk_bt, Hkv, D)))
        p = tmp_path / llm_hip.disk_block_path(d)
        p.parent.mkdir(parents=True, exist_ok=True)
        p.write_bytes(llm_hip.encode_disk_block(d, hidden, layers))
        paths.append((d, p))

    # read: validate each block against its expected descriptor, join, restore into fresh pools
    blocks = []
    for start, (d, p) in zip(range(0, persisted, disk_bt), paths):
        expect = llm_hip.disk_block_descriptor(ident, ns_hash, 1, start, tokens[:start + disk_bt])
        blk = DiskBlock(p.read_bytes())
        blk.validate(expect, ident)
        blocks.append(blk)
    assert llm_hip.disk_blocks_assemble_check(blocks) == persisted
    assert np.array_equal(blocks[-1].hidden(), hidden)
    dst = []
    for li in range(n_layers):
        batch = workloads.paged_batch([persisted], BT, 0.5, 900 + li)  # another permutation, a larger pool
        pool = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
        for start, blk in zip(range(0, persisted, disk_bt), blocks):
            rows = blk.layer(li)
            assert (rows.token_count, rows.key_value_heads, rows.head_dim) == (disk_bt, Hkv, D)
            ctx.append_f32(pool, to_dev(slots_of(batch.tables[0], start, start + disk_bt)),
                           to_dev(rows.keys.ravel()), to_dev(rows.values.ravel()))
        dst.append((batch, pool))
    torch.cuda.synchronize()
    assert ctx.device_errors() == 0

    # the restored rows are the original rows, bit for bit (codes and, through the f32 view, scales)
    esz = 2 if fmt == llm_hip.KV_BF16 else 1
    for (sb, sp), (db, dp) in zip(src, dst):
        a = export(ctx, sp, slots_of(sb.tables[0], 0, persisted), Hkv, D)
        b = export(ctx, dp, slots_of(db.tables[0], 0, persisted), Hkv, D)
        assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
        assert np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
        so = oracle.Pool.from_raw(fmt, BT, Hkv, D, sb.n_blocks, sp.raw())
        do = oracle.Pool.from_raw(fmt, BT, Hkv, D, db.n_blocks, dp.raw())
        for tensor in (0, 1):
            st1, r1 = so.gather_raw(sb.tables[0], 0, persisted, tensor)
            st2, r2 = do.gather_raw(db.tables[0], 0, persisted, tensor)
            assert st1 == st2 == oracle.OK
            assert np.array_equal(r1.view(np.uint8), r2.view(np.uint8)), tensor
        assert r1.size * esz == persisted * Hkv * D * esz

    # decode over the restored prefix == decode over the original, bit for bit
    q = oracle.normal_bf16(77, Hq * D)
    scale = 1.0 / math.sqrt(D)
    outs = []
    for batch, pool in (src[0], dst[0]):
        lens = np.array([persisted], np.int32)
        desc = ctx.decode_desc(to_dev(lens), to_dev(batch.tables[:, :persisted // BT].copy()), Hq, persisted)
        out = torch.empty(Hq * D, dtype=torch.int16, device="cuda")
        ctx.paged_decode(pool, desc, to_dev(q), out, scale)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    assert ctx.device_errors() == 0
    for blk in blocks:
        blk.close()
