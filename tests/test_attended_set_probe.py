"""The position-coded probe (tests/attended_set.py) on the CPU oracle: it reads the
oracle's own attended set exactly, and it fails for each plausible gather / mask
mistake planted in the oracle's inputs -- a duplicated block (a table entry
pointing at the next block), a dropped block, a window one position wider or
narrower, one token past the end attended -- so a GPU kernel passing the probe
attends exactly the reference's set."""
import numpy as np
import pytest

import oracle
from attended_set import BT, D, check_decode, check_prefill, coded_rows, code, counts
from llm_hip import workloads

Q_HEADS, KV_HEADS = 8, 4


def coded_pool(lens, seed, max_blocks=None):
    batch = workloads.paged_batch(lens, BT, 0.10, seed)
    tables = batch.tables
    rows_k = [oracle.normal_bf16(seed, int(L) * KV_HEADS * D).reshape(int(L), KV_HEADS, D) for L in lens]
    rows_v = [coded_rows(0, int(L), KV_HEADS) for L in lens]
    pool = oracle.build_bf16_pool(rows_k, rows_v, tables, lens, BT, KV_HEADS, D, batch.n_blocks)
    return pool, batch


def decode_q0(pool, lens, tables, window):
    q = np.zeros(len(lens) * Q_HEADS * D, np.uint16)
    st, out = pool.decode(Q_HEADS, lens, tables, window, q, 0.1)
    assert st == oracle.OK
    return oracle.f32_to_bf16(out)


def test_codes_are_balanced_and_tell_blocks_apart():
    pos = np.arange(8192)
    for h in range(4):
        c = np.bincount(code(pos, h), minlength=D)
        assert c.max() == c.min() == 64, h
    # the folded code separates blocks 128 apart, which the plain block code cannot
    assert code(np.array([5 * 16]), 0) == code(np.array([133 * 16]), 0)
    assert code(np.array([5 * 16]), 2) != code(np.array([133 * 16]), 2)
    assert counts(0, 4096, 4).sum(axis=1).tolist() == [4096] * 4


@pytest.mark.parametrize("window", [0, 17, 100])
def test_probe_reads_the_oracle_decode_set(window):
    lens = np.array([1, 16, 17, 333, 1000], np.int32)
    pool, batch = coded_pool(lens, 5)
    check_decode(decode_q0(pool, lens, batch.tables, window), lens, window, Q_HEADS, KV_HEADS, 1.0, "oracle")


def test_probe_catches_a_duplicated_block():
    lens = np.array([1000], np.int32)
    pool, batch = coded_pool(lens, 6)
    bad = batch.tables.copy()
    bad[0, 20] = bad[0, 21]  # block 20's entry points at block 21: its data read twice, block 20 never
    with pytest.raises(AssertionError):
        check_decode(decode_q0(pool, lens, bad, 0), lens, 0, Q_HEADS, KV_HEADS, 1.0)


def test_probe_catches_a_block_read_instead_of_the_one_128_blocks_away():
    """Blocks j and j + 128 carry the same block code and the same token codes; the
    folded code tells them apart."""
    lens = np.array([4096], np.int32)
    pool, batch = coded_pool(lens, 7)
    bad = batch.tables.copy()
    bad[0, 3] = batch.tables[0, 131]
    with pytest.raises(AssertionError):
        check_decode(decode_q0(pool, lens, bad, 0), lens, 0, Q_HEADS, KV_HEADS, 1.0)


def test_probe_catches_the_window_edge_block_swapped_with_an_inner_one():
    """Swapping two wholly attended blocks leaves the attended set (and any attention
    output) unchanged; swapping the partly masked first block of a window with an inner
    one masks the wrong tokens, which the probe sees."""
    lens = np.array([1000], np.int32)
    pool, batch = coded_pool(lens, 12)
    swapped = batch.tables.copy()
    swapped[0, 57], swapped[0, 60] = batch.tables[0, 60], batch.tables[0, 57]
    check_decode(decode_q0(pool, lens, swapped, 100), lens, 100, Q_HEADS, KV_HEADS, 1.0)
    edge = batch.tables.copy()
    edge[0, 56], edge[0, 60] = batch.tables[0, 60], batch.tables[0, 56]  # block 56 holds the window start (900)
    with pytest.raises(AssertionError):
        check_decode(decode_q0(pool, lens, edge, 100), lens, 100, Q_HEADS, KV_HEADS, 1.0)


def test_probe_catches_a_dropped_block():
    L = 2048
    lens = np.array([L], np.int32)
    pool, batch = coded_pool(lens, 8)
    st, keys, vals = pool.gather_f32(batch.tables[0], 0, L)
    assert st == oracle.OK
    keep = np.ones(L, bool)
    keep[16 * 50:16 * 51] = False  # block 50 never read
    n = int(keep.sum())
    vl = KV_HEADS * D
    st, out = oracle.attention_mix(np.zeros(Q_HEADS * D, np.float32), keys.reshape(L, vl)[keep].ravel(),
                                   vals.reshape(L, vl)[keep].ravel(), n, Q_HEADS, KV_HEADS, D, 0.1)
    assert st == oracle.OK
    with pytest.raises(AssertionError):
        check_decode(oracle.f32_to_bf16(out), lens, 0, Q_HEADS, KV_HEADS, 1.0)


@pytest.mark.parametrize("window,shift", [(100, 1), (100, -1), (4096, 1), (4096, -1)])
def test_probe_catches_a_window_off_by_one(window, shift):
    lens = np.array([5000, 777], np.int32)
    pool, batch = coded_pool(lens, 9)
    with pytest.raises(AssertionError):
        check_decode(decode_q0(pool, lens, batch.tables, window + shift), lens, window, Q_HEADS, KV_HEADS, 1.0)


def test_probe_catches_a_token_past_the_end():
    lens = np.array([70], np.int32)  # the last block has room: slot 70 holds position 70's code
    pool, batch = coded_pool(np.array([71], np.int32), 10)
    with pytest.raises(AssertionError):
        check_decode(decode_q0(pool, lens + 1, batch.tables, 0), lens, 0, Q_HEADS, KV_HEADS, 1.0)
    check_decode(decode_q0(pool, lens, batch.tables, 0), lens, 0, Q_HEADS, KV_HEADS, 1.0)


@pytest.mark.parametrize("window", [0, 40])
def test_probe_reads_the_oracle_prefill_set_and_catches_a_shifted_window(window):
    prefix, chunk = 100, 37
    lens = np.array([prefix + chunk, prefix + chunk], np.int32)
    pool, batch = coded_pool(lens, 11)
    starts = np.array([0, chunk, 2 * chunk], np.int32)
    q = np.zeros(2 * chunk * Q_HEADS * D, np.uint16)
    st, out = pool.prefill(Q_HEADS, starts, lens, batch.tables, window, q, 0.1)
    assert st == oracle.OK
    check_prefill(oracle.f32_to_bf16(out), starts, lens, window, Q_HEADS, KV_HEADS, 1.0, "oracle prefill")
    if window:
        st, out = pool.prefill(Q_HEADS, starts, lens, batch.tables, window + 1, q, 0.1)
        with pytest.raises(AssertionError):
            check_prefill(oracle.f32_to_bf16(out), starts, lens, window, Q_HEADS, KV_HEADS, 1.0)
