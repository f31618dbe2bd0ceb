"""Benchmark of the MI355X paged-attention hot path (one JSON line on stdout).

A "step" is one batched decode pass over BASELINE configs[1] (C2): 32
sequences with context lengths uniform in [256, 4096], 16 query / 8 KV heads,
head_dim 128, bf16 K/V in 16-token blocks whose tables are a seeded
permutation of a shared pool (+10% free blocks), one new token per sequence.
K/V/Q are synthetic N(0,1) bf16 already resident in HBM when timing starts.

`value` is the decode kernel's achieved HBM bandwidth in GB/s: the algorithmic
bytes of one step (K+V rows attended, q, out, block tables, lengths) divided by
the mean step time from HIP events on the launch stream over --steps steps.
Every timed run starts from the GPU's steady state under load: before its
--warmup steps the step is repeated, untimed, for --settle-ms of wall time
(the clocks ramp up over the first 15-40 ms of sustained work after the GPU
has idled, e.g. while the host builds a workload).
`secondary` adds the other BASELINE configs (C1, C3 prefill MFMA utilisation,
C4 window decode/prefill, C5 int8/fp8 decode) measured the same way.
`cpu_baseline` times the CPU oracle (a C restatement of the reference's
single-threaded per-head loop) on the same pool, on this host, on one thread
(the reference's own setting) and, under `all_threads`, on all of this
process's host threads (at most 16); each secondary config carries the same
two timings under `cpu` (C5 and the prefills on a stated, scaled sample).

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--settle-ms 150] [--no-secondary] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kir-ai_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged decode attn: HBM GB/s (% of peak) + µs/step at B=32; prefill MFMA util"
D = 128
BT = 16
SETTLE = {"s": 0.15}  # untimed settle before each timed run (--settle-ms)
HOST = {"us": None}   # host time per call of the last time_steps run (issue loop wall time / steps)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class DecodeWorkload:
    """A paged batch resident on the device plus its descriptor."""

    def __init__(self, ctx, lens, Hq, Hkv, fmt, window=0, resident_from=None, seed=0, free_frac=0.10, head_dim=D):
        import torch
        import llm_hip
        from llm_hip import workloads

        self.torch = torch
        self.ctx = ctx
        self.Hq, self.Hkv, self.fmt, self.window = Hq, Hkv, fmt, window
        self.D = D = head_dim
        self.batch = workloads.paged_batch(lens, BT, free_frac, seed, resident_from)
        b = self.batch
        self.pool = ctx.pool(fmt, BT, Hkv, D, b.n_blocks)
        # every resident block gets N(0,1) rows, quantised on write for int8/fp8
        ids = [int(b.tables[i, j]) for i in range(b.seq_lens.size)
               for j in range(int(b.first_block[i]), (int(b.seq_lens[i]) + BT - 1) // BT)]
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        chunk = 4096
        for s in range(0, len(ids), chunk):
            idx = torch.tensor(ids[s:s + chunk], dtype=torch.int32, device="cuda")
            n = idx.numel()
            k = torch.randn((n, BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
            v = torch.randn((n, BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
            ctx.write_blocks(self.pool, idx, k, v)
        B = b.seq_lens.size
        self.q = torch.randn((B, Hq, D), generator=g, device="cuda").to(torch.bfloat16)
        self.out = torch.empty_like(self.q)
        self.d_lens = torch.from_numpy(b.seq_lens).cuda()
        self.d_tab = torch.from_numpy(b.tables).cuda()
        rows, _ = self.attended_rows()
        self.desc = ctx.decode_desc(self.d_lens, self.d_tab, Hq, int(b.seq_lens.max()), window,
                                    total_tokens_hint=int(rows.sum()))
        self.scale = 1.0 / math.sqrt(D)
        torch.cuda.synchronize()
        if ctx.device_errors() != 0:
            raise RuntimeError("device error flags set while building the workload")
        self.llm_hip = llm_hip
        self._bound = {}

    def attended_rows(self):
        import numpy as np

        lens = np.asarray(self.batch.seq_lens).astype(np.int64)
        lo = np.maximum(0, lens - self.window) if self.window > 0 else np.zeros_like(lens)
        return lens - lo, lo

    def algorithmic_bytes(self) -> int:
        return decode_bytes(self.batch.seq_lens, self.Hq, self.Hkv, self.fmt, self.window, self.D)

    def bound(self, key, name, *args):
        """The C call `name` with its arguments converted once (Context.bind), per stream."""
        f = self._bound.get(key)
        if f is None:
            f = self._bound[key] = self.ctx.bind(name, *args)
        return f

    def step(self, stream):
        self.bound(("decode", stream), "llh_paged_decode", self.pool, self.desc, self.q, self.out, self.scale,
                   stream)()

    def prepare_append(self):
        """The new token of every sequence (position len-1): its pool slot and N(0,1) K/V rows."""
        import numpy as np

        b = self.batch
        lens = b.seq_lens.astype(np.int64)
        pos = lens - 1
        blocks = b.tables[np.arange(lens.size), (pos // BT) % b.max_blocks].astype(np.int64)
        self.d_slots = self.torch.from_numpy(blocks * BT + pos % BT).cuda()
        g = self.torch.Generator(device="cuda")
        g.manual_seed(int(lens.sum()))
        self.k_new = self.torch.randn((lens.size, self.Hkv, self.D), generator=g, device="cuda").to(self.torch.bfloat16)
        self.v_new = self.torch.randn((lens.size, self.Hkv, self.D), generator=g, device="cuda").to(self.torch.bfloat16)

    def append_step(self, stream):
        """kir-ai's decode step order (native_attention.rs:307-329): append the new token, then attend."""
        self.bound(("append", stream), "llh_kv_append", self.pool, self.d_slots, self.k_new, self.v_new,
                   self.d_slots.numel(), stream)()
        self.step(stream)

    def fused_step(self, stream):
        """The same step as append_step in one call (llh_paged_decode_append)."""
        self.bound(("fused", stream), "llh_paged_decode_append", self.pool, self.desc, self.k_new, self.v_new, self.q,
                   self.out, self.scale, stream)()

    def append_bytes(self) -> int:
        """Algorithmic bytes of the append: the new rows read (bf16) and written (pool format), slots."""
        B = self.batch.seq_lens.size
        elem = 2 if self.fmt in (self.llm_hip.KV_BF16, self.llm_hip.KV_F16) else 1
        scales = B * self.Hkv * 2 * 2 if self.fmt == self.llm_hip.KV_INT8 else 0
        return B * self.Hkv * self.D * 2 * 2 + B * self.Hkv * self.D * elem * 2 + scales + B * 8


def settle(fn, stream, seconds: float) -> None:
    """Repeats the step, untimed, for `seconds` of wall time with the GPU kept
    busy (at most three batches of 8 steps queued ahead): after an idle spell
    the GPU's clocks ramp up over the first 15-40 ms of sustained load (C2 step
    48.8 -> 47.3 us, C5 fp8 240 -> 187 us), so a run timed from a cold start
    measures the ramp, not the kernels."""
    import torch

    t0 = time.perf_counter()
    pending = []
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn(stream)
        e = torch.cuda.Event()
        e.record(stream)
        pending.append(e)
        if len(pending) > 3:
            pending.pop(0).synchronize()


def time_steps(fn, steps: int, warmup: int, kernel_timing=None):
    """Mean ms per step from HIP events recorded on the launch stream.

    The timed steps follow a settle phase (`settle`) and `warmup` untimed steps.
    With kernel_timing = (ctx, kind), the library also records HIP events around
    its main kernel in every timed step (same stream); returns (step ms, kernel ms)."""
    import torch

    stream = torch.cuda.Stream()  # default priority
    settle(fn, stream, SETTLE["s"])
    for _ in range(warmup):
        fn(stream)
    torch.cuda.synchronize()
    if kernel_timing:
        kernel_timing[0].kernel_time(kernel_timing[1], reset=True)
        kernel_timing[0].set_kernel_timing(True)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    t0 = time.perf_counter()
    for _ in range(steps):
        fn(stream)
    HOST["us"] = round((time.perf_counter() - t0) / steps * 1e6, 2)  # the host's issue cost per call
    e1.record(stream)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    if not kernel_timing:
        return step_ms
    kernel_timing[0].set_kernel_timing(False)
    total, n = kernel_timing[0].kernel_time(kernel_timing[1], reset=True)
    return step_ms, total / max(n, 1)


def time_graph(fns, replays: int, min_calls: int = 128):
    """Mean ms per step of a HIP graph holding the calls fn(stream) of fns, in order,
    repeated until it holds at least min_calls of them (a graph launch costs about as much
    as ten small kernels, so short graphs would time the launch), replayed `replays` times
    after a settle phase: the GPU's own time per step, without the host's per-call launch
    cost."""
    import torch

    fns = list(fns) * max(1, -(-min_calls // len(fns)))
    replays = max(3, replays // len(fns) + 1)
    s = torch.cuda.Stream()  # default priority
    for f in fns:  # eager once, outside the capture
        f(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f in fns:
            f(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < SETTLE["s"]:
            g.replay()
            s.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(s)
        for _ in range(replays):
            g.replay()
        e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (replays * len(fns))
    del g
    return ms


def cpu_baseline_decode(w: DecodeWorkload, budget_s: float):
    """Times the oracle (single-threaded reference loop) on whole decode steps of the same pool."""
    import numpy as np
    import oracle

    b = w.batch
    opool = oracle.Pool.from_raw(w.fmt, BT, w.Hkv, D, b.n_blocks, w.pool.raw())
    q = w.q.view(w.torch.int16).cpu().numpy().view(np.uint16).ravel()
    reps, t0 = 0, time.perf_counter()
    while True:
        st, _ = opool.decode(w.Hq, b.seq_lens, b.tables, w.window, q, w.scale, threads=1)
        if st != 0:
            raise RuntimeError(f"oracle decode failed: {st}")
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 20:
            break
    sec_per_step = el / reps
    return {
        "value": round(w.algorithmic_bytes() / sec_per_step / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{reps} full C2 decode step(s) (32 seqs x 16 heads) of the oracle's per-head loop, "
                  f"single thread, {el:.1f} s; {sec_per_step * 1e6:.0f} us/step",
        "us_per_step": round(sec_per_step * 1e6, 1),
        "host": host_info(),
    }


def host_threads() -> int:
    """Threads of the all-cores CPU timing: this process's CPU set, at most 16 (one GPU's share of the box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _timed(fn, budget_s: float, max_reps: int = 20) -> tuple[float, int]:
    """Mean seconds per call of fn over at least one call, until budget_s or max_reps."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= max_reps:
            return el / reps, reps


def cpu_decode_times(w: DecodeWorkload, budget_s: float, sample_seqs: int = 0) -> dict:
    """The oracle's decode step on w's pool on 1 thread and on all host threads.  With
    sample_seqs > 0 (workloads whose sequences all have one length) each call decodes the
    first sample_seqs sequences and the time is scaled by B / sample_seqs."""
    import numpy as np
    import oracle

    b = w.batch
    B = b.seq_lens.size
    k = B if sample_seqs <= 0 else min(B, sample_seqs)
    opool = oracle.Pool.from_raw(w.fmt, BT, w.Hkv, D, b.n_blocks, w.pool.raw())
    q = w.q.view(w.torch.int16).cpu().numpy().view(np.uint16).ravel()[: k * w.Hq * D]
    lens, tabs = b.seq_lens[:k], b.tables[:k]
    res = {"threads": host_threads(), "sample": f"{k} of {B} sequences per call" + ("" if k == B else f", scaled x{B / k:g}")}
    for key, th in (("us_per_step_1_thread", 1), ("us_per_step_all_threads", res["threads"])):
        def call():
            st, _ = opool.decode(w.Hq, lens, tabs, w.window, q, w.scale, threads=th)
            if st != 0:
                raise RuntimeError(f"oracle decode failed: {st}")
        sec, reps = _timed(call, budget_s)
        res[key] = round(sec * B / k * 1e6, 1)
        res[key.replace("us_per_step", "calls")] = reps
    res["gbs_all_threads"] = round(w.algorithmic_bytes() / (res["us_per_step_all_threads"] * 1e-6) / 1e9, 3)
    res["tokens_per_s_all_threads"] = round(B / (res["us_per_step_all_threads"] * 1e-6), 1)
    return res


def cpu_prefill_times(keep, B: int, prefix: int, chunk: int, Hq: int, Hkv: int, window: int, rows: int,
                      budget_s: float) -> dict:
    """The oracle's prefill on `rows` query rows of sequence 0 (the middle of its chunk), on 1 thread
    and on all host threads, scaled to the whole step by the count of unmasked (query, key) pairs
    (the oracle's work is proportional to it)."""
    import numpy as np
    import oracle
    import llm_hip

    pool, q, out, starts, clens, tab = keep
    opool = oracle.Pool.from_raw(llm_hip.KV_BF16, BT, Hkv, D, int(pool.info.n_blocks), pool.raw())
    qh = q.view(torch_int16()).cpu().numpy().view(np.uint16).ravel()
    cs, cl, tb = starts.cpu().numpy(), clens.cpu().numpy(), tab.cpu().numpy()
    lo_row = (chunk - rows) // 2
    pairs = lambda i: (prefix + i) - (max(0, prefix + i - window + 1) if window > 0 else 0) + 1
    scale_up = B * sum(pairs(i) for i in range(chunk)) / sum(pairs(i) for i in range(lo_row, lo_row + rows))
    buf = np.zeros(int(cs[-1]) * Hq * D, dtype=np.float32)
    res = {"threads": host_threads(), "sample": f"rows {lo_row}..{lo_row + rows - 1} of sequence 0, all {Hq} heads, "
                                                f"scaled x{scale_up:.1f} by unmasked (query, key) pairs"}
    for key, th in (("us_per_step_1_thread", 1), ("us_per_step_all_threads", res["threads"])):
        def call():
            st = opool.prefill_rows(0, Hq, cs, cl, tb, window, qh, 1.0 / math.sqrt(D), lo_row, lo_row + rows, buf,
                                    threads=th)
            if st != 0:
                raise RuntimeError(f"oracle prefill failed: {st}")
        sec, reps = _timed(call, budget_s, max_reps=5)
        res[key] = round(sec * scale_up * 1e6, 1)
        res[key.replace("us_per_step", "calls")] = reps
    res["tokens_per_s_all_threads"] = round(B * chunk / (res["us_per_step_all_threads"] * 1e-6), 1)
    return res


def torch_int16():
    import torch

    return torch.int16


def host_info() -> str:
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{model} (nproc={os.cpu_count()})"


def prefill_case(ctx, B, prefix, chunk, Hq, Hkv, window, seed, resident_from_pos=None, fmt=None, head_dim=D):
    """Prefill workload: B sequences of prefix + chunk tokens, all K/V resident (bf16 pool
    unless fmt names a quantised one)."""
    import torch
    import llm_hip
    from llm_hip import workloads

    D = head_dim
    fmt = llm_hip.KV_BF16 if fmt is None else fmt
    ctxlen = prefix + chunk
    lens = [ctxlen] * B
    first = None if resident_from_pos is None else [resident_from_pos // BT] * B
    batch = workloads.paged_batch(lens, BT, 0.10, seed, first)
    pool = ctx.pool(fmt, BT, Hkv, D, batch.n_blocks)
    ids = [int(batch.tables[i, j]) for i in range(B) for j in range(int(batch.first_block[i]), (ctxlen + BT - 1) // BT)]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    idx = torch.tensor(ids, dtype=torch.int32, device="cuda")
    k = torch.randn((len(ids), BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((len(ids), BT, Hkv, D), generator=g, device="cuda").to(torch.bfloat16)
    ctx.write_blocks(pool, idx, k, v)
    del k, v
    q = torch.randn((B * chunk, Hq, D), generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    starts = torch.tensor([i * chunk for i in range(B + 1)], dtype=torch.int32, device="cuda")
    clens = torch.tensor(lens, dtype=torch.int32, device="cuda")
    tab = torch.from_numpy(batch.tables).cuda()
    desc = ctx.prefill_desc(starts, clens, tab, Hq, chunk, window, total_q_rows=B * chunk)
    keep = (pool, q, out, starts, clens, tab)
    scale = 1.0 / math.sqrt(D)

    def step(stream):
        ctx.paged_prefill(pool, desc, q, out, scale, stream=stream)

    # FLOPs of unmasked (query, key) pairs only: 4 * D per pair per head
    pairs = 0
    for i in range(chunk):
        pos = prefix + i
        lo = max(0, pos - window + 1) if window > 0 else 0
        pairs += pos - lo + 1
    flops = 4 * D * pairs * Hq * B
    return step, flops, keep


def measure_neighbours(ctx, steps: int, warmup: int) -> list:
    """The steps either side of decode attention, at C2's shape: the new token's K/V append
    (32 rows into 16-token blocks; bf16, and int8 quantised on write) and the o_proj of
    Qwen3-0.6B (W bf16 1024 x 2048, 32 attention outputs), alone and fused behind the decode.
    W rotates over copies totalling > 2 x 256 MB so each step reads it from HBM."""
    import numpy as np
    import torch
    import llm_hip
    from llm_hip import workloads

    out = []
    g = torch.Generator(device="cuda")
    g.manual_seed(workloads.SEED_BASE + 7)
    B, Hkv, Hq = 32, 8, 16
    # decode: the C2 batch's 32 new tokens (one row per sequence, scattered slots);
    # prefill: C3's 8 x 512-token chunks, whole 16-token blocks (llh_kv_write_blocks), and
    # the same chunks at the Qwen3.6 shape (head_dim 256, Hkv 2, bf16)
    for fmt, nm, hd, H, shape, kern in (
            (llm_hip.KV_BF16, "bf16", D, 4, "C3", "write_blocks_d128_kernel"),
            (llm_hip.KV_INT8, "int8", D, 4, "C3", "write_blocks_d128_kernel"),
            (llm_hip.KV_FP8_E4M3, "fp8", D, 4, "C3", "write_blocks_d128_kernel"),
            (llm_hip.KV_F16, "fp16", D, 4, "C3", "write_blocks_d128_kernel"),
            (llm_hip.KV_BF16, "bf16, head_dim 256", 256, 2, "Q36", "write_blocks16_d256_kernel")):
        nblk = 8 * 512 // BT
        pool = ctx.pool(fmt, BT, H, hd, 8192)
        ids = torch.randperm(8192, generator=g, device="cuda")[:nblk].to(torch.int32)
        k = torch.randn((nblk, BT, H, hd), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((nblk, BT, H, hd), generator=g, device="cuda").to(torch.bfloat16)
        ms = time_steps(lambda s: ctx.write_blocks(pool, ids, k, v, stream=s), steps, warmup)
        host_us = HOST["us"]
        # the same write replayed from a HIP graph (the GPU's own time per call, which a
        # slow host's issue time can hide); writing the same rows again leaves the pool as it was
        before = pool.raw()
        gms = time_graph([lambda s: ctx.write_blocks(pool, ids, k, v, stream=s)], steps)
        if any(not np.array_equal(a, b) for a, b in zip(before.values(), pool.raw().values())):
            raise RuntimeError("block write: graph replay changed the pool")
        esz = 2 if fmt in (llm_hip.KV_BF16, llm_hip.KV_F16) else 1
        T = nblk * BT
        scales = {llm_hip.KV_INT8: T * H * 2 * 2, llm_hip.KV_FP8_E4M3: nblk * H * 4 * 2}.get(fmt, 0)
        nbytes = T * H * hd * 2 * 2 + T * H * hd * esz * 2 + nblk * 4 + scales
        out.append({"config": f"KV write {shape} prefill chunks ({nblk} blocks = {T} tokens, Hkv{H}, {nm})",
                    "us_per_step": round(ms * 1e3, 2), "host_us_per_call": host_us, "bytes_per_step": nbytes,
                    "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "graph_us_per_step": round(gms * 1e3, 2),
                    "graph_hbm_frac": round(nbytes / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "kernel": kern})
        del pool
    for fmt, nm, T, H in ((llm_hip.KV_BF16, "bf16", B, Hkv), (llm_hip.KV_INT8, "int8", B, Hkv),
                          (llm_hip.KV_FP8_E4M3, "fp8", B, Hkv), (llm_hip.KV_F16, "fp16", B, Hkv)):
        pool = ctx.pool(fmt, BT, H, D, 8192)
        slots = torch.randperm(8192 * BT, generator=g, device="cuda")[:T].to(torch.int64)
        k = torch.randn((T, H, D), generator=g, device="cuda").to(torch.bfloat16)
        v = torch.randn((T, H, D), generator=g, device="cuda").to(torch.bfloat16)
        ms = time_steps(lambda s: ctx.append(pool, slots, k, v, stream=s), steps, warmup)
        host_us = HOST["us"]
        # the same append replayed from a HIP graph (the GPU's own time per call); appending the
        # same rows again leaves the pool as it was, which the replay must reproduce
        before = pool.raw()
        gms = time_graph([lambda s: ctx.append(pool, slots, k, v, stream=s)], steps)
        if any(not np.array_equal(a, b) for a, b in zip(before.values(), pool.raw().values())):
            raise RuntimeError("append: graph replay changed the pool")
        esz = 2 if fmt in (llm_hip.KV_BF16, llm_hip.KV_F16) else 1
        # fp8: the block's scale is read and written per token (an earlier row re-encode is not counted)
        scales = {llm_hip.KV_INT8: T * H * 2 * 2, llm_hip.KV_FP8_E4M3: T * H * 4 * 2 * 2}.get(fmt, 0)
        nbytes = T * H * D * 2 * 2 + T * H * D * esz * 2 + T * 8 + scales
        out.append({"config": f"KV append C2 batch ({T} tokens, Hkv{H}, {nm})", "us_per_step": round(ms * 1e3, 2),
                    "host_us_per_call": host_us, "graph_us_per_step": round(gms * 1e3, 2), "bytes_per_step": nbytes, "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                    "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "kernel": "append_kernel (launch-bound at this size)"})
        if ctx.device_errors() != 0:
            raise RuntimeError("append: device error flags set")
        del pool
    rows, cols = 1024, Hq * D
    wbytes = rows * cols * 2
    ws = [torch.randn((rows, cols), generator=g, device="cuda").to(torch.bfloat16)
          for _ in range(2 * LLC_BYTES // wbytes + 2)]
    x = torch.randn((B, cols), generator=g, device="cuda").to(torch.bfloat16)
    y = torch.empty((B, rows), dtype=torch.float32, device="cuda")
    st = {"i": 0}

    def proj(s):
        ctx.matvec_bf16(ws[st["i"] % len(ws)], rows, cols, x, B, y, stream=s)
        st["i"] += 1

    ms = time_steps(proj, steps, warmup)
    nbytes = wbytes + B * cols * 2 + B * rows * 4
    out.append({"config": f"o_proj matvec W {rows}x{cols} bf16, {B} rows", "us_per_step": round(ms * 1e3, 2),
                "host_us_per_call": HOST["us"],
                "bytes_per_step": nbytes, "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "w_copies": len(ws),
                "kernel": "matvec_bf16_kernel (MFMA)"})
    lens = list(workloads.uniform_lengths(B, 256, 4096, workloads.SEED_BASE + 1))
    w = DecodeWorkload(ctx, lens, Hq, Hkv, llm_hip.KV_BF16, seed=workloads.SEED_BASE + 3)
    st["i"] = 0

    def fused(s):
        ctx.paged_decode_output_projection(w.pool, w.desc, w.q, ws[st["i"] % len(ws)], rows, y, w.scale, stream=s)
        st["i"] += 1

    ms_f = time_steps(fused, steps, warmup)
    ms_d = time_steps(lambda s: w.step(s), steps, warmup)
    out.append({"config": "C2 decode + o_proj fused (llh_paged_decode_output_projection)", "us_per_step": round(ms_f * 1e3, 2),
                "decode_alone_us": round(ms_d * 1e3, 2), "projection_added_us": round((ms_f - ms_d) * 1e3, 2),
                "note": "one pool copy: the K/V of consecutive steps may be partly cache resident"})
    if ctx.device_errors() != 0:
        raise RuntimeError("o_proj: device error flags set")
    del w, ws
    torch.cuda.empty_cache()
    return out


def measure_trait_c1(ctx, calls: int, cpu_seconds: float, with_cpu: bool) -> dict:
    """Per-call latency of the trait hook full_attention_cache_mix_f32_in_place
    (native_matvec.rs:656-668) on a C1-shaped layer cache (512 tokens, 8 kv heads x 128,
    16 query heads): the synchronous call kir-ai makes once per layer per token, host
    timed end to end (f32 q in, f32 out), on the tuned kernels and on the reference-order
    kernel, with the reference's CPU loop (the oracle) on the same rows beside it."""
    import numpy as np
    import llm_hip
    import oracle

    rng = np.random.default_rng(0x6B69722D00)
    cache = llm_hip.LayerKvCache.new(ctx, 512, 8, D)
    backend = llm_hip.HipNativeMatvecBackend(ctx)
    for _ in range(512):
        k = rng.standard_normal(8 * D).astype(np.float32)
        v = rng.standard_normal(8 * D).astype(np.float32)
        backend.append_kv_cache_sliding_f32(cache, k, v)
    q = rng.standard_normal(16 * D).astype(np.float32)
    out = np.zeros(16 * D, np.float32)
    res = {"config": "trait hook full_attention_cache_mix_f32_in_place, C1 cache (512 x Hkv8 x 128, Hq16), per call",
           "calls": calls}
    saved = ctx.get_option(llm_hip.OPT_TRAIT_REFERENCE_ORDER)
    for key, ref_order in (("tuned_us_per_call", 0), ("reference_order_us_per_call", 1)):
        ctx.set_option(llm_hip.OPT_TRAIT_REFERENCE_ORDER, ref_order)
        for _ in range(10):
            backend.full_attention_cache_mix_f32_in_place(cache, q, 512, 16, 8, D, 0.0883883, out)
        t0 = time.perf_counter()
        for _ in range(calls):
            backend.full_attention_cache_mix_f32_in_place(cache, q, 512, 16, 8, D, 0.0883883, out)
        res[key] = round((time.perf_counter() - t0) / calls * 1e6, 2)
    ctx.set_option(llm_hip.OPT_TRAIT_REFERENCE_ORDER, saved)
    res["tuned_calls_counted"] = ctx.metrics()["trait_tuned_calls"] >= calls
    if with_cpu:
        keys, vals = cache.keys(), cache.values()
        sec, reps = _timed(lambda: oracle.attention_mix(q, keys, vals, 512, 16, 8, D, 0.0883883), cpu_seconds, 200)
        res["cpu_oracle_us_per_call"] = round(sec * 1e6, 1)
        res["cpu_threads"] = 1
    cache.close()
    return res


def measure_copy(mb: int) -> dict:
    """A plain device-to-device copy of `mb` MiB: the measured bandwidth ceiling, and the
    known-size kernel that calibrates the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = mb * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    def step(stream):
        with torch.cuda.stream(stream):
            dst.copy_(src)

    ms = time_steps(step, 20, 3)
    return {"bytes": 2 * n, "us": round(ms * 1e3, 2), "gbs": round(2 * n / (ms * 1e-3) / 1e9, 1)}


LLC_BYTES = 256 << 20  # MI355X Infinity Cache (memory-side last-level cache)


def measure_decode(ctx, name, lens, Hq, Hkv, fmt, steps, warmup, window=0, resident_from=None, seed=0, free=0.10,
                   append=False, fused=False, graph=False, head_dim=D):
    """Mean step time over `steps` decode steps.  Steps rotate over enough independent
    copies of the workload (same lengths, own pool, own block permutation and data) that
    the bytes read between two visits of one copy exceed the 256 MB Infinity Cache: every
    step reads its K/V from HBM, not from cache.  append=True times kir-ai's whole decode
    step instead: the new token's K/V append, then attention over the cache holding it.  fused=True
    times the same step through llh_paged_decode_append (one call).  graph=True also times
    the step replayed from a HIP graph (llh_paged_decode_noalloc, one call per copy): the
    GPU's own time per step, free of the host's per-call launch cost, which sets the pace of
    small steps issued one call at a time (host_us_per_call)."""
    first = DecodeWorkload(ctx, lens, Hq, Hkv, fmt, window, resident_from, seed, free, head_dim)
    nbytes = first.algorithmic_bytes() + (first.append_bytes() if append or fused else 0)
    copies = [first]
    while (len(copies) - 1) * nbytes < 2 * LLC_BYTES:
        copies.append(DecodeWorkload(ctx, lens, Hq, Hkv, fmt, window, resident_from, seed + 1000 * len(copies), free,
                                     head_dim))
    if append or fused:
        for c in copies:
            c.prepare_append()
    state = {"i": 0}

    def step(stream):
        c = copies[state["i"] % len(copies)]
        if fused:
            c.fused_step(stream)
        elif append:
            c.append_step(stream)
        else:
            c.step(stream)
        state["i"] += 1

    # step time over all timed steps, then the decode kernel alone (library-recorded events)
    streamed0, calls0 = ctx.metrics()["stream_decode_calls"], state["i"]
    ms = time_steps(step, steps, warmup)
    host_us = HOST["us"]
    streamed, calls = ctx.metrics()["stream_decode_calls"] - streamed0, state["i"] - calls0
    _, kms = time_steps(step, steps, 0, kernel_timing=(ctx, "decode"))
    if ctx.device_errors() != 0:
        raise RuntimeError(f"{name}: device error flags set during timing")
    gbs = nbytes / (ms * 1e-3) / 1e9
    # the event pair around the main kernel also spans its dispatch; a figure above the step
    # time is not a kernel duration and is not reported (rocprof's trace gives the duration)
    kernel_ok = kms <= ms
    extra = {}
    if graph:
        import torch

        def noalloc(c):
            return lambda s: ctx.paged_decode_noalloc(c.pool, c.desc, c.q, c.out, c.scale, stream=s)

        eager = []
        for c in copies:
            c.step(torch.cuda.current_stream())
        torch.cuda.synchronize()
        eager = [c.out.clone() for c in copies]
        # the no-allocation entry runs split-K where the stream kernel's partials exceed
        # its static scratch: then its replay would time another kernel
        noalloc(first)(torch.cuda.current_stream())
        torch.cuda.synchronize()
        if not torch.equal(first.out, eager[0]):
            extra = {"graph_us_per_step": None,
                     "graph_note": "llh_paged_decode_noalloc runs split-K for this step (the stream kernel's "
                                   "partials exceed its scratch): no graph figure for the eager kernel"}
        else:
            gms = time_graph([noalloc(c) for c in copies], steps)
            same = all(torch.equal(c.out, e) for c, e in zip(copies, eager))
            if not same or ctx.device_errors() != 0:
                raise RuntimeError(f"{name}: graph replay output differs from the eager call")
            extra = {"graph_us_per_step": round(gms * 1e3, 2),
                     "graph_hbm_frac": round(nbytes / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return first, {
        "config": name,
        "us_per_step": round(ms * 1e3, 2),
        "kernel_us": round(kms * 1e3, 2) if kernel_ok else None,
        "kernel_gbs": round(first.algorithmic_bytes() / (kms * 1e-3) / 1e9, 1) if kernel_ok else None,
        "hbm_gbs": round(gbs, 1),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(len(lens) / (ms * 1e-3), 1),
        "bytes_per_step": nbytes,
        "rotating_copies": len(copies),
        "kernel": (("paged_decode_d256_stream_kernel" if head_dim == 256 else "paged_decode_stream_kernel")
                   if streamed == calls else
                   "paged_decode_d256_kernel (split-K)" if head_dim == 256 else "paged_decode_kernel (split-K)"),
        "host_us_per_call": host_us,
        **extra,
    }


def decode_bytes(lens, Hq: int, Hkv: int, fmt: int, window: int = 0, head_dim: int = D) -> int:
    """Algorithmic bytes of one decode step: K and V of every attended position (+ int8 /
    fp8 scales), q and out, the block-table entries read and the lengths."""
    import numpy as np

    lens = np.asarray(lens, np.int64)
    lo = np.maximum(0, lens - window) if window > 0 else np.zeros_like(lens)
    rows = lens - lo
    elem = 2 if fmt in (0, 4) else 1  # bf16, fp16: 2 bytes; int8, fp8: 1
    kv = int(rows.sum()) * Hkv * head_dim * elem * 2
    blocks = ((lens + BT - 1) // BT) - lo // BT
    scales = int(rows.sum()) * Hkv * 4 if fmt == 1 else (int(blocks.sum()) * Hkv * 8 if fmt == 2 else 0)
    return kv + scales + 2 * lens.size * Hq * head_dim * 2 + int(blocks.sum()) * 4 + lens.size * 4


def prefill_flops(B: int, prefix: int, chunk: int, Hq: int, window: int, head_dim: int = D) -> int:
    """4 * head_dim FLOPs per unmasked (query, key) pair per head."""
    pairs = 0
    for i in range(chunk):
        pos = prefix + i
        lo = max(0, pos - window + 1) if window > 0 else 0
        pairs += pos - lo + 1
    return 4 * head_dim * pairs * Hq * B


def summarize(root: str) -> int:
    """Writes profiles/*.md from rocprofv3 csv output: ROOT/<section>/kt (--kernel-trace --stats),
    ROOT/<section>/fetch and /write (--pmc FETCH_SIZE, --pmc WRITE_SIZE) and, where present,
    ROOT/<section>/ctr (one --pmc pass of other counters: MFMA for prefill, issue and wait
    cycles for decode), each made by `bench.py --only <section>`.  FETCH_SIZE and WRITE_SIZE
    are scaled by what they read for the run's own 512 MiB copy."""
    import csv
    import glob
    import statistics
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "kir-ai_amd"))
    from llm_hip import workloads

    def short(n):
        n = n.replace("void ", "").replace("llh::(anonymous namespace)::", "").replace("llh::", "")
        return n.split("(")[0].strip()

    def rows_of(sec, sub, suffix):
        out = []
        for f in glob.glob(os.path.join(root, sec, sub, "**", "*" + suffix), recursive=True):
            out.extend(csv.DictReader(open(f)))
        return out

    c2lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    c2b = decode_bytes(c2lens, 16, 8, 0)
    append_b = 32 * 8 * D * 2 * 2 * 2 + 32 * 8  # bf16 rows read and written, K and V, slots
    alg = {  # section -> {kernel prefix: (unit, amount)}
        "c2": {"paged_decode_stream_kernel": ("B", c2b)},
        "c2append": {"paged_decode_stream_kernel": ("B", c2b), "append_kernel": ("B", append_b)},
        "c2fused": {"paged_decode_stream_kernel": ("B", c2b + append_b)},
        "c1": {"paged_decode_kernel": ("B", decode_bytes([512], 16, 8, 0))},
        "c4": {"paged_decode_kernel": ("B", decode_bytes([32768] * 4, 16, 8, 0, 4096))},
        "c5int8": {"paged_decode_stream_kernel": ("B", decode_bytes([8192] * 64, 32, 8, 1))},
        "c5fp8": {"paged_decode_stream_kernel": ("B", decode_bytes([8192] * 64, 32, 8, 2))},
        "c2f16": {"paged_decode_stream_kernel": ("B", decode_bytes(c2lens, 16, 8, 4))},
        "c3f16": {"paged_prefill_kernel": ("F", prefill_flops(8, 1536, 512, 32, 0))},
        "q36f16": {"paged_decode_d256_stream_kernel": ("B", decode_bytes(c2lens, 16, 2, 4, 0, 256)),
                   "paged_decode_d256_kernel": ("B", decode_bytes(c2lens, 16, 2, 4, 0, 256))},
        "q36prefillf16": {"paged_prefill_d256_kernel": ("F", prefill_flops(8, 1536, 512, 16, 0, 256))},
        "q36": {"paged_decode_d256_stream_kernel": ("B", decode_bytes(c2lens, 16, 2, 0, 0, 256)),
                "paged_decode_d256_kernel": ("B", decode_bytes(c2lens, 16, 2, 0, 0, 256))},
        "q36prefill": {"paged_prefill_d256_kernel": ("F", prefill_flops(8, 1536, 512, 16, 0, 256))},
        "c3": {"paged_prefill_kernel": ("F", prefill_flops(8, 1536, 512, 32, 0))},
        "c3int8": {"paged_prefill_kernel": ("F", prefill_flops(8, 1536, 512, 32, 0))},
        "c3fp8": {"paged_prefill_kernel": ("F", prefill_flops(8, 1536, 512, 32, 0))},
        "c4prefill": {"paged_prefill_kernel": ("F", prefill_flops(4, 31744, 1024, 16, 4096))},
        "neighbours": {"matvec_bf16_kernel": ("B", 1024 * 2048 * 2 + 32 * 2048 * 2 + 32 * 1024 * 4)},
    }
    groups = (
        ("decode_c2_bf16.md", "Paged GQA decode, C2 (B=32, L~U[256,4096], Hq16/Hkv8, bf16 KV), and kir-ai's step "
                              "order (append the new token, then attend: two calls, and one call)", ("c2", "c2append", "c2fused")),
        ("decode_c1_c4_bf16.md", "Paged GQA decode, C1 (B=1, L=512) and C4 (4 x 32768, window 4096), bf16 KV",
         ("c1", "c4")),
        ("decode_c5_int8_fp8.md", "Quantized-KV decode, C5 (B=64, L=8192, Hq32/Hkv8): int8 (fp16 per (token, head) "
                                  "scales) and fp8 e4m3 (per (block, head) scales)", ("c5int8", "c5fp8")),
        ("f16_kv.md", "fp16 KV pools (the reference's Metal mirror dtype): decode on C2 (B=32, L~U[256,4096], "
                      "Hq16/Hkv8) and prefill on C3 (8 x (1536 + 512), Hq32/Hkv4); the Qwen3.6 head_dim-256 shape "
                      "(Hq16/Hkv2) on the same lengths", ("c2f16", "c3f16", "q36f16", "q36prefillf16")),
        ("decode_q36_d256.md", "Paged GQA decode at head_dim 256, the Qwen3.6 full-attention shape (Hq16/Hkv2, "
                               "bf16 KV): decode on C2's lengths (B=32, L~U[256,4096]) and prefill on C3's chunking "
                               "(8 x (1536 + 512))", ("q36", "q36prefill")),
        ("prefill_mfma.md", "Chunked causal prefill (MFMA): C3 (8 x (1536 + 512), Hq32/Hkv4) over bf16, int8 and fp8 "
                            "blocks, C4 (4 x (31744 + 1024), window 4096)", ("c3", "c3int8", "c3fp8", "c4prefill")),
        ("kv_write_oproj.md", "KV writes (whole blocks, per-token append) and the output projection",
         ("neighbours",)),
    )
    med = statistics.median
    wrote = 0
    for fname, title, secs in groups:
        body, cmds, cal_notes = "", [], []
        for sec in secs:
            if not os.path.isdir(os.path.join(root, sec)):
                continue
            run = f"python3 /root/repo/bench.py --only {sec} --no-cpu"
            cmds.append(f"    cd /tmp && rocprofv3 --kernel-trace --stats --output-format csv -d <dir>/{sec}/kt -o run -- {run}")
            tr = {}
            for r in rows_of(sec, "kt", "kernel_trace.csv"):
                k = (short(r["Kernel_Name"]), int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]))
                tr.setdefault(k, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
            ctr = {}
            for sub in ("fetch", "write", "ctr"):
                got = rows_of(sec, sub, "counter_collection.csv")
                if got and sub != "ctr":
                    cmds.append(f"    cd /tmp && rocprofv3 --pmc {sub.upper()}_SIZE --output-format csv "
                                f"-d <dir>/{sec}/{sub} -o run -- {run} --steps 10 --warmup 2 --settle-ms 20")
                elif got:
                    names = sorted({r["Counter_Name"] for r in got})
                    cmds.append(f"    cd /tmp && rocprofv3 --pmc {' '.join(names)} --output-format csv "
                                f"-d <dir>/{sec}/{sub} -o run -- {run} --steps 10 --warmup 2 --settle-ms 20")
                for r in got:
                    k = (short(r["Kernel_Name"]), int(r["Grid_Size"]))
                    ctr.setdefault((k, r["Counter_Name"]), []).append(float(r["Counter_Value"]))
            copies = [k for (k, c) in ctr if k[0].startswith("__amd_rocclr_copyBuffer") and c == "FETCH_SIZE"]
            fcal = wcal = None
            if copies:
                ck = max(copies, key=lambda k: med(ctr[(k, "FETCH_SIZE")]))
                fcal = 512 * 1024 / med(ctr[(ck, "FETCH_SIZE")])
                wcal = 512 * 1024 / med(ctr[(ck, "WRITE_SIZE")]) if (ck, "WRITE_SIZE") in ctr else None
                cal_notes.append(f"{sec}: FETCH_SIZE x{fcal:.4f}" + (f", WRITE_SIZE x{wcal:.4f}" if wcal else ""))
            for k in sorted(tr, key=lambda k: -med(tr[k])):
                if not k[0] or k[0].startswith("__amd") or "::" in k[0] or "elementwise" in k[0] or k[0].startswith(
                        "_ZN") or k[0].startswith("Cijk"):
                    continue  # the copy, torch's and rocprim's kernels of the set-up
                d = tr[k]
                unit = next((v for pfx, v in alg.get(sec, {}).items() if k[0].startswith(pfx)), None)
                rate = "-"
                if unit and unit[0] == "B":
                    rate = f"{unit[1] / (med(d) * 1e-6) / 1e9:.0f} GB/s"
                elif unit:
                    tf = unit[1] / (med(d) * 1e-6) / 1e12
                    rate = f"{tf:.1f} TFLOP/s = {100 * tf / BF16_PEAK_TFLOPS:.1f}% of 2.5 PF"
                f = ctr.get((k, "FETCH_SIZE"))
                w = ctr.get((k, "WRITE_SIZE"))
                traffic = (med(f) * fcal + (med(w) * wcal if w and wcal else 0)) * 1024 if f and fcal else None
                ratio = f"{traffic / unit[1]:.3f}" if traffic and unit and unit[0] == "B" else "-"
                body += (f"| {sec.upper() if sec != 'c2' else 'C2'} | `{k[0]}` | {k[1]} | {len(d)} | {med(d):.2f} | "
                         f"{statistics.mean(d):.2f} | {unit[1] if unit else '-'} | {rate} | "
                         f"{med(f) if f else float('nan'):.0f} | {med(w) if w else float('nan'):.0f} | "
                         f"{traffic if traffic else float('nan'):.0f} | {ratio} |\n")
            mf = [(k, c) for (k, c) in ctr if not c.endswith("_SIZE") and not k[0].startswith("__amd")
                  and "::" not in k[0] and not k[0].startswith("_ZN")]  # library kernels of the set-up and checks
            for k, c in sorted(mf):
                body += f"| {sec.upper()} | `{k[0]}` | {k[1]} | counter `{c}` | {med(ctr[(k, c)]):.4g} per dispatch |  |  |  |  |  |  |  |\n"
            for k in sorted({k for (k, c) in mf}):
                g = {c: med(ctr[(k, c)]) for (kk, c) in mf if kk == k}
                if "SQ_WAVE_CYCLES" in g and "SQ_ACTIVE_INST_ANY" in g:
                    wc = g["SQ_WAVE_CYCLES"]
                    body += (f"| {sec.upper()} | `{k[0]}` | {k[1]} | derived | of wave cycles: issuing "
                             f"{100 * g['SQ_ACTIVE_INST_ANY'] / wc:.0f} %, waiting on counters / barrier "
                             f"{100 * g.get('SQ_WAIT_ANY', 0) / wc:.0f} %, waiting to issue "
                             f"{100 * g.get('SQ_WAIT_INST_ANY', 0) / wc:.0f} %, VALU active "
                             f"{100 * g.get('SQ_ACTIVE_INST_VALU', 0) / wc:.0f} %; VALU instructions per vector "
                             f"load {g.get('SQ_INSTS_VALU', 0) / max(g.get('SQ_INSTS_VMEM_RD', 1), 1):.1f} "
                             f"|  |  |  |  |  |  |  |\n")
        if not body:
            continue
        text = (f"# {title}\n\nMI355X (gfx950), rocprofv3 from ROCm 7.2.  Made by `python bench.py --summarize <dir>` "
                f"from the csv output of these commands (run on the GPU box; <dir> is the output root):\n\n"
                + "\n".join(cmds) + "\n\nCounter scale factors from each run's own 512 MiB device copy "
                "(`__amd_rocclr_copyBuffer`, 512 MiB read and written): " + "; ".join(cal_notes) + ".\n\n"
                "| section | kernel | grid (work-items) | dispatches | median us | mean us | algorithmic bytes or FLOPs "
                "per dispatch | rate at the median | FETCH KiB/dispatch (raw) | WRITE KiB/dispatch (raw) | "
                "HBM bytes/dispatch (scaled) | HBM traffic / algorithmic bytes |\n"
                "|---|---|---|---|---|---|---|---|---|---|---|---|\n" + body)
        with open(os.path.join(ROOT, "profiles", fname), "w") as fh:
            fh.write(text)
        wrote += 1
        log(f"wrote profiles/{fname}")
    return 0 if wrote else 1


def traffic_from_profile(kernel: str):
    """HBM bytes per launch of the C2 decode kernel from the committed rocprofv3 --pmc summary
    (FETCH_SIZE and WRITE_SIZE, each scaled by the copy-kernel calibration; written by
    `bench.py --summarize`), or None."""
    path = os.path.join(ROOT, "profiles", "decode_c2_bf16.md")
    try:
        for line in open(path):
            cells = [c.strip() for c in line.split("|")]
            if len(cells) > 12 and cells[1] == "C2" and cells[2].strip("`").startswith(kernel):
                return int(float(cells[11]))
    except (OSError, ValueError):
        pass
    return None


# sections of the secondary measurements (--only runs one, for a profiler run)
SECTIONS = ("c1", "c2", "c2append", "c2fused", "c4", "c5int8", "c5fp8", "q36", "neighbours", "trait", "c3", "c4prefill",
            "c3int8", "c3fp8", "q36prefill", "c2f16", "c3f16", "q36f16", "q36prefillf16")


def run_sections(ctx, args, lens, sel) -> list:
    """The secondary measurements: all of them, or the one --only names."""
    import torch
    import llm_hip
    from llm_hip import workloads

    secondary = []
    # secondaries time at least 100 steps whatever --steps is (the driver passes few)
    sec_steps, sec_warm = max(100, args.steps), max(10, args.warmup)
    if sel("c1"):
        w1, r = measure_decode(ctx, "C1 B=1 L=512", [512], 16, 8, llm_hip.KV_BF16, sec_steps, sec_warm,
                               seed=workloads.SEED_BASE, free=0.0, graph=True)
        if not args.no_cpu:
            r["cpu"] = cpu_decode_times(w1, 1.0)
        del w1
        secondary.append(r)
        log(f"C1: {r}")
    if sel("c2append"):
        _, r = measure_decode(ctx, "C2 append + attend (kir-ai's step order: llh_kv_append then llh_paged_decode)",
                              lens, 16, 8, llm_hip.KV_BF16, sec_steps, sec_warm, seed=workloads.SEED_BASE + 1,
                              append=True)
        secondary.append(r)
        log(f"C2 append+attend: {r}")
        torch.cuda.empty_cache()
    if sel("c2fused"):
        _, r = measure_decode(ctx, "C2 append + attend in one call (llh_paged_decode_append)", lens, 16, 8,
                              llm_hip.KV_BF16, sec_steps, sec_warm, seed=workloads.SEED_BASE + 1, fused=True)
        secondary.append(r)
        log(f"C2 fused append+attend: {r}")
        torch.cuda.empty_cache()
    if sel("c4"):
        L, W = 32768, 4096
        _, r = measure_decode(ctx, "C4 decode 4x32768 W=4096", [L] * 4, 16, 8, llm_hip.KV_BF16, sec_steps,
                              sec_warm, window=W, resident_from=[(L - W) // BT] * 4, seed=workloads.SEED_BASE + 3,
                              graph=True)
        secondary.append(r)
        log(f"C4 decode: {r}")
    for fmt, nm in ((llm_hip.KV_INT8, "int8"), (llm_hip.KV_FP8_E4M3, "fp8")):
        if not sel("c5" + nm):
            continue
        wq, r = measure_decode(ctx, f"C5 decode {nm} B=64 L=8192 Hq32/Hkv8", [8192] * 64, 32, 8, fmt,
                               sec_steps, sec_warm, seed=workloads.SEED_BASE + 4, free=0.0)
        if not args.no_cpu:
            r["cpu"] = cpu_decode_times(wq, 1.0, sample_seqs=4)
        secondary.append(r)
        log(f"C5 {nm}: {r}")
        del wq
        torch.cuda.empty_cache()
        # kir-ai's step order on the same shape: append the new token (quantised), then attend, in one call
        _, r = measure_decode(ctx, f"C5 {nm} append + attend in one call (llh_paged_decode_append)", [8192] * 64, 32,
                              8, fmt, sec_steps, sec_warm, seed=workloads.SEED_BASE + 4, free=0.0, fused=True)
        r["decode_alone_us"] = secondary[-1]["us_per_step"]
        # int8: the stream kernel quantises the token itself (+ merge); fp8: the append
        # kernel (slots from the descriptor), then the stream kernel and merge
        r["launches"] = 2 if fmt == llm_hip.KV_INT8 else 3
        secondary.append(r)
        log(f"C5 {nm} fused append+attend: {r}")
        torch.cuda.empty_cache()
    if sel("q36"):
        # Qwen3.6 full-attention layer (fixtures/qwen36/config.json: Hq16 / Hkv2, head_dim 256) on C2's
        # lengths, bf16 blocks: the head_dim-256 kernel
        _, r = measure_decode(ctx, "Q36 decode B=32 L~U[256,4096] Hq16/Hkv2 D=256", lens, 16, 2, llm_hip.KV_BF16,
                              sec_steps, sec_warm, seed=workloads.SEED_BASE + 5, graph=True, head_dim=256)
        secondary.append(r)
        log(f"Q36 decode: {r}")
        # kir-ai's step order on the same shape, in one call: the append kernel, then the stream kernel
        _, r = measure_decode(ctx, "Q36 append + attend in one call (llh_paged_decode_append)", lens, 16, 2,
                              llm_hip.KV_BF16, sec_steps, sec_warm, seed=workloads.SEED_BASE + 5, fused=True,
                              head_dim=256)
        r["decode_alone_us"] = secondary[-1]["us_per_step"]
        secondary.append(r)
        log(f"Q36 append+attend: {r}")
    if sel("c2f16"):
        # C2's shape over an fp16 pool (the element type of the reference's Metal KV mirror)
        _, r = measure_decode(ctx, "C2 decode over fp16 blocks", lens, 16, 8, llm_hip.KV_F16, sec_steps, sec_warm,
                              seed=workloads.SEED_BASE + 1)
        secondary.append(r)
        log(f"C2 f16: {r}")
        torch.cuda.empty_cache()
    if sel("q36f16"):
        # the Qwen3.6 full-attention shape over an fp16 pool: the head_dim-256 kernel, fp16 instance
        _, r = measure_decode(ctx, "Q36 decode over fp16 blocks", lens, 16, 2, llm_hip.KV_F16, sec_steps, sec_warm,
                              seed=workloads.SEED_BASE + 5, graph=True, head_dim=256)
        secondary.append(r)
        log(f"Q36 f16: {r}")
        # append + attend in one call over the fp16 pool (the stream kernel's fused instance)
        _, r = measure_decode(ctx, "Q36 fp16 append + attend in one call (llh_paged_decode_append)", lens, 16, 2,
                              llm_hip.KV_F16, sec_steps, sec_warm, seed=workloads.SEED_BASE + 5, fused=True,
                              head_dim=256)
        r["decode_alone_us"] = secondary[-1]["us_per_step"]
        secondary.append(r)
        log(f"Q36 f16 append+attend: {r}")
        torch.cuda.empty_cache()
    if sel("neighbours"):
        secondary.extend(measure_neighbours(ctx, sec_steps, sec_warm))
    if sel("trait"):
        r = measure_trait_c1(ctx, 200, 2.0, not args.no_cpu)
        secondary.append(r)
        log(f"trait C1: {r}")
    for key, name, B, prefix, chunk, Hq, Hkv, window, res, fmt, hd in (
            ("c3", "C3 prefill 8x(1536+512) Hq32/Hkv4", 8, 1536, 512, 32, 4, 0, None, llm_hip.KV_BF16, D),
            ("c4prefill", "C4 prefill 4x(31744+1024) W=4096", 4, 31744, 1024, 16, 8, 4096, 31744 - 4096,
             llm_hip.KV_BF16, D),
            ("c3int8", "C3 prefill over int8 blocks", 8, 1536, 512, 32, 4, 0, None, llm_hip.KV_INT8, D),
            ("c3fp8", "C3 prefill over fp8 blocks", 8, 1536, 512, 32, 4, 0, None, llm_hip.KV_FP8_E4M3, D),
            ("c3f16", "C3 prefill over fp16 blocks", 8, 1536, 512, 32, 4, 0, None, llm_hip.KV_F16, D),
            # Qwen3.6 full-attention layer (Hq16 / Hkv2, head_dim 256) on C3's chunking: the head_dim-256 kernel
            ("q36prefill", "Q36 prefill 8x(1536+512) Hq16/Hkv2 D=256", 8, 1536, 512, 16, 2, 0, None, llm_hip.KV_BF16,
             256),
            ("q36prefillf16", "Q36 prefill over fp16 blocks", 8, 1536, 512, 16, 2, 0, None, llm_hip.KV_F16, 256)):
        if not sel(key):
            continue
        step, flops, keep = prefill_case(ctx, B, prefix, chunk, Hq, Hkv, window, workloads.SEED_BASE + 2, res, fmt,
                                         hd)
        pms = time_steps(step, sec_steps, sec_warm)
        host_us = HOST["us"]
        _, pkms = time_steps(step, sec_steps, 0, kernel_timing=(ctx, "prefill"))
        if ctx.device_errors() != 0:
            raise RuntimeError(f"{name}: device error flags set")
        tf = flops / (pms * 1e-3) / 1e12
        r = {"config": name, "us_per_step": round(pms * 1e3, 2),
             "kernel_us": round(pkms * 1e3, 2) if pkms <= pms else None, "tflops": round(tf, 1),
             "mfma_util": round(tf / BF16_PEAK_TFLOPS, 4), "tokens_per_s": round(B * chunk / (pms * 1e-3), 1),
             "flops_per_step": flops, "host_us_per_call": host_us}
        if not args.no_cpu and fmt == llm_hip.KV_BF16 and hd == D:
            r["cpu"] = cpu_prefill_times(keep, B, prefix, chunk, Hq, Hkv, window, 16, 1.0)
        secondary.append(r)
        log(f"{name}: {r}")
        del keep
        torch.cuda.empty_cache()
    return secondary


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--settle-ms", type=float, default=150.0,
                    help="untimed wall time of repeated steps before each timed run (GPU clock ramp)")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-mb", type=int, default=512,
                    help="size of the plain device copy that measures the copy-bandwidth ceiling (0 = skip)")
    ap.add_argument("--only", choices=sorted(SECTIONS),
                    help="run one measurement (and the copy that calibrates the counters) for a profiler run; "
                         "prints its record instead of the headline line")
    ap.add_argument("--summarize", metavar="DIR",
                    help="write profiles/*.md from rocprofv3 csv output under DIR/<section>/{kt,fetch,write,ctr}")
    args = ap.parse_args()
    if args.summarize:
        return summarize(args.summarize)
    SETTLE["s"] = max(0.0, args.settle_ms / 1e3)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode (the batch shards by sequence with "
              "no communication). Run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import llm_hip
    from llm_hip import workloads

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    ctx = llm_hip.Context(0)
    only = args.only

    def sel(name):
        return only is None or only == name

    lens = workloads.uniform_lengths(32, 256, 4096, workloads.SEED_BASE + 1)
    if only is not None and only != "c2":
        records = run_sections(ctx, args, lens, sel)
        if args.copy_mb > 0:
            records.append({"copy": measure_copy(args.copy_mb)})
        print(json.dumps({"only": only, "records": records}), flush=True)
        ctx.close()
        return 0

    # ---- headline: C2 batched paged decode ----
    log(f"C2 decode: B=32 sum(L)={int(lens.sum())}")
    w, c2 = measure_decode(ctx, "C2", lens, 16, 8, llm_hip.KV_BF16, args.steps, args.warmup,
                           seed=workloads.SEED_BASE + 1, graph=True)
    ms = c2["us_per_step"] / 1e3
    value = c2["hbm_gbs"]
    log(f"C2: {c2['us_per_step']} us/step, {value} GB/s ({100 * value / HBM_PEAK_GBS:.1f}% of 8 TB/s); "
        f"decode kernel {c2['kernel_us']} us = {c2['kernel_gbs']} GB/s")

    copy = None
    if args.copy_mb > 0:
        copy = measure_copy(args.copy_mb)
        log(f"device copy {args.copy_mb} MiB: {copy['gbs']} GB/s (read + write)")

    cpu = None
    if not args.no_cpu:
        log("CPU baseline (oracle, 1 thread) on the C2 pool ...")
        cpu = cpu_baseline_decode(w, args.cpu_seconds)
        log(f"CPU: {cpu['us_per_step']} us/step")
        mt = cpu_decode_times(w, 3.0)
        cpu["all_threads"] = {k: mt[k] for k in ("threads", "us_per_step_all_threads", "gbs_all_threads", "calls_all_threads")}
        log(f"CPU, {mt['threads']} threads: {mt['us_per_step_all_threads']} us/step")
    del w
    torch.cuda.empty_cache()

    secondary = [] if args.no_secondary or only == "c2" else run_sections(ctx, args, lens, sel)

    line = {
        "metric": METRIC,
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 K/V/Q resident in HBM; seeded lengths and block permutation; steps rotate over "
                "independent copies so each step reads beyond the 256 MB Infinity Cache",
        "config": {
            "workload": "C2 batched paged GQA decode: B=32, L~U[256,4096] (seeded), Hq=16, Hkv=8, D=128, "
                        "bf16 KV in 16-token blocks, permuted pool +10% free, 1 new token/seq",
            "global_batch": 32,
            "sum_context_tokens": int(lens.sum()),
            "hbm_frac_of_peak": round(value / HBM_PEAK_GBS, 4),
            "us_per_step": c2["us_per_step"],
            "host_us_per_call": c2["host_us_per_call"],
            "graph_us_per_step": c2["graph_us_per_step"],
            "tokens_per_s": c2["tokens_per_s"],
            "bytes_per_step": c2["bytes_per_step"],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{c2['kernel']}, G=2, bf16 (the merge launch is excluded)"
                      if c2["kernel_gbs"] else "the whole step (kernel events exceeded the step time)",
            "achieved": c2["kernel_gbs"] or c2["hbm_gbs"],
            "kernel_us": c2["kernel_us"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round((c2["kernel_gbs"] or c2["hbm_gbs"]) / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profile(c2["kernel"].split(" ")[0]),
        },
        "cpu_baseline": cpu,
        "copy_ceiling": copy,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
