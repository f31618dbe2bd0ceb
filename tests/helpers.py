"""Test helpers: seeded inputs, device upload, and the parity bar."""
from __future__ import annotations

import numpy as np

import oracle

MAXPOS = 1 << 20  # PRNG stride between sequences (positions per sequence)


def rows_bf16(seed: int, b: int, lo: int, hi: int, kv_heads: int, head_dim: int) -> np.ndarray:
    """Token rows [hi-lo][kv_heads][head_dim] bf16 bits of sequence b (seeded, N(0,1))."""
    n = (hi - lo) * kv_heads * head_dim
    off = (b * MAXPOS + lo) * kv_heads * head_dim
    return oracle.normal_bf16(seed, n, off).reshape(hi - lo, kv_heads, head_dim)


# query magnitudes from bf16 subnormal to 1e30, zero included
MAGNITUDES = np.array([1.0, 1e-30, 6.0, 1e-3, 1e-39, 0.0, 3e4, 1e30], np.float32)


def magnitude_rows(q_bf16: np.ndarray, heads: int, head_dim: int) -> np.ndarray:
    """q (bf16 bits, rows x heads x head_dim) with (row, head) scaled by MAGNITUDES in turn
    and dim 3 of every 7th row 100x its row: rows and heads of very different size side
    by side (scores up to ~1e31 in log2 units)."""
    qf = oracle.bf16_to_f32(q_bf16.ravel()).reshape(-1, heads, head_dim).copy()
    rows = qf.shape[0]
    qf *= MAGNITUDES[(np.arange(rows)[:, None] + np.arange(heads)[None, :]) % MAGNITUDES.size][:, :, None]
    qf[::7, :, 3] *= np.float32(100.0)
    return oracle.f32_to_bf16(qf.ravel())


def to_dev(a: np.ndarray):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def from_dev_bf16(t) -> np.ndarray:
    return t.cpu().numpy().view(np.uint16)


def assert_parity(gpu_bf16: np.ndarray, ref_f32: np.ndarray, max_abs: float = 2e-2, mean_abs: float = 2e-3,
                  what: str = ""):
    """BASELINE bar: bf16 output (fp32 accumulation) within max-abs 2e-2 and mean-abs 2e-3
    of the reference fp32 result rounded to bf16."""
    g = oracle.bf16_to_f32(gpu_bf16.ravel())
    r = oracle.bf16_to_f32(oracle.f32_to_bf16(ref_f32.ravel()))
    assert g.shape == r.shape, (g.shape, r.shape)
    assert np.all(np.isfinite(g)), f"{what}: non-finite GPU output"
    d = np.abs(g - r)
    assert d.max() <= max_abs and d.mean() <= mean_abs, (
        f"{what}: max-abs {d.max():.3e} (bar {max_abs}), mean-abs {d.mean():.3e} (bar {mean_abs})")
    return float(d.max()), float(d.mean())
