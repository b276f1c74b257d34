"""Shared helpers for the parity tests (CPU oracle vs HIP kernels)."""

from __future__ import annotations

import numpy as np
import torch

# Tolerances against the float64 oracle (max-abs), per output dtype.
# f32 and bf16 are the stated targets; f16 follows the reference's own dense
# attention check, allclose(atol=1e-3, rtol=1e-3)
# (csrc/flash_attention/test_flash_attention.py:51).
ATOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2, torch.float16: 1e-3}
RTOL = {torch.float32: 0.0, torch.bfloat16: 0.0, torch.float16: 1e-3}


def np64(t: torch.Tensor) -> np.ndarray:
    """Exact float64 copy of a (possibly bf16 / f16, possibly GPU) tensor."""
    return t.detach().to("cpu").to(torch.float32).numpy().astype(np.float64)


def np32(t: torch.Tensor) -> np.ndarray:
    """Exact float32 copy (bf16 / f16 values are exact in float32); used for big pools.

    bf16 widens by moving its bits into the high half of a float32 word
    (bf16 is the top 16 bits of float32), which numpy does far faster than a
    CPU tensor cast; f16 goes through numpy's own float16.
    """
    t = t.detach().to("cpu").contiguous()
    if t.dtype == torch.bfloat16:
        return (t.view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.float16).astype(np.float32)
    return t.to(torch.float32).numpy()


def np_tables(meta) -> np.ndarray:
    return meta.block_tables.to("cpu").numpy().astype(np.int64)


def assert_close(got: torch.Tensor, want: np.ndarray, dtype: torch.dtype, what: str = "", mask=None):
    g = np64(got)
    w = np.asarray(want, dtype=np.float64)
    if mask is not None:
        g, w = g[mask], w[mask]
    nan_g, nan_w = np.isnan(g), np.isnan(w)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN pattern differs ({nan_g.sum()} vs {nan_w.sum()})"
    ok = ~nan_w
    err = np.abs(g[ok] - w[ok])
    tol = ATOL[dtype] + RTOL[dtype] * np.abs(w[ok])
    worst = float(err.max()) if err.size else 0.0
    assert np.all(err <= tol), f"{what}: max abs err {worst:.3e} exceeds tolerance (atol {ATOL[dtype]}, rtol {RTOL[dtype]})"
    return worst


def sample_rows(cu_seqlens, per_seq: int, rng: np.random.Generator, tile: int = 32):
    """Token rows to check on big prefill workloads: first, last, tile edges and random."""
    rows = set()
    cu = [int(x) for x in cu_seqlens]
    for b in range(len(cu) - 1):
        lo, hi = cu[b], cu[b + 1]
        if hi <= lo:
            continue
        cand = {lo, hi - 1, min(hi - 1, lo + tile - 1), min(hi - 1, lo + tile)}
        cand.update(int(x) for x in rng.integers(lo, hi, size=per_seq))
        rows.update(cand)
    return sorted(rows)
