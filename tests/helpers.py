"""Shared helpers for the parity tests (CPU oracle vs HIP kernels)."""

from __future__ import annotations

import json
import os

import numpy as np
import torch

# Tolerances against the float64 oracle (max-abs), per output dtype.
# f32 and bf16 are the stated targets; f16 follows the reference's own dense
# attention check, allclose(atol=1e-3, rtol=1e-3)
# (csrc/flash_attention/test_flash_attention.py:51).
ATOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2, torch.float16: 1e-3}
RTOL = {torch.float32: 0.0, torch.bfloat16: 0.0, torch.float16: 1e-3}
# The max-abs bound holds for the value before its final rounding to the
# output type; that rounding adds half an ulp at |want| (0.0078 for a bf16
# output in [2, 4), where the grid is 2^-6 wide).  Without it no kernel that
# stores bf16 meets 1e-2 on rows of a few visible keys with |out| >= 2: the
# reference's own arithmetic (fp32 softmax, weights cast to bf16 before P.V,
# bf16 store; femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:
# 122-160, restated in oracle/ref_arith.py) exceeds a plain 1e-2 against the
# float64 oracle there and stays within 1e-2 + half an ulp
# (tests/test_oracle.py::test_ref_arith_needs_the_output_rounding_allowance).
# Below |want| = 1.28 a bf16 half ulp is at most 2^-9 x 1.28 = 0.0025.

# Scale-aware bound, checked beside the max-abs one.  Attention outputs
# shrink with context length (N(0,1) inputs give an output RMS of about
# 1/sqrt(visible keys): 0.0096 at 32k keys), so a max-abs 1e-2 alone would
# pass a kernel returning half the right answer there.  Per output row (one
# query token of one head, the head_dim axis):
#     |got - want| <= ROW_REL * max|want row| + half an ulp of the output type at max|want row|.
# 16-bit outputs: 2^-7 covers the rounding of P to the storage type (at most
# 2^-8 relative per probability, random over keys) and the output rounding;
# f32 outputs: 2^-14.
ROW_REL = {torch.float32: 2.0 ** -14, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -7}
MANT_BITS = {torch.float32: 24, torch.bfloat16: 8, torch.float16: 11}

# Per-check statistics of the last assert_close calls (what, max abs error,
# worst error / row bound, relative RMS error); appended to the file named by
# FEMTO_PARITY_LOG as JSON lines when that variable is set.
STATS: list = []


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


def half_ulp(x: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Half a unit in the last place of ``dtype`` at magnitude ``x`` (x >= 0; 0 at 0)."""
    _, e = np.frexp(x)  # x = f * 2^e, 0.5 <= f < 1
    return np.where(x > 0, np.ldexp(1.0, e - MANT_BITS[dtype] - 1), 0.0)


def row_bound(want: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """The scale-aware per-element bound, broadcast over each row's last axis."""
    m = np.where(np.isnan(want), 0.0, np.abs(want)).max(axis=-1, keepdims=True)
    return np.broadcast_to(ROW_REL[dtype] * m + half_ulp(m, dtype), want.shape)


def assert_close(got: torch.Tensor, want: np.ndarray, dtype: torch.dtype, what: str = "", mask=None, factor=1.0):
    """Max-abs (ATOL / RTOL) and per-row scale-aware (ROW_REL) parity; returns the max abs error.
    ``factor`` scales both bounds (assert_agree)."""
    g = got if isinstance(got, np.ndarray) else np64(got)
    w = np.asarray(want, dtype=np.float64)
    rb = factor * row_bound(w, dtype)
    if mask is not None:
        g, w, rb = g[mask], w[mask], rb[mask]
    nan_g, nan_w = np.isnan(g), np.isnan(w)
    assert np.array_equal(nan_g, nan_w), f"{what}: NaN pattern differs ({nan_g.sum()} vs {nan_w.sum()})"
    ok = ~nan_w
    err = np.abs(g[ok] - w[ok])
    tol = factor * (ATOL[dtype] + RTOL[dtype] * np.abs(w[ok]) + half_ulp(np.abs(w[ok]), dtype))
    worst = float(err.max()) if err.size else 0.0
    rbo = rb[ok]
    ratio = float((err / np.where(rbo > 0, rbo, np.inf)).max()) if err.size else 0.0
    if err.size and np.any((rbo == 0) & (err > 0)):
        ratio = float("inf")
    wn = float(np.sqrt(np.sum(w[ok] ** 2)))
    rel_rms = float(np.sqrt(np.sum(err ** 2)) / wn) if wn > 0 else 0.0
    rec = {"what": what, "dtype": str(dtype).replace("torch.", ""), "max_abs": worst,
           "row_bound_ratio": ratio, "rel_rms": rel_rms, "n": int(err.size)}
    STATS.append(rec)
    log = os.environ.get("FEMTO_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps(rec) + "\n")
    assert np.all(err <= tol), (f"{what}: max abs err {worst:.3e} exceeds tolerance ({factor:g} x (atol "
                                f"{ATOL[dtype]}, rtol {RTOL[dtype]}, + half an output ulp))")
    assert ratio <= 1.0, (f"{what}: error reaches {ratio:.2f}x the per-row bound ({factor:g} x "
                          f"({ROW_REL[dtype]:.2e} x max|row| + half ulp)); relative RMS error {rel_rms:.2e}")
    return worst


def assert_agree(got: torch.Tensor, other: torch.Tensor, dtype: torch.dtype, what: str = "", mask=None):
    """Two kernel results for the same call (e.g. with and without the key split), each of which must
    lie within the bounds of assert_close from the exact value: by the triangle inequality they differ
    by at most twice those bounds, which is what this checks.  Each result's own check is against the
    oracle; this one catches a path that is consistently off where the oracle checks only sample rows.
    (Seen on random batches: 1 of 1,800 split / unsplit pairs differs by 1.03x a single bound while
    both pass the oracle.)"""
    o = other if isinstance(other, np.ndarray) else np64(other)
    return assert_close(got, o, dtype, what, mask=mask, factor=2.0)


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
