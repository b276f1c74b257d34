"""Seeded random batches through the HIP prefill kernel, checked against the oracle.

Each case draws a batch the hand-written cases may not reach: 1-10
sequences whose chunks are empty, one token (decode rows), short or a few
hundred tokens, after no, short or long cached prefixes, with a random head
layout and storage type.  One call covers the query-tile mapping, the key
split of long tiles (whenever a sequence's keys far exceed the mean work per
resident workgroup), and the decode rows, fused into the launch or run
before it by head ratio.  Each call must match the oracle (the reference's
attention, femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:83-160)
and the call without key split, and leave the split counters zero-filled.
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_agree, assert_close, np32, np64, np_tables, sample_rows
from test_prefill_split_gpu import _gemm, _unsplit, _workspace_is_zero, split_plan

HEADS = [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4), (28, 4), (40, 8), (8, 1), (4, 1), (6, 2), (3, 3)]
# Oracle work allowed per case (rows x keys x query heads) before rows are sampled.
FULL_CHECK = 2e8


def random_batch(seed):
    rng = np.random.default_rng(seed)
    H, KVH = HEADS[int(rng.integers(len(HEADS)))]
    dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float16
    chunks = []
    for _ in range(int(rng.integers(1, 11))):
        r = rng.random()
        prefix = 0 if r < 0.3 else int(rng.integers(1, 200)) if r < 0.7 else int(rng.integers(200, 4000))
        r = rng.random()
        n = 0 if r < 0.1 else 1 if r < 0.3 else int(rng.integers(2, 64)) if r < 0.7 else int(rng.integers(64, 400))
        chunks.append((prefix, n))
    if all(n == 0 for _, n in chunks):
        chunks[0] = (chunks[0][0], 1)
    return chunks, H, KVH, dtype


def test_generator_reaches_every_kind_of_sequence():
    """Over the seeds used below: empty chunks, one-token rows, long prefixes,
    fresh prompts and both storage types all occur, and on a 256-CU GPU most
    calls cut some query tiles into key pieces."""
    seen = set()
    split = 0
    for seed in range(64):
        chunks, H, KVH, dtype = random_batch(7000 + seed)
        split += max(split_plan(chunks, H, KVH, 256)) > 1
        seen.add(dtype)
        for p, n in chunks:
            seen.add("empty" if n == 0 else "one" if n == 1 else "chunk")
            seen.add("fresh" if p == 0 else "long" if p >= 200 else "short")
    assert seen >= {torch.bfloat16, torch.float16, "empty", "one", "chunk", "fresh", "long", "short"}
    assert split >= 32


# range(64), plus seed 3865 (batch 10865: 64 / 8 heads, bf16, eight sequences), whose split and
# unsplit results differ by slightly more than one row bound while both lie within the oracle's.
@pytest.mark.gpu
@pytest.mark.parametrize("seed", [*range(64), 3865])
def test_random_batch(ops, gpu, monkeypatch, seed):
    chunks, H, KVH, dtype = random_batch(7000 + seed)
    what = f"seed {7000 + seed}: H={H} KVH={KVH} {dtype} chunks {chunks}"
    print(what, flush=True)
    w = workloads.make_paged_workload("random", chunks, H, KVH, dtype=dtype, seed=7000 + seed)
    q, meta = w.gemm_call(device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    out = _gemm(ops, q, meta, wd)
    assert _workspace_is_zero(gpu), f"split counters not reset after {what}"
    cu = meta.raw_cu_seqlens
    work = sum((cu[b + 1] - cu[b]) * (p + n) for b, (p, n) in enumerate(chunks)) * H
    rows = None
    if work > FULL_CHECK:
        rows = sorted(set(sample_rows(cu, 12, np.random.default_rng(seed))))
    want = oa.paged_prefill(np64(q.cpu()), np32(w.k_pool), np32(w.v_pool), cu, np_tables(meta),
                            meta.kv_lens.tolist(), np.asarray(meta.raw_positions), rows=rows)
    mask = None
    if rows is not None:
        mask = np.zeros(want.shape, dtype=bool)
        mask[:, rows] = True
    assert_close(out, want, dtype, what, mask=mask)
    # the call without key split takes the same tiles whole; one-token rows
    # run on the decode kernel either way
    ref = _unsplit(ops, q, meta, wd, monkeypatch)
    assert_agree(out, ref, dtype, what + " vs unsplit")


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(24))
def test_random_batch_arbitrary_positions(ops, gpu, monkeypatch, seed):
    """The same kind of batches with each token's position drawn anywhere:
    mostly inside its context, a few past it (all keys visible) and a few at
    -1 (no key visible: a NaN row, as in the reference).  Key pieces then
    see fewer or more key tiles than the engine's layout implies, and
    some rows of a piece see none."""
    chunks, H, KVH, dtype = random_batch(7500 + seed)
    what = f"seed {7500 + seed}: H={H} KVH={KVH} {dtype} chunks {chunks}, arbitrary positions"
    print(what, flush=True)
    w = workloads.make_paged_workload("random_pos", chunks, H, KVH, dtype=dtype, seed=7500 + seed)
    q, meta = w.gemm_call(device=gpu)
    rng = np.random.default_rng(7500 + seed)
    cu = meta.raw_cu_seqlens
    pos = np.asarray(meta.raw_positions).copy()
    for b, kvl in enumerate(meta.kv_lens.tolist()):
        for t in range(cu[b], cu[b + 1]):
            r = rng.random()
            pos[t] = -1 if r < 0.05 else kvl + int(rng.integers(0, 50)) if r < 0.1 else int(rng.integers(0, max(1, kvl)))
    meta.raw_positions = [int(x) for x in pos]
    meta.positions = torch.tensor(pos, dtype=torch.int32, device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    out = _gemm(ops, q, meta, wd)
    assert _workspace_is_zero(gpu), f"split counters not reset after {what}"
    work = sum((cu[b + 1] - cu[b]) * (p + n) for b, (p, n) in enumerate(chunks)) * H
    rows = None
    if work > FULL_CHECK:
        rows = sorted(set(sample_rows(cu, 12, np.random.default_rng(seed))))
    want = oa.paged_prefill(np64(q.cpu()), np32(w.k_pool), np32(w.v_pool), cu, np_tables(meta),
                            meta.kv_lens.tolist(), pos, rows=rows)
    mask = None
    if rows is not None:
        mask = np.zeros(want.shape, dtype=bool)
        mask[:, rows] = True
    assert_close(out, want, dtype, what, mask=mask)
    # Without key split: the oracle's bar too, and at most one output unit
    # in the last place from the split result (rows that see a few keys
    # reach magnitudes of 2-4, where a bf16 unit is 2^-6, and the split's
    # partials can move a value across a rounding boundary).
    ref = _unsplit(ops, q, meta, wd, monkeypatch)
    assert_close(ref, want, dtype, what + ", unsplit", mask=mask)
    a, b = np64(out), np64(ref)
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dtype]  # relative spacing bound
    both = ~(np.isnan(a) | np.isnan(b))
    assert np.array_equal(np.isnan(a), np.isnan(b)), what + ": NaN rows differ from the unsplit call"
    assert np.all(np.abs(a - b)[both] <= 1e-2 + ulp * np.maximum(np.abs(a), np.abs(b))[both]), what + " vs unsplit"


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(16))
def test_random_batch_head_dims(ops, gpu, monkeypatch, seed):
    """The same kind of batches at a head_dim below 128 (a multiple of 16, as the reference's CUDA
    prefill check allows, csrc/paged_attention/paged_attention_gemm.cu:347-348)."""
    chunks, H, KVH, dtype = random_batch(7600 + seed)
    D = int(np.random.default_rng(7600 + seed).choice([16, 32, 48, 64, 80, 96, 112]))
    what = f"seed {7600 + seed}: H={H} KVH={KVH} D={D} {dtype} chunks {chunks}"
    print(what, flush=True)
    w = workloads.make_paged_workload("random_hd", chunks, H, KVH, head_dim=D, dtype=dtype, seed=7600 + seed)
    q, meta = w.gemm_call(device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    out = _gemm(ops, q, meta, wd)
    assert out.shape[-1] == D
    assert _workspace_is_zero(gpu), f"split counters not reset after {what}"
    cu = meta.raw_cu_seqlens
    work = sum((cu[b + 1] - cu[b]) * (p + n) for b, (p, n) in enumerate(chunks)) * H
    rows = None
    if work > FULL_CHECK:
        rows = sorted(set(sample_rows(cu, 12, np.random.default_rng(seed))))
    want = oa.paged_prefill(np64(q.cpu()), np32(w.k_pool), np32(w.v_pool), cu, np_tables(meta),
                            meta.kv_lens.tolist(), np.asarray(meta.raw_positions), rows=rows)
    mask = None
    if rows is not None:
        mask = np.zeros(want.shape, dtype=bool)
        mask[:, rows] = True
    assert_close(out, want, dtype, what, mask=mask)
    ref = _unsplit(ops, q, meta, wd, monkeypatch)
    assert_agree(out, ref, dtype, what + " vs unsplit")
