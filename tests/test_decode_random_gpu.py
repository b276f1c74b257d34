"""Seeded random batches through the HIP decode kernel, checked against the oracle.

The decode kernel cuts the concatenated pages of the whole batch into equal
slices, one per wave, so a sequence may be split between waves at any page
and a wave may cover the ends of several sequences; the merge kernel then
combines the slices of each (sequence, head).  Each case draws a batch that
moves those cuts around: 1-160 sequences whose contexts are empty, one key,
a page boundary, short or up to 8192 keys (the reference's limit,
csrc/paged_attention/paged_attention_gemv.cu:271-274), with a random head
layout and storage type.  Every row must match the oracle (the reference's
decode attention, paged_attention_gemv.cu:20-220, float64 restatement).
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_close, np32, np64, np_tables

HEADS = [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4), (28, 4), (40, 8), (8, 1), (4, 1), (6, 2), (3, 3)]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def random_batch(seed):
    rng = np.random.default_rng(seed)
    H, KVH = HEADS[int(rng.integers(len(HEADS)))]
    dtype = DTYPES[int(rng.integers(len(DTYPES)))]
    n = int(rng.choice([1, 2, int(rng.integers(3, 40)), int(rng.integers(40, 160))]))
    lens = []
    for _ in range(n):
        r = rng.random()
        L = (0 if r < 0.05 else 1 if r < 0.1 else 16 * int(rng.integers(1, 8)) + int(rng.integers(-1, 2)) if r < 0.3
             else int(rng.integers(2, 600)) if r < 0.88 else int(rng.integers(600, 8193)))
        lens.append(max(0, L))
    return lens, H, KVH, dtype


def test_generator_reaches_every_kind_of_batch():
    """Over the seeds used below: empty and one-key contexts, page-boundary
    lengths, long contexts, single sequences, large batches and all three
    storage types occur."""
    seen = set()
    for seed in range(48):
        lens, H, KVH, dtype = random_batch(9000 + seed)
        seen.add(dtype)
        seen.add("single" if len(lens) == 1 else "large" if len(lens) >= 40 else "small")
        for L in lens:
            seen.add("empty" if L == 0 else "one" if L == 1 else "long" if L >= 4096 else
                     "edge" if L % 16 in (0, 1, 15) else "other")
    assert seen >= {*DTYPES, "single", "large", "small", "empty", "one", "long", "edge"}


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(48))
def test_random_decode_batch(ops, gpu, decode_path, seed):
    lens, H, KVH, dtype = random_batch(9000 + seed)
    what = f"seed {9000 + seed} ({decode_path}): H={H} KVH={KVH} {dtype} {len(lens)} seqs, max len {max(lens)}"
    print(what, flush=True)
    # decode: the query token is the last of each context (a context of 0
    # keys is a chunk of one token with kv_len 0)
    w = workloads.make_paged_workload("random_decode", [(max(0, L - 1), 1) for L in lens], H, KVH, dtype=dtype,
                                      seed=9000 + seed)
    q, meta = w.gemv_call(device=gpu)
    kv_lens = torch.tensor(lens, dtype=torch.int32, device=gpu)
    wd = w.to(gpu)
    out = ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, kv_lens,
                                   max(1, max(lens)))
    torch.cuda.synchronize()
    want = oa.paged_decode(np64(q), np32(w.k_pool), np32(w.v_pool), np_tables(meta), lens)
    assert_close(out, want, dtype, what)
