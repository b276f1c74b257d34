"""Invariances of the HIP attention kernels, checked on the GPU.

* Physical placement: moving every pool block to another place and rewriting
  the block tables to match leaves the outputs bit-identical (decode, and
  prefill without the key split, whose merge order depends on which piece
  finishes last).  This pins the gather ``pool[tables[b][j // 16], h / n_rep,
  j % 16]`` independently of the oracle.
* GQA: n_rep = 2 gives the same outputs as MHA over KV heads replicated in
  pairs (femtovllm/models/qwen/qwen3.py:504-523 repeats each KV head n_rep
  times for consecutive query heads).
* Chunking: the tokens of one sequence give bit-identical outputs whether they
  come in one chunk or in two (the second attending the first through the
  cache, with positions continuing), as the engine's chunked prefill relies on
  (model_runner.py:187-202).
"""

import dataclasses

import numpy as np
import pytest
import torch

from femtovllm import workloads
from femtovllm.metadata import build_varlen_metadata
from helpers import assert_agree, assert_close

pytestmark = pytest.mark.gpu


def _gemm(ops, q, meta, w):
    out = ops.paged_attention_gemm(q, w.k_pool, w.v_pool, meta.cu_seqlens, meta.max_q_len, meta.Q_TILE_SIZE,
                                   meta.cu_q_tiles, meta.q_tile_to_seq_idx, meta.block_tables, meta.kv_lens,
                                   meta.positions)
    torch.cuda.synchronize()
    return out


def _gemv(ops, q, meta, w):
    out = ops.paged_attention_gemv(q, w.k_pool, w.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    torch.cuda.synchronize()
    return out


@pytest.fixture
def no_split(monkeypatch):
    from femtovllm import _C

    monkeypatch.setattr(_C, "_prefill_workspace", lambda *args: (None, 0))


def _permuted(w, seed):
    """The same workload with pool block i moved to perm[i] and the tables rewritten."""
    nb = w.k_pool.shape[0]
    perm = torch.from_numpy(np.random.default_rng(seed).permutation(nb))
    k = torch.empty_like(w.k_pool)
    v = torch.empty_like(w.v_pool)
    k[perm] = w.k_pool
    v[perm] = w.v_pool
    tables = [[int(perm[x]) if x >= 0 else x for x in row] for row in w.raw_block_tables]
    return dataclasses.replace(w, raw_block_tables=tables, k_pool=k, v_pool=v)


def test_prefill_placement_is_bit_identical(ops, gpu, no_split):
    w = workloads.make_paged_workload("perm_prefill", [(300, 200), (0, 77), (1500, 64), (40, 1)], 16, 8, seed=41)
    wp = _permuted(w, 42)
    assert wp.raw_block_tables != w.raw_block_tables
    outs = []
    for x in (w, wp):
        q, meta = x.gemm_call(device=gpu)
        outs.append(_gemm(ops, q.to(gpu), meta, x.to(gpu)))
    assert torch.equal(outs[0], outs[1])


def test_decode_placement_is_bit_identical(ops, gpu):
    w = workloads.make_paged_workload("perm_decode", [(int(L) - 1, 1) for L in (17, 300, 2049, 4000, 5)], 16, 8,
                                      seed=43)
    wp = _permuted(w, 44)
    outs = []
    for x in (w, wp):
        q, meta = x.gemv_call(device=gpu)
        outs.append(_gemv(ops, q.to(gpu), meta, x.to(gpu)))
    assert torch.equal(outs[0], outs[1])


def _replicated_kv(w):
    """MHA twin of a GQA workload: KV head k of the twin is head k // n_rep of w."""
    n_rep = w.n_heads // w.n_kv_heads
    k = w.k_pool.repeat_interleave(n_rep, dim=1).contiguous()
    v = w.v_pool.repeat_interleave(n_rep, dim=1).contiguous()
    return dataclasses.replace(w, n_kv_heads=w.n_heads, k_pool=k, v_pool=v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gqa_equals_replicated_mha(ops, gpu, dtype):
    w = workloads.make_paged_workload("gqa_mha", [(700, 130), (0, 64), (64, 1)], 16, 8, dtype=dtype, seed=45)
    m = _replicated_kv(w)
    outs = []
    for x in (w, m):
        q, meta = x.gemm_call(device=gpu)
        outs.append(_gemm(ops, q.to(gpu), meta, x.to(gpu)))
    # Same math per row; only how rows are grouped into waves differs.
    assert_agree(outs[0], outs[1], dtype, "GQA vs replicated MHA (prefill)")

    d = workloads.make_paged_workload("gqa_mha_dec", [(900, 1), (33, 1), (4095, 1)], 16, 8, dtype=dtype, seed=46)
    dm = _replicated_kv(d)
    outs = []
    for x in (d, dm):
        q, meta = x.gemv_call(device=gpu)
        outs.append(_gemv(ops, q.to(gpu), meta, x.to(gpu)))
    assert_agree(outs[0], outs[1], dtype, "GQA vs replicated MHA (decode)")


@pytest.mark.parametrize("heads", [(16, 8), (32, 8)])
def test_two_chunks_equal_one(ops, gpu, no_split, heads):
    """A 512-token chunk after a 1000-token prefix, as one call and as two
    256-token calls: the per-token outputs are bit-identical."""
    H, KVH = heads
    prefix, n, n1 = 1000, 512, 256
    w = workloads.make_paged_workload("chunks", [(prefix, n)], H, KVH, seed=47)
    wd = w.to(gpu)
    q, meta = w.gemm_call(device=gpu)
    whole = _gemm(ops, q.to(gpu), meta, wd)
    parts = []
    for start, count in ((0, n1), (n1, n - n1)):
        meta_p = build_varlen_metadata([(prefix + start, count)], w.raw_block_tables, device=gpu)
        q_p = w.q[:, start:start + count].contiguous().to(gpu)
        parts.append(_gemm(ops, q_p, meta_p, wd))
    assert torch.equal(whole, torch.cat(parts, dim=1))
