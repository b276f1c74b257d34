"""Pools past 4 GiB: block offsets that need 64-bit arithmetic.

A KV pool sized for long-context serving on a 288 GB GPU runs to tens of GB,
so the byte offset block * block_stride * element_size passes 2^32 (and the
element offset 2^31).  Every kernel runs once on a compact pool and once on a
4.3 GiB pool holding the same blocks at its end (block ids >= 131,072 at
32 KiB per block); outputs, and the blocks the writers fill, must be
bit-identical.  The attention ops read pools the reference indexes as
k_pool[tables[b][j // 16], h / n_rep, j % 16] (paged_attention_gemv.cu:84-107,
paged_attention_gemm.py:6-162); the writers follow qwen3.py:240-264, 322-366.
"""

import dataclasses

import numpy as np
import pytest
import torch

from femtovllm import workloads
from femtovllm.rope import rope_tables

pytestmark = pytest.mark.gpu

# 140,000 blocks x (8 KV heads x 16 rows x 128 dims x 2 bytes) = 4.27 GiB per pool.
BIG_BLOCKS = 140_000


@pytest.fixture
def no_split(monkeypatch):
    from femtovllm import _C

    monkeypatch.setattr(_C, "_prefill_workspace", lambda *args: (None, 0))


def _moved_to_end(w, gpu):
    """w with its pool blocks moved to the end of a BIG_BLOCKS pool on the GPU."""
    nb = w.k_pool.shape[0]
    base = BIG_BLOCKS - nb
    assert base * w.k_pool[0].numel() * w.k_pool.element_size() > 2**32
    shape = (BIG_BLOCKS,) + tuple(w.k_pool.shape[1:])
    k = torch.empty(shape, dtype=w.k_pool.dtype, device=gpu)
    v = torch.empty(shape, dtype=w.v_pool.dtype, device=gpu)
    k[base:] = w.k_pool.to(gpu)
    v[base:] = w.v_pool.to(gpu)
    tables = [[x + base if x >= 0 else x for x in row] for row in w.raw_block_tables]
    return dataclasses.replace(w, raw_block_tables=tables, k_pool=k, v_pool=v, q=w.q.to(gpu)), base


def test_decode_on_large_pool(ops, gpu):
    w = workloads.make_paged_workload("big_decode", [(int(L) - 1, 1) for L in (17, 300, 2049, 4000)], 16, 8,
                                      seed=51, poison=False)
    outs = []
    for x in (w.to(gpu), _moved_to_end(w, gpu)[0]):
        q, meta = x.gemv_call(device=gpu)
        outs.append(ops.paged_attention_gemv(q, x.k_pool, x.v_pool, meta.block_tables, meta.kv_lens,
                                             meta.max_kv_len))
        torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_prefill_on_large_pool(ops, gpu, no_split):
    w = workloads.make_paged_workload("big_prefill", [(300, 200), (0, 77), (1500, 64), (40, 1)], 16, 8, seed=52,
                                      poison=False)
    outs = []
    for x in (w.to(gpu), _moved_to_end(w, gpu)[0]):
        q, meta = x.gemm_call(device=gpu)
        outs.append(ops.paged_attention_gemm(q, x.k_pool, x.v_pool, meta.cu_seqlens, meta.max_q_len,
                                             meta.Q_TILE_SIZE, meta.cu_q_tiles, meta.q_tile_to_seq_idx,
                                             meta.block_tables, meta.kv_lens, meta.positions))
        torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def _writer_case(gpu, seed):
    """A prefill workload, its metadata, and new q / k / v rows for every token."""
    w = workloads.make_paged_workload("big_write", [(300, 200), (0, 77), (1500, 64)], 16, 8, seed=seed,
                                      poison=False)
    rng = np.random.default_rng(seed)
    T = w.num_tokens
    new = [torch.from_numpy(rng.standard_normal((T, h, 128), dtype=np.float32)).to(torch.bfloat16).to(gpu)
           for h in (16, 8, 8)]
    return w, new


def test_cache_write_on_large_pool(ops, gpu):
    w, (_, k_new, v_new) = _writer_case(gpu, 53)
    small = w.to(gpu)
    big, base = _moved_to_end(w, gpu)
    for x in (small, big):
        _, meta = x.gemm_call(device=gpu)
        ops.kv_cache_write(k_new, v_new, x.k_pool, x.v_pool, meta.positions, meta.block_tables,
                           cu_seqlens=meta.cu_seqlens, max_q_len=meta.max_q_len)
    torch.cuda.synchronize()
    assert not torch.equal(small.k_pool, w.k_pool.to(gpu)), "the write changed nothing"
    assert torch.equal(big.k_pool[base:], small.k_pool)
    assert torch.equal(big.v_pool[base:], small.v_pool)


def test_prologue_on_large_pool(ops, gpu):
    w, (q_new, k_new, v_new) = _writer_case(gpu, 54)
    g = torch.Generator().manual_seed(54)
    wq = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(gpu)
    wk = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(gpu)
    cos, sin = rope_tables(4096, 128, device=gpu)
    small = w.to(gpu)
    big, base = _moved_to_end(w, gpu)
    q_outs = []
    for x in (small, big):
        _, meta = x.gemm_call(device=gpu)
        q_outs.append(ops.qk_norm_rope_cache_write(q_new, k_new, v_new, wq, wk, 1e-6, cos, sin, meta.positions,
                                                   x.k_pool, x.v_pool, meta.block_tables,
                                                   cu_seqlens=meta.cu_seqlens, max_q_len=meta.max_q_len))
    torch.cuda.synchronize()
    assert torch.equal(q_outs[0], q_outs[1])
    assert torch.equal(big.k_pool[base:], small.k_pool)
    assert torch.equal(big.v_pool[base:], small.v_pool)

