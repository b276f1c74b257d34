"""Device-side varlen metadata (femto_build_varlen_metadata) equals the host build.

The host builder restates the reference's ModelRunner rules
(femtovllm/engine/model_runner.py:187-202 prefill, 283-293 decode, 46-72
block-table padding); every tensor must match it exactly.
"""

import time

import numpy as np
import pytest
import torch

from femtovllm.metadata import build_varlen_metadata, build_varlen_metadata_device

pytestmark = pytest.mark.gpu

FIELDS = ("positions", "cu_seqlens", "cu_q_tiles", "q_tile_to_seq_idx", "kv_lens", "block_tables")


def random_batch(rng, B, max_prefix, max_tokens, decode=False):
    chunks, tables, nxt = [], [], 0
    for _ in range(B):
        p = int(rng.integers(0, max_prefix + 1))
        n = 1 if decode else int(rng.integers(0, max_tokens + 1))
        pages = -(-(p + n) // 16)
        extra = int(rng.integers(0, 3))
        tables.append(list(range(nxt, nxt + pages + extra)))
        nxt += pages + extra
        chunks.append((p, n))
    return chunks, tables


def check(gpu, chunks, tables, q_tile=32):
    host = build_varlen_metadata(chunks, tables, Q_TILE_SIZE=q_tile, device="cpu")
    dev = build_varlen_metadata_device(chunks, tables, Q_TILE_SIZE=q_tile, device=gpu)
    torch.cuda.synchronize()
    for f in FIELDS:
        a, b = getattr(dev, f).cpu(), getattr(host, f)
        assert a.shape == b.shape and torch.equal(a, b), f"{f} differs"
    assert dev.max_q_len == host.max_q_len and dev.max_kv_len == host.max_kv_len


@pytest.mark.parametrize("case", ["prefill", "decode", "large_batch", "long_chunks", "zero_tokens", "tile16"])
def test_matches_host_build(gpu, case):
    rng = np.random.default_rng(61)
    if case == "prefill":
        chunks, tables = random_batch(rng, 8, 2048, 512)
    elif case == "decode":
        chunks, tables = random_batch(rng, 256, 8000, 1, decode=True)
    elif case == "large_batch":
        chunks, tables = random_batch(rng, 3000, 500, 40)
    elif case == "long_chunks":
        chunks, tables = random_batch(rng, 3, 30000, 9000)
    elif case == "zero_tokens":
        chunks, tables = [(0, 0), (16, 0), (5, 3)], [[], [0], [1]]
    else:
        chunks, tables = random_batch(rng, 20, 100, 100)
    check(gpu, chunks, tables, q_tile=16 if case == "tile16" else 32)


def test_feeds_the_attention_ops(ops, gpu):
    """The device-built metadata drives prefill and decode exactly like the host-built one."""
    from femtovllm import workloads

    w = workloads.make_paged_workload("md", [(100, 60), (0, 40), (250, 9)], 16, 8, seed=62)
    wd = w.to(gpu)
    q = w.q.to(gpu)
    args = lambda m: (m.cu_seqlens, m.max_q_len, m.Q_TILE_SIZE, m.cu_q_tiles, m.q_tile_to_seq_idx, m.block_tables,
                      m.kv_lens, m.positions)
    mh = build_varlen_metadata(w.chunks, w.raw_block_tables, device=gpu)
    md = build_varlen_metadata_device(w.chunks, w.raw_block_tables, device=gpu)
    a = ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, *args(mh))
    b = ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, *args(md))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_host_time(gpu):
    """Informative: host-side cost of the two builders for a 256-sequence prefill batch of 16k tokens."""
    rng = np.random.default_rng(63)
    chunks, tables = random_batch(rng, 256, 4000, 128)
    for fn in (build_varlen_metadata, build_varlen_metadata_device):
        fn(chunks, tables, device=gpu)
    torch.cuda.synchronize()
    for fn in (build_varlen_metadata, build_varlen_metadata_device):
        t0 = time.perf_counter()
        for _ in range(5):
            fn(chunks, tables, device=gpu)
        torch.cuda.synchronize()
        print(f"{fn.__name__}: {(time.perf_counter() - t0) / 5 * 1e3:.2f} ms per build")
