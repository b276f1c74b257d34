"""The allocation-free decode entry point, femto_paged_attention_gemv_noalloc.

It runs the same kernels as femto_paged_attention_gemv, with the partial
softmax states in the library's own device scratch array instead of a caller
workspace.  Checked through the C ABI against femto_paged_attention_gemv on
two calls in a row (the second smaller: the array keeps the first call's
contents), against the float64 oracle where the scratch forces a coarser
split, and for the size limit.
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_close, np32, np64, np_tables

pytestmark = pytest.mark.gpu


def _pool_args(q, out, k_pool, tables, kv_lens):
    return (q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), out.stride(1))


def gemv_with_workspace(C, q, k_pool, v_pool, tables, kv_lens, max_kv_len):
    out = torch.empty_like(q)
    ws, ws_bytes = C._decode_workspace(q.device, q.size(1), q.size(0), max_kv_len)
    rc = C._lib.femto_paged_attention_gemv(
        C._DTYPE[q.dtype], *_pool_args(q, out, k_pool, tables, kv_lens),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.size(0), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        tables.data_ptr(), tables.size(1), tables.stride(0), kv_lens.data_ptr(), q.size(1), q.size(0), max_kv_len,
        ws, ws_bytes, C._stream(q.device))
    assert rc == 0, C._lib.femto_attn_last_error().decode()
    return out


def gemv_noalloc(C, q, k_pool, v_pool, tables, kv_lens, max_kv_len, out=None):
    out = torch.empty_like(q) if out is None else out
    rc = C._lib.femto_paged_attention_gemv_noalloc(
        C._DTYPE[q.dtype], *_pool_args(q, out, k_pool, tables, kv_lens),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.size(0), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        tables.data_ptr(), tables.size(1), tables.stride(0), kv_lens.data_ptr(), q.size(1), q.size(0), max_kv_len,
        C._stream(q.device))
    return rc, out


def case(w, gpu):
    q, meta = w.gemv_call(device=gpu)
    wd = w.to(gpu)
    return q.to(gpu).contiguous(), wd, meta


def test_noalloc_matches_workspace_entry_two_calls(gpu):
    """Two calls in a row, the second with a smaller batch: bit-identical to the
    workspace entry point (same kernels, same split) and within the bf16 / f32
    tolerance of the oracle."""
    from femtovllm import _C

    big = workloads.decode_bf16_qwen3_0p6b()  # 64 sequences, contexts U[256, 4096]
    small = workloads.make_paged_workload("small", [(L - 1, 1) for L in (5, 300, 17, 1200, 2)], 16, 8,
                                          dtype=torch.float32, seed=71)
    for w in (big, small):
        q, wd, meta = case(w, gpu)
        # poison the output buffer so unwritten rows would show
        rc, got = gemv_noalloc(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len,
                               out=torch.full_like(q, float("nan")))
        assert rc == 0, _C._lib.femto_attn_last_error().decode()
        ref = gemv_with_workspace(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"{w.name}: noalloc output differs from the workspace entry point"
        want = oa.paged_decode(np64(q), np32(w.k_pool), np32(w.v_pool), np_tables(meta), meta.kv_lens.tolist())
        assert_close(got, want, w.dtype, f"noalloc {w.name}")


@pytest.fixture
def split_route(gpu):
    """The split route (scratch in use) for every length, restored afterwards."""
    from femtovllm import _C

    prev = _C._lib.femto_attn_set_decode_single_max_kv(-1)
    yield
    _C._lib.femto_attn_set_decode_single_max_kv(prev)


def test_noalloc_coarser_split_when_scratch_is_tight(gpu, split_route):
    """600 sequences x 32 heads: the default split needs more partial slots than
    the scratch holds, so sequences are cut into fewer slices; still within
    tolerance of the oracle and of the workspace entry point."""
    from femtovllm import _C

    rng = np.random.default_rng(72)
    lens = [int(x) for x in rng.integers(1, 600, size=600)]
    w = workloads.make_paged_workload("tight", [(L - 1, 1) for L in lens], 32, 8, seed=72)
    q, wd, meta = case(w, gpu)
    need = _C._lib.femto_paged_attention_gemv_workspace_size(600, 32, meta.max_kv_len)
    assert need > (64 << 20), "the case must not fit the scratch with the default split"
    rc, got = gemv_noalloc(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    assert rc == 0, _C._lib.femto_attn_last_error().decode()
    ref = gemv_with_workspace(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    torch.cuda.synchronize()
    want = oa.paged_decode(np64(q), np32(w.k_pool), np32(w.v_pool), np_tables(meta), meta.kv_lens.tolist())
    assert_close(got, want, torch.bfloat16, "noalloc, coarse split")
    assert (got.float() - ref.float()).abs().max().item() <= 2e-2


def test_noalloc_rejects_calls_beyond_the_scratch(gpu, split_route):
    """num_seqs * n_heads past the limit fails with a message and launches nothing
    (on the split route; the one-launch route uses no scratch)."""
    from femtovllm import _C

    B = 40000
    q = torch.zeros((2, B, 128), dtype=torch.bfloat16, device=gpu)
    pool = torch.zeros((1, 2, 16, 128), dtype=torch.bfloat16, device=gpu)
    tables = torch.zeros((B, 1), dtype=torch.int32, device=gpu)
    kv_lens = torch.ones(B, dtype=torch.int32, device=gpu)
    rc, _ = gemv_noalloc(_C, q, pool, pool, tables, kv_lens, 1)
    assert rc == 1
    msg = _C._lib.femto_attn_last_error().decode()
    assert "scratch" in msg and "femto_paged_attention_gemv" in msg


@pytest.mark.parametrize("lens", [(1500, 40, 3000, 700), (300, 17, 511, 2)], ids=["split_route", "one_launch_route"])
def test_noalloc_under_graph_capture(gpu, lens):
    """The allocation-free call captured in a HIP graph (after one call outside
    capture, which sets up the device) and replayed with new q and kv_lens:
    every replay matches the oracle and an eager call on the same inputs."""
    from femtovllm import _C

    w = workloads.make_paged_workload("graph", [(L - 1, 1) for L in lens], 16, 8, seed=73)
    q, wd, meta = case(w, gpu)
    kv_lens = meta.kv_lens.clone()
    out = torch.empty_like(q)
    rc, _ = gemv_noalloc(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, kv_lens, meta.max_kv_len, out=out)
    assert rc == 0, _C._lib.femto_attn_last_error().decode()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc, _ = gemv_noalloc(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, kv_lens, meta.max_kv_len, out=out)
    assert rc == 0, _C._lib.femto_attn_last_error().decode()
    gen = torch.Generator().manual_seed(74)
    rng = np.random.default_rng(74)
    for rep in range(3):
        q_new = torch.randn(q.shape, generator=gen).to(q.dtype)
        new_lens = [int(rng.integers(1, L + 1)) for L in lens]
        q.copy_(q_new.to(gpu))
        kv_lens.copy_(torch.tensor(new_lens, dtype=torch.int32))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        eager = gemv_with_workspace(_C, q, wd.k_pool, wd.v_pool, meta.block_tables, kv_lens, meta.max_kv_len)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}: graph output differs from the eager call"
        want = oa.paged_decode(np64(q_new), np32(w.k_pool), np32(w.v_pool), np_tables(meta), new_lens)
        assert_close(out, want, w.dtype, f"graph replay {rep}, lens {new_lens}")
