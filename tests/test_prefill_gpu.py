"""Parity of the HIP MFMA prefill kernel (femto_paged_attention_gemm) with the oracle.

Reference behaviour: paged_attention_gemm_triton
(femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:165-235) and
PagedAttentionGemmCuda (csrc/paged_attention/paged_attention_gemm.cu:304-395)
behind femtovllm.ops.paged_attention_gemm (femtovllm/ops/__init__.py:110-156).
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from femtovllm.metadata import build_varlen_metadata
from helpers import assert_agree, assert_close, np32, np64, np_tables, sample_rows

pytestmark = pytest.mark.gpu


def run_gemm(ops, q, meta, k_pool, v_pool, device, impl=None):
    out = ops.paged_attention_gemm(
        q.to(device), k_pool, v_pool, meta.cu_seqlens, meta.max_q_len, meta.Q_TILE_SIZE, meta.cu_q_tiles,
        meta.q_tile_to_seq_idx, meta.block_tables, meta.kv_lens, meta.positions, impl=impl,
    )
    torch.cuda.synchronize()
    return out


def oracle_prefill(q, meta, k_pool, v_pool, rows=None):
    return oa.paged_prefill(np64(q), np32(k_pool), np32(v_pool), meta.raw_cu_seqlens, np_tables(meta),
                            meta.kv_lens.tolist(), np.asarray(meta.raw_positions), rows=rows)


def check_workload(ops, w, gpu, seqs=None, rows_per_seq=None, what=""):
    q, meta = w.gemm_call(seqs=seqs, device=gpu)
    wd = w.to(gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    rows = None
    if rows_per_seq is not None:
        rows = sample_rows(meta.raw_cu_seqlens, rows_per_seq, np.random.default_rng(0))
    want = oracle_prefill(q, meta, w.k_pool, w.v_pool, rows=rows)
    mask = None
    if rows is not None:
        mask = np.zeros(want.shape, dtype=bool)
        mask[:, rows] = True
    return assert_close(out, want, w.dtype, what, mask=mask)


def test_reference_fixture_structure(ops, gpu):
    """cu_seqlens [0,8,24], kv_lens [59,44], tables [[0,4,5,6],[1,8,9,-1]], H=8, KVH=4."""
    w = workloads.reference_fixture()
    err = check_workload(ops, w, gpu, what="reference fixture")
    print(f"reference fixture max abs err {err:.2e}")


@pytest.mark.parametrize("impl", ["cuda", "triton"])
def test_impl_flag_routes_to_hip(ops, gpu, impl):
    from femtovllm.protocol import ImplCustomKernel

    w = workloads.reference_fixture()
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu, impl=ImplCustomKernel(impl))
    assert_close(out, oracle_prefill(q, meta, w.k_pool, w.v_pool), torch.bfloat16, impl)


def test_chunked_prefill_8x512(ops, gpu):
    """Every one of the 4096 rows of the 8 x 512 chunked batch."""
    w = workloads.prefill_bf16_chunked()
    err = check_workload(ops, w, gpu, what="8x512 chunked prefill")
    print(f"8x512 max abs err {err:.2e}")


@pytest.fixture(scope="module")
def long_context(gpu):
    """The 32k-token Llama-3-8B-shaped sequence, on the host and on the GPU."""
    w = workloads.prefill_bf16_long_llama3_8b()
    return w, w.to(gpu), np32(w.k_pool), np32(w.v_pool)


@pytest.mark.parametrize("chunk", range(16))
def test_long_context_chunks(ops, gpu, long_context, chunk):
    """All 16 successive 2048-token chunks, on sampled rows (tile edges included)."""
    w, wd, kp, vp = long_context
    q, meta = workloads.long_context_chunk(w, chunk, device=gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    rows = sample_rows(meta.raw_cu_seqlens, 24, np.random.default_rng(chunk))
    want = oa.paged_prefill(np64(q), kp, vp, meta.raw_cu_seqlens, np_tables(meta), meta.kv_lens.tolist(),
                            np.asarray(meta.raw_positions), rows=rows)
    mask = np.zeros(want.shape, dtype=bool)
    mask[:, rows] = True
    assert_close(out, want, torch.bfloat16, f"long-context chunk {chunk}", mask=mask)


@pytest.mark.parametrize("chunk", [0, 7, 15])
def test_long_context_chunks_every_row(ops, gpu, long_context, chunk):
    """Every row of the first, a middle and the last 2048-token chunk (32 heads,
    up to 32,768 keys), under the scale-aware per-row bound; the oracle runs over
    512-row slices to bound its memory."""
    w, wd, kp, vp = long_context
    q, meta = workloads.long_context_chunk(w, chunk, device=gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    qn, tables = np64(q), np_tables(meta)
    want = np.empty(tuple(out.shape), dtype=np.float64)
    for r0 in range(0, out.shape[1], 512):
        rows = list(range(r0, min(out.shape[1], r0 + 512)))
        part = oa.paged_prefill(qn, kp, vp, meta.raw_cu_seqlens, tables, meta.kv_lens.tolist(),
                                np.asarray(meta.raw_positions), rows=rows)
        want[:, rows] = part[:, rows]
    err = assert_close(out, want, torch.bfloat16, f"long-context chunk {chunk}, every row")
    print(f"chunk {chunk}: max abs err {err:.2e}")


def test_long_context_whole_prompt_one_call(ops, gpu, long_context):
    """The 32,768-token sequence as one fresh prompt in a single call, the largest chunk a call takes
    here (1,024 query tiles per KV head, 16 dispatch rounds of the resident slots): sampled rows, the
    edges of the first and of several later query tiles, and the last rows, which see every key."""
    w, wd, kp, vp = long_context
    q, meta = workloads.long_context_chunk(w, 0, chunk=32768, device=gpu)
    assert q.shape[1] == 32768 and meta.kv_lens.tolist() == [32768]
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    rows = set(sample_rows(meta.raw_cu_seqlens, 40, np.random.default_rng(32768)))
    rows.update({2047, 2048, 16383, 16384, 32735, 32736, 32766})
    rows = sorted(rows)
    want = oa.paged_prefill(np64(q), kp, vp, meta.raw_cu_seqlens, np_tables(meta), meta.kv_lens.tolist(),
                            np.asarray(meta.raw_positions), rows=rows)
    mask = np.zeros(want.shape, dtype=bool)
    mask[:, rows] = True
    err = assert_close(out, want, torch.bfloat16, "32k-token prompt in one call", mask=mask)
    print(f"32k prompt, {len(rows)} rows: max abs err {err:.2e}")


@pytest.fixture(scope="module")
def mixed(gpu):
    """The unified Qwen3-8B-shaped batch and the oracle for every row of it.

    Sequence 0 is a 1024-token chunk on a 4096-token prefix, sequences
    1..127 are decode rows with contexts U[512, 8192]; the even sequences
    share their first 64 physical blocks.
    """
    w = workloads.mixed_bf16_qwen3_8b()
    q, meta = w.gemm_call()
    want = oracle_prefill(q, meta, w.k_pool, w.v_pool)  # (H, 1024 + 127, D), every row
    return w, w.to(gpu), want


def test_mixed_batch_single_call(ops, gpu, mixed):
    """All 128 sequences in one paged_attention_gemm call (the CUSTOM_GEMM route,
    femtovllm/models/qwen/qwen3.py:575-580): every prefill and decode row."""
    w, wd, want = mixed
    q, meta = w.gemm_call(device=gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    err = assert_close(out, want, torch.bfloat16, "mixed batch, one call")
    print(f"mixed single call max abs err {err:.2e}")


def test_mixed_batch_prefill_plus_decode_route(ops, gpu, mixed):
    """The reference's default route (femtovllm/engine/model_runner.py:97-141): a
    paged_attention_gemm call for the chunk and a paged_attention_gemv call for
    the 127 decode rows (H=32, KVH=8, up to 8192 keys over shared blocks)."""
    w, wd, want = mixed
    qp, mp = w.gemm_call(seqs=[0], device=gpu)
    outp = run_gemm(ops, qp, mp, wd.k_pool, wd.v_pool, gpu)
    qd, md = w.gemv_call(seqs=range(1, 128), device=gpu)
    outd = ops.paged_attention_gemv(qd.to(gpu), wd.k_pool, wd.v_pool, md.block_tables, md.kv_lens, md.max_kv_len)
    torch.cuda.synchronize()
    assert md.max_kv_len <= 8192
    e1 = assert_close(outp, want[:, :1024], torch.bfloat16, "mixed route: prefill call")
    e2 = assert_close(outd, want[:, 1024:], torch.bfloat16, "mixed route: decode call")
    print(f"mixed route max abs err: prefill {e1:.2e}, decode {e2:.2e}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads", [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4), (6, 1)])
def test_prefill_gqa_and_dtypes(ops, gpu, dtype, heads):
    H, KVH = heads
    rng = np.random.default_rng(H * 7 + KVH)
    chunks = [(int(rng.integers(0, 300)), int(rng.integers(1, 200))) for _ in range(4)] + [(0, 1), (31, 33)]
    w = workloads.make_paged_workload("gqa", chunks, H, KVH, dtype=dtype, seed=H + 3 * KVH)
    check_workload(ops, w, gpu, what=f"prefill H={H} KVH={KVH} {dtype}")


def test_arbitrary_positions(ops, gpu):
    """The mask comes from positions[], not from the chunk layout."""
    w = workloads.make_paged_workload("pos", [(60, 40), (0, 70)], 16, 8, seed=21)
    q, meta = w.gemm_call(device=gpu)
    rng = np.random.default_rng(21)
    pos = []
    for (p, n) in w.chunks:
        pos.extend(int(x) for x in rng.integers(0, p + n, size=n))
    meta.positions = torch.tensor(pos, dtype=torch.int32, device=gpu)
    meta.raw_positions = pos
    wd = w.to(gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    assert_close(out, oracle_prefill(q, meta, w.k_pool, w.v_pool), torch.bfloat16, "arbitrary positions")


def test_causal_boundary_spike_is_exact(ops, gpu):
    """Key j = positions[t] is selected bit-exactly; key positions[t] + 1 is not.

    Token i (position 50 + i) queries along its own dim i.  Even tokens get a
    spike key at their own position, odd tokens one position later.
    """
    H, KVH = 2, 1
    L, n = 150, 100
    w = workloads.make_paged_workload("causal", [(L - n, n)], H, KVH, seed=22)
    w.k_pool.zero_()
    w.q.zero_()
    table = w.raw_block_tables[0]
    for i in range(n):
        p = L - n + i + (i % 2)
        w.q[:, i, i] = 3000.0
        if p < L:
            w.k_pool[table[p // 16], 0, p % 16, i] = 1.0
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu).cpu()
    for i in range(0, n, 2):
        p = L - n + i
        want = w.v_pool[table[p // 16], 0, p % 16]
        for h in range(H):
            assert torch.equal(out[h, i], want), f"token {i}: key at its own position not selected exactly"
    want = oracle_prefill(q, meta, w.k_pool, w.v_pool)
    assert_close(out, want, torch.bfloat16, "causal boundary")


def test_empty_sequences_and_kv_len_zero(ops, gpu):
    """Zero-length chunks produce no rows; kv_len == 0 rows are NaN as in the reference."""
    w = workloads.make_paged_workload("empty", [(10, 5), (20, 0), (0, 3)], 8, 4, seed=23)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    assert_close(out, oracle_prefill(q, meta, w.k_pool, w.v_pool), torch.bfloat16, "empty seq")
    kv0 = meta.kv_lens.clone()
    kv0[2] = 0
    out = ops.paged_attention_gemm(q.to(gpu), wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len, 32,
                                   meta.cu_q_tiles, meta.q_tile_to_seq_idx, meta.block_tables, kv0, meta.positions)
    torch.cuda.synchronize()
    assert torch.isnan(out[:, 5:8].float()).all()
    assert not torch.isnan(out[:, :5].float()).any()


def test_one_token_chunk_equals_decode(ops, gpu):
    w = workloads.make_paged_workload("dec", [(L - 1, 1) for L in (33, 700, 1500)], 16, 8, seed=24)
    wd = w.to(gpu)
    q, meta = w.gemm_call(device=gpu)
    a = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    b = ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    assert (a.float() - b.float()).abs().max().item() <= 2e-2


def test_strided_q_and_errors(ops, gpu):
    w = workloads.make_paged_workload("st", [(30, 50)], 16, 8, seed=25)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    strided = q.transpose(0, 1).contiguous().to(gpu).transpose(0, 1)
    a = run_gemm(ops, strided, meta, wd.k_pool, wd.v_pool, gpu)
    b = run_gemm(ops, strided.contiguous(), meta, wd.k_pool, wd.v_pool, gpu)
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        run_gemm(ops, q.cpu(), meta, wd.k_pool, wd.v_pool, "cpu")
    with pytest.raises(NotImplementedError):
        run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu, impl="opencl")
    with pytest.raises(RuntimeError):
        qf = q.float().to(gpu)
        run_gemm(ops, qf, meta, wd.k_pool.float(), wd.v_pool.float(), gpu)


def test_mixed_batch_tp8_share_both_routes(ops, gpu):
    """One GPU's share of the unified batch under 8-way tensor parallelism
    (4 query heads, 1 KV head): the single call and the prefill + decode
    route, every decode row and sampled rows of the 1024-token chunk."""
    w = workloads.mixed_bf16_qwen3_8b_tp8_share()
    q, meta = w.gemm_call()
    cu = meta.raw_cu_seqlens
    rows = sorted(set(sample_rows(cu[:2], 48, np.random.default_rng(3))) | set(range(1024, cu[-1])))
    want = oa.paged_prefill(np64(q), np32(w.k_pool), np32(w.v_pool), cu, np_tables(meta), meta.kv_lens.tolist(),
                            np.asarray(meta.raw_positions), rows=rows)
    mask = np.zeros(want.shape, dtype=bool)
    mask[:, rows] = True
    wd = w.to(gpu)
    qg, mg = w.gemm_call(device=gpu)
    out = run_gemm(ops, qg, mg, wd.k_pool, wd.v_pool, gpu)
    assert_close(out, want, torch.bfloat16, "tp8 share mixed batch, one call", mask=mask)
    qp, mp = w.gemm_call(seqs=[0], device=gpu)
    outp = run_gemm(ops, qp, mp, wd.k_pool, wd.v_pool, gpu)
    qd, md = w.gemv_call(seqs=range(1, 128), device=gpu)
    outd = ops.paged_attention_gemv(qd.to(gpu), wd.k_pool, wd.v_pool, md.block_tables, md.kv_lens, md.max_kv_len)
    torch.cuda.synchronize()
    assert_close(torch.cat([outp, outd], dim=1), want, torch.bfloat16, "tp8 share mixed batch, two calls",
                 mask=mask)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [16, 48, 64, 96, 112])
def test_prefill_head_dim_below_128(ops, gpu, monkeypatch, dtype, head_dim):
    """head_dim < 128 in multiples of 16, as the reference's check allows (TORCH_CHECK_LE(dim_d, kDimHead),
    csrc/paged_attention/paged_attention_gemm.cu:347-348): fresh prompts, cached prefixes, a key-split
    long sequence and one-token rows (the fused decode workers), against the oracle and against the
    call without key split; the pools' unused blocks and tail rows are NaN."""
    from test_prefill_split_gpu import _unsplit

    chunks = [(0, 70), (300, 45), (5000, 96), (17, 1), (2000, 1), (0, 1), (64, 33)]
    H, KVH = 16, 8 if head_dim != 48 else 4
    w = workloads.make_paged_workload("hd", chunks, H, KVH, head_dim=head_dim, dtype=dtype, seed=head_dim)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    out = run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
    assert out.shape == (H, q.shape[1], head_dim)
    want = oracle_prefill(q, meta, w.k_pool, w.v_pool)
    what = f"prefill head_dim {head_dim} {dtype}"
    assert_close(out, want, dtype, what)
    ref = _unsplit(ops, q.to(gpu), meta, wd, monkeypatch)
    assert_agree(out, ref, dtype, what + " vs unsplit")


@pytest.mark.parametrize("head_dim", [136, 72, 8])
def test_prefill_head_dim_rejects(ops, gpu, head_dim):
    w = workloads.make_paged_workload("hdx", [(10, 20)], 8, 8, head_dim=head_dim, seed=3)
    q, meta = w.gemm_call(device=gpu)
    wd = w.to(gpu)
    with pytest.raises(RuntimeError, match="head_dim must be"):
        run_gemm(ops, q, meta, wd.k_pool, wd.v_pool, gpu)
