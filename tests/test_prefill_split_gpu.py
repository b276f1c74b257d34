"""Key split of long query tiles in the HIP prefill kernel.

With a workspace, femto_paged_attention_gemm cuts the query tiles of
sequences much longer than the average work per resident workgroup into up
to eight pieces over their keys; the last piece to finish merges the others'
partial softmax states within the launch.  The results must match the oracle
(the reference's attention, paged_attention_gemm.py:83-160) and the unsplit
kernel, and every call must leave the split counters zero-filled.
"""

import dataclasses

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_agree, assert_close, np32, np64, np_tables, sample_rows

pytestmark = pytest.mark.gpu


def _gemm(ops, q, meta, wd):
    out = ops.paged_attention_gemm(q, wd.k_pool, wd.v_pool, meta.cu_seqlens, meta.max_q_len, meta.Q_TILE_SIZE,
                                   meta.cu_q_tiles, meta.q_tile_to_seq_idx, meta.block_tables, meta.kv_lens,
                                   meta.positions)
    torch.cuda.synchronize()
    return out


def _unsplit(ops, q, meta, wd, monkeypatch):
    from femtovllm import _C

    with monkeypatch.context() as m:
        m.setattr(_C, "_prefill_workspace", lambda *args: (None, 0))
        return _gemm(ops, q, meta, wd)


def _workspace_is_zero(device):
    """The key-split counters of every cached workspace (its first
    femto_paged_attention_gemm_split_bytes() bytes from the 256-byte aligned
    start) are back to zeros."""
    from femtovllm import _C

    split = int(_C._lib.femto_paged_attention_gemm_split_bytes())
    for key, ws in _C._prefill_workspaces.items():
        off = (-ws.data_ptr()) % 256
        if key[0] == device.index and int(torch.count_nonzero(ws[off:off + split])) != 0:
            return False
    return True


def split_plan(chunks, n_heads, n_kv_heads, cus):
    """Pieces per query tile of each sequence, by the kernel's rule: T = the
    causal-estimated key tiles per resident workgroup (two per CU), pieces =
    round(key tiles / T) capped at 8; while the pieces do not all fit in the
    resident slots at once, T grows by half (three times at most), then the
    call is not split."""
    n_rep = n_heads // n_kv_heads
    G = 4 if n_rep % 4 == 0 else 2 if n_rep % 2 == 0 else 1
    BT = 32 * (4 // G)
    groups = n_kv_heads * (n_rep // G)
    resident = 2 * cus
    est = 0
    for pos, n in chunks:
        kvl = pos + n
        if n > 0 and kvl > 0:
            mean_keys = min(kvl, max(1, kvl - n + (n + BT) // 2))
            est += -(-n // BT) * -(-mean_keys // 64)
    T = max(8, -(-est * groups // resident))
    for _ in range(4):
        pieces = [min(8, max(1, (2 * -(-(p + n) // 64) + T) // (2 * T))) if p + n > 0 else 1 for p, n in chunks]
        if groups * sum(-(-n // BT) * pp for (p, n), pp in zip(chunks, pieces)) <= resident:
            return pieces
        T += T // 2
    return [1] * len(chunks)


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


def _check(ops, w, gpu, monkeypatch, rows_per_seq=6, what=""):
    q, meta = w.gemm_call(device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    out = _gemm(ops, q, meta, wd)
    assert _workspace_is_zero(gpu), f"split counters not reset after {what}"
    cu = meta.raw_cu_seqlens
    # sequences of one token run on the decode kernel (its own rounding), so
    # they are checked against the oracle, every one, and not against the
    # unsplit MFMA result
    one = [cu[b] for b in range(len(cu) - 1) if cu[b + 1] - cu[b] == 1]
    rows = sorted(set(sample_rows(cu, rows_per_seq, np.random.default_rng(1))) | set(one))
    want = oa.paged_prefill(np64(q.cpu()), np32(w.k_pool), np32(w.v_pool), cu, np_tables(meta),
                            meta.kv_lens.tolist(), np.asarray(meta.raw_positions), rows=rows)
    mask = np.zeros(want.shape, dtype=bool)
    mask[:, rows] = True
    err = assert_close(out, want, w.dtype, what, mask=mask)
    ref = _unsplit(ops, q, meta, wd, monkeypatch)
    multi = np.ones(want.shape, dtype=bool)
    multi[:, one] = False
    assert_agree(out, ref, w.dtype, what + " vs unsplit", mask=multi)
    return err


# One long sequence among short ones: the long one's query tiles are split
# into 8, 6, 3 or 2 pieces.
@pytest.mark.parametrize("long_prefix,pieces", [(6000, 8), (2600, 6), (1300, 3), (800, 2)])
def test_long_sequence_among_short(ops, gpu, monkeypatch, long_prefix, pieces):
    chunks = [(long_prefix, 192)] + [(int(p), 64) for p in np.linspace(0, 300, 40)]
    assert split_plan(chunks, 16, 8, _cus())[0] == pieces
    w = workloads.make_paged_workload(f"split{long_prefix}", chunks, 16, 8, seed=long_prefix)
    err = _check(ops, w, gpu, monkeypatch, what=f"long prefix {long_prefix}")
    print(f"long prefix {long_prefix}: {pieces} pieces, max abs err {err:.2e}")


def test_partial_slots_need_no_zeros(ops, gpu, monkeypatch):
    """Only the counters must start at zero: every partial slot a merge reads
    was written in the same call.  With everything behind the counters (the
    partial slots) filled with 0xff bytes, NaN in every float, a call split
    into 8 pieces per long query tile still matches the oracle."""
    from femtovllm import _C

    chunks = [(6000, 192)] + [(int(p), 64) for p in np.linspace(0, 300, 40)]
    assert split_plan(chunks, 16, 8, _cus())[0] == 8
    w = workloads.make_paged_workload("dirty_slots", chunks, 16, 8, seed=6000)
    q, meta = w.gemm_call(device=gpu)
    _gemm(ops, q.to(gpu), meta, w.to(gpu))  # the cached workspace exists from here on
    counters = int(_C._lib.femto_paged_attention_gemm_split_bytes())
    filled = 0
    for key, ws in _C._prefill_workspaces.items():
        if key[0] == gpu.index:
            off = (-ws.data_ptr()) % 256
            ws[off + counters:].fill_(0xFF)
            filled += 1
    torch.cuda.synchronize()
    assert filled
    _check(ops, w, gpu, monkeypatch, what="partial slots full of 0xff bytes")


def test_fresh_prompt_is_split_by_causal_length(ops, gpu, monkeypatch):
    """A single 1024-token prompt without prefix: its late query tiles see
    about twice the average keys and are split in two."""
    chunks = [(0, 1024)]
    assert split_plan(chunks, 16, 8, _cus()) == [2]
    w = workloads.make_paged_workload("fresh", chunks, 16, 8, seed=77)
    _check(ops, w, gpu, monkeypatch, rows_per_seq=48, what="fresh 1024-token prompt")


def test_pieces_shrink_to_fit_resident_slots(ops, gpu, monkeypatch):
    """Four long sequences whose first split needs more pieces than resident
    slots: T grows until only the two longest are split (in three)."""
    chunks = [(3000, 512), (200, 512), (4000, 256), (100, 1024)]
    assert split_plan(chunks, 16, 8, _cus()) == [3, 1, 3, 1]
    w = workloads.make_paged_workload("shrink", chunks, 16, 8, seed=79)
    _check(ops, w, gpu, monkeypatch, rows_per_seq=24, what="pieces shrunk to fit")


def test_full_gpu_call_is_not_split(ops, gpu, monkeypatch):
    """A 2048-token prompt with 32 heads fills every resident slot with query
    tiles already: the call runs unsplit, bit-identical to no workspace."""
    chunks = [(0, 2048)]
    assert split_plan(chunks, 32, 8, _cus()) == [1]
    w = workloads.make_paged_workload("full", chunks, 32, 8, seed=78)
    q, meta = w.gemm_call(device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    assert torch.equal(_gemm(ops, q, meta, wd), _unsplit(ops, q, meta, wd, monkeypatch))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads", [(16, 8), (32, 8), (12, 4), (6, 1), (8, 8)])
def test_split_gqa_and_dtypes(ops, gpu, monkeypatch, dtype, heads):
    H, KVH = heads
    chunks = [(3000, 100), (5, 33), (40, 64), (0, 1), (200, 70)]
    assert split_plan(chunks, H, KVH, _cus())[0] > 1
    w = workloads.make_paged_workload("splitgqa", chunks, H, KVH, dtype=dtype, seed=H * 10 + KVH)
    _check(ops, w, gpu, monkeypatch, what=f"split H={H} KVH={KVH} {dtype}")


def test_arbitrary_positions_with_split(ops, gpu, monkeypatch):
    """Positions that are not the last q_len keys: some pieces see no visible
    key for some rows (their state is empty and must merge away)."""
    chunks = [(4000, 96), (10, 64), (30, 64), (50, 64)]
    assert split_plan(chunks, 16, 8, _cus())[0] == 8
    w = workloads.make_paged_workload("splitpos", chunks, 16, 8, seed=91)
    q, meta = w.gemm_call(device=gpu)
    rng = np.random.default_rng(92)
    pos = np.asarray(meta.raw_positions).copy()
    s0, s1 = meta.raw_cu_seqlens[0], meta.raw_cu_seqlens[1]
    pos[s0:s1] = rng.integers(0, meta.kv_lens.tolist()[0], size=s1 - s0)  # any visible limit inside the context
    meta.raw_positions = [int(x) for x in pos]
    meta.positions = torch.tensor(pos, dtype=torch.int32, device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    out = _gemm(ops, q, meta, wd)
    assert _workspace_is_zero(gpu)
    want = oa.paged_prefill(np64(q.cpu()), np32(w.k_pool), np32(w.v_pool), meta.raw_cu_seqlens, np_tables(meta),
                            meta.kv_lens.tolist(), pos, rows=list(range(s0, s1)))
    mask = np.zeros(want.shape, dtype=bool)
    mask[:, s0:s1] = True
    assert_close(out, want, w.dtype, "arbitrary positions, split", mask=mask)


def test_back_to_back_shapes_share_workspace(ops, gpu, monkeypatch):
    """Calls of different shapes reuse one workspace: counters and partial
    slots of one call must not leak into the next."""
    cases = [
        [(6000, 192)] + [(10, 64)] * 30,
        [(0, 2048)],
        [(2000, 512)] * 2 + [(0, 17)] * 50,
        [(9000, 64), (8000, 64), (10, 32)],
    ]
    for i, chunks in enumerate(cases):
        w = workloads.make_paged_workload(f"reuse{i}", chunks, 16, 8, seed=300 + i)
        _check(ops, w, gpu, monkeypatch, rows_per_seq=4, what=f"shape sequence case {i}")


@pytest.mark.parametrize("num_seqs", [300, 700])
def test_many_sequences(ops, gpu, monkeypatch, num_seqs):
    """More sequences than one workgroup pass covers (256): the kernel's
    per-sequence passes run over several chunks, and the work item of a
    query tile past the first 256 sequences is found in a later chunk.  A
    few long contexts among them are split when their pieces fit."""
    rng = np.random.default_rng(num_seqs)
    chunks = []
    for i in range(num_seqs):
        if i % 97 == 5:
            chunks.append((int(rng.integers(3000, 6000)), int(rng.integers(64, 200))))  # long context
        elif i % 3 == 0:
            chunks.append((int(rng.integers(0, 400)), 1))  # decode token
        else:
            chunks.append((int(rng.integers(0, 300)), int(rng.integers(1, 40))))
    w = workloads.make_paged_workload(f"many{num_seqs}", chunks, 16, 8, seed=num_seqs)
    _check(ops, w, gpu, monkeypatch, rows_per_seq=1, what=f"{num_seqs} sequences")


def test_many_sequences_with_one_split(ops, gpu, monkeypatch):
    """300 sequences of one decode token each and one long chunk at the end,
    one KV head (so the pieces fit the resident slots): the long sequence
    (index 300) is split and lives in the second chunk of the kernel's
    per-sequence passes."""
    chunks = [(int(p), 1) for p in np.linspace(10, 500, 300)] + [(8000, 128)]
    assert split_plan(chunks, 2, 1, _cus())[-1] == 8
    w = workloads.make_paged_workload("many_split", chunks, 2, 1, seed=261)
    _check(ops, w, gpu, monkeypatch, rows_per_seq=2, what="300 decode + 1 long")


def test_tp8_share_long_chunk(ops, gpu, monkeypatch):
    """One GPU's share under 8-way tensor parallelism (4 query heads, 1 KV
    head): a 2048-token chunk after a 6144-token prefix has 64 query tiles for
    the whole GPU, and each is split into 8 pieces.

    The handoff crosses XCDs on every tile: the work list is piece-major
    (piece p of query tile i is item i + 64 p) and each XCD (workgroup id
    mod 8) takes a contiguous eighth of the 512 items, so the 8 pieces of a
    tile run on 8 different XCDs and the merging piece reads partials that
    the other 7 wrote through their own L2s."""
    chunks = [(6144, 2048)]
    assert split_plan(chunks, 4, 1, _cus()) == [8]
    w = workloads.make_paged_workload("tp8", chunks, 4, 1, seed=1004)
    _check(ops, w, gpu, monkeypatch, rows_per_seq=64, what="tp8 share chunk")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_values_beyond_fp16_range(ops, gpu, monkeypatch, dtype):
    """bf16 key-split partials travel as fp16 scaled by a per-lane power of
    two.  V scaled by 2^18 (past fp16's 65504, exact in bf16) must give the
    output scaled by 2^18, split and unsplit (f16 storage keeps fp32
    partials and is checked the same way at 2^10)."""
    chunks = [(6000, 192)] + [(int(p), 64) for p in np.linspace(0, 300, 40)]
    assert split_plan(chunks, 16, 8, _cus())[0] == 8
    w = workloads.make_paged_workload("split_range", chunks, 16, 8, dtype=dtype, seed=81, poison=False)
    scale = 2.0**18 if dtype == torch.bfloat16 else 2.0**10
    q, meta = w.gemm_call(device=gpu)
    q = q.to(gpu)
    wd = w.to(gpu)
    big = dataclasses.replace(wd, v_pool=wd.v_pool * scale)
    assert torch.isfinite(big.v_pool).all()
    out = _gemm(ops, q, meta, wd)
    out_big = _gemm(ops, q, meta, big)
    assert torch.isfinite(out_big).all()
    assert_agree(out_big.float() / scale, out, dtype, "V x 2^k, split")
    ref_big = _unsplit(ops, q, meta, big, monkeypatch)
    assert_agree(out_big.float() / scale, ref_big.float() / scale, dtype, "V x 2^k vs unsplit")
    assert _workspace_is_zero(gpu)


def test_too_small_workspace_is_rejected(ops, gpu):
    """The C ABI checks the workspace against one slot per resident workgroup."""
    from femtovllm import _C

    need = _C._lib.femto_paged_attention_gemm_workspace_size(2, 10, 5, 16, 8, 4)
    assert need >= _cus() * 2 * 67584
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    q = torch.zeros((16, 10, 128), dtype=torch.bfloat16, device=gpu)
    pool = torch.zeros((8, 8, 16, 128), dtype=torch.bfloat16, device=gpu)
    out = torch.empty_like(q)
    cu = torch.tensor([0, 5, 10], dtype=torch.int32, device=gpu)
    tables = torch.zeros((2, 4), dtype=torch.int32, device=gpu)
    kv = torch.tensor([5, 5], dtype=torch.int32, device=gpu)
    pos = torch.arange(10, dtype=torch.int32, device=gpu) % 5
    args = [2, q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
            pool.data_ptr(), pool.data_ptr(), 8, 8, 16, 128, pool.stride(0), pool.stride(1), pool.stride(2),
            cu.data_ptr(), 2, 10, 5, 16, tables.data_ptr(), 4, tables.stride(0), kv.data_ptr(), pos.data_ptr()]
    rc = _C._lib.femto_paged_attention_gemm(*args, ws.data_ptr(), need - 256, None)
    assert rc == 1 and "workspace" in _C._lib.femto_attn_last_error().decode()
    rc = _C._lib.femto_paged_attention_gemm(*args, ws.data_ptr(), need, None)
    torch.cuda.synchronize()
    assert rc == 0 and int(torch.count_nonzero(ws)) == 0
