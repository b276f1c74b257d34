"""Parity of the HIP decode kernel (femto_paged_attention_gemv) with the oracle.

Reference behaviour: PagedAttentionGemvCuda
(csrc/paged_attention/paged_attention_gemv.cu:223-308) behind
femtovllm.ops.paged_attention_gemv (femtovllm/ops/__init__.py:82-107).
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from femtovllm.metadata import build_varlen_metadata
from helpers import assert_close, np32, np64, np_tables

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("decode_path")]


def run_decode(ops, w, device, seqs=None):
    q, meta = w.gemv_call(seqs=seqs, device=device)
    wd = w.to(device)
    out = ops.paged_attention_gemv(q.to(device), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    torch.cuda.synchronize()
    return out, q, meta


def oracle_decode(w, q, meta):
    return oa.paged_decode(np64(q), np32(w.k_pool), np32(w.v_pool), np_tables(meta), meta.kv_lens.tolist())


def test_decode_fp32_four_sequences(ops, gpu):
    w = workloads.decode_fp32_small()
    out, q, meta = run_decode(ops, w, gpu)
    err = assert_close(out, oracle_decode(w, q, meta), torch.float32, "fp32 decode")
    print(f"fp32 decode max abs err {err:.2e}")


def test_decode_bf16_qwen3_shape(ops, gpu):
    w = workloads.decode_bf16_qwen3_0p6b()
    out, q, meta = run_decode(ops, w, gpu)
    err = assert_close(out, oracle_decode(w, q, meta), torch.bfloat16, "bf16 decode B=64")
    print(f"bf16 decode max abs err {err:.2e}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("heads", [(8, 8), (16, 8), (32, 8), (64, 8), (12, 4), (6, 1)])
def test_decode_gqa_and_dtypes(ops, gpu, dtype, heads):
    H, KVH = heads
    rng = np.random.default_rng(H * 100 + KVH)
    lens = [int(x) for x in rng.integers(1, 700, size=5)] + [16, 17]
    w = workloads.make_paged_workload("gqa", [(L - 1, 1) for L in lens], H, KVH, dtype=dtype, seed=H + KVH)
    out, q, meta = run_decode(ops, w, gpu)
    assert_close(out, oracle_decode(w, q, meta), dtype, f"decode H={H} KVH={KVH} {dtype}")


def test_decode_long_context_split_merge(ops, gpu):
    """Contexts up to kMaxKVLenNonSplit exercise the multi-split merge."""
    lens = [8192, 1, 4097, 8191, 300]
    w = workloads.make_paged_workload("long", [(L - 1, 1) for L in lens], 16, 8, seed=11)
    out, q, meta = run_decode(ops, w, gpu)
    assert_close(out, oracle_decode(w, q, meta), torch.bfloat16, "long decode")


def test_decode_gather_is_bit_exact(ops, gpu):
    """A dominant key at logical index j* returns V[j*] bit for bit, for every j*."""
    L = 100
    B = L
    H, KVH, D = 4, 2, 128
    w = workloads.make_paged_workload("spike", [(L - 1, 1)] * B, H, KVH, seed=12)
    w.k_pool.zero_()
    ktab = w.raw_block_tables
    for b in range(B):
        page, row = ktab[b][b // 16], b % 16
        w.k_pool[page, :, row, 0] = 1.0
    w.q.zero_()
    w.q[:, :, 0] = 2000.0
    out, q, meta = run_decode(ops, w, gpu)
    out = out.cpu()
    for b in range(B):
        page, row = ktab[b][b // 16], b % 16
        for h in range(H):
            want = w.v_pool[page, h // 2, row]
            assert torch.equal(out[h, b], want), f"seq {b} head {h}: gather of key {b} not exact"


def test_decode_empty_context_returns_zeros(ops, gpu):
    w = workloads.make_paged_workload("empty", [(4, 1), (0, 1)], 8, 4, seed=13)
    q, meta = w.gemv_call(device=gpu)
    kv_lens = meta.kv_lens.clone()
    kv_lens[1] = 0
    wd = w.to(gpu)
    out = ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, kv_lens, meta.max_kv_len)
    assert torch.all(out[:, 1] == 0)
    want = oa.paged_decode(np64(q), np32(w.k_pool), np32(w.v_pool), np_tables(meta), [5, 0])
    assert_close(out, want, torch.bfloat16, "empty context")


def test_decode_strided_q_matches_contiguous(ops, gpu):
    """q as the caller passes it, (tokens, H, D).transpose(0, 1), needs no copy."""
    w = workloads.make_paged_workload("strided", [(99, 1), (40, 1), (7, 1)], 16, 8, seed=14)
    wd = w.to(gpu)
    q, meta = w.gemv_call(device=gpu)
    q_thd = q.transpose(0, 1).contiguous().to(gpu)  # (B, H, D)
    strided = q_thd.transpose(0, 1)
    assert not strided.is_contiguous()
    a = ops.paged_attention_gemv(strided, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    b = ops.paged_attention_gemv(strided.contiguous(), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                 meta.max_kv_len)
    assert torch.equal(a, b)


def test_decode_back_to_back_calls_reuse_workspace(ops, gpu):
    """Consecutive calls of different sizes share the per-stream workspace."""
    big = workloads.make_paged_workload("ws1", [(5000, 1)] * 3 + [(200, 1)], 16, 8, seed=15)
    small = workloads.make_paged_workload("ws2", [(3000, 1), (100, 1)], 16, 8, seed=16)
    for w in (big, small, big):
        out, q, meta = run_decode(ops, w, gpu)
        assert_close(out, oracle_decode(w, q, meta), torch.bfloat16, f"workspace reuse {w.name}")


def test_decode_shape_changes_share_workspace(ops, gpu):
    """Regression: calls of different shapes share one workspace.

    An earlier design kept split counters in the workspace at a shape-
    dependent offset, so a later call could find an earlier call's partials
    there; any state carried between calls in the workspace would fail here.
    """
    shapes = [
        ("a", [(L - 1, 1) for L in (4000, 3000, 2500, 100) * 16], 16, 8),
        ("b", [(L - 1, 1) for L in (230, 273, 161, 269, 98, 16, 17)], 16, 8),
        ("c", [(L - 1, 1) for L in (900, 1800)], 32, 8),
        ("d", [(L - 1, 1) for L in (700, 60, 1300)], 8, 8),
    ]
    for name, chunks, H, KVH in shapes:
        w = workloads.make_paged_workload(name, chunks, H, KVH, dtype=torch.float16, seed=len(chunks) + H)
        out, q, meta = run_decode(ops, w, gpu)
        assert_close(out, oracle_decode(w, q, meta), torch.float16, f"shape change {name}")


def test_decode_large_batch(ops, gpu):
    """1100 short sequences: each wave's slice holds many sequence segments."""
    rng = np.random.default_rng(19)
    lens = [int(x) for x in rng.integers(1, 300, size=1100)]
    w = workloads.make_paged_workload("many", [(L - 1, 1) for L in lens], 16, 8, seed=19)
    out, q, meta = run_decode(ops, w, gpu)
    assert_close(out, oracle_decode(w, q, meta), torch.bfloat16, "1100 sequences")


def test_decode_out_of_pool_block_is_a_zero_page(ops, gpu):
    """A table entry outside the pool is never dereferenced; it reads as zeros."""
    w = workloads.make_paged_workload("badblk", [(47, 1)], 8, 4, seed=17, poison=False)
    q, meta = w.gemv_call(device=gpu)
    tables = meta.block_tables.clone()
    tables[0, 1] = w.k_pool.shape[0] + 1000
    wd = w.to(gpu)
    out = ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, tables, meta.kv_lens, meta.max_kv_len)
    kp, vp = np32(w.k_pool), np32(w.v_pool)
    kp = np.concatenate([kp, np.zeros_like(kp[:1])])
    vp = np.concatenate([vp, np.zeros_like(vp[:1])])
    t = np_tables(meta)
    t[0, 1] = kp.shape[0] - 1
    want = oa.paged_decode(np64(q), kp, vp, t, meta.kv_lens.tolist())
    assert_close(out, want, torch.bfloat16, "out-of-pool block")


def test_decode_errors(ops, gpu):
    w = workloads.make_paged_workload("err", [(3, 1)], 8, 4, seed=18)
    q, meta = w.gemv_call(device=gpu)
    wd = w.to(gpu)
    with pytest.raises(ValueError):
        ops.paged_attention_gemv(q, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    with pytest.raises(NotImplementedError):
        ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                 meta.max_kv_len, impl="opencl")
    with pytest.raises(RuntimeError):
        ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables.long(), meta.kv_lens,
                                 meta.max_kv_len)
    with pytest.raises(RuntimeError):
        ops.paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, 8193)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.bfloat16, 96), (torch.float16, 8),
                                     (torch.float16, 120), (torch.float32, 64), (torch.float32, 4),
                                     (torch.float32, 100)])
def test_decode_head_dim_below_128(ops, gpu, dtype, D):
    """head_dim <= 128 as the reference's decode accepts (TORCH_CHECK_LE(dim_d, kDimHead),
    csrc/paged_attention/paged_attention_gemv.cu:256-257): rows of D elements, scale
    1/sqrt(D); NaN-poisoned tails and unused blocks sit right after the rows read."""
    rng = np.random.default_rng(D)
    lens = [int(x) for x in rng.integers(1, 1500, size=6)] + [16, 1]
    w = workloads.make_paged_workload("head_dim", [(L - 1, 1) for L in lens], 16, 4, head_dim=D, dtype=dtype,
                                      seed=D + 5)
    from femtovllm import _C

    q, meta = w.gemv_call(device=gpu)
    wd = w.to(gpu)
    out = _C._paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                   meta.max_kv_len)
    torch.cuda.synchronize()
    assert out.shape == (16, len(lens), D)
    assert_close(out, oracle_decode(w, q, meta), dtype, f"decode head_dim {D} {dtype}")


def test_decode_head_dim_errors(ops, gpu):
    from femtovllm import _C

    for D, dtype in ((136, torch.bfloat16), (100, torch.bfloat16), (6, torch.float32)):
        w = workloads.make_paged_workload("hd_err", [(30, 1)], 4, 2, head_dim=D, dtype=dtype, seed=1)
        q, meta = w.gemv_call(device=gpu)
        wd = w.to(gpu)
        with pytest.raises(RuntimeError, match="head_dim"):
            _C._paged_attention_gemv(q.to(gpu), wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens,
                                     meta.max_kv_len)
