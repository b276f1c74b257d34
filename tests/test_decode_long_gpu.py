"""Decode past kMaxKVLenNonSplit (8192 keys): the split-KV lift.

The reference caps decode at 8192 keys (csrc/utils/constants.cuh:36-39 leaves
split-K "to be implemented"; PagedAttentionGemvCuda checks max_kv_len <=
kMaxKVLenNonSplit, csrc/paged_attention/paged_attention_gemv.cu:271-274).  The
HIP decode kernel cuts every context into wave slices and merges their partial
softmax states, so any length runs.  These tests call the C ABI directly
(femto_paged_attention_gemv, which has no length check) and the Python
operator with ``femtovllm._DEV.split_kv_decode`` set, and compare every row with
the float64 oracle at the bf16 tolerance, for H/KVH = 32/8 (four query heads
per wave) and 16/8 (two).
"""

import numpy as np
import pytest
import torch

import femtovllm
import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_close, np32, np64, np_tables

pytestmark = pytest.mark.gpu

LENGTHS = (8193, 16384, 32768, 131072)


@pytest.fixture(scope="module")
def long_decode(gpu):
    """Four decode rows of 8193 .. 131072 keys over one 8-KV-head pool, q for 32 heads."""
    w = workloads.make_paged_workload("decode_long", [(L - 1, 1) for L in LENGTHS], 32, 8, seed=1010)
    q, meta = w.gemv_call(device=gpu)
    return w, w.to(gpu), q, meta, np32(w.k_pool), np32(w.v_pool)


def c_abi_decode(C, q, k_pool, v_pool, tables, kv_lens, max_kv_len):
    """femto_paged_attention_gemv through ctypes, with the workspace it asks for."""
    out = torch.empty_like(q)
    ws, ws_bytes = C._decode_workspace(q.device, q.size(1), q.size(0), max_kv_len)
    rc = C._lib.femto_paged_attention_gemv(
        2, q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.size(0), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        tables.data_ptr(), tables.size(1), tables.stride(0), kv_lens.data_ptr(), q.size(1), q.size(0), max_kv_len,
        ws, ws_bytes, C._stream(q.device))
    assert rc == 0, C._lib.femto_attn_last_error().decode()
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("n_heads", [32, 16])
def test_c_abi_decode_beyond_8192(gpu, long_decode, n_heads):
    from femtovllm import _C

    w, wd, q, meta, kp, vp = long_decode
    qh = q[:n_heads].contiguous().to(gpu)
    assert meta.max_kv_len == max(LENGTHS) > _C.kMaxKVLenNonSplit
    out = c_abi_decode(_C, qh, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    want = oa.paged_decode(np64(qh), kp, vp, np_tables(meta), meta.kv_lens.tolist())
    err = assert_close(out, want, torch.bfloat16, f"decode beyond 8192, H={n_heads} KVH=8")
    print(f"H={n_heads}: max abs err {err:.2e} over contexts {LENGTHS}")


def test_ops_decode_beyond_8192_behind_dev_flag(ops, gpu, long_decode, monkeypatch):
    w, wd, q, meta, kp, vp = long_decode
    qd = q.to(gpu)
    args = (qd, wd.k_pool, wd.v_pool, meta.block_tables, meta.kv_lens, meta.max_kv_len)
    with pytest.raises(RuntimeError, match="kMaxKVLenNonSplit"):
        ops.paged_attention_gemv(*args)  # the reference's check by default
    monkeypatch.setattr(femtovllm._DEV, "split_kv_decode", True)
    out = ops.paged_attention_gemv(*args)
    torch.cuda.synchronize()
    want = oa.paged_decode(np64(q), kp, vp, np_tables(meta), meta.kv_lens.tolist())
    assert_close(out, want, torch.bfloat16, "ops decode beyond 8192, H=32 KVH=8")
