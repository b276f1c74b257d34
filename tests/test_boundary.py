"""CPU tests of the drop-in boundary: the C ABI library and the Python mirror.

No GPU work is launched here: every C-ABI call below fails argument
validation before any HIP call, and tensor-level checks run on CPU tensors.
"""

import ctypes
import os
import re
import subprocess

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "femto_attn.h")


@pytest.fixture(scope="module")
def C():
    from femtovllm import _C

    return _C


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(femto_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(C):
    declared = header_functions()
    assert "femto_paged_attention_gemv" in declared and "femto_paged_attention_gemm" in declared
    nm = subprocess.run(["nm", "-D", "--defined-only", C.LIBRARY_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT\s+(femto_\w+)", nm.stdout))
    missing = [f for f in declared if f not in exported]
    assert not missing, f"declared in femto_attn.h but not exported: {missing}"
    lib = ctypes.CDLL(C.LIBRARY_PATH)
    for f in declared:
        getattr(lib, f)


def test_library_is_built_for_gfx950(C):
    out = subprocess.run(["strings", C.LIBRARY_PATH], capture_output=True, text=True).stdout
    assert "gfx950" in out


def test_constants_match_reference(C):
    # csrc/utils/constants.cuh:8, 39, 75 via csrc/bindings.cpp:62-66
    assert C.kMaxKVLenNonSplit == 8192
    assert C.kKVLenPerPage == 16
    assert C.kDimHead == 128
    from femtovllm import ops

    assert (ops.MAX_KV_LEN_NON_SPLIT, ops.KV_LEN_PER_PAGE, ops.DIM_HEAD) == (8192, 16, 128)


def test_workspace_size(C):
    f = C._lib.femto_paged_attention_gemv_workspace_size
    assert f(0, 16, 4096) == 0
    small = f(4, 16, 17)
    big = f(64, 16, 4096)
    assert big > small >= 0
    assert big % 4 == 0


def _gemv(C, **kw):
    a = dict(dtype=2, q=16, qsh=128, qsb=2048, out=16, osh=128, osb=2048, k=16, v=16, nb=8, kvh=8, bs=16, d=128,
             ps0=16384, ps1=2048, ps2=128, tables=16, npages=4, ts=4, kv_lens=16, nseq=4, h=16, maxkv=64,
             ws=None, wsb=0, stream=None)
    a.update(kw)
    return C._lib.femto_paged_attention_gemv(*a.values())


def test_gemv_validation_errors(C):
    last = lambda: C._lib.femto_attn_last_error().decode()
    # decode takes head_dim <= 128 in 16-byte chunks (the reference's TORCH_CHECK_LE)
    assert _gemv(C, d=136) == 2 and "head_dim must be at most 128" in last()
    assert _gemv(C, d=100) == 2 and "multiple of 16 bytes" in last()
    assert _gemv(C, d=0) == 2 and "head_dim" in last()
    assert _gemv(C, bs=32) == 1 and "block_size must be 16" in last()
    assert _gemv(C, h=12) == 1 and "multiple of n_kv_heads" in last()
    assert _gemv(C, dtype=7) == 2
    assert _gemv(C, q=8) == 1 and "aligned" in last()
    assert _gemv(C, ps2=100) == 1 and "strides" in last()
    assert _gemv(C, nb=0) == 1 and "at least one block" in last()
    assert _gemv(C, nseq=0) == 0  # nothing to do
    # a split plan without a workspace is rejected before launch
    assert _gemv(C, maxkv=8192, nseq=64) == 1 and "workspace" in last()


def test_gemm_rejects_fp32(C):
    rc = C._lib.femto_paged_attention_gemm(0, 16, 128, 128, 16, 128, 128, 16, 16, 8, 8, 16, 128, 16384, 2048, 128,
                                           16, 2, 10, 5, 16, 16, 4, 4, 16, 16, None, 0, None)
    assert rc == 2
    assert "not implemented for 'Float'" in C._lib.femto_attn_last_error().decode()


def _gemm(C, **kw):
    a = dict(dtype=2, q=16, qsh=128, qst=128, out=16, osh=128, ost=128, k=16, v=16, nb=8, kvh=8, bs=16, d=128,
             ps0=16384, ps1=2048, ps2=128, cu=16, nseq=2, ntok=10, maxq=5, h=16, tables=16, npages=4, ts=4,
             kv_lens=16, pos=16, ws=None, wsb=0, stream=None)
    a.update(kw)
    return C._lib.femto_paged_attention_gemm(*a.values())


def test_gemm_head_dim_rule(C):
    """Prefill takes head_dim <= 128 as the reference checks (paged_attention_gemm.cu:347-348), in
    multiples of 16; the checks run before anything touches the (fake) pointers."""
    last = lambda: C._lib.femto_attn_last_error().decode()
    assert _gemm(C, d=136) == 2 and "head_dim must be at most 128" in last()
    assert _gemm(C, d=72, ps2=72) == 2 and "multiple of 16" in last()
    assert _gemm(C, d=0) == 2 and "head_dim" in last()
    for d in (16, 64, 112):
        # accepted; the call then fails on its (deliberately too small) workspace before any launch,
        # with or without a GPU, so the fake pointers are never used
        rc = _gemm(C, d=d, ps2=d, ps1=16 * d, ps0=8 * 16 * d, ws=256, wsb=64)
        assert rc != 0 and "head_dim" not in last(), (d, rc, last())


def test_gemm_workspace_size_and_checks(C):
    # The size is one slot per resident workgroup of the current device (0
    # without a device, as here); empty calls and bad head counts need none.
    size = C._lib.femto_paged_attention_gemm_workspace_size
    assert size(0, 16, 16, 16, 8, 4) == 0 and size(2, 0, 1, 16, 8, 4) == 0
    assert size(8, 4096, 512, 12, 8, 4) == 0  # heads not a multiple of kv heads
    assert C._lib.femto_paged_attention_gemm_split_bytes() == 0
    # with a workspace the call sizes it against the device: without one it fails cleanly
    rc = C._lib.femto_paged_attention_gemm(2, 16, 128, 128, 16, 128, 128, 16, 16, 8, 8, 16, 128, 16384, 2048, 128,
                                           16, 2, 10, 5, 16, 16, 4, 4, 16, 16, 256, 64, None)
    assert rc != 0 and C._lib.femto_attn_last_error().decode()


def test_flash_validation(C):
    rc = C._lib.femto_flash_attention(2, 16, 1, 1, 1, 16, 1, 1, 1, 16, 1, 1, 1, 16, 4, 4, 4, 1, 4, 4, 8, 8, 128, None)
    assert rc == 1 and "strides" in C._lib.femto_attn_last_error().decode()
    rc = C._lib.femto_flash_attention(2, 16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, 16, 0, 0, 0, 1, 4, 4, 8, 8, 64, None)
    assert rc == 2


def test_ops_reject_cpu_tensors():
    from femtovllm import ops

    q = torch.zeros(16, 2, 128, dtype=torch.bfloat16)
    pool = torch.zeros(4, 8, 16, 128, dtype=torch.bfloat16)
    t = torch.zeros(2, 1, dtype=torch.int32)
    with pytest.raises(ValueError):
        ops.paged_attention_gemv(q, pool, pool, t, t[:, 0], 16)
    with pytest.raises(ValueError):
        ops.paged_attention_gemm(q, pool, pool, t[:, 0], 1, 32, t[:, 0], t[:, 0], t, t[:, 0], t[:, 0])


def test_dev_flags_and_enums_mirror_reference():
    import femtovllm
    from femtovllm.protocol import AttentionBackend, ImplCustomKernel

    assert femtovllm._DEV.impl_custom_gemm == ImplCustomKernel.TRITON
    assert femtovllm._DEV.impl_custom_gemv == ImplCustomKernel.CUDA
    assert femtovllm._DEV.route_prefill_decode
    assert AttentionBackend("custom_gemm_gemv") is AttentionBackend.CUSTOM_GEMM_GEMV
    assert ImplCustomKernel("cuda") is ImplCustomKernel.CUDA


# Every name the reference's engine imports from femtovllm.protocol, by importing module
# (femtovllm/__init__.py:4, models/qwen/qwen3.py:14, engine/model_runner.py:10,
# engine/core_engine.py:11, engine/sequence.py:5, engine/scheduler/v3.py:9,
# engine/kv_cache_manager/v3.py:6, entrypoints/llm.py:10, inputs/input_builder.py:6).
REFERENCE_PROTOCOL_IMPORTS = {
    "femtovllm/__init__.py": ["AttentionBackend", "ImplCustomKernel", "SamplingParams"],
    "femtovllm/models/qwen/qwen3.py": ["AttentionBackend", "VarlenAttnMetadata"],
    "femtovllm/engine/model_runner.py": ["ImplCustomKernel", "VarlenAttnMetadata"],
    "femtovllm/engine/core_engine.py": ["ReqId", "SamplingParams", "StepDelta", "StopReason"],
    "femtovllm/engine/sequence.py": ["ReqId", "SamplingParams", "SeqId", "StopReason"],
    "femtovllm/engine/scheduler/v3.py": ["StopReason"],
    "femtovllm/engine/kv_cache_manager/v3.py": ["SeqId"],
    "femtovllm/entrypoints/llm.py": ["SamplingParams"],
    "femtovllm/inputs/input_builder.py": ["SamplingParams"],
}


def test_protocol_exports_every_name_the_engine_imports():
    import dataclasses

    import femtovllm.protocol as P

    for module, names in REFERENCE_PROTOCOL_IMPORTS.items():
        for n in names:
            assert hasattr(P, n), f"femtovllm.protocol lacks {n} (imported by {module})"
    # field names and order of the reference's dataclasses / NamedTuple (protocol.py:35-100)
    assert [f.name for f in dataclasses.fields(P.VarlenAttnMetadata)] == [
        "positions", "raw_positions", "cu_seqlens", "raw_cu_seqlens", "max_q_len", "Q_TILE_SIZE",
        "raw_cu_q_tiles", "cu_q_tiles", "raw_q_tile_to_seq_idx", "q_tile_to_seq_idx", "k_cache_pools",
        "v_cache_pools", "kv_lens", "max_kv_len", "block_tables", "raw_block_tables", "is_decoding"]
    assert [f.name for f in dataclasses.fields(P.SamplingParams)] == [
        "temperature", "presence_penalty", "stop_token_ids", "max_new_tokens"]
    sp = P.SamplingParams(stop_token_ids=[1, 2])
    c = sp.clone()
    assert c == sp and c.stop_token_ids is not sp.stop_token_ids
    assert P.SamplingParams().max_new_tokens == 5000 and P.SamplingParams().temperature == 1.0
    assert P.StepDelta._fields == ("req_id", "seq_id", "new_token_id", "stop_reason")
    assert [m.value for m in P.StopReason] == ["EOS", "LENGTH", "OOM", "HARDWARE_LIMIT"]
    import femtovllm

    assert femtovllm.SamplingParams is P.SamplingParams


def test_metadata_follows_model_runner():
    """femtovllm/engine/model_runner.py:187-202 on the reference test's layout."""
    from femtovllm.metadata import build_varlen_metadata

    m = build_varlen_metadata([(51, 8), (28, 16)], [[0, 4, 5, 6], [1, 8, 9]], Q_TILE_SIZE=16)
    assert m.raw_cu_seqlens == [0, 8, 24]
    assert m.kv_lens.tolist() == [59, 44]
    assert m.raw_positions == list(range(51, 59)) + list(range(28, 44))
    assert m.raw_cu_q_tiles == [0, 1, 2]
    assert m.raw_q_tile_to_seq_idx == [0, 1]
    assert m.block_tables.tolist() == [[0, 4, 5, 6], [1, 8, 9, -1]]
    assert m.max_q_len == 16 and m.max_kv_len == 59
    assert not m.is_decoding and m.k_cache_pools == [] and m.v_cache_pools == []


def test_workloads_follow_generation_rules():
    import numpy as np

    from femtovllm import workloads

    w = workloads.decode_fp32_small()
    assert [p + n for p, n in w.chunks] == [17, 64, 200, 511]
    assert w.k_pool.shape == (256, 8, 16, 128) and w.q.shape == (16, 4, 128)
    used = sorted(b for t in w.raw_block_tables for b in t)
    assert len(used) == len(set(used)) == sum(-(-L // 16) for L in (17, 64, 200, 511))
    unused = sorted(set(range(256)) - set(used))
    assert torch.isnan(w.k_pool[unused]).all()
    # tail rows of a last page are poisoned, visible rows are finite
    t0 = w.raw_block_tables[0]
    assert torch.isnan(w.k_pool[t0[-1], :, 1:]).all() and torch.isfinite(w.k_pool[t0[-1], :, :1]).all()
    assert workloads.prefill_flops([(0, 2048)], 32, 128) == 4 * 128 * 32 * (2048 * 2049 // 2)
    b = workloads.decode_bytes(w, unique_blocks=False)
    assert b == (17 + 64 + 200 + 511) * 8 * 128 * 4 * 2 + 2 * 16 * 4 * 128 * 4 + 4 * 51 + 16
