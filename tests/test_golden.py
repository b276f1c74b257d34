"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces the committed outputs.  GPU: the HIP kernels match
them at the stated tolerances.
"""

import os

import numpy as np
import pytest
import torch

import oracle.attention as oa
from helpers import assert_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return dict(np.load(os.path.join(HERE, name)))


def bf16(bits):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def f64(bits):
    return bf16(bits).to(torch.float32).numpy().astype(np.float64)


def test_oracle_reproduces_prefill_fixture():
    g = load("paged_prefill_fixture.npz")
    out = oa.paged_prefill(f64(g["q"]), f64(g["k_pool"]), f64(g["v_pool"]), g["cu_seqlens"], g["tables"],
                           g["kv_lens"], g["positions"])
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-6)


def test_oracle_reproduces_decode_fixture():
    g = load("paged_decode_fixture.npz")
    out = oa.paged_decode(f64(g["q"]), f64(g["k_pool"]), f64(g["v_pool"]), g["tables"], g["kv_lens"])
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-6)


def test_oracle_reproduces_dense_fixture():
    g = load("dense_fixture.npz")
    out = oa.dense_attention(f64(g["q"]), f64(g["k"]), f64(g["v"]))
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-6)


@pytest.mark.gpu
def test_kernels_match_fixtures(ops, gpu):
    from femtovllm import _C

    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.int32).to(gpu)
    g = load("paged_prefill_fixture.npz")
    out = ops.paged_attention_gemm(bf16(g["q"]).to(gpu), bf16(g["k_pool"]).to(gpu), bf16(g["v_pool"]).to(gpu),
                                   i32(g["cu_seqlens"]), 16, 32, i32([0, 1, 2]), i32([0, 1]), i32(g["tables"]),
                                   i32(g["kv_lens"]), i32(g["positions"]))
    torch.cuda.synchronize()
    assert_close(out, g["out"], torch.bfloat16, "prefill fixture")

    g = load("paged_decode_fixture.npz")
    out = ops.paged_attention_gemv(bf16(g["q"]).to(gpu), bf16(g["k_pool"]).to(gpu), bf16(g["v_pool"]).to(gpu),
                                   i32(g["tables"]), i32(g["kv_lens"]), int(g["kv_lens"].max()))
    torch.cuda.synchronize()
    assert_close(out, g["out"], torch.bfloat16, "decode fixture")

    g = load("dense_fixture.npz")
    out = _C.FlashAttentionWarpCuda(bf16(g["q"]).to(gpu), bf16(g["k"]).to(gpu), bf16(g["v"]).to(gpu))
    torch.cuda.synchronize()
    assert_close(out, g["out"], torch.bfloat16, "dense fixture")
