"""Parity of the dense flash-attention entry (femto_flash_attention) with the oracle.

Reference behaviour: FlashAttentionWarpCuda
(csrc/flash_attention/flash_attention_warp.cu:301-376): dense, non-causal,
GQA, q (B, H, Tq, 128), k/v (B, KVH, Tkv, 128).
"""

import numpy as np
import pytest
import torch

import oracle.attention as oa
from femtovllm import workloads
from helpers import assert_close, np64

pytestmark = pytest.mark.gpu


def rand(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


@pytest.fixture(scope="module")
def C(gpu):
    from femtovllm import _C

    return _C


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize(
    "shape",
    [
        (4, 2, 2, 64, 64),     # csrc/flash_attention/test_flash_attention.py:9-18
        (2, 4, 4, 16, 16),     # benchmarks/flash_attention/scripts/benchmark.py:56-57
        (2, 4, 4, 256, 256),
        (2, 8, 2, 100, 333),   # GQA, ragged lengths
        (1, 32, 8, 129, 1),
        (3, 6, 6, 1, 77),
    ],
)
def test_dense_attention(C, gpu, dtype, shape):
    B, H, KVH, Tq, Tkv = shape
    q = rand((B, H, Tq, 128), dtype, 1)
    k = rand((B, KVH, Tkv, 128), dtype, 2)
    v = rand((B, KVH, Tkv, 128), dtype, 3)
    out = C.FlashAttentionWarpCuda(q.to(gpu), k.to(gpu), v.to(gpu))
    torch.cuda.synchronize()
    want = oa.dense_attention(np64(q), np64(k), np64(v))
    assert_close(out, want, dtype, f"dense {shape} {dtype}")


DENSE_HEADS = [(2, 2), (4, 4), (8, 2), (16, 8), (32, 8), (12, 4), (6, 2), (5, 1), (3, 3), (64, 8)]


@pytest.mark.parametrize("seed", range(32))
def test_dense_attention_random_shapes(C, gpu, seed):
    """Seeded random shapes: batch 1-4, ten head layouts, query and key
    lengths from 1 to a few hundred (ragged against the 32-, 64- or
    128-row query tiles and the 64-key tiles), f16 and bf16."""
    rng = np.random.default_rng(500 + seed)
    H, KVH = DENSE_HEADS[int(rng.integers(len(DENSE_HEADS)))]
    B = int(rng.integers(1, 5))
    Tq = int(rng.choice([1, int(rng.integers(2, 64)), int(rng.integers(64, 300))]))
    Tkv = int(rng.choice([1, int(rng.integers(2, 128)), int(rng.integers(128, 700))]))
    dtype = torch.float16 if rng.random() < 0.5 else torch.bfloat16
    q = rand((B, H, Tq, 128), dtype, 600 + seed)
    k = rand((B, KVH, Tkv, 128), dtype, 700 + seed)
    v = rand((B, KVH, Tkv, 128), dtype, 800 + seed)
    out = C.FlashAttentionWarpCuda(q.to(gpu), k.to(gpu), v.to(gpu))
    torch.cuda.synchronize()
    want = oa.dense_attention(np64(q), np64(k), np64(v))
    assert_close(out, want, dtype, f"dense B={B} H={H} KVH={KVH} Tq={Tq} Tkv={Tkv} {dtype}")


@pytest.mark.parametrize("tkv", [2048, 8192, 32768])
def test_dense_attention_long_key_shapes(C, gpu, tkv):
    """q 1 x 32 x 2048 against k/v 1 x 8 x tkv in bf16 (the long-key shapes the dense entry is timed
    on), on 40 query rows, tile edges included; rows of a dense call are independent, so the oracle
    runs on the sampled rows alone."""
    q = rand((1, 32, 2048, 128), torch.bfloat16, 11)
    k = rand((1, 8, tkv, 128), torch.bfloat16, 12)
    v = rand((1, 8, tkv, 128), torch.bfloat16, 13)
    out = C.FlashAttentionWarpCuda(q.to(gpu), k.to(gpu), v.to(gpu))
    torch.cuda.synchronize()
    rng = np.random.default_rng(tkv)
    rows = sorted({0, 31, 32, 63, 64, 127, 128, 2047} | {int(x) for x in rng.integers(0, 2048, size=32)})
    want = oa.dense_attention(np64(q[:, :, rows]), np64(k), np64(v))
    assert_close(out[:, :, rows], want, torch.bfloat16, f"dense q 2048 x 32 heads, Tkv={tkv}")


def test_dense_equals_paged_identity_table(C, ops, gpu):
    """Dense attention == paged prefill with contiguous pages and no causal limit."""
    B, H, KVH, T = 1, 8, 4, 96
    q = rand((B, H, T, 128), torch.bfloat16, 4)
    k = rand((B, KVH, T, 128), torch.bfloat16, 5)
    v = rand((B, KVH, T, 128), torch.bfloat16, 6)
    dense = C.FlashAttentionWarpCuda(q.to(gpu), k.to(gpu), v.to(gpu))
    k_pool = k[0].reshape(KVH, T // 16, 16, 128).transpose(0, 1).contiguous().to(gpu)
    v_pool = v[0].reshape(KVH, T // 16, 16, 128).transpose(0, 1).contiguous().to(gpu)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=gpu)
    paged = ops.paged_attention_gemm(
        q[0].to(gpu), k_pool, v_pool, i32([0, T]), T, 32, i32([0, 3]), i32([0, 0, 0]),
        i32([list(range(T // 16))]), i32([T]), i32([T - 1] * T),
    )
    torch.cuda.synchronize()
    assert torch.equal(dense[0], paged)


def test_dense_errors(C, gpu):
    q = rand((1, 2, 8, 128), torch.bfloat16, 7).to(gpu)
    with pytest.raises(RuntimeError):
        kt = q.transpose(2, 3).contiguous().transpose(2, 3)  # same shape, not contiguous
        C.FlashAttentionWarpCuda(q, kt, kt)
    with pytest.raises(RuntimeError):
        C.FlashAttentionWarpCuda(q.float(), q.float(), q.float())
    with pytest.raises(RuntimeError):
        C.FlashAttentionWarpCuda(q[..., :64].contiguous(), q[..., :64].contiguous(), q[..., :64].contiguous())
