"""Write the golden fixtures in this directory from the float64 oracle.

    python tests/golden/make_golden.py

Layouts follow the reference's own (print-only) test scripts, with seeded
inputs (the reference tests draw unseeded random data, so they hold no
values to copy):

* paged_prefill_fixture.npz -- femtovllm/ops/triton/paged_attention/
  test_paged_attention_gemm.py:18-102: cu_seqlens [0, 8, 24], kv_lens
  [59, 44], tables [[0,4,5,6],[1,8,9,-1]], H=8, KVH=4, D=128, positions
  kv_len - q_len + i (pool cut to the 10 blocks the tables use);
* paged_decode_fixture.npz -- csrc/paged_attention/test_paged_attention_gemv.py:25-56
  re-parameterised to 16-token pages and D=128 (kv_lens 16*4-5, 16*3-4);
* dense_fixture.npz -- csrc/flash_attention/test_flash_attention.py:9-18 at
  B=1, H=2, T=16 (GQA variant: KVH=1).

Inputs are bf16 values stored as uint16 bit patterns; outputs are the oracle's
float64 results stored as float32.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle.attention as oa  # noqa: E402


def bf16(shape, gen):
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(torch.bfloat16)


def bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def f64(t):
    return t.to(torch.float32).numpy().astype(np.float64)


def main():
    gen = torch.Generator().manual_seed(2024)
    tables = np.array([[0, 4, 5, 6], [1, 8, 9, -1]], dtype=np.int32)
    k_pool, v_pool = bf16((10, 4, 16, 128), gen), bf16((10, 4, 16, 128), gen)

    kv_lens = np.array([59, 44], dtype=np.int32)
    cu = np.array([0, 8, 24], dtype=np.int32)
    pos = np.concatenate([np.arange(59 - 8, 59), np.arange(44 - 16, 44)]).astype(np.int32)
    q = bf16((8, 24, 128), gen)
    out = oa.paged_prefill(f64(q), f64(k_pool), f64(v_pool), cu, tables, kv_lens, pos)
    np.savez(os.path.join(HERE, "paged_prefill_fixture.npz"), q=bits(q), k_pool=bits(k_pool), v_pool=bits(v_pool),
             tables=tables, kv_lens=kv_lens, cu_seqlens=cu, positions=pos, out=out.astype(np.float32))

    qd = bf16((8, 2, 128), gen)
    out = oa.paged_decode(f64(qd), f64(k_pool), f64(v_pool), tables, kv_lens)
    np.savez(os.path.join(HERE, "paged_decode_fixture.npz"), q=bits(qd), k_pool=bits(k_pool), v_pool=bits(v_pool),
             tables=tables, kv_lens=kv_lens, out=out.astype(np.float32))

    q, k, v = bf16((1, 2, 16, 128), gen), bf16((1, 1, 16, 128), gen), bf16((1, 1, 16, 128), gen)
    out = oa.dense_attention(f64(q), f64(k), f64(v))
    np.savez(os.path.join(HERE, "dense_fixture.npz"), q=bits(q), k=bits(k), v=bits(v), out=out.astype(np.float32))


if __name__ == "__main__":
    main()
