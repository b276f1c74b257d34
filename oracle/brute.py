"""Pure-Python brute-force attention for tiny inputs -- TEST INFRASTRUCTURE ONLY.

A third, deliberately naive restatement (scalar loops, ``math.exp``, direct
``pool[page][head][row][d]`` indexing) used by tests/test_oracle.py to pin
``oracle.attention`` on tiny shapes.  Same semantics and citations as
``oracle/attention.py``: gather by ``block_table[b][j // 16]`` / ``j % 16``
(csrc/paged_attention/paged_attention_gemv.cu:80-105), kv head ``h // n_rep``
(paged_attention_gemv.cu:34), visibility ``j < kv_len and j <= positions[i]``
(femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:110-120).
"""

from __future__ import annotations

import math


def _row(q_vec, keys, vals, dim):
    scale = 1.0 / math.sqrt(dim)
    if not keys:
        return None
    scores = [sum(q_vec[d] * k[d] for d in range(dim)) * scale for k in keys]
    m = max(scores)
    w = [math.exp(s - m) for s in scores]
    tot = sum(w)
    return [sum(w[j] * vals[j][d] for j in range(len(keys))) / tot for d in range(dim)]


def paged_prefill(q, k_pool, v_pool, cu_seqlens, block_tables, kv_lens, positions, page_size=16):
    """Nested-list inputs; returns nested list (H, T, D); rows with no key are None."""
    n_heads = len(q)
    n_kv = len(k_pool[0])
    n_rep = n_heads // n_kv
    dim = len(q[0][0])
    out = [[None] * len(q[0]) for _ in range(n_heads)]
    for b in range(len(cu_seqlens) - 1):
        for t in range(cu_seqlens[b], cu_seqlens[b + 1]):
            for h in range(n_heads):
                g = h // n_rep
                keys, vals = [], []
                for j in range(kv_lens[b]):
                    if j > positions[t]:
                        continue
                    page = block_tables[b][j // page_size]
                    keys.append(k_pool[page][g][j % page_size])
                    vals.append(v_pool[page][g][j % page_size])
                out[h][t] = _row(q[h][t], keys, vals, dim)
    return out
