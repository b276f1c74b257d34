"""CPU restatement of the reference's own PyTorch attention path -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/`` (as a second, library-backed check of
``oracle.attention``) and by the ``cpu_baseline`` leg of ``bench.py`` (timed
on the host cores as the reference's CPU path).  It never runs inside the
shipped operators.

It follows ``QwenSelfAttention.forward_varlen_pytorch``
(femtovllm/models/qwen/qwen3.py:389-544) from the point where the new K/V
are already in the pools: per sequence, gather the pages of the block table
(qwen3.py:460-497), replicate each KV head ``n_rep`` times consecutively
(qwen3.py:504-523) and call ``torch.nn.functional.scaled_dot_product_attention``
with the right-bottom mask (qwen3.py:188-198, 527-535).  Decode uses the
same gather with no mask (csrc/paged_attention/test_paged_attention_gemv.py:65-89).
Unlike the reference loop it honours arbitrary ``positions`` (the mask is
``j <= positions[i]``), which equals the right-bottom mask for contiguous
chunks.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _gather(pool: torch.Tensor, table_row, kv_len: int) -> torch.Tensor:
    page_size = pool.shape[2]
    need = -(-kv_len // page_size)
    pages = [int(p) for p in table_row if int(p) >= 0][:need]
    return torch.cat([pool[p] for p in pages], dim=1)[:, :kv_len]


def _rep(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    kvh, length, dim = x.shape
    return x.unsqueeze(1).expand(kvh, n_rep, length, dim).reshape(kvh * n_rep, length, dim)


def paged_decode(q, k_pool, v_pool, raw_block_tables, kv_lens) -> torch.Tensor:
    """``q`` (H, B, D) -> (H, B, D) in q's dtype, on the CPU."""
    n_heads, num_seqs, dim = q.shape
    n_rep = n_heads // k_pool.shape[1]
    outs = []
    for b in range(num_seqs):
        kv_len = int(kv_lens[b])
        k = _rep(_gather(k_pool, raw_block_tables[b], kv_len), n_rep)
        v = _rep(_gather(v_pool, raw_block_tables[b], kv_len), n_rep)
        outs.append(F.scaled_dot_product_attention(q[:, b : b + 1], k, v))
    return torch.cat(outs, dim=1)


def paged_prefill(q, k_pool, v_pool, raw_cu_seqlens, raw_block_tables, raw_kv_lens, positions):
    """``q`` (H, T, D) -> (H, T, D) in q's dtype, on the CPU."""
    n_heads, num_tokens, dim = q.shape
    n_rep = n_heads // k_pool.shape[1]
    outs = []
    for b in range(len(raw_cu_seqlens) - 1):
        lo, hi = int(raw_cu_seqlens[b]), int(raw_cu_seqlens[b + 1])
        kv_len = int(raw_kv_lens[b])
        k = _rep(_gather(k_pool, raw_block_tables[b], kv_len), n_rep)
        v = _rep(_gather(v_pool, raw_block_tables[b], kv_len), n_rep)
        pos = positions[lo:hi].to(torch.int64)
        mask = torch.arange(kv_len)[None, :] <= pos[:, None]
        outs.append(F.scaled_dot_product_attention(q[:, lo:hi], k, v, attn_mask=mask))
    return torch.cat(outs, dim=1)


def dense_attention(q, k, v) -> torch.Tensor:
    """``q`` (B, H, Tq, D), ``k``/``v`` (B, KVH, Tkv, D), non-causal."""
    return F.scaled_dot_product_attention(q, k, v, enable_gqa=q.shape[1] != k.shape[1])
