"""CPU oracle for the paged-attention hot path -- TEST INFRASTRUCTURE ONLY.

This module checks results and is never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped operators (``femtovllm.ops`` / ``femtovllm._C``) run
the HIP kernels in ``libfemto_attn.so`` and raise when that library is absent.

It restates, in float64 numpy, the attention semantics of FemtoVLLM
(fishAndShrimp/nano-vllm-practice).  Citations are paths inside that
repository:

* paged KV gather -- ``k_pool[page, kv_head, row, :]`` with
  ``page = block_table[b][j // 16]`` and ``row = j % 16``
  (csrc/paged_attention/paged_attention_gemv.cu:80-105,
  femtovllm/ops/triton/paged_attention/test_paged_attention_gemm.py:156-160,
  femtovllm/models/qwen/qwen3.py:460-497);
* GQA: query head ``h`` reads kv head ``h // n_rep``, the consecutive
  replication of qwen3.py:504-523 and paged_attention_gemv.cu:34;
* decode: every query attends to all ``kv_lens[b]`` keys, no causal mask
  (csrc/paged_attention/test_paged_attention_gemv.py:79-87);
* prefill / chunked varlen: key ``j`` is visible to query token ``i`` of
  sequence ``b`` iff ``j < kv_lens[b]`` and ``j <= positions[i]``
  (femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:110-120,
  csrc/paged_attention/paged_attention_gemm.cu:179-184); for contiguous
  chunks this is the right-bottom mask of qwen3.py:188-198;
* dense flash attention: non-causal GQA over the whole ``kv_len``
  (csrc/flash_attention/flash_attention_warp.cu:20-299);
* scale ``1/sqrt(head_dim)`` (paged_attention_gemm.py:225,
  paged_attention_gemv.cu:115).

Edge conventions follow the reference kernels exactly:

* decode with ``kv_len == 0`` returns zeros (the GEMV's P.V loop is empty and
  its output is the untouched zero accumulator, paged_attention_gemv.cu:203-218);
* a prefill or dense row with no visible key returns NaN (``acc / sum`` with
  both zero, paged_attention_gemm.py:157 and flash_attention_warp.cu:290).

Pinning (what checks each function, all in tests/test_oracle.py):
``gather_seq_kv`` -- spike keys scanned over every logical index and a
physical-block permutation invariance test; ``paged_decode`` /
``paged_prefill`` / ``dense_attention`` -- torch's
``scaled_dot_product_attention`` (a library routine, independent of this
code), a pure-Python triple loop on tiny inputs, closed forms (``kv_len == 1``
returns the V row; ``q == 0`` returns the mean of the visible V rows), the
causal boundary spike and GQA head-mapping spikes; planted mistakes
(``h % n_kv`` instead of ``h // n_rep``, ``<`` instead of ``<=``, a shifted
page row) are shown to fail those checks.
"""

from __future__ import annotations

import math

import numpy as np

KV_LEN_PER_PAGE = 16


def kv_head_of(h: int, n_heads: int, n_kv_heads: int) -> int:
    """GQA: query head h reads kv head h // n_rep (consecutive replication,
    femtovllm/models/qwen/qwen3.py:504-523; paged_attention_gemv.cu:34)."""
    return h // (n_heads // n_kv_heads)


def visible(j: np.ndarray, kv_len: int, pos: np.ndarray) -> np.ndarray:
    """Key j is visible to a query at position pos iff j < kv_len and j <= pos
    (femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:110-120)."""
    return (j < kv_len) & (j <= pos)


def softmax_scale(dim: int) -> float:
    """1/sqrt(head_dim) (paged_attention_gemm.py:225; paged_attention_gemv.cu:115)."""
    return 1.0 / math.sqrt(dim)


def page_slot(j: int, page_size: int = KV_LEN_PER_PAGE):
    """Logical key j -> (table column, row inside the page) = (j // 16, j % 16)."""
    return j // page_size, j % page_size


def gather_seq_kv(pool: np.ndarray, table_row, kv_len: int) -> np.ndarray:
    """Gather one sequence's keys (or values) through its block table.

    ``pool`` is ``(num_blocks, n_kv_heads, 16, D)``; returns
    ``(n_kv_heads, kv_len, D)``.  Follows the reference oracle
    (femtovllm/ops/triton/paged_attention/test_paged_attention_gemm.py:156-160):
    drop ``-1`` padding, concatenate the pages in table order, cut at kv_len.
    """
    page_size = pool.shape[2]
    pages = [int(p) for p in table_row if int(p) >= 0]
    need = -(-kv_len // page_size)
    if len(pages) < need:
        raise ValueError(f"block table holds {len(pages)} pages, kv_len {kv_len} needs {need}")
    col, row = page_slot(np.arange(kv_len), page_size)
    phys = np.asarray(pages, dtype=np.int64)[col] if kv_len else np.zeros(0, dtype=np.int64)
    return np.ascontiguousarray(pool[phys, :, row].transpose(1, 0, 2))


def _softmax_attend(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray, scale: float):
    """``q`` (Tq, D), ``k``/``v`` (Tk, D), boolean ``mask`` (Tq, Tk)."""
    q = q.astype(np.float64, copy=False)
    k = k.astype(np.float64, copy=False)
    v = v.astype(np.float64, copy=False)
    s = (q @ k.T) * scale
    s = np.where(mask, s, -np.inf)
    with np.errstate(invalid="ignore"):
        m = s.max(axis=1, keepdims=True) if s.shape[1] else np.full((s.shape[0], 1), -np.inf)
        p = np.exp(s - m)
        p = np.where(mask, p, 0.0)
        l = p.sum(axis=1, keepdims=True)
        o = (p @ v) / l
    return o


def paged_decode(q, k_pool, v_pool, block_tables, kv_lens) -> np.ndarray:
    """Decode attention, one query token per sequence.

    ``q`` (H, B, D); pools (NB, KVH, 16, D); ``block_tables`` (B, maxP) int
    with -1 padding; ``kv_lens`` (B,).  Returns (H, B, D) float64.
    Restates PagedAttentionGemvKernel (csrc/paged_attention/paged_attention_gemv.cu:16-221).
    """
    q = np.asarray(q)
    n_heads, num_seqs, dim = q.shape
    n_kv = k_pool.shape[1]
    scale = softmax_scale(dim)
    out = np.zeros((n_heads, num_seqs, dim), dtype=np.float64)
    for b in range(num_seqs):
        kv_len = int(kv_lens[b])
        if kv_len == 0:
            continue
        k = gather_seq_kv(k_pool, block_tables[b], kv_len)
        v = gather_seq_kv(v_pool, block_tables[b], kv_len)
        mask = np.ones((1, kv_len), dtype=bool)
        for g in range(n_kv):
            kg, vg = k[g].astype(np.float64), v[g].astype(np.float64)
            for h in range(n_heads):
                if kv_head_of(h, n_heads, n_kv) == g:
                    out[h, b] = _softmax_attend(q[h, b : b + 1], kg, vg, mask, scale)[0]
    return out


def paged_prefill(
    q, k_pool, v_pool, cu_seqlens, block_tables, kv_lens, positions, rows=None
) -> np.ndarray:
    """Chunked varlen causal prefill over the paged cache.

    ``q`` (H, T, D) with sequences laid out by ``cu_seqlens``; key ``j`` is
    visible to token ``i`` of sequence ``b`` iff ``j < kv_lens[b]`` and
    ``j <= positions[i]`` (femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:110-120).
    ``rows`` optionally restricts the computation to a subset of token
    indices (the other rows are returned as NaN); used to check large
    workloads on a sample of rows.  Returns (H, T, D) float64.
    """
    q = np.asarray(q)
    n_heads, num_tokens, dim = q.shape
    n_kv = k_pool.shape[1]
    scale = softmax_scale(dim)
    cu = [int(x) for x in cu_seqlens]
    positions = np.asarray(positions).astype(np.int64)
    out = np.full((n_heads, num_tokens, dim), np.nan, dtype=np.float64)
    wanted = None if rows is None else set(int(r) for r in rows)
    for b in range(len(cu) - 1):
        lo, hi = cu[b], cu[b + 1]
        toks = [t for t in range(lo, hi) if wanted is None or t in wanted]
        if not toks:
            continue
        kv_len = int(kv_lens[b])
        k = gather_seq_kv(k_pool, block_tables[b], kv_len)
        v = gather_seq_kv(v_pool, block_tables[b], kv_len)
        j = np.arange(kv_len)
        toks = np.asarray(toks)
        mask = visible(j[None, :], kv_len, positions[toks][:, None])
        for g in range(n_kv):
            kg, vg = k[g].astype(np.float64), v[g].astype(np.float64)
            for h in range(n_heads):
                if kv_head_of(h, n_heads, n_kv) == g:
                    out[h, toks] = _softmax_attend(q[h, toks], kg, vg, mask, scale)
    return out


def dense_attention(q, k, v) -> np.ndarray:
    """Dense non-causal GQA attention, the FlashAttentionWarpCuda contract.

    ``q`` (B, H, Tq, D); ``k``/``v`` (B, KVH, Tkv, D).  Returns (B, H, Tq, D)
    float64 (csrc/flash_attention/flash_attention_warp.cu:20-299).
    """
    q = np.asarray(q)
    batch, n_heads, q_len, dim = q.shape
    n_kv, kv_len = k.shape[1], k.shape[2]
    scale = softmax_scale(dim)
    out = np.zeros((batch, n_heads, q_len, dim), dtype=np.float64)
    mask = np.ones((q_len, kv_len), dtype=bool)
    for b in range(batch):
        for h in range(n_heads):
            g = kv_head_of(h, n_heads, n_kv)
            out[b, h] = _softmax_attend(q[b, h], k[b, g], v[b, g], mask, scale)
    return out


def cache_write(k_pool, v_pool, k_new, v_new, block_tables, cu_seqlens, positions):
    """Scatter new K/V rows into the paged pools (returns updated copies).

    Restates the per-sequence slicing loops that write the cache before the
    attention ops (femtovllm/models/qwen/qwen3.py:322-366 for prefill,
    240-264 for decode).  ``k_new``/``v_new`` are (T, KVH, D).  Sequence b
    owns tokens ``cu_seqlens[b] .. cu_seqlens[b+1]`` (``cu_seqlens=None``:
    token b alone, the decode layout); its first token sits at logical
    position ``p0 = positions[cu_seqlens[b]]`` and the rest follow it
    (``remaining_cache`` advances by the tokens written, qwen3.py:330-364),
    so token i of the sequence lands at ``p0 + i``: block
    ``block_tables[b][(p0 + i) // 16]``, row ``(p0 + i) % 16``.  The loop
    walks table columns from ``p0 // 16`` and breaks at the first ``-1``
    (qwen3.py:335-338); a column past the table or a block id outside the
    pool ends the walk the same way.
    """
    k_pool = np.array(k_pool, copy=True)
    v_pool = np.array(v_pool, copy=True)
    num_blocks, page_size = k_pool.shape[0], k_pool.shape[2]
    tables = [list(map(int, row)) for row in block_tables]
    n_seq = len(tables)
    cu = list(range(n_seq + 1)) if cu_seqlens is None else [int(x) for x in cu_seqlens]
    for b in range(n_seq):
        q0, q1 = cu[b], cu[b + 1]
        if q1 <= q0:
            continue
        p0 = int(positions[q0])
        if p0 < 0:
            continue
        for i in range(q1 - q0):
            col, row = page_slot(p0 + i, page_size)
            page = tables[b][col] if col < len(tables[b]) else -1
            if page < 0 or page >= num_blocks:
                break
            k_pool[page, :, row] = k_new[q0 + i]
            v_pool[page, :, row] = v_new[q0 + i]
    return k_pool, v_pool
