"""Seeded synthetic paged-attention workloads.

Shapes follow the decode / chunked-prefill / mixed-batch cases the engine
produces (femtovllm/engine/model_runner.py:159-339): a paged KV pool
``(num_blocks, n_kv_heads, 16, head_dim)`` whose blocks are handed out by a
random permutation of the pool, -1 padded block tables, ``cu_seqlens`` /
``positions`` / ``kv_lens`` built by :mod:`femtovllm.metadata`.

Generation rules (identical inputs for the GPU kernels and any CPU check):

* integer draws (context lengths, block placement) come from
  ``numpy.random.default_rng(seed)``;
* Q, K and V are drawn as float32 N(0, 1) from a seeded CPU
  ``torch.Generator`` and then cast to the workload dtype;
* with ``poison=True`` every pool block no sequence uses, and every row past
  ``kv_len`` in a sequence's (unshared) last page, is set to NaN, so a
  kernel that reads outside the visible keys produces NaN.
"""

from __future__ import annotations

import dataclasses
import math

import numpy as np
import torch

from femtovllm.metadata import build_varlen_metadata

PAGE = 16


@dataclasses.dataclass
class PagedWorkload:
    name: str
    dtype: torch.dtype
    n_heads: int
    n_kv_heads: int
    head_dim: int
    chunks: list  # (num_computed_tokens, num_tokens) per sequence
    raw_block_tables: list
    q: torch.Tensor  # (H, T, D), tokens in chunk order
    k_pool: torch.Tensor
    v_pool: torch.Tensor

    @property
    def num_tokens(self) -> int:
        return sum(n for _, n in self.chunks)

    def token_offsets(self) -> list:
        off = [0]
        for _, n in self.chunks:
            off.append(off[-1] + n)
        return off

    def to(self, device) -> "PagedWorkload":
        return dataclasses.replace(
            self,
            q=self.q.to(device),
            k_pool=self.k_pool.to(device),
            v_pool=self.v_pool.to(device),
        )

    def select(self, seqs) -> tuple:
        """(chunks, tables, q) restricted to sequence indices ``seqs``."""
        off = self.token_offsets()
        seqs = list(seqs)
        chunks = [self.chunks[s] for s in seqs]
        tables = [self.raw_block_tables[s] for s in seqs]
        idx = torch.cat([torch.arange(off[s], off[s + 1]) for s in seqs]) if seqs else torch.zeros(0, dtype=torch.long)
        q = self.q.index_select(1, idx.to(self.q.device))
        return chunks, tables, q

    def gemm_call(self, seqs=None, device=None, Q_TILE_SIZE: int = 32):
        """Arguments of ``ops.paged_attention_gemm`` for sequences ``seqs``."""
        seqs = range(len(self.chunks)) if seqs is None else seqs
        chunks, tables, q = self.select(seqs)
        device = device or self.q.device
        meta = build_varlen_metadata(chunks, tables, Q_TILE_SIZE=Q_TILE_SIZE, device=device)
        return q, meta

    def gemv_call(self, seqs=None, device=None):
        """Arguments of ``ops.paged_attention_gemv``: every sequence must be a decode row."""
        seqs = range(len(self.chunks)) if seqs is None else seqs
        chunks, tables, q = self.select(seqs)
        if any(n != 1 for _, n in chunks):
            raise ValueError("gemv_call needs one query token per sequence")
        device = device or self.q.device
        meta = build_varlen_metadata(chunks, tables, device=device)
        return q, meta


def _place_blocks(rng, pages_per_seq, num_blocks, shared_seqs=(), shared_blocks=0):
    """Block tables from a random permutation of the pool, consumed in order.

    Sequences listed in ``shared_seqs`` start with the same
    ``min(shared_blocks, pages)`` physical blocks (a prefix-tree hit).
    """
    perm = [int(x) for x in rng.permutation(num_blocks)]
    cursor = 0
    shared = []
    if shared_seqs:
        shared = perm[:shared_blocks]
        cursor = shared_blocks
    tables = []
    shared_set = set(shared_seqs)
    for s, npages in enumerate(pages_per_seq):
        table = []
        if s in shared_set:
            table = shared[: min(shared_blocks, npages)]
        rest = npages - len(table)
        if cursor + rest > num_blocks:
            raise ValueError("pool too small for the block tables")
        table = table + perm[cursor : cursor + rest]
        cursor += rest
        tables.append(table)
    return tables


def _randn(shape, gen, dtype, chunk_elems=1 << 26):
    """float32 N(0,1) from ``gen`` cast to ``dtype``, generated in slabs."""
    out = torch.empty(shape, dtype=dtype)
    flat = out.view(-1)
    n = flat.numel()
    i = 0
    while i < n:
        j = min(n, i + chunk_elems)
        flat[i:j] = torch.randn(j - i, generator=gen, dtype=torch.float32).to(dtype)
        i = j
    return out


def make_paged_workload(
    name: str,
    chunks: list,
    n_heads: int,
    n_kv_heads: int,
    head_dim: int = 128,
    dtype: torch.dtype = torch.bfloat16,
    seed: int = 0,
    num_blocks: int | None = None,
    pool_factor: float = 1.2,
    shared_seqs=(),
    shared_blocks: int = 0,
    poison: bool = True,
    rng: np.random.Generator | None = None,
) -> PagedWorkload:
    rng = np.random.default_rng(seed) if rng is None else rng
    gen = torch.Generator().manual_seed(seed)
    pages = [-(-(p + n) // PAGE) for p, n in chunks]
    shared_set = set(shared_seqs)
    unique = sum(pages) - sum(min(shared_blocks, pg) for s, pg in enumerate(pages) if s in shared_set)
    if shared_set:
        unique += shared_blocks
    if num_blocks is None:
        num_blocks = max(1, math.ceil(pool_factor * unique))
    tables = _place_blocks(rng, pages, num_blocks, shared_seqs, shared_blocks)

    total_tokens = sum(n for _, n in chunks)
    q = _randn((n_heads, total_tokens, head_dim), gen, dtype)
    k_pool = _randn((num_blocks, n_kv_heads, PAGE, head_dim), gen, dtype)
    v_pool = _randn((num_blocks, n_kv_heads, PAGE, head_dim), gen, dtype)

    if poison:
        used = np.zeros(num_blocks, dtype=bool)
        for t in tables:
            used[t] = True
        unused = torch.from_numpy(np.nonzero(~used)[0])
        k_pool[unused] = float("nan")
        v_pool[unused] = float("nan")
        shared_pages = set()
        for s in shared_set:
            shared_pages.update(tables[s][: min(shared_blocks, pages[s])])
        for (p, n), t in zip(chunks, tables):
            kv_len = p + n
            tail = kv_len % PAGE
            if tail and t and t[-1] not in shared_pages:
                k_pool[t[-1], :, tail:] = float("nan")
                v_pool[t[-1], :, tail:] = float("nan")

    return PagedWorkload(
        name=name,
        dtype=dtype,
        n_heads=n_heads,
        n_kv_heads=n_kv_heads,
        head_dim=head_dim,
        chunks=list(chunks),
        raw_block_tables=tables,
        q=q,
        k_pool=k_pool,
        v_pool=v_pool,
    )


# ---------------------------------------------------------------------------
# The five measured configurations.
# ---------------------------------------------------------------------------


def decode_fp32_small(poison=True) -> PagedWorkload:
    """fp32 decode: 4 sequences, kv_lens {17, 64, 200, 511}, H=16, KVH=8, 256-block pool."""
    lens = [17, 64, 200, 511]
    return make_paged_workload(
        "decode_fp32_b4", [(L - 1, 1) for L in lens], 16, 8, dtype=torch.float32,
        seed=1001, num_blocks=256, poison=poison,
    )


def decode_bf16_qwen3_0p6b(poison=True) -> PagedWorkload:
    """bf16 decode, Qwen3-0.6B attention shape: B=64, L ~ U[256, 4096], H=16, KVH=8."""
    rng = np.random.default_rng(1002)
    lens = [int(x) for x in rng.integers(256, 4096, size=64, endpoint=True)]
    return make_paged_workload(
        "decode_bf16_qwen3_0.6b_b64", [(L - 1, 1) for L in lens], 16, 8,
        seed=1002, poison=poison, rng=rng,
    )


def decode_bf16_short(poison=True) -> PagedWorkload:
    """bf16 decode of short contexts, Qwen3-0.6B attention shape: B=64, L ~ U[64, 512], H=16, KVH=8."""
    rng = np.random.default_rng(1006)
    lens = [int(x) for x in rng.integers(64, 512, size=64, endpoint=True)]
    return make_paged_workload(
        "decode_bf16_qwen3_0.6b_b64_short", [(L - 1, 1) for L in lens], 16, 8,
        seed=1006, poison=poison, rng=rng,
    )


def prefill_bf16_chunked(poison=True) -> PagedWorkload:
    """bf16 chunked prefill: 8 x 512-token chunks after prefixes U[0, 2048], H=16, KVH=8."""
    rng = np.random.default_rng(1003)
    prefixes = [int(x) for x in rng.integers(0, 2048, size=8, endpoint=True)]
    return make_paged_workload(
        "prefill_bf16_8x512", [(p, 512) for p in prefixes], 16, 8,
        seed=1003, poison=poison, rng=rng,
    )


def prefill_bf16_uneven(poison=True) -> PagedWorkload:
    """bf16 chunked prefill of four uneven sequences, H=16, KVH=8: chunks of 512,
    512, 256 and 1024 tokens after prefixes of 3000, 200, 4000 and 100 tokens
    (two long contexts among short ones; fewer query tiles than the GPU holds)."""
    return make_paged_workload(
        "prefill_bf16_uneven4", [(3000, 512), (200, 512), (4000, 256), (100, 1024)], 16, 8,
        seed=1005, poison=poison,
    )


def prefill_bf16_long_llama3_8b(poison=True) -> PagedWorkload:
    """bf16 long context, Llama-3-8B attention shape: one 32768-token sequence, H=32, KVH=8.

    The workload holds the whole sequence as a single chunk; ``long_context_chunk``
    cuts it into the 16 successive 2048-token calls.
    """
    return make_paged_workload(
        "prefill_bf16_llama3_8b_32k", [(0, 32768)], 32, 8,
        seed=1004, poison=poison,
    )


def prefill_bf16_long_tp8_share(poison=True) -> PagedWorkload:
    """One GPU's share of the long-context workload under 8-way tensor parallelism
    (Llama-3-8B shape split by KV head): 4 query heads and 1 KV head, one
    32768-token sequence, cut into chunks by ``long_context_chunk``."""
    return make_paged_workload(
        "prefill_bf16_llama3_8b_32k_tp8", [(0, 32768)], 4, 1,
        seed=1004, poison=poison,
    )


def long_context_chunk(w: PagedWorkload, c: int, chunk: int = 2048, device=None, Q_TILE_SIZE=32):
    """Chunk ``c`` of the long-context sequence: ``chunk`` new tokens after a ``chunk*c`` prefix."""
    device = device or w.q.device
    q = w.q[:, c * chunk : (c + 1) * chunk]
    pages = (c + 1) * chunk // PAGE
    meta = build_varlen_metadata([(c * chunk, chunk)], [w.raw_block_tables[0][:pages]], Q_TILE_SIZE=Q_TILE_SIZE, device=device)
    return q, meta


def mixed_bf16_qwen3_8b(poison=True) -> PagedWorkload:
    """bf16 unified batch, Qwen3-8B attention shape (H=32, KVH=8).

    Sequence 0 is a 1024-token chunk after a 4096-token cached prefix;
    sequences 1..127 are decode rows with L ~ U[512, 8192].  The even
    sequences share their first min(64, pages) physical blocks.
    """
    rng = np.random.default_rng(1005)
    lens = [int(x) for x in rng.integers(512, 8192, size=127, endpoint=True)]
    chunks = [(4096, 1024)] + [(L - 1, 1) for L in lens]
    return make_paged_workload(
        "mixed_bf16_qwen3_8b", chunks, 32, 8, seed=1005, poison=poison, rng=rng,
        shared_seqs=tuple(range(0, 128, 2)), shared_blocks=64,
    )


def mixed_bf16_qwen3_8b_tp8_share(poison=True) -> PagedWorkload:
    """One GPU's share of the unified batch under 8-way tensor parallelism
    (Qwen3-8B shape split by KV head): 4 query heads and 1 KV head, the same
    sequences, context lengths and shared prefix blocks as ``mixed_bf16_qwen3_8b``."""
    rng = np.random.default_rng(1005)
    lens = [int(x) for x in rng.integers(512, 8192, size=127, endpoint=True)]
    chunks = [(4096, 1024)] + [(L - 1, 1) for L in lens]
    return make_paged_workload(
        "mixed_bf16_qwen3_8b_tp8", chunks, 4, 1, seed=1005, poison=poison, rng=rng,
        shared_seqs=tuple(range(0, 128, 2)), shared_blocks=64,
    )


def reference_fixture(dtype=torch.bfloat16) -> PagedWorkload:
    """The structure of the reference's paged prefill test.

    cu_seqlens [0, 8, 24], kv_lens [59, 44], tables [[0,4,5,6],[1,8,9]],
    32 blocks, H=8, KVH=4, D=128
    (femtovllm/ops/triton/paged_attention/test_paged_attention_gemm.py:18-102).
    """
    gen = torch.Generator().manual_seed(7)
    kv_lens = [59, 44]
    q_lens = [8, 16]
    chunks = [(L - n, n) for L, n in zip(kv_lens, q_lens)]
    tables = [[0, 4, 5, 6], [1, 8, 9]]
    q = _randn((8, 24, 128), gen, dtype)
    k_pool = _randn((32, 4, PAGE, 128), gen, dtype)
    v_pool = _randn((32, 4, PAGE, 128), gen, dtype)
    return PagedWorkload("reference_fixture", dtype, 8, 4, 128, chunks, tables, q, k_pool, v_pool)


# ---------------------------------------------------------------------------
# Algorithmic work (what the roofline numbers are computed from).
# ---------------------------------------------------------------------------


def decode_bytes(w: PagedWorkload, seqs=None, unique_blocks: bool = True) -> int:
    """HBM bytes a decode call must move at minimum.

    K and V once per KV head for every visible key, Q in and O out, the
    block-table entries read and ``kv_lens``.  With ``unique_blocks`` a
    physical block shared by several tables is counted once (its most-used
    row count), which is the strict figure for a prefix-shared pool.
    """
    seqs = range(len(w.chunks)) if seqs is None else list(seqs)
    s = torch.finfo(w.dtype).bits // 8
    row_bytes = w.n_kv_heads * w.head_dim * s * 2
    if unique_blocks:
        rows = {}
        for b in seqs:
            p, n = w.chunks[b]
            L = p + n
            for i, blk in enumerate(w.raw_block_tables[b][: -(-L // PAGE)]):
                r = min(PAGE, L - i * PAGE)
                rows[blk] = max(rows.get(blk, 0), r)
        kv = sum(rows.values()) * row_bytes
    else:
        kv = sum(sum(w.chunks[b]) for b in seqs) * row_bytes
    nseq = len(seqs)
    qo = 2 * w.n_heads * nseq * w.head_dim * s
    tables = 4 * sum(-(-sum(w.chunks[b]) // PAGE) for b in seqs)
    return kv + qo + tables + 4 * nseq


def prefill_flops(chunks, n_heads: int, head_dim: int) -> int:
    """Causal-exact FLOPs: 4*D*H per visible (query, key) pair."""
    pairs = 0
    for p, n in chunks:
        pairs += n * p + n * (n + 1) // 2
    return 4 * head_dim * n_heads * pairs
