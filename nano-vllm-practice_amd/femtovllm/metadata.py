"""Host-side varlen metadata, built the way the reference's ModelRunner builds it.

``build_varlen_metadata`` reproduces femtovllm/engine/model_runner.py:187-202
(prefill route) and 283-293 (decode route); ``pad_block_tables`` reproduces
model_runner.py:46-72 (tables padded with -1, not 0).  The tensors it returns
are exactly what ``femtovllm.ops.paged_attention_gemm`` /
``paged_attention_gemv`` receive from the engine.

Both return the reference's ``VarlenAttnMetadata`` (femtovllm/protocol.py:58-81,
mirrored in :mod:`femtovllm.protocol`).

``build_varlen_metadata_device`` produces the same tensors on the GPU from
one host-to-device copy of the per-sequence counts and the block tables (CSR)
and two small kernels, instead of per-token Python lists and one copy per
tensor; its ``raw_*`` list fields are ``None`` except ``raw_block_tables``.
"""

from __future__ import annotations

import itertools

import numpy as np
import torch

from femtovllm.protocol import VarlenAttnMetadata


def pad_block_tables(raw_block_tables: list) -> list:
    """Pad every table to the longest with -1 (model_runner.py:54-66)."""
    if not raw_block_tables:
        return []
    width = max(len(t) for t in raw_block_tables)
    return [list(t) + [-1] * (width - len(t)) for t in raw_block_tables]


def build_varlen_metadata(
    chunks: list,
    raw_block_tables: list,
    Q_TILE_SIZE: int = 32,
    device: str | torch.device = "cpu",
    k_cache_pools: list | None = None,
    v_cache_pools: list | None = None,
    is_decoding: bool = False,
) -> VarlenAttnMetadata:
    """Metadata for one prefill (or unified) call.

    ``chunks`` holds ``(num_computed_tokens, num_tokens)`` per scheduled
    sequence.  As in model_runner.py:187-202: ``kv_len = pos + num_tokens``,
    ``positions = range(pos, kv_len)``, ``ceil(num_tokens / Q_TILE_SIZE)``
    query tiles per sequence.  A decode sequence is the chunk ``(L - 1, 1)``
    (model_runner.py:283-289).
    """
    raw_positions: list = []
    raw_cu_seqlens = [0]
    raw_cu_q_tiles = [0]
    raw_q_tile_to_seq_idx: list = []
    raw_kv_lens: list = []
    max_q_len = -1
    max_kv_len = -1
    for seq_idx, (pos, num_tokens) in enumerate(chunks):
        kv_len = pos + num_tokens
        raw_positions.extend(range(pos, kv_len))
        raw_cu_seqlens.append(raw_cu_seqlens[-1] + num_tokens)
        num_q_tiles = (num_tokens + Q_TILE_SIZE - 1) // Q_TILE_SIZE
        raw_cu_q_tiles.append(raw_cu_q_tiles[-1] + num_q_tiles)
        raw_q_tile_to_seq_idx.extend([seq_idx] * num_q_tiles)
        raw_kv_lens.append(kv_len)
        max_q_len = max(max_q_len, num_tokens)
        max_kv_len = max(max_kv_len, kv_len)

    def i32(x):
        return torch.tensor(x, dtype=torch.int32, device=device)

    padded = pad_block_tables(raw_block_tables)
    return VarlenAttnMetadata(
        positions=i32(raw_positions),
        raw_positions=raw_positions,
        cu_seqlens=i32(raw_cu_seqlens),
        raw_cu_seqlens=raw_cu_seqlens,
        max_q_len=max_q_len,
        Q_TILE_SIZE=Q_TILE_SIZE,
        cu_q_tiles=i32(raw_cu_q_tiles),
        raw_cu_q_tiles=raw_cu_q_tiles,
        q_tile_to_seq_idx=i32(raw_q_tile_to_seq_idx),
        raw_q_tile_to_seq_idx=raw_q_tile_to_seq_idx,
        k_cache_pools=list(k_cache_pools or []),
        v_cache_pools=list(v_cache_pools or []),
        kv_lens=i32(raw_kv_lens),
        max_kv_len=max_kv_len,
        block_tables=torch.tensor(padded, dtype=torch.int32, device=device).reshape(len(padded), -1),
        raw_block_tables=[list(t) for t in raw_block_tables],
        is_decoding=is_decoding,
    )


def build_varlen_metadata_device(
    chunks: list,
    raw_block_tables: list,
    Q_TILE_SIZE: int = 32,
    device: str | torch.device = "cuda",
    k_cache_pools: list | None = None,
    v_cache_pools: list | None = None,
    is_decoding: bool = False,
) -> VarlenAttnMetadata:
    """``build_varlen_metadata`` with the tensors built by HIP kernels on ``device``.

    ``chunks`` holds ``(num_computed_tokens, num_tokens)`` per sequence, as
    for the host version; the result's tensors are identical.
    """
    from femtovllm import _C

    num_seqs = len(chunks)
    if num_seqs != len(raw_block_tables):
        raise ValueError("chunks and raw_block_tables differ in length")
    comp = [int(p) for p, _ in chunks]
    ntok = [int(n) for _, n in chunks]
    if any(n < 0 for n in ntok) or any(p < 0 for p in comp):
        raise ValueError("negative num_computed_tokens or num_tokens")
    lens = [len(t) for t in raw_block_tables]
    offsets = [0]
    for n in lens:
        offsets.append(offsets[-1] + n)
    flat = np.fromiter(itertools.chain.from_iterable(raw_block_tables), dtype=np.int32, count=offsets[-1])
    head = np.array(comp + ntok + offsets, dtype=np.int32)
    packed = torch.from_numpy(np.concatenate([head, flat])).pin_memory().to(device, non_blocking=True)
    max_q_len = max(ntok) if ntok else -1
    total_tokens = sum(ntok)
    total_tiles = sum((n + Q_TILE_SIZE - 1) // Q_TILE_SIZE for n in ntok)
    kv = [p + n for p, n in chunks]
    width = max(lens) if lens else 0
    flat_len = int(flat.size)
    positions, cu_seqlens, cu_q_tiles, tile_map, kv_lens, tables = _C._build_varlen_metadata(
        packed, num_seqs, flat_len, width, Q_TILE_SIZE, max(max_q_len, 0), total_tokens, total_tiles)
    return VarlenAttnMetadata(
        positions=positions, raw_positions=None,
        cu_seqlens=cu_seqlens, raw_cu_seqlens=None,
        max_q_len=max_q_len, Q_TILE_SIZE=Q_TILE_SIZE,
        cu_q_tiles=cu_q_tiles, raw_cu_q_tiles=None,
        q_tile_to_seq_idx=tile_map, raw_q_tile_to_seq_idx=None,
        k_cache_pools=list(k_cache_pools or []), v_cache_pools=list(v_cache_pools or []),
        kv_lens=kv_lens, max_kv_len=max(kv) if kv else -1,
        block_tables=tables,
        raw_block_tables=[list(t) for t in raw_block_tables],
        is_decoding=is_decoding,
    )
