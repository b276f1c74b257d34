"""Attention operators with the reference's call signatures.

``paged_attention_gemv`` and ``paged_attention_gemm`` keep the signatures,
defaults, constants and error behaviour of femtovllm/ops/__init__.py:21-156
of the reference, so the engine, scheduler, prefix tree and block tables
drive them unchanged.  Both run hand-written HIP kernels for gfx950
(``libfemto_attn.so`` through :mod:`femtovllm._C`); importing this module
raises ``ImportError`` when that library is missing (ops/__init__.py:6-16).

``impl`` is kept for signature compatibility: ``ImplCustomKernel.CUDA`` and,
for the prefill op, ``ImplCustomKernel.TRITON`` (the reference's default)
both select the HIP kernels; anything else raises ``NotImplementedError``
as in the reference (ops/__init__.py:106-107, 155-156).

``kv_cache_write`` and ``qk_norm_rope_cache_write`` have no operator
counterpart in the reference: the first replaces the per-sequence slicing
loops that write the new K/V into the paged pools before the attention ops
(femtovllm/models/qwen/qwen3.py:240-264 for decode, 322-366 for prefill),
taking the same metadata; the second also fuses the q/k RMSNorm and the
rotary embedding that precede those loops (qwen3.py:230-238, 312-320).

One deliberate difference: ``q`` arrives as ``q.transpose(0, 1)`` of a
``(tokens, n_heads, head_dim)`` tensor (femtovllm/models/qwen/qwen3.py:270,
372).  The reference copies it with ``.contiguous()``; the HIP kernels take
the head and token strides directly, so no copy is made as long as the
head dimension is contiguous.
"""

import torch

import femtovllm
from femtovllm.protocol import ImplCustomKernel

try:
    from femtovllm import _C as _hip_backend
except ImportError as e:
    raise ImportError(
        "Failed to load the femtovllm HIP backend (libfemto_attn.so).\n"
        "Build it for gfx950 with:\n"
        "    python nano-vllm-practice_amd/build.py"
    ) from e

MAX_KV_LEN_NON_SPLIT = _hip_backend.kMaxKVLenNonSplit

KV_LEN_PER_PAGE = _hip_backend.kKVLenPerPage
# The kernels are built for this exact head dim (register tiling), as in the
# reference (femtovllm/ops/__init__.py:24-26).
DIM_HEAD = _hip_backend.kDimHead


def _ensure_valid_tensor(t: torch.Tensor, name: str) -> torch.Tensor:
    """Require a GPU tensor (ValueError otherwise, ops/__init__.py:36-39).

    Strided views are passed through; only a tensor whose innermost
    dimension is not contiguous is copied.
    """
    if not t.is_cuda:
        raise ValueError(f"Argument '{name}' must be a CUDA tensor. Got device={t.device}")
    if t.stride(-1) != 1:
        return t.contiguous()
    return t


def paged_attention_gemv(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    kv_page_tables: torch.Tensor,
    kv_lens: torch.Tensor,
    max_kv_len: int,
    #####
    impl: ImplCustomKernel = None,
):
    """Decode attention over the paged KV cache.

    q (n_heads, num_seqs, head_dim); pools (num_blocks, n_kv_heads, 16,
    head_dim); kv_page_tables (num_seqs, max_pages) int32, -1 padded;
    kv_lens (num_seqs,) int32.  Returns (n_heads, num_seqs, head_dim).
    ``max_kv_len`` above ``MAX_KV_LEN_NON_SPLIT`` raises ``RuntimeError`` as in
    the reference unless ``femtovllm._DEV.split_kv_decode`` is set.
    """
    q = _ensure_valid_tensor(q, "q")

    impl = femtovllm._DEV.impl_custom_gemv if (impl is None) else impl

    if impl == ImplCustomKernel.CUDA:
        return _hip_backend._paged_attention_gemv(
            q,
            k_pool,
            v_pool,
            kv_page_tables,
            kv_lens,
            max_kv_len,
            require_contiguous_q=False,
            # getattr: a reference checkout's DevFlags has no such field
            max_kv_len_limit=None if getattr(femtovllm._DEV, "split_kv_decode", False) else MAX_KV_LEN_NON_SPLIT,
        )
    else:
        raise NotImplementedError()


def paged_attention_gemm(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    cu_seqlens: torch.Tensor,
    max_q_len: int,
    Q_TILE_SIZE: int,
    cu_q_tiles: torch.Tensor,
    q_tile_to_seq_idx: torch.Tensor,
    kv_page_tables: torch.Tensor,
    kv_lens: torch.Tensor,
    positions: torch.Tensor,
    #####
    impl: ImplCustomKernel = None,
):
    """Chunked / varlen / causal prefill over the paged KV cache.

    q (n_heads, num_tokens, head_dim) with sequences delimited by
    cu_seqlens; token t sees key j iff j < kv_lens[seq] and
    j <= positions[t].  ``Q_TILE_SIZE``, ``cu_q_tiles`` and
    ``q_tile_to_seq_idx`` describe the reference Triton kernel's launch grid;
    the HIP kernel derives its own tiles from ``cu_seqlens`` and ignores them.
    Returns (n_heads, num_tokens, head_dim).
    """
    q = _ensure_valid_tensor(q, "q")

    impl = femtovllm._DEV.impl_custom_gemm if (impl is None) else impl

    if impl == ImplCustomKernel.CUDA or impl == ImplCustomKernel.TRITON:
        return _hip_backend._paged_attention_gemm(
            q,
            k_pool,
            v_pool,
            cu_seqlens,
            max_q_len,
            kv_page_tables,
            kv_lens,
            positions,
            require_contiguous_q=False,
        )
    else:
        raise NotImplementedError()


def kv_cache_write(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache_pool: torch.Tensor,
    v_cache_pool: torch.Tensor,
    positions: torch.Tensor,
    kv_page_tables: torch.Tensor,
    cu_seqlens: torch.Tensor = None,
    max_q_len: int = 1,
):
    """Write the new K/V rows into the paged pools (in place, bit-exact).

    k, v (num_tokens, n_kv_heads, head_dim), as produced by the projections
    (femtovllm/models/qwen/qwen3.py:231-238); pools (num_blocks, n_kv_heads,
    16, head_dim).  Prefill: sequence b owns tokens cu_seqlens[b] ..
    cu_seqlens[b+1] and writes them at positions[cu_seqlens[b]] + 0, 1, ...
    (qwen3.py:322-366); decode (``cu_seqlens=None``, as in the decode
    metadata of femtovllm/engine/model_runner.py:316-330): token b at
    positions[b] (qwen3.py:240-264).  max_q_len is the metadata's
    ``max_q_len``.  Position p goes to block kv_page_tables[b][p // 16], row
    p % 16; as in the reference loops, a sequence's writes stop at the first
    table entry that is -1 (and at block ids outside the pool).
    """
    for name, t in (("k", k), ("v", v)):
        if not t.is_cuda:
            raise ValueError(f"Argument '{name}' must be a CUDA tensor. Got device={t.device}")
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    _hip_backend._kv_cache_write(k, v, k_cache_pool, v_cache_pool, positions, kv_page_tables, cu_seqlens, max_q_len)


def qk_norm_rope_cache_write(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    eps: float,
    cos: torch.Tensor,
    sin: torch.Tensor,
    positions: torch.Tensor,
    k_cache_pool: torch.Tensor,
    v_cache_pool: torch.Tensor,
    kv_page_tables: torch.Tensor,
    cu_seqlens: torch.Tensor = None,
    max_q_len: int = 1,
    out: torch.Tensor = None,
):
    """The attention layer's prologue in one kernel; returns the rotated q.

    q (num_tokens, n_heads, 128), k and v (num_tokens, n_kv_heads, 128) as
    produced by the projections; ``q_norm_weight`` / ``k_norm_weight`` and
    ``eps`` of the layer's ``q_norm`` / ``k_norm`` RMSNorms; ``cos`` / ``sin``
    the rotary tables of ``QwenRotaryEmbedding`` (float32, (max_seqlen,
    128)); ``positions`` each token's position.  Computes
    ``rotary_embd(q_norm(q))`` (returned, in ``out`` if given, which may be
    ``q``) and ``rotary_embd(k_norm(k))``, and writes that k and v into the
    pools exactly as :func:`kv_cache_write` (qwen3.py:230-264, 312-366).
    Each output element is rounded once from fp32.
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not t.is_cuda:
            raise ValueError(f"Argument '{name}' must be a CUDA tensor. Got device={t.device}")
    return _hip_backend._qk_norm_rope_cache_write(q, k, v, q_norm_weight, k_norm_weight, eps, cos, sin, positions,
                                                   k_cache_pool, v_cache_pool, kv_page_tables, cu_seqlens,
                                                   max_q_len, out)
