"""The reference's ``femtovllm._C`` extension surface, backed by libfemto_attn.so.

Same names, attributes and argument meaning as the pybind11 module of the
reference (csrc/bindings.cpp:35-98):

* ``PagedAttentionGemvCuda(q, k_pool, v_pool, kv_page_tables, kv_lens, max_kv_len)``
* ``PagedAttentionGemmCuda(q, k_pool, v_pool, cu_seqlens, max_q_len, kv_page_tables, kv_lens, positions)``
* ``FlashAttentionWarpCuda(q, k, v)``
* ``kMaxKVLenNonSplit``, ``kKVLenPerPage``, ``kDimHead``

The functions run hand-written HIP kernels for gfx950 through the library's
C ABI (include/femto_attn.h) on torch's current stream.  Argument checks
raise ``RuntimeError`` where the reference's ``TORCH_CHECK``s do
(csrc/paged_attention/paged_attention_gemv.cu:231-274,
csrc/paged_attention/paged_attention_gemm.cu:314-353,
csrc/flash_attention/flash_attention_warp.cu:306-349).  Importing this module
raises ``ImportError`` when the library has not been built, exactly as the
reference fails without its compiled extension (femtovllm/ops/__init__.py:6-16).

Differences from the reference, all supersets: f32 decode is accepted (the
reference dispatches f16/bf16 only), and the decode kernel splits long
contexts internally, so ``max_kv_len`` only sizes the split workspace (the
``kMaxKVLenNonSplit`` check is kept for API parity; ``femtovllm._DEV.split_kv_decode``
lifts it).  head_dim is at most 128 as the reference checks, in whole 16-byte
chunks for decode and in multiples of 16 for prefill; dense attention takes
exactly 128, as the reference's.
"""

from __future__ import annotations

import ctypes
import os

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libfemto_attn.so")


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        raise ImportError(
            "femtovllm HIP backend is not built: missing "
            f"{_LIB_PATH}\nBuild it with: python nano-vllm-practice_amd/build.py"
        )
    lib = ctypes.CDLL(_LIB_PATH)
    i, i64, p, sz = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
    lib.femto_attn_last_error.restype = ctypes.c_char_p
    lib.femto_attn_last_error.argtypes = []
    for name in ("femto_attn_max_kv_len_non_split", "femto_attn_kv_len_per_page", "femto_attn_dim_head"):
        getattr(lib, name).restype = i
        getattr(lib, name).argtypes = []
    lib.femto_paged_attention_gemv_workspace_size.restype = sz
    lib.femto_paged_attention_gemv_workspace_size.argtypes = [i, i, i]
    lib.femto_attn_set_decode_single_max_kv.restype = i
    lib.femto_attn_set_decode_single_max_kv.argtypes = [i]
    lib.femto_paged_attention_gemv.restype = i
    lib.femto_paged_attention_gemv.argtypes = [
        i, p, i64, i64, p, i64, i64, p, p, i64, i, i, i, i64, i64, i64, p, i, i64, p, i, i, i, p, sz, p,
    ]
    lib.femto_paged_attention_gemv_noalloc.restype = i
    lib.femto_paged_attention_gemv_noalloc.argtypes = [
        i, p, i64, i64, p, i64, i64, p, p, i64, i, i, i, i64, i64, i64, p, i, i64, p, i, i, i, p,
    ]
    lib.femto_paged_attention_gemm.restype = i
    lib.femto_paged_attention_gemm.argtypes = [
        i, p, i64, i64, p, i64, i64, p, p, i64, i, i, i, i64, i64, i64, p, i, i, i, i, p, i, i64, p, p, p, sz, p,
    ]
    lib.femto_paged_attention_gemm_workspace_size.restype = sz
    lib.femto_paged_attention_gemm_workspace_size.argtypes = [i, i, i, i, i, i]
    lib.femto_paged_attention_gemm_split_bytes.restype = sz
    lib.femto_paged_attention_gemm_split_bytes.argtypes = []
    lib.femto_kv_cache_write.restype = i
    lib.femto_kv_cache_write.argtypes = [
        i, p, i64, i64, p, i64, i64, p, p, i64, i, i, i, i64, i64, i64, p, i, i, i, p, p, i, i64, p,
    ]
    lib.femto_qk_norm_rope_cache_write.restype = i
    lib.femto_qk_norm_rope_cache_write.argtypes = [
        i, p, i64, i64, p, i64, i64, p, i64, i64, p, i64, i64, p, p, ctypes.c_float, p, p, i64, i,
        p, p, i64, i, i, i, i, i64, i64, i64, p, i, i, i, p, p, i, i64, p,
    ]
    lib.femto_build_varlen_metadata.restype = i
    lib.femto_build_varlen_metadata.argtypes = [i, p, p, p, p, i, i, i, p, p, p, p, p, p, p]
    lib.femto_flash_attention.restype = i
    lib.femto_flash_attention.argtypes = [
        i, p, i64, i64, i64, p, i64, i64, i64, p, i64, i64, i64, p, i64, i64, i64, i, i, i, i, i, i, p,
    ]
    return lib


_lib = _load()

kMaxKVLenNonSplit = int(_lib.femto_attn_max_kv_len_non_split())
kKVLenPerPage = int(_lib.femto_attn_kv_len_per_page())
kDimHead = int(_lib.femto_attn_dim_head())

LIBRARY_PATH = _LIB_PATH

_DTYPE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}
_DTYPE_NAME = {torch.float32: "Float", torch.float16: "Half", torch.bfloat16: "BFloat16"}


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _raise_on(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_lib.femto_attn_last_error().decode())


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _dtype_code(t: torch.Tensor, fn: str) -> int:
    code = _DTYPE.get(t.dtype)
    _check(code is not None, f'"{fn}" not implemented for \'{t.dtype}\'')
    return code


# Split-KV workspaces, one per (device, stream), grown on demand; calls on
# one stream are ordered, so they can share it.
_workspaces: dict = {}


def _cached_workspace(cache: dict, device: torch.device, nbytes: int, zero: bool):
    if nbytes == 0:
        return None, 0
    key = (device.index, _stream(device))
    ws = cache.get(key)
    if ws is None or ws.numel() < nbytes + 256:
        alloc = torch.zeros if zero else torch.empty
        ws = alloc(nbytes + 256, dtype=torch.uint8, device=device)
        cache[key] = ws
    ptr = ws.data_ptr()
    aligned = (ptr + 255) & ~255
    return aligned, ws.numel() - (aligned - ptr)


def _decode_workspace(device: torch.device, num_seqs: int, n_heads: int, max_kv_len: int):
    nbytes = int(_lib.femto_paged_attention_gemv_workspace_size(num_seqs, n_heads, max_kv_len))
    return _cached_workspace(_workspaces, device, nbytes, zero=False)


# Workspaces of the prefill call, one per (device, stream): the key-split
# counters at the front must be zero-filled before the first use and are left
# so; the partial slots and the decode-row part behind them need no
# initialisation (a grown workspace is zero-filled whole).
_prefill_workspaces: dict = {}


def _prefill_workspace(device: torch.device, num_seqs: int, num_tokens: int, max_q_len: int, n_heads: int,
                       n_kv_heads: int, num_pages_per_seq: int):
    nbytes = int(_lib.femto_paged_attention_gemm_workspace_size(num_seqs, num_tokens, max_q_len, n_heads,
                                                                 n_kv_heads, num_pages_per_seq))
    return _cached_workspace(_prefill_workspaces, device, nbytes, zero=True)


def _check_paged(fn, q, k_pool, v_pool, tables, kv_lens, require_contiguous_q, decode=False):
    for name, t in (("q", q), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check(t.is_cuda, f"{fn}: {name} must be a GPU tensor")
    if require_contiguous_q:
        _check(q.is_contiguous(), f"{fn}: q must be contiguous")
    _check(k_pool.is_contiguous() and v_pool.is_contiguous(), f"{fn}: k_pool and v_pool must be contiguous")
    _check(q.dim() == 3, f"{fn}: q must be 3-D (n_heads, tokens, head_dim), got {q.dim()}-D")
    _check(k_pool.dim() == 4 and v_pool.dim() == 4, f"{fn}: pools must be 4-D (num_blocks, n_kv_heads, 16, head_dim)")
    _check(q.size(-1) == k_pool.size(-1) and q.size(-1) == v_pool.size(-1), f"{fn}: head_dim of q and pools differ")
    _check(tuple(k_pool.shape) == tuple(v_pool.shape), f"{fn}: k_pool and v_pool shapes differ")
    _check(q.dtype == k_pool.dtype == v_pool.dtype, f"{fn}: q, k_pool and v_pool must share a dtype")
    _check(q.stride(-1) == 1, f"{fn}: q must be contiguous in head_dim")
    _check(tables.dtype == torch.int32, f"{fn}: kv_page_tables must be int32")
    _check(kv_lens.dtype == torch.int32, f"{fn}: kv_lens must be int32")
    _check(tables.dim() == 2 and (tables.size(1) <= 1 or tables.stride(1) == 1), f"{fn}: kv_page_tables must be 2-D, row-major")
    _check(kv_lens.is_contiguous(), f"{fn}: kv_lens must be contiguous")
    for name, t in (("kv_page_tables", tables), ("kv_lens", kv_lens)):
        _check(t.device == q.device, f"{fn}: {name} must be on {q.device}")
    _check(k_pool.size(2) == kKVLenPerPage, f"{fn}: block_size must be {kKVLenPerPage}, got {k_pool.size(2)}")
    # head_dim <= 128, TORCH_CHECK_LE(dim_d, kDimHead) (paged_attention_gemv.cu:256-257,
    # paged_attention_gemm.cu:347-348); decode in whole 16-byte chunks (the wave loads rows 16 bytes
    # per lane), prefill in multiples of 16 (one step of the score MFMAs).
    _check(q.size(-1) <= kDimHead, f"{fn}: head_dim must be <= {kDimHead}, got {q.size(-1)}")
    if decode:
        _check((q.size(-1) * q.element_size()) % 16 == 0,
               f"{fn}: head_dim must be a multiple of 16 bytes ({16 // q.element_size()} elements), got {q.size(-1)}")
    else:
        _check(q.size(-1) % 16 == 0, f"{fn}: head_dim must be a multiple of 16, got {q.size(-1)}")
    _check(q.size(0) % k_pool.size(1) == 0, f"{fn}: n_heads must be a multiple of n_kv_heads")


def _paged_attention_gemv(q, k_pool, v_pool, kv_page_tables, kv_lens, max_kv_len, require_contiguous_q=True,
                          max_kv_len_limit=kMaxKVLenNonSplit):
    """Decode through the C ABI.  ``max_kv_len_limit`` is the reference's
    ``kMaxKVLenNonSplit`` check (paged_attention_gemv.cu:271-274); ``None``
    lifts it, since the kernel splits contexts of any length over waves."""
    fn = "PagedAttentionGemvCuda"
    _check_paged(fn, q, k_pool, v_pool, kv_page_tables, kv_lens, require_contiguous_q, decode=True)
    n_heads, num_seqs, dim = q.shape
    _check(num_seqs == kv_page_tables.size(0), f"{fn}: q.size(1) must equal kv_page_tables.size(0)")
    _check(num_seqs == kv_lens.size(0), f"{fn}: q.size(1) must equal kv_lens.size(0)")
    if max_kv_len_limit is not None:
        _check(int(max_kv_len) <= max_kv_len_limit, f"{fn}: max_kv_len {max_kv_len} > kMaxKVLenNonSplit {max_kv_len_limit}")
    dtype = _dtype_code(q, fn)
    out = torch.empty((n_heads, num_seqs, dim), dtype=q.dtype, device=q.device)
    if num_seqs == 0:
        return out
    ws, ws_bytes = _decode_workspace(q.device, num_seqs, n_heads, int(max_kv_len))
    rc = _lib.femto_paged_attention_gemv(
        dtype,
        q.data_ptr(), q.stride(0), q.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(),
        k_pool.size(0), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        kv_page_tables.data_ptr(), kv_page_tables.size(1), kv_page_tables.stride(0),
        kv_lens.data_ptr(), num_seqs, n_heads, int(max_kv_len),
        ws, ws_bytes,
        _stream(q.device),
    )
    _raise_on(rc)
    return out


def _paged_attention_gemm(q, k_pool, v_pool, cu_seqlens, max_q_len, kv_page_tables, kv_lens, positions,
                          require_contiguous_q=True):
    fn = "PagedAttentionGemmCuda"
    _check_paged(fn, q, k_pool, v_pool, kv_page_tables, kv_lens, require_contiguous_q)
    for name, t in (("cu_seqlens", cu_seqlens), ("positions", positions)):
        _check(t.dtype == torch.int32, f"{fn}: {name} must be int32")
        _check(t.is_contiguous(), f"{fn}: {name} must be contiguous")
        _check(t.device == q.device, f"{fn}: {name} must be on {q.device}")
    num_seqs = cu_seqlens.numel() - 1
    _check(num_seqs == kv_page_tables.size(0), f"{fn}: cu_seqlens.numel()-1 must equal kv_page_tables.size(0)")
    _check(num_seqs == kv_lens.size(0), f"{fn}: cu_seqlens.numel()-1 must equal kv_lens.size(0)")
    n_heads, num_tokens, dim = q.shape
    _check(num_tokens == positions.numel(), f"{fn}: q.size(1) must equal positions.numel()")
    _check(q.dtype != torch.float32, f'"{fn}" not implemented for \'Float\'')
    dtype = _dtype_code(q, fn)
    out = torch.empty((n_heads, num_tokens, dim), dtype=q.dtype, device=q.device)
    if num_seqs <= 0 or num_tokens == 0:
        return out
    max_q_len = int(max_q_len)
    ws, ws_bytes = _prefill_workspace(q.device, num_seqs, num_tokens, max_q_len, n_heads, k_pool.size(1),
                                      kv_page_tables.size(1))
    rc = _lib.femto_paged_attention_gemm(
        dtype,
        q.data_ptr(), q.stride(0), q.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(),
        k_pool.size(0), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        cu_seqlens.data_ptr(), num_seqs, num_tokens, max_q_len, n_heads,
        kv_page_tables.data_ptr(), kv_page_tables.size(1), kv_page_tables.stride(0),
        kv_lens.data_ptr(), positions.data_ptr(),
        ws, ws_bytes, _stream(q.device),
    )
    _raise_on(rc)
    return out


def _kv_cache_write(k, v, k_pool, v_pool, positions, kv_page_tables, cu_seqlens=None, max_q_len=1):
    """Scatter k, v (tokens, n_kv_heads, head_dim) into the paged pools in place."""
    fn = "kv_cache_write"
    for name, t in (("k", k), ("v", v), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check(t.is_cuda, f"{fn}: {name} must be a GPU tensor")
    _check(k.dim() == 3 and v.dim() == 3, f"{fn}: k and v must be 3-D (tokens, n_kv_heads, head_dim)")
    _check(tuple(k.shape) == tuple(v.shape), f"{fn}: k and v shapes differ")
    _check(k.stride(-1) == 1 and v.stride(-1) == 1, f"{fn}: k and v must be contiguous in head_dim")
    _check(k_pool.dim() == 4 and tuple(k_pool.shape) == tuple(v_pool.shape),
           f"{fn}: pools must be 4-D (num_blocks, n_kv_heads, 16, head_dim) of one shape")
    _check(k_pool.is_contiguous() and v_pool.is_contiguous(), f"{fn}: k_pool and v_pool must be contiguous")
    _check(k.size(1) == k_pool.size(1) and k.size(2) == k_pool.size(3), f"{fn}: k/v heads or head_dim differ from the pools")
    _check(k.dtype == v.dtype == k_pool.dtype == v_pool.dtype, f"{fn}: k, v and the pools must share a dtype")
    _check(k_pool.size(2) == kKVLenPerPage, f"{fn}: block_size must be {kKVLenPerPage}, got {k_pool.size(2)}")
    _check(kv_page_tables.dtype == torch.int32 and positions.dtype == torch.int32, f"{fn}: positions and kv_page_tables must be int32")
    _check(kv_page_tables.dim() == 2 and (kv_page_tables.size(1) <= 1 or kv_page_tables.stride(1) == 1),
           f"{fn}: kv_page_tables must be 2-D, row-major")
    _check(positions.is_contiguous(), f"{fn}: positions must be contiguous")
    tensors = [("positions", positions), ("kv_page_tables", kv_page_tables)]
    num_tokens = k.size(0)
    num_seqs = kv_page_tables.size(0)
    if cu_seqlens is None:
        _check(num_tokens == num_seqs, f"{fn}: without cu_seqlens every sequence has one token")
        _check(positions.numel() == num_seqs, f"{fn}: positions.numel() must equal the number of sequences")
        cu_ptr = None
    else:
        _check(cu_seqlens.dtype == torch.int32 and cu_seqlens.is_contiguous(), f"{fn}: cu_seqlens must be contiguous int32")
        _check(cu_seqlens.numel() - 1 == num_seqs, f"{fn}: cu_seqlens.numel()-1 must equal kv_page_tables.size(0)")
        _check(positions.numel() == num_tokens, f"{fn}: positions.numel() must equal k.size(0)")
        tensors.append(("cu_seqlens", cu_seqlens))
        cu_ptr = cu_seqlens.data_ptr()
    for name, t in tensors:
        _check(t.device == k.device, f"{fn}: {name} must be on {k.device}")
    dtype = _dtype_code(k, fn)
    if num_seqs == 0 or num_tokens == 0:
        return
    rc = _lib.femto_kv_cache_write(
        dtype,
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(),
        k_pool.size(0), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        cu_ptr, num_seqs, num_tokens, int(max_q_len),
        positions.data_ptr(), kv_page_tables.data_ptr(), kv_page_tables.size(1), kv_page_tables.stride(0),
        _stream(k.device),
    )
    _raise_on(rc)


def _qk_norm_rope_cache_write(q, k, v, q_weight, k_weight, eps, cos, sin, positions, k_pool, v_pool,
                              kv_page_tables, cu_seqlens=None, max_q_len=1, out=None):
    """RMSNorm + RoPE of q and k, q to ``out``, rotated k and v into the pools; returns ``out``."""
    fn = "qk_norm_rope_cache_write"
    for name, t in (("q", q), ("k", k), ("v", v), ("q_weight", q_weight), ("k_weight", k_weight),
                    ("cos", cos), ("sin", sin), ("k_pool", k_pool), ("v_pool", v_pool)):
        _check(t.is_cuda, f"{fn}: {name} must be a GPU tensor")
        _check(t.device == q.device, f"{fn}: {name} must be on {q.device}")
    _check(q.dim() == 3 and k.dim() == 3 and v.dim() == 3, f"{fn}: q, k, v must be 3-D (tokens, heads, head_dim)")
    _check(tuple(k.shape) == tuple(v.shape) and q.size(0) == k.size(0) and q.size(2) == k.size(2),
           f"{fn}: q, k, v shapes disagree")
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check(t.stride(-1) == 1, f"{fn}: {name} must be contiguous in head_dim")
    _check(q.size(2) == kDimHead, f"{fn}: head_dim must be {kDimHead}")
    _check(q_weight.numel() == kDimHead and k_weight.numel() == kDimHead and q_weight.is_contiguous()
           and k_weight.is_contiguous(), f"{fn}: norm weights must be contiguous ({kDimHead},)")
    _check(q.dtype == k.dtype == v.dtype == q_weight.dtype == k_weight.dtype == k_pool.dtype == v_pool.dtype,
           f"{fn}: q, k, v, the norm weights and the pools must share a dtype")
    _check(cos.dtype == torch.float32 and sin.dtype == torch.float32, f"{fn}: cos / sin tables must be float32")
    _check(cos.dim() == 2 and tuple(cos.shape) == tuple(sin.shape) and cos.stride() == sin.stride()
           and cos.stride(1) == 1 and cos.size(1) >= kDimHead, f"{fn}: cos / sin must be (rows, >= {kDimHead}) row-major alike")
    _check(k_pool.dim() == 4 and tuple(k_pool.shape) == tuple(v_pool.shape) and k_pool.is_contiguous()
           and v_pool.is_contiguous(), f"{fn}: pools must be contiguous 4-D tensors of one shape")
    _check(k.size(1) == k_pool.size(1) and k_pool.size(3) == kDimHead, f"{fn}: k heads or head_dim differ from the pools")
    _check(k_pool.size(2) == kKVLenPerPage, f"{fn}: block_size must be {kKVLenPerPage}")
    _check(q.size(1) % k.size(1) == 0, f"{fn}: n_heads must be a multiple of n_kv_heads")
    _check(positions.dtype == torch.int32 and positions.is_contiguous() and positions.device == q.device,
           f"{fn}: positions must be a contiguous int32 tensor on {q.device}")
    _check(kv_page_tables.dtype == torch.int32 and kv_page_tables.dim() == 2 and kv_page_tables.device == q.device
           and (kv_page_tables.size(1) <= 1 or kv_page_tables.stride(1) == 1), f"{fn}: kv_page_tables must be 2-D row-major int32")
    num_tokens, num_seqs = q.size(0), kv_page_tables.size(0)
    _check(positions.numel() == num_tokens, f"{fn}: positions.numel() must equal the number of tokens")
    if cu_seqlens is None:
        _check(num_tokens == num_seqs, f"{fn}: without cu_seqlens every sequence has one token")
        cu_ptr = None
    else:
        _check(cu_seqlens.dtype == torch.int32 and cu_seqlens.is_contiguous() and cu_seqlens.device == q.device,
               f"{fn}: cu_seqlens must be a contiguous int32 tensor on {q.device}")
        _check(cu_seqlens.numel() - 1 == num_seqs, f"{fn}: cu_seqlens.numel()-1 must equal kv_page_tables.size(0)")
        cu_ptr = cu_seqlens.data_ptr()
    if out is None:
        out = torch.empty_like(q)
    _check(tuple(out.shape) == tuple(q.shape) and out.dtype == q.dtype and out.stride(-1) == 1 and out.device == q.device,
           f"{fn}: out must match q")
    dtype = _dtype_code(q, fn)
    if num_tokens == 0 or num_seqs == 0:
        return out
    rc = _lib.femto_qk_norm_rope_cache_write(
        dtype,
        q.data_ptr(), q.stride(0), q.stride(1),
        k.data_ptr(), k.stride(0), k.stride(1),
        v.data_ptr(), v.stride(0), v.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1),
        q_weight.data_ptr(), k_weight.data_ptr(), float(eps),
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.size(0),
        k_pool.data_ptr(), v_pool.data_ptr(),
        k_pool.size(0), q.size(1), k_pool.size(1), k_pool.size(2), k_pool.size(3),
        k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        cu_ptr, num_seqs, num_tokens, int(max_q_len),
        positions.data_ptr(), kv_page_tables.data_ptr(), kv_page_tables.size(1), kv_page_tables.stride(0),
        _stream(q.device),
    )
    _raise_on(rc)
    return out


def _build_varlen_metadata(packed, num_seqs, num_block_ids, table_width, q_tile_size, max_q_len, num_tokens_total,
                           num_tiles_total):
    """Run the device builder on ``packed`` = [num_computed | num_tokens | block_offsets | block_ids]
    (int32, on the GPU); returns (positions, cu_seqlens, cu_q_tiles, q_tile_to_seq_idx, kv_lens, block_tables)."""
    dev = packed.device
    i32 = lambda n: torch.empty(n, dtype=torch.int32, device=dev)
    positions, cu_seqlens, cu_q_tiles = i32(num_tokens_total), i32(num_seqs + 1), i32(num_seqs + 1)
    tile_map, kv_lens = i32(num_tiles_total), i32(num_seqs)
    tables = torch.empty((num_seqs, table_width), dtype=torch.int32, device=dev)
    base = packed.data_ptr()
    off = lambda k: base + 4 * k
    rc = _lib.femto_build_varlen_metadata(
        num_seqs, off(0), off(num_seqs), off(2 * num_seqs), off(3 * num_seqs + 1), table_width,
        q_tile_size, max_q_len, positions.data_ptr(), cu_seqlens.data_ptr(), cu_q_tiles.data_ptr(),
        tile_map.data_ptr(), kv_lens.data_ptr(), tables.data_ptr(), _stream(dev),
    )
    _raise_on(rc)
    return positions, cu_seqlens, cu_q_tiles, tile_map, kv_lens, tables


def PagedAttentionGemvCuda(q, k_pool, v_pool, kv_page_tables, kv_lens, max_kv_len):
    """Decode attention; out (n_heads, num_seqs, head_dim) like ``torch.empty_like(q)``."""
    return _paged_attention_gemv(q, k_pool, v_pool, kv_page_tables, kv_lens, max_kv_len)


def PagedAttentionGemmCuda(q, k_pool, v_pool, cu_seqlens, max_q_len, kv_page_tables, kv_lens, positions):
    """Varlen causal prefill; out (n_heads, num_tokens, head_dim)."""
    return _paged_attention_gemm(q, k_pool, v_pool, cu_seqlens, max_q_len, kv_page_tables, kv_lens, positions)


def FlashAttentionWarpCuda(q, k, v):
    """Dense non-causal GQA attention, q (B, H, Tq, 128), k/v (B, KVH, Tkv, 128)."""
    fn = "FlashAttentionWarpCuda"
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check(t.is_cuda, f"{fn}: {name} must be a GPU tensor")
        _check(t.is_contiguous(), f"{fn}: {name} must be contiguous")
        _check(t.data_ptr() % 16 == 0, f"{fn}: {name} must be 16-byte aligned")
        _check(t.dim() == 4, f"{fn}: {name} must be 4-D")
    _check(q.size(0) == k.size(0) == v.size(0), f"{fn}: batch sizes differ")
    _check(k.size(1) == v.size(1), f"{fn}: k and v head counts differ")
    _check(q.size(1) % k.size(1) == 0, f"{fn}: n_heads must be a multiple of n_kv_heads")
    _check(k.size(2) == v.size(2), f"{fn}: k and v lengths differ")
    _check(q.size(3) == k.size(3) == v.size(3), f"{fn}: head_dim differs")
    _check(q.size(3) == kDimHead, f"{fn}: head_dim must be {kDimHead}")
    _check(q.dtype == k.dtype == v.dtype, f"{fn}: q, k and v must share a dtype")
    _check(q.dtype != torch.float32, f'"{fn}" not implemented for \'Float\'')
    dtype = _dtype_code(q, fn)
    out = torch.empty_like(q)
    B, H, Tq, D = q.shape
    rc = _lib.femto_flash_attention(
        dtype,
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        k.data_ptr(), k.stride(0), k.stride(1), k.stride(2),
        v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
        B, H, k.size(1), Tq, k.size(2), D,
        _stream(q.device),
    )
    _raise_on(rc)
    return out
