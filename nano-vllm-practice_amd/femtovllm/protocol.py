"""Names shared by the operator layer, the engine and its entry points.

Every name the reference's ``femtovllm.protocol`` defines
(femtovllm/protocol.py:8-100) is defined here with the same fields, values
and order, so engine modules that import them (femtovllm/__init__.py:4,
femtovllm/models/qwen/qwen3.py:14, femtovllm/engine/model_runner.py:10,
femtovllm/engine/core_engine.py:11, femtovllm/engine/sequence.py:5,
femtovllm/engine/scheduler/v3.py:9, femtovllm/engine/kv_cache_manager/v3.py:6,
femtovllm/entrypoints/llm.py:10, femtovllm/inputs/input_builder.py:6) find
them when this package provides ``femtovllm.protocol``.  Only the enums and
``VarlenAttnMetadata`` are read by the attention path itself.
"""

from __future__ import annotations

import dataclasses
import enum
from typing import NamedTuple, Optional, Union

import torch


class StopReason(str, enum.Enum):
    """Why a sequence finished (protocol.py:8-17): normal ends, then aborts."""

    EOS = "EOS"
    LENGTH = "LENGTH"

    OOM = "OOM"
    # The scheduler aborts a sequence whose context passes the decode
    # kernel's limit (femtovllm/engine/scheduler/v3.py:80-81).
    HARDWARE_LIMIT = "HARDWARE_LIMIT"


class AttentionBackend(str, enum.Enum):
    """Which varlen attention route a model layer takes (protocol.py:20-25)."""

    PYTORCH = "pytorch"
    CUSTOM_GEMM = "custom_gemm"
    CUSTOM_GEMM_GEMV = "custom_gemm_gemv"


class ImplCustomKernel(str, enum.Enum):
    """Kernel family selector kept for signature compatibility (protocol.py:28-32).

    Both members run the same HIP kernels for gfx950; there is no second
    backend behind ``TRITON``.
    """

    CUDA = "cuda"
    TRITON = "triton"


@dataclasses.dataclass
class SamplingParams:
    """Per-request sampling and stopping settings (protocol.py:35-56)."""

    temperature: float = 1.0
    presence_penalty: float = 1.0

    stop_token_ids: list = dataclasses.field(default_factory=list)
    max_new_tokens: int = 5000

    def clone(self) -> "SamplingParams":
        """A copy whose ``stop_token_ids`` list is not shared."""
        return dataclasses.replace(self, stop_token_ids=list(self.stop_token_ids))


@dataclasses.dataclass
class VarlenAttnMetadata:
    """Per-step attention metadata the ModelRunner hands to every layer (protocol.py:58-81).

    The attention ops read ``positions``, ``cu_seqlens``, ``max_q_len``,
    ``Q_TILE_SIZE``, ``cu_q_tiles``, ``q_tile_to_seq_idx``, ``kv_lens``,
    ``max_kv_len`` and ``block_tables`` (int32, -1 padded); the decode
    route leaves the prefill-only fields ``None`` and sets ``is_decoding``
    (femtovllm/engine/model_runner.py:238-261, 312-335).
    """

    positions: torch.Tensor
    raw_positions: list

    cu_seqlens: Optional[torch.Tensor]
    raw_cu_seqlens: Optional[list]
    max_q_len: int

    Q_TILE_SIZE: Optional[int]
    raw_cu_q_tiles: Optional[list]
    cu_q_tiles: Optional[torch.Tensor]
    raw_q_tile_to_seq_idx: Optional[list]
    q_tile_to_seq_idx: Optional[torch.Tensor]

    k_cache_pools: list
    v_cache_pools: list
    kv_lens: torch.Tensor
    max_kv_len: int

    block_tables: torch.Tensor
    raw_block_tables: list

    is_decoding: bool


ReqId = Union[int, str]
SeqId = Union[int, str]


class StepDelta(NamedTuple):
    """One streamed token of one sequence (protocol.py:88-100)."""

    req_id: ReqId
    seq_id: SeqId
    new_token_id: int
    stop_reason: Optional[StopReason]
