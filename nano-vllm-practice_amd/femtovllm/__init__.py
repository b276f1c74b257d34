"""MI355X-native FemtoVLLM attention hot path.

``femtovllm.ops`` keeps the reference's operator signatures
(femtovllm/ops/__init__.py:82-156) and ``femtovllm._C`` the reference's
extension surface (csrc/bindings.cpp:35-98); both run hand-written HIP
kernels for gfx950 from ``libfemto_attn.so``.

``_DEV`` mirrors the reference's global developer flags
(femtovllm/__init__.py:7-23): ``ops`` reads ``impl_custom_gemm`` /
``impl_custom_gemv`` when ``impl`` is not given, and ``split_kv_decode``
(the one added flag).
"""

import dataclasses

from femtovllm.protocol import AttentionBackend, ImplCustomKernel, SamplingParams


@dataclasses.dataclass
class DevFlags:
    varlen_attn_backend: AttentionBackend = AttentionBackend.CUSTOM_GEMM_GEMV
    impl_custom_gemm: ImplCustomKernel = ImplCustomKernel.TRITON
    impl_custom_gemv: ImplCustomKernel = ImplCustomKernel.CUDA

    fake_varlen_by_batch: bool = False

    scheduler_version: int = 3

    # Not in the reference: when True, ops.paged_attention_gemv accepts
    # max_kv_len above MAX_KV_LEN_NON_SPLIT (8192), the limit the reference
    # leaves "to be implemented" (csrc/utils/constants.cuh:36-39); the HIP
    # decode kernel splits any context over its waves.  The engine's
    # HARDWARE_LIMIT (femtovllm/engine/core_engine.py:27) reads the exported
    # constant, which stays 8192.
    split_kv_decode: bool = False

    @property
    def route_prefill_decode(self) -> bool:
        return self.varlen_attn_backend == AttentionBackend.CUSTOM_GEMM_GEMV


_DEV = DevFlags()

__all__ = ["AttentionBackend", "ImplCustomKernel", "SamplingParams", "DevFlags", "_DEV"]
