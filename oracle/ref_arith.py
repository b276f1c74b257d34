"""The reference prefill kernel's arithmetic on one query row -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` import this module; it checks tolerances and is never the
product.  Where ``oracle.attention`` computes attention exactly (float64),
this restates the precision of the reference's Triton prefill kernel
(femtovllm/ops/triton/paged_attention/paged_attention_gemm.py:89-160 of
fishAndShrimp/nano-vllm-practice) for a bf16 cache, one 16-key page at a time:

* scores ``q . k`` accumulated in fp32 and scaled in fp32 (``tl.dot`` and
  ``* scale_softmax``, lines 108, 110);
* the online softmax in fp32: running max, ``exp(m_old - m)`` rescale of the
  row sum and accumulator, ``exp(qk - m)`` weights, row sum of the fp32
  weights (lines 122-138);
* the weights cast to bf16 before the P.V product, accumulated in fp32
  (``tl.cast(qk, DTYPE)``, ``tl.dot``, lines 152-153);
* ``acc / sum`` cast to bf16 on store (lines 155-160).

The tests use it to show what a plain max-abs bound can ask of any kernel that
computes in this precision (see ``tests/helpers.py``).  Pinned in
tests/test_oracle.py: equal scores give the bf16 rounding of the exact mean,
and over random rows it stays within the documented bound of the float64
oracle.
"""

from __future__ import annotations

import numpy as np

PAGE = 16


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bf16 value (ties to even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32)


def prefill_row_bf16(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """One query row over its visible keys ``k``, ``v`` (L, D), all given as
    float32 copies of bf16 values; returns the bf16 output row as float32."""
    q = np.asarray(q, dtype=np.float32)
    m = np.float32(-np.inf)
    s = np.float32(0.0)
    acc = np.zeros(q.shape[-1], dtype=np.float32)
    for p0 in range(0, k.shape[0], PAGE):
        kp, vp = k[p0:p0 + PAGE], v[p0:p0 + PAGE]
        # products of bf16 values are exact in fp32; the sum is rounded once
        qk = (kp.astype(np.float64) @ q.astype(np.float64)).astype(np.float32) * np.float32(scale)
        m_old = m
        m = np.maximum(m, qk.max())
        delta = np.float32(np.exp(np.float32(m_old - m))) if np.isfinite(m_old) else np.float32(0.0)
        s = np.float32(s * delta)
        acc = (acc * delta).astype(np.float32)
        w = np.exp((qk - m).astype(np.float32)).astype(np.float32)
        s = np.float32(s + w.sum(dtype=np.float32))
        acc = (acc + (bf16_round(w).astype(np.float64) @ vp.astype(np.float64))).astype(np.float32)
    return bf16_round(acc / s)
