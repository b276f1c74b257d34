"""CPU oracle for the attention prologue -- TEST INFRASTRUCTURE ONLY.

Reference results for the fused QK-norm + RoPE + cache-write kernel: only
``tests/`` and the ``cpu_baseline`` leg of ``bench.py`` may use it; the
shipped operator runs the HIP kernel in ``libfemto_attn.so``.

Restates, in float64 numpy, the steps that femtovllm/models/qwen/qwen3.py
applies to the projected q and k before the attention ops (lines 230-238
and 312-320):

* ``q_norm`` / ``k_norm``: ``torch.nn.RMSNorm(d_head, eps)`` per head
  (qwen3.py:181-183): ``x / sqrt(mean(x**2) + eps) * weight``;
* ``rotary_embd``: ``cos[p] * x + sin[p] * concat(-x2, x1)`` with
  ``(x1, x2) = x.chunk(2)`` and per-token positions ``p``
  (QwenRotaryEmbedding.forward, qwen3.py:97-138), the tables built as in
  ``QwenRotaryEmbedding.__init__`` (qwen3.py:22-52): ``theta = p *
  base**(-2i/d)`` for ``i < d/2``, duplicated to ``d`` columns.
"""

import numpy as np


def rope_tables(max_seqlen: int, d_head: int, base: float = 1000000.0):
    """(cos, sin), each (max_seqlen, d_head) float32, as QwenRotaryEmbedding builds them (qwen3.py:35-52)."""
    i = np.arange(d_head // 2, dtype=np.float32)
    inv_freq = (np.float32(1.0) / np.float32(base)) ** (np.float32(2.0) * i / np.float32(d_head))
    theta = np.arange(max_seqlen, dtype=np.float32)[:, None] * inv_freq[None, :]
    theta = np.concatenate([theta, theta], axis=-1)
    return np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)


def rms_norm(x, weight, eps):
    """``torch.nn.RMSNorm`` over the last axis (float64)."""
    x = np.asarray(x, dtype=np.float64)
    rms = np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x / rms * np.asarray(weight, dtype=np.float64)


def rope(x, cos, sin, positions):
    """Rotary embedding of ``x`` (T, heads, D) at per-token ``positions`` (qwen3.py:111-138)."""
    x = np.asarray(x, dtype=np.float64)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    rot = np.concatenate([-x2, x1], axis=-1)
    pos = np.asarray(positions, dtype=np.int64)
    c = np.asarray(cos, dtype=np.float64)[pos][:, None, :]
    s = np.asarray(sin, dtype=np.float64)[pos][:, None, :]
    return c * x + s * rot


def qk_norm_rope(q, k, q_weight, k_weight, eps, cos, sin, positions):
    """The prologue's q and k: RMSNorm per head, then RoPE at each token's position."""
    return (rope(rms_norm(q, q_weight, eps), cos, sin, positions),
            rope(rms_norm(k, k_weight, eps), cos, sin, positions))
