"""Rotary-embedding tables for ``ops.qk_norm_rope_cache_write``.

Built as ``QwenRotaryEmbedding.__init__`` builds its ``cos`` / ``sin``
buffers (femtovllm/models/qwen/qwen3.py:22-52): ``inv_freq_i = (1/base) **
(2 i / d_head)`` for ``i < d_head/2`` in float32, ``theta = p * inv_freq``
for ``p < max_seqlen``, duplicated to ``d_head`` columns.  A model that
already holds the buffers passes them directly (as float32).
"""

import torch


def rope_tables(max_seqlen: int, d_head: int, base: float = 1000000.0, device=None):
    """(cos, sin), each (max_seqlen, d_head) float32."""
    if d_head % 2 != 0:
        raise ValueError(f"d_head must be even, now {d_head=}")
    inv_freq = torch.arange(d_head // 2, device=device).float()
    inv_freq = (1.0 / base) ** (2 * inv_freq / d_head)
    theta = torch.arange(max_seqlen, device=device).float()[:, None] * inv_freq[None, :]
    theta = torch.cat((theta, theta), dim=-1)
    return torch.cos(theta), torch.sin(theta)
