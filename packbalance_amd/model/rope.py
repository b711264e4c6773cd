"""Rotary position embeddings with per-document position ids (harness, plain PyTorch).

Same math as the reference ``packbalance/model/rope.py:9-42``: an fp32
cos/sin cache indexed by per-document ``position_ids``; ``rotate_half``
(NeoX) applied to q and k in their dtype.  The reference's host-synchronising
range check (``int(position_ids.max())``, rope.py:21) is left out: the
harness builds its position ids itself.
"""

from __future__ import annotations

import torch
from torch import nn


class RotaryEmbedding(nn.Module):
    def __init__(self, head_dim: int, max_seq_len: int, theta: float = 10000.0) -> None:
        super().__init__()
        if head_dim % 2:
            raise ValueError("RoPE requires an even head_dim")
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        freqs = torch.outer(torch.arange(max_seq_len, dtype=torch.float32), inv_freq)
        self.register_buffer("cos_cached", freqs.cos(), persistent=False)
        self.register_buffer("sin_cached", freqs.sin(), persistent=False)

    def forward(self, position_ids: torch.Tensor):
        return self.cos_cached[position_ids], self.sin_cached[position_ids]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin):
    cos = torch.cat((cos, cos), dim=-1).unsqueeze(1).to(dtype=q.dtype)
    sin = torch.cat((sin, sin), dim=-1).unsqueeze(1).to(dtype=q.dtype)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)
