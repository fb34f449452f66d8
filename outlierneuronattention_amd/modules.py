"""Rotary position embedding on the outlier channels.

Same tables and rotation as the reference (src/modules/modules.py:5-45):
``inv_freq = base^(-(0, 2, .., dim-2)/dim)``, float32 ``cos``/``sin`` of
``cat(freqs, freqs)`` for 131072 positions (grown on demand), and the
half-split rotation ``[x1, x2] -> [-x2, x1]``.
"""
from __future__ import annotations

import torch
import torch.nn as nn


def _tables(dim: int, n: int, base: float, device=None):
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim))
    pos = torch.arange(n, dtype=torch.float32, device=device)
    ang = torch.outer(pos, inv_freq)
    full = torch.cat((ang, ang), dim=-1)
    return inv_freq, full.cos(), full.sin()


class RotaryEmbedding(nn.Module):
    def __init__(self, dim: int, max_seq_len: int = 131072, base: float = 10000.0):
        super().__init__()
        self.dim = dim
        self.base = base
        inv_freq, cos, sin = _tables(dim, max_seq_len, base)
        self.register_buffer("inv_freq", inv_freq, persistent=False)
        self.max_seq_len_cached = max_seq_len
        self.register_buffer("cos_cached", cos, persistent=False)
        self.register_buffer("sin_cached", sin, persistent=False)

    def forward(self, seq_len: int):
        """``(cos, sin)`` rows ``[0, seq_len)``; the tables grow when needed,
        from the current ``inv_freq`` (which a context-extension patch such
        as :func:`outlierneuronattention_amd.yarn.patch_model_yarn` may have
        replaced), in float32 (src/modules/modules.py:19-26)."""
        if seq_len > self.max_seq_len_cached:
            self.max_seq_len_cached = seq_len
            pos = torch.arange(seq_len, dtype=torch.float32, device=self.inv_freq.device)
            ang = torch.outer(pos, self.inv_freq)
            full = torch.cat((ang, ang), dim=-1)
            self.register_buffer("cos_cached", full.cos(), persistent=False)
            self.register_buffer("sin_cached", full.sin(), persistent=False)
        return self.cos_cached[:seq_len], self.sin_cached[:seq_len]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """q, k ``[B, H, N, d]``; cos, sin ``[N, d]`` broadcast over batch and heads."""
    cos = cos[None, None]
    sin = sin[None, None]
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin
