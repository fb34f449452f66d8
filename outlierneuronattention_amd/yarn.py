"""YaRN context extension of the rotary tables (src/yarn.py:17-86).

``patch_model_yarn`` rewrites every layer's ``rotary_emb`` for a context
``scale = target_seq_len / original_seq_len`` (or a given ``scale``):

* frequencies: rotary pair ``i`` (of ``dim / 2``) keeps its original
  frequency ``theta_i = base^(-2i/dim)`` below the correction index
  ``low = floor(d(beta_fast))``, is interpolated fully (divided by ``scale``)
  above ``high = ceil(d(beta_slow))``, and ramps linearly in between, where
  ``d(beta) = dim * ln(L / (2 pi beta)) / (2 ln base)`` is the pair whose
  wavelength fits ``beta`` times into the original context ``L`` (the YaRN
  paper's "NTK-by-parts" boundaries).  The ``geometric`` mode (the reference's
  default) scales ``theta_i`` by ``scale^(-ramp_i)``; ``arithmetic`` blends
  ``ramp_i * theta_i / scale + (1 - ramp_i) * theta_i``;
* attention temperature: both tables are multiplied by
  ``mscale = 1 + mscale_coeff * ln(scale)`` (or a given ``mscale``), which
  scales every rotated q.k logit by ``mscale^2``;
* the tables (``max(current rows, target_seq_len)`` rows) are stored in
  ``dtype`` (bfloat16 by default), the new ``inv_freq`` in float32.

With ``scale <= 1`` the original frequencies are kept and only ``mscale``
(1 unless given) and ``dtype`` change.  The module paths read the tables as
they are, and so does the fused decode step, whose in-kernel RoPE accepts
16-bit tables.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

MODES = ("geometric", "arithmetic")


def yarn_find_correction_dim(beta: float, dim: int, base: float, max_seq_len: float) -> float:
    """``d(beta) = dim * ln(L / (2 pi beta)) / (2 ln base)`` (fractional pair index)."""
    return (dim * math.log(max_seq_len / (2.0 * math.pi * beta))) / (2.0 * math.log(base))


def yarn_inv_freq(dim: int, base: float, scale: float, original_seq_len: int, beta_fast: float = 32.0,
                  beta_slow: float = 1.0, mode: str = "geometric", device=None) -> torch.Tensor:
    """float32 ``inv_freq [dim / 2]`` after YaRN scaling (see the module docstring)."""
    mode = str(getattr(mode, "value", mode)).lower()
    if mode not in MODES:
        raise ValueError(f"unknown YaRN mode {mode!r}; expected one of {MODES}")
    theta = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim))
    if scale <= 1.0:
        return theta
    n = dim // 2
    low = max(0, math.floor(yarn_find_correction_dim(beta_fast, dim, base, original_seq_len)))
    high = min(n - 1, math.ceil(yarn_find_correction_dim(beta_slow, dim, base, original_seq_len)))
    if high <= low:
        high = low + 1e-3
    ramp = ((torch.arange(n, dtype=torch.float32, device=device) - low) / (high - low)).clamp(0.0, 1.0)
    if mode == "geometric":
        return theta * scale ** (-ramp)
    return ramp * (theta / scale) + (1.0 - ramp) * theta


def patch_model_yarn(model: nn.Module, target_seq_len: int, original_seq_len: int, beta_fast: float = 32.0,
                     beta_slow: float = 1.0, dtype: torch.dtype = torch.bfloat16, scale: Optional[float] = None,
                     yarn_mode: Optional[str] = None, mscale_coeff: float = 0.1,
                     mscale: Optional[float] = None) -> int:
    """Rewrite the rotary tables of every ``model.layers[i].attn.rotary_emb``;
    returns how many were patched."""
    mode = "geometric" if yarn_mode is None else str(getattr(yarn_mode, "value", yarn_mode)).lower()
    if scale is None:
        scale = max(1.0, float(target_seq_len) / float(original_seq_len))
    base = float(getattr(getattr(model, "config", None), "rope_base", 10000.0))
    if mscale is not None:
        m = float(mscale)
    else:
        m = 1.0 + mscale_coeff * math.log(scale) if scale > 1.0 else 1.0
    patched = 0
    for layer in getattr(model, "layers", []):
        rot = getattr(getattr(layer, "attn", None), "rotary_emb", None)
        if rot is None:
            continue
        dev = rot.inv_freq.device
        inv_freq = yarn_inv_freq(rot.dim, base, scale, original_seq_len, beta_fast, beta_slow, mode, device=dev)
        rows = max(rot.max_seq_len_cached, int(target_seq_len))
        ang = torch.outer(torch.arange(rows, dtype=torch.float32, device=dev), inv_freq)
        full = torch.cat((ang, ang), dim=-1)
        rot.inv_freq = inv_freq
        rot.register_buffer("cos_cached", (full.cos() * m).to(dtype), persistent=False)
        rot.register_buffer("sin_cached", (full.sin() * m).to(dtype), persistent=False)
        rot.max_seq_len_cached = rows
        patched += 1
    return patched
