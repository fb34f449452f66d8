"""The hybrid prefill of one HOFA layer's attention core as one call.

``prefill_fwd`` runs the two pathways the reference runs back to back in its
inference ``forward`` (src/HybridOutlierFactorizedAttention.py:201-208:
``chunk_gla_inlier_fwd`` writes ``(1 - mix) * gla_scale * RMSNorm(GLA)``,
then ``exact_attention_triton`` adds ``mix * softmax-attention`` into the same
bf16 buffer) with one difference in rounding: the GLA result is handed to the
attention kernel in float32 and the sum is rounded to the output dtype once,
where the reference rounds the GLA part to bf16 first and the sum again.
The second rounding would cost the stated bf16 bar: at cfg2 (outputs up to
about 4, half a bf16 ulp 0.016 there) two roundings reach 0.027 max-abs
against the float32 oracle, above 2e-2.
"""
from __future__ import annotations

from typing import Optional

import torch

from .chunk_gla_inlier import chunk_gla_inlier_fwd
from .exact_attention import exact_attention


def prefill_fwd(q, k, v, log_gamma, r: int, sm_scale: float, mix, gla_scale, *, log_alpha=None,
                g: Optional[torch.Tensor] = None, eps: float, q_o=None, k_o=None, out=None,
                chunk_states=None, n_out=None, rstd=None, o=None, lse=None):
    """``Y = (1 - mix) * gla_scale * RMSNorm(GLA(q_I, k_I, v, decay)) + mix * softmax(q_O k_O^T sm_scale) v``.

    q, k, v ``[B,H,T,d_h]`` (unit last stride); the GLA reads channels
    ``[r, d_h)`` of q/k, the attention ``q_o``/``k_o`` (``[B,H,T,r]``, RoPE'd)
    or, when they are None, channels ``[0, r)`` of q/k.  ``r == 0`` is the pure
    GLA (``mix`` may then be None).  Returns ``(Y, states_out)`` with
    ``states_out`` as from :func:`chunk_gla_inlier_fwd`.  ``chunk_states``,
    ``n_out``, ``rstd`` (GLA) and ``o``, ``lse`` (attention) are the optional
    saves of a training forward.
    """
    B, H, T, D = v.shape
    dt = v.dtype
    Y = out if out is not None else torch.empty(B, H, T, D, dtype=dt, device=v.device)
    if r == 0:
        _, states = chunk_gla_inlier_fwd(q, k, v, log_gamma, 0, 64, log_alpha=log_alpha, mix_g=mix,
                                         gla_scale=gla_scale, out=Y, g=g, eps=eps, chunk_states=chunk_states,
                                         n_out=n_out, rstd=rstd)
        return Y, states
    part = Y if dt == torch.float32 else torch.empty(B, H, T, D, dtype=torch.float32, device=v.device)
    _, states = chunk_gla_inlier_fwd(q, k, v, log_gamma, r, 64, log_alpha=log_alpha, mix_g=mix, gla_scale=gla_scale,
                                     out=part, g=g, eps=eps, chunk_states=chunk_states, n_out=n_out, rstd=rstd)
    exact_attention(q if q_o is None else q_o, k if k_o is None else k_o, v, r, sm_scale, mix, out=Y, o=o, lse=lse,
                    acc=None if part is Y else part)
    return Y, states
