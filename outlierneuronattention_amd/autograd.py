"""Autograd function over the HOFA attention core (training path).

``hofa_core(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, r, sm_scale)``
computes, for every head and token,

    Y = (1 - mix) * gla_scale * RMSNorm(GLA(q[..., r:], k[..., r:], v, g))
        + mix * softmax_causal(q_o k_o^T * sm_scale) v,
    g[t, c] = log_gamma[t] * exp(log_alpha[c])       (log_gamma[t] without alpha)

with RMSNorm eps = finfo(float32).eps.  This is the Train module's hybrid
forward after projections, gates and RoPE (SDPA + fla ``chunk_gla`` +
``RMSNorm * gla_scale`` + ``lerp``, src/HybridOutlierFactorizedAttentionTrain.py:233-294).
``q_o``/``k_o`` are the RoPE'd outlier channels, ``q``/``k`` the projections
whose channels ``[r, d_head)`` feed the GLA.  With ``r == 0`` (and no mix) it
is the pure-GLA branch ``gla_scale * RMSNorm(GLA)`` (:201-223).
"""
from __future__ import annotations

import torch

from .chunk_gla_inlier import chunk_gla_inlier_fwd
from .exact_attention import exact_attention

FP32_EPS = float(torch.finfo(torch.float32).eps)


class _HOFACore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, r, sm_scale):
        B, H, T, D = v.shape
        if mix is None:  # pure GLA: Y = gla_scale * RMSNorm(GLA)
            mix_eff = torch.zeros(B, H, T, dtype=v.dtype, device=v.device)
        else:
            mix_eff = mix
        y = torch.empty(B, H, T, D, dtype=v.dtype, device=v.device)
        chunk_gla_inlier_fwd(q, k, v, log_gamma, r, 64, log_alpha=log_alpha, mix_g=mix_eff, gla_scale=gla_scale,
                             out=y, eps=FP32_EPS)
        if r > 0:
            exact_attention(q_o, k_o, v, r, sm_scale, mix_eff, out=y)
        ctx.mark_non_differentiable()
        return y

    @staticmethod
    def backward(ctx, dy):
        raise NotImplementedError("the backward kernels of the HOFA core are not available in this build")


def hofa_core(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, r: int, sm_scale: float):
    return _HOFACore.apply(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, int(r), float(sm_scale))
