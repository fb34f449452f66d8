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
whose channels ``[r, d_head)`` feed the GLA; ``q_o = k_o = None`` means the
outlier channels are ``q[..., :r]`` / ``k[..., :r]`` themselves (no RoPE), and
their gradients land in ``dq[..., :r]`` / ``dk[..., :r]`` directly.  With
``r == 0`` (and no mix) it is the pure-GLA branch ``gla_scale * RMSNorm(GLA)`` (:201-223).

The backward runs the HIP kernel pair ``hofa_gla_bwd`` (epilogue + inlier
GLA) then ``hofa_attn_bwd`` (outlier softmax attention, accumulating into
dv); the reference relies on autograd through SDPA and fla instead.
"""
from __future__ import annotations

import torch

from .chunk_gla_inlier import chunk_gla_inlier_bwd, chunk_states_numel
from .exact_attention import exact_attention_bwd
from .prefill import prefill_fwd

FP32_EPS = float(torch.finfo(torch.float32).eps)


def _rows_ok(t: torch.Tensor) -> torch.Tensor:
    """The kernels need unit last stride and 16-byte aligned rows."""
    es = t.element_size()
    if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1]):
        return t
    return t.contiguous()


def _grad_like(g: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """Reduce a full-shape gradient to a broadcast input's shape and dtype."""
    if tuple(g.shape) != tuple(ref.shape):
        g = g.sum_to_size(ref.shape) if g.numel() != ref.numel() else g.reshape(ref.shape)
    return g.to(ref.dtype)


class _HOFACore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, r, sm_scale):
        B, H, T, D = v.shape
        J = D - r
        dev = v.device
        train = any(ctx.needs_input_grad[:9])
        mix_eff = torch.zeros(B, H, T, dtype=v.dtype, device=dev) if mix is None else mix
        y = torch.empty(B, H, T, D, dtype=v.dtype, device=dev)
        n = rstd = cs = o = lse = None
        if train:
            n = torch.empty(B, H, T, D, dtype=v.dtype, device=dev)
            rstd = torch.empty(B * H * T, dtype=torch.float32, device=dev)
            cs = torch.empty(chunk_states_numel(B, H, T, D, J), dtype=torch.int16, device=dev)
        if r > 0 and train and mix is not None:
            o = torch.empty(B, H, T, D, dtype=v.dtype, device=dev)
            lse = torch.empty(B * H * T, dtype=torch.float32, device=dev)
        prefill_fwd(q, k, v, log_gamma, r, sm_scale, mix_eff, gla_scale, log_alpha=log_alpha, eps=FP32_EPS,
                    q_o=q_o, k_o=k_o, out=y, chunk_states=cs, n_out=n, rstd=rstd, o=o, lse=lse)
        if train:
            ctx.save_for_backward(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, n, rstd, cs, o, lse)
            ctx.r, ctx.sm_scale = r, sm_scale
        return y

    @staticmethod
    def backward(ctx, dy):
        q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, n, rstd, cs, o, lse = ctx.saved_tensors
        r, sm_scale = ctx.r, ctx.sm_scale
        dy = _rows_ok(dy.to(v.dtype))
        attn = r > 0 and mix is not None
        g = chunk_gla_inlier_bwd(q, k, v, log_gamma, r, dy, n, rstd, cs, gla_scale, log_alpha=log_alpha, mix_g=mix,
                                 o=o, want_attn_grad=attn)
        dq, dk, dv = g["dq"], g["dk"], g["dv"]
        shared = q_o is None  # outlier channels are q[..., :r]: their gradient goes into dq[..., :r]
        dq_o = dk_o = None
        if attn:
            if shared:
                exact_attention_bwd(q, k, v, g["dout_attn"], lse, g["delta"], r, sm_scale, dq=dq, dk=dk, dv=dv,
                                    dv_accumulate=True)
            else:
                dq_o, dk_o, _ = exact_attention_bwd(q_o, k_o, v, g["dout_attn"], lse, g["delta"], r, sm_scale,
                                                    dv=dv, dv_accumulate=True)
        if r > 0 and not (attn and shared):
            dq[..., :r].zero_()
            dk[..., :r].zero_()
            if not shared:
                dq_o = dq_o if dq_o is not None else torch.zeros_like(q_o)
                dk_o = dk_o if dk_o is not None else torch.zeros_like(k_o)
        d_lg = _grad_like(g["d_log_gamma"], log_gamma)
        d_la = _grad_like(g["d_log_alpha"], log_alpha) if log_alpha is not None else None
        d_mix = _grad_like(g["d_mix"], mix) if mix is not None else None
        d_gs = _grad_like(g["d_gla_scale"], gla_scale)
        if dq_o is not None:
            dq_o, dk_o = dq_o.to(q_o.dtype), dk_o.to(k_o.dtype)
        return dq_o, dk_o, dq, dk, dv, d_lg, d_la, d_mix, d_gs, None, None


def hofa_core(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, r: int, sm_scale: float):
    q, k, v = _rows_ok(q), _rows_ok(k), _rows_ok(v)
    if q_o is not None:
        q_o, k_o = _rows_ok(q_o), _rows_ok(k_o)
    return _HOFACore.apply(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, int(r), float(sm_scale))
