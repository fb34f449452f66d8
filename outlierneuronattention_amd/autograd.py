"""The HOFA attention core as ``torch.library`` operators (training path).

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

Two custom operators carry it, so ``torch.compile`` traces the core as single
graph nodes (their fake implementations give output shapes, dtypes and
strides without running anything):

* ``hofa::prefill_fwd`` -> ``(Y, states_out, N, rstd, chunk_states, O, lse)``;
  the last five are the saves of a training forward (empty when ``save`` is
  False, or ``O``/``lse`` without the attention pathway);
* ``hofa::prefill_bwd`` -> ``(dq_o, dk_o, dq, dk, dv, d_log_gamma,
  d_log_alpha, d_mix, d_gla_scale)`` in float32 for the decay and gate
  gradients (empty for inputs that were None).

``prefill_bwd`` is registered as the autograd formula of ``prefill_fwd``.  Its
eager implementation runs the HIP kernel pair ``hofa_gla_bwd`` (epilogue +
inlier GLA) then ``hofa_attn_bwd`` (outlier softmax attention, accumulating
into dv); the reference relies on autograd through SDPA and fla instead.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch
from torch import Tensor

from .chunk_gla_inlier import CHUNK, chunk_gla_inlier_bwd, chunk_states_numel
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


def _pow2_at_least_16(n: int) -> int:
    return max(1 << (max(n, 1) - 1).bit_length(), 16)


def _none(dev) -> Tensor:
    return torch.empty(0, device=dev)


# --------------------------------------------------------------------- forward
@torch.library.custom_op("hofa::prefill_fwd", mutates_args=())
def prefill_fwd_op(q: Tensor, k: Tensor, v: Tensor, log_gamma: Tensor, log_alpha: Optional[Tensor],
                   mix: Optional[Tensor], gla_scale: Tensor, q_o: Optional[Tensor], k_o: Optional[Tensor],
                   r: int, sm_scale: float, save: bool
                   ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Hybrid prefill of one layer's attention core; see the module docstring.
    The RMSNorm eps is finfo(float32).eps, as in the Train module (a fixed
    part of the operator rather than an argument: a float argument fed from a
    Python global becomes a symbolic input under ``torch.compile(dynamic=True)``)."""
    q, k, v = _rows_ok(q), _rows_ok(k), _rows_ok(v)
    if q_o is not None:
        q_o, k_o = _rows_ok(q_o), _rows_ok(k_o)
    B, H, T, D = v.shape
    J = D - r
    dev = v.device
    mix_eff = torch.zeros(B, H, T, dtype=v.dtype, device=dev) if mix is None else mix
    y = torch.empty(B, H, T, D, dtype=v.dtype, device=dev)
    n = rstd = cs = o = lse = None
    if save:
        n = torch.empty(B, H, T, D, dtype=v.dtype, device=dev)
        rstd = torch.empty(B * H * T, dtype=torch.float32, device=dev)
        cs = torch.empty(chunk_states_numel(B, H, T, D, J), dtype=torch.int16, device=dev)
        if r > 0 and mix is not None:
            o = torch.empty(B, H, T, D, dtype=v.dtype, device=dev)
            lse = torch.empty(B * H * T, dtype=torch.float32, device=dev)
    _, states = prefill_fwd(q, k, v, log_gamma, r, sm_scale, mix_eff, gla_scale, log_alpha=log_alpha, eps=FP32_EPS,
                            q_o=q_o, k_o=k_o, out=y, chunk_states=cs, n_out=n, rstd=rstd, o=o, lse=lse)
    e = lambda t: _none(dev) if t is None else t  # noqa: E731  (one fresh empty tensor per absent output)
    return y, states, e(n), e(rstd), e(cs), e(o), e(lse)


@prefill_fwd_op.register_fake
def _(q, k, v, log_gamma, log_alpha, mix, gla_scale, q_o, k_o, r, sm_scale, save):
    B, H, T, D = v.shape
    J = D - r
    dev = v.device
    e = lambda: torch.empty(0, device=dev)  # noqa: E731
    y = v.new_empty(B, H, T, D)
    states = torch.empty(B, H, _pow2_at_least_16(J), _pow2_at_least_16(D), dtype=torch.float32, device=dev)
    if not save:
        return y, states, e(), e(), e(), e(), e()
    nc = (T + CHUNK - 1) // CHUNK
    n = v.new_empty(B, H, T, D)
    rstd = torch.empty(B * H * T, dtype=torch.float32, device=dev)
    cs = torch.empty(B * H * nc * 4 * D * J, dtype=torch.int16, device=dev)
    if r > 0 and mix is not None:
        return y, states, n, rstd, cs, v.new_empty(B, H, T, D), torch.empty(B * H * T, dtype=torch.float32,
                                                                              device=dev)
    return y, states, n, rstd, cs, e(), e()


# -------------------------------------------------------------------- backward
@torch.library.custom_op("hofa::prefill_bwd", mutates_args=())
def prefill_bwd_op(dy: Tensor, q_o: Optional[Tensor], k_o: Optional[Tensor], q: Tensor, k: Tensor, v: Tensor,
                   log_gamma: Tensor, log_alpha: Optional[Tensor], mix: Optional[Tensor], gla_scale: Tensor,
                   n: Tensor, rstd: Tensor, chunk_states: Tensor, o: Tensor, lse: Tensor, r: int, sm_scale: float
                   ) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Gradients of ``prefill_fwd``'s ``Y`` given ``dy`` and its saves."""
    q, k, v = _rows_ok(q), _rows_ok(k), _rows_ok(v)
    if q_o is not None:
        q_o, k_o = _rows_ok(q_o), _rows_ok(k_o)
    dy = _rows_ok(dy.to(v.dtype))
    dev = v.device
    attn = r > 0 and mix is not None
    o_, lse_ = (o, lse) if attn else (None, None)
    g = chunk_gla_inlier_bwd(q, k, v, log_gamma, r, dy, n, rstd, chunk_states, gla_scale, log_alpha=log_alpha,
                             mix_g=mix, o=o_, want_attn_grad=attn)
    dq, dk, dv = g["dq"], g["dk"], g["dv"]
    shared = q_o is None  # outlier channels are q[..., :r]: their gradient goes into dq[..., :r]
    dq_o = dk_o = None
    if attn:
        if shared:
            exact_attention_bwd(q, k, v, g["dout_attn"], lse_, g["delta"], r, sm_scale, dq=dq, dk=dk, dv=dv,
                                dv_accumulate=True)
        else:
            dq_o, dk_o, _ = exact_attention_bwd(q_o, k_o, v, g["dout_attn"], lse_, g["delta"], r, sm_scale,
                                                dv=dv, dv_accumulate=True)
    if r > 0 and not (attn and shared):
        dq[..., :r].zero_()
        dk[..., :r].zero_()
        if not shared:
            dq_o = dq_o if dq_o is not None else torch.zeros_like(q_o)
            dk_o = dk_o if dk_o is not None else torch.zeros_like(k_o)
    e = lambda t: _none(dev) if t is None else t  # noqa: E731  (one fresh empty tensor per absent output)
    return (e(dq_o), e(dk_o), dq, dk, dv, g["d_log_gamma"], e(g.get("d_log_alpha")), e(g.get("d_mix")),
            g["d_gla_scale"])


@prefill_bwd_op.register_fake
def _(dy, q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, n, rstd, chunk_states, o, lse, r, sm_scale):
    B, H, T, D = v.shape
    J = D - r
    dev = v.device
    e = lambda: torch.empty(0, device=dev)  # noqa: E731
    f32 = dict(dtype=torch.float32, device=dev)
    dq_o = torch.empty_like(q_o) if q_o is not None else e()
    dk_o = torch.empty_like(k_o) if q_o is not None else e()
    return (dq_o, dk_o, torch.empty_like(q), torch.empty_like(k), v.new_empty(B, H, T, D),
            torch.empty(B, H, T, **f32), torch.empty(H, J, **f32) if log_alpha is not None else e(),
            torch.empty(B, H, T, **f32) if mix is not None else e(), torch.empty(H, D, **f32))


# -------------------------------------------------------------------- autograd
def _setup_context(ctx, inputs, output):
    q, k, v, log_gamma, log_alpha, mix, gla_scale, q_o, k_o, r, sm_scale, save = inputs
    _, states, n, rstd, cs, o, lse = output
    # only Y carries a gradient: no zero tensors for the other outputs' gradients
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(states, n, rstd, cs, o, lse)
    if not save:
        ctx.r = None
        return
    ctx.save_for_backward(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, n, rstd, cs, o, lse)
    ctx.r, ctx.sm_scale = r, sm_scale


def _backward(ctx, dy, *_):
    if ctx.r is None:
        raise RuntimeError("hofa::prefill_fwd was run with save=False; call it with save=True to differentiate")
    if dy is None:
        return (None,) * 12
    q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, n, rstd, cs, o, lse = ctx.saved_tensors
    dq_o, dk_o, dq, dk, dv, d_lg, d_la, d_mix, d_gs = torch.ops.hofa.prefill_bwd(
        dy, q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, n, rstd, cs, o, lse, ctx.r, ctx.sm_scale)
    return (dq, dk, dv, _grad_like(d_lg, log_gamma),
            _grad_like(d_la, log_alpha) if log_alpha is not None else None,
            _grad_like(d_mix, mix) if mix is not None else None,
            _grad_like(d_gs, gla_scale),
            dq_o.to(q_o.dtype) if q_o is not None else None,
            dk_o.to(k_o.dtype) if k_o is not None else None,
            None, None, None)


prefill_fwd_op.register_autograd(_backward, setup_context=_setup_context)


def hofa_core(q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale, r: int, sm_scale: float):
    """``Y`` of the hybrid core (see the module docstring), differentiable
    through ``hofa::prefill_bwd`` when any input requires a gradient."""
    inputs = (q_o, k_o, q, k, v, log_gamma, log_alpha, mix, gla_scale)
    save = torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in inputs)
    return torch.ops.hofa.prefill_fwd(q, k, v, log_gamma, log_alpha, mix, gla_scale, q_o, k_o, int(r),
                                      float(sm_scale), save)[0]


# ---------------------------------------------------------------------- decode
@torch.library.custom_op("hofa::decode_step", mutates_args=("state_out",))
def decode_step_op(q: Tensor, k: Tensor, v: Tensor, cache_k: Tensor, cache_v: Tensor, state_in: Tensor,
                   state_out: Tensor, log_gamma: Tensor, mix: Tensor, norm_w: Tensor, r: int, seq_len: int,
                   sm_scale: float, log_alpha: Optional[Tensor] = None, seq_len_dev: Optional[Tensor] = None
                   ) -> Tensor:
    """One decode token (``fused_hofa_decode``); writes ``state_out``, returns ``Y``."""
    from .hofa_decode import fused_hofa_decode
    return fused_hofa_decode(q, k, v, cache_k, cache_v, state_in, state_out, log_gamma, mix, norm_w, r, seq_len,
                             sm_scale, log_alpha=log_alpha, seq_len_dev=seq_len_dev)


@decode_step_op.register_fake
def _(q, k, v, cache_k, cache_v, state_in, state_out, log_gamma, mix, norm_w, r, seq_len, sm_scale, log_alpha=None,
      seq_len_dev=None):
    return torch.empty_like(q)


__all__: List[str] = ["hofa_core", "prefill_fwd_op", "prefill_bwd_op", "decode_step_op"]
