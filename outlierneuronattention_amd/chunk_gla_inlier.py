"""Inlier-pathway prefill: drop-in for ``src/chunk_gla_inlier.py``.

``chunk_gla_inlier_fwd`` keeps the reference signature and return value
(src/chunk_gla_inlier.py:153-237) and runs ``csrc/hofa_gla.hip`` through the C
ABI (``hofa_gla_fwd`` in include/hofa.h).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

CHUNK = 64  # kernel chunk length; results do not depend on the caller's chunk_size


def _pow2_at_least_16(n: int) -> int:
    return max(1 << (max(n, 1) - 1).bit_length(), 16)


def chunk_states_numel(B: int, H: int, T: int, D: int, J: int) -> int:
    """Elements of the 16-bit per-chunk entering-state buffer saved for the backward pass."""
    return B * H * ((T + CHUNK - 1) // CHUNK) * 4 * D * J


def gla_fwd_args(Q, K, V, log_gamma, r, log_alpha, mix_g, gla_scale, y, state_view, g, eps, chunk_states,
                 n_out=None, rstd=None, round_operands=False):
    B, H, T, D = Q.shape
    r = int(r)
    J = D - r
    if K.shape != Q.shape or V.shape[:3] != (B, H, T) or V.shape[-1] != D:
        raise _lib.HofaError(f"Q/K/V shapes disagree: {tuple(Q.shape)} {tuple(K.shape)} {tuple(V.shape)}")
    a = _lib.GlaFwdArgs()
    a.B, a.H, a.T, a.D, a.R = B, H, T, D, r
    a.eps = float(eps)
    a.round_operands = 1 if round_operands else 0
    a.q, a.k, a.v, a.y = _lib.view(Q), _lib.view(K), _lib.view(V), _lib.view(y)
    keep = []
    if g is not None:
        _lib.expect_shape(g, (B, H, T, J), "g")
        if g.dtype != torch.float32:
            raise _lib.HofaError("g must be float32")
        a.g = _lib.view(g)
    else:
        a.log_gamma = _lib.view(log_gamma, _lib.per_token_strides(log_gamma, B, H, T, "log_gamma"))
        if log_alpha is not None:
            la, st = _lib.per_head_strides(log_alpha, H, J, "log_alpha")
            keep.append(la)
            a.log_alpha = _lib.view(la, st)
    if mix_g is not None and gla_scale is not None:
        a.fuse_norm_gate = 1
        a.mix = _lib.view(mix_g, _lib.per_token_strides(mix_g, B, H, T, "mix_g"))
        gs, st = _lib.per_head_strides(gla_scale, H, D, "gla_scale")
        keep.append(gs)
        a.gla_scale = _lib.view(gs, st)
    _lib.expect_shape(state_view, (B, H, J, D), "state_out")
    a.state_out = _lib.view(state_view)
    if chunk_states is not None:
        if chunk_states.numel() != chunk_states_numel(B, H, T, D, J) or chunk_states.element_size() != 2 \
                or not chunk_states.is_contiguous():
            raise _lib.HofaError("chunk_states must be a contiguous 16-bit tensor of B*H*ceil(T/64)*4*D*J elements")
        a.chunk_states = chunk_states.data_ptr()
    if n_out is not None:
        _lib.expect_shape(n_out, (B, H, T, D), "n_out")
        if rstd is None or rstd.dtype != torch.float32 or not rstd.is_contiguous() or rstd.numel() != B * H * T:
            raise _lib.HofaError("n_out needs rstd: a contiguous float32 tensor of B*H*T elements")
        a.n_out = _lib.view(n_out)
        a.rstd = rstd.data_ptr()
    return a, keep


def chunk_gla_inlier_fwd(Q, K, V, log_gamma, r, chunk_size, log_alpha=None, mix_g=None, gla_scale=None, out=None,
                         states_in=None, requires_grad=False, *, g: Optional[torch.Tensor] = None,
                         eps: float = 1e-5, chunk_states: Optional[torch.Tensor] = None,
                         n_out: Optional[torch.Tensor] = None, rstd: Optional[torch.Tensor] = None,
                         round_operands: bool = False):
    """Chunked GLA over channels ``[r, d_head)``; returns ``(Y, states_out)``.

    Same contract as the reference (src/chunk_gla_inlier.py:153-237):
    ``Y = (1 - mix_g) * gla_scale * RMSNorm(Y_I; eps=1e-5)`` when both
    ``mix_g`` and ``gla_scale`` are given, else ``Y_I``; ``states_out`` is
    ``[B, H, j_pad, d_pad]`` float32 (powers of two, at least 16) holding the
    final state in ``[:, :, :j, :d_head]`` (zeros elsewhere).  ``chunk_size``
    only shapes the reference's reduction order and is not needed here.
    ``g`` (float32 ``[B,H,T,j]``) gives a general per-channel log decay
    instead of ``log_gamma`` (x ``exp(log_alpha)``).  For a backward pass:
    ``chunk_states`` (16-bit, ``chunk_states_numel(...)`` elements) receives
    the state entering every chunk as hi/lo operand pairs, ``n_out``
    (``[B,H,T,d_head]``, dtype of Q) ``RMSNorm(Y_I)`` and ``rstd`` (float32,
    ``B*H*T``) the per-token reciprocal RMS.  By default every matrix-product
    operand is a hi/lo bf16 pair, which tracks an fp32 computation;
    ``round_operands`` (bf16/f16 inputs, no ``chunk_states``) rounds each
    operand and the carried state to bf16 once, as the reference kernel does
    (src/chunk_gla_inlier.py:96-121), with the reference's larger error.
    """
    if requires_grad or states_in is not None:
        raise NotImplementedError("per-chunk state export through states_in is not supported; "
                                  "pass chunk_states instead")
    _lib.require_gpu(Q, K, V, log_gamma, log_alpha, mix_g, gla_scale, out, g, chunk_states, n_out, rstd)
    lib = _lib.load()
    B, H, T, D = Q.shape
    J = D - int(r)
    Y = out if out is not None else torch.empty(B, H, T, D, dtype=Q.dtype, device=Q.device)
    _lib.expect_shape(Y, (B, H, T, D), "out")
    # the kernel writes the state and the zero rows of its padding (D is 64 or 128: no column padding)
    j_pad, d_pad = _pow2_at_least_16(J), _pow2_at_least_16(D)
    if d_pad != D:
        raise _lib.HofaError(f"chunk_gla_inlier_fwd: head dim {D} unsupported")
    states_out = torch.empty(B, H, j_pad, d_pad, dtype=torch.float32, device=Q.device)
    state_view = states_out[:, :, :J, :D]
    if round_operands and chunk_states is not None:
        raise _lib.HofaError("round_operands is for inference: a backward pass (chunk_states) needs hi/lo operands")
    a, keep = gla_fwd_args(Q, K, V, log_gamma, r, log_alpha, mix_g, gla_scale, Y, state_view, g, eps, chunk_states,
                           n_out, rstd, round_operands and Q.dtype != torch.float32)
    a.state_pad_rows = j_pad - J
    nbytes = lib.hofa_gla_fwd_workspace_bytes(ctypes.byref(a))
    if nbytes == 0:
        _lib.check(-1, "chunk_gla_inlier_fwd")
    stream = _lib.stream_handle(Q.device)
    ws = _lib.WORKSPACES.get(Q.device, stream, "gla_fwd", nbytes)
    _lib.check(lib.hofa_gla_fwd(ctypes.byref(a), ws.data_ptr(), ws.numel(), stream), "chunk_gla_inlier_fwd")
    del keep
    return Y, states_out


def chunk_gla_inlier_bwd(Q, K, V, log_gamma, r, dy, n, rstd, chunk_states, gla_scale, *, log_alpha=None, mix_g=None,
                         o=None, g=None, dq=None, dk=None, dv=None, want_attn_grad=False):
    """Backward of ``Y = (1 - mix_g) * gla_scale * RMSNorm(GLA(Q_I, K_I, V, g)) [+ mix_g * O]``.

    ``n``, ``rstd`` and ``chunk_states`` come from the forward
    (:func:`chunk_gla_inlier_fwd` with ``n_out``/``rstd``/``chunk_states``),
    ``o`` is the outlier attention output ``O`` (for ``d_mix``).  Returns a
    dict with ``dq``/``dk`` (columns ``[r, d)`` written, the rest untouched),
    ``dv``, ``d_log_gamma`` (or ``d_g`` for a general float32 ``g``),
    ``d_log_alpha`` (``[H, j]`` float32, when ``log_alpha`` is given),
    ``d_mix`` (``[B,H,T]`` float32), ``d_gla_scale`` (``[H, d]`` float32) and,
    with ``want_attn_grad``, ``dout_attn = mix_g * dy`` and ``delta`` for
    :func:`exact_attention_bwd`.  The reference trains this path through
    autograd of fla's ``chunk_gla`` and torch ops
    (src/HybridOutlierFactorizedAttentionTrain.py:263-294).
    """
    _lib.require_gpu(Q, K, V, log_gamma, dy, n, rstd, chunk_states, gla_scale, log_alpha, mix_g, o, g, dq, dk, dv)
    lib = _lib.load()
    B, H, T, D = Q.shape
    r = int(r)
    J = D - r
    dev = Q.device
    if K.shape != Q.shape or tuple(V.shape) != (B, H, T, D):
        raise _lib.HofaError(f"Q/K/V shapes disagree: {tuple(Q.shape)} {tuple(K.shape)} {tuple(V.shape)}")
    for name, t in (("dy", dy), ("n", n)):
        _lib.expect_shape(t, (B, H, T, D), name)
    if rstd.dtype != torch.float32 or not rstd.is_contiguous() or rstd.numel() != B * H * T:
        raise _lib.HofaError("rstd must be a contiguous float32 tensor of B*H*T elements")
    if chunk_states.numel() != chunk_states_numel(B, H, T, D, J) or chunk_states.element_size() != 2 \
            or not chunk_states.is_contiguous():
        raise _lib.HofaError("chunk_states must be the contiguous 16-bit buffer written by the forward")
    dq = torch.empty_like(Q) if dq is None else dq
    dk = torch.empty_like(K) if dk is None else dk
    dv = torch.empty(B, H, T, D, dtype=V.dtype, device=dev) if dv is None else dv
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        _lib.expect_shape(t, (B, H, T, D), name)
    out = {"dq": dq, "dk": dk, "dv": dv}
    a = _lib.GlaBwdArgs()
    a.B, a.H, a.T, a.D, a.R = B, H, T, D, r
    a.q, a.k, a.v = _lib.view(Q), _lib.view(K), _lib.view(V)
    a.dy, a.n = _lib.view(dy), _lib.view(n)
    a.rstd, a.chunk_states = rstd.data_ptr(), chunk_states.data_ptr()
    a.dq, a.dk, a.dv = _lib.view(dq), _lib.view(dk), _lib.view(dv)
    keep = []
    if g is not None:
        _lib.expect_shape(g, (B, H, T, J), "g")
        if g.dtype != torch.float32:
            raise _lib.HofaError("g must be float32")
        a.g = _lib.view(g)
        out["d_g"] = torch.empty(B, H, T, J, dtype=torch.float32, device=dev)
        a.d_g = _lib.view(out["d_g"])
    else:
        a.log_gamma = _lib.view(log_gamma, _lib.per_token_strides(log_gamma, B, H, T, "log_gamma"))
        out["d_log_gamma"] = torch.empty(B, H, T, dtype=torch.float32, device=dev)
        a.d_log_gamma = _lib.view(out["d_log_gamma"])
        if log_alpha is not None:
            la, st = _lib.per_head_strides(log_alpha, H, J, "log_alpha")
            keep.append(la)
            a.log_alpha = _lib.view(la, st)
            out["d_log_alpha"] = torch.empty(H, J, dtype=torch.float32, device=dev)
            a.d_log_alpha = _lib.view(out["d_log_alpha"])
    gs, st = _lib.per_head_strides(gla_scale, H, D, "gla_scale")
    keep.append(gs)
    a.gla_scale = _lib.view(gs, st)
    out["d_gla_scale"] = torch.empty(H, D, dtype=torch.float32, device=dev)
    a.d_gla_scale = _lib.view(out["d_gla_scale"])
    if mix_g is not None:
        a.mix = _lib.view(mix_g, _lib.per_token_strides(mix_g, B, H, T, "mix_g"))
        out["d_mix"] = torch.empty(B, H, T, dtype=torch.float32, device=dev)
        a.d_mix = _lib.view(out["d_mix"])
    if o is not None:
        _lib.expect_shape(o, (B, H, T, D), "o")
        a.o = _lib.view(o)
    if want_attn_grad:
        if mix_g is None or o is None:
            raise _lib.HofaError("want_attn_grad needs mix_g and o")
        out["dout_attn"] = torch.empty(B, H, T, D, dtype=Q.dtype, device=dev)
        out["delta"] = torch.empty(B * H * T, dtype=torch.float32, device=dev)
        a.dout_attn = _lib.view(out["dout_attn"])
        a.delta = out["delta"].data_ptr()
    nbytes = lib.hofa_gla_bwd_workspace_bytes(ctypes.byref(a))
    if nbytes == 0:
        _lib.check(-1, "chunk_gla_inlier_bwd")
    stream = _lib.stream_handle(dev)
    ws = _lib.WORKSPACES.get(dev, stream, "gla_bwd", nbytes)
    _lib.check(lib.hofa_gla_bwd(ctypes.byref(a), ws.data_ptr(), ws.numel(), stream), "chunk_gla_inlier_bwd")
    del keep
    return out
