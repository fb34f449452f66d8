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


def gla_fwd_args(Q, K, V, log_gamma, r, log_alpha, mix_g, gla_scale, y, state_view, g, eps, chunk_states):
    B, H, T, D = Q.shape
    r = int(r)
    J = D - r
    if K.shape != Q.shape or V.shape[:3] != (B, H, T) or V.shape[-1] != D:
        raise _lib.HofaError(f"Q/K/V shapes disagree: {tuple(Q.shape)} {tuple(K.shape)} {tuple(V.shape)}")
    a = _lib.GlaFwdArgs()
    a.B, a.H, a.T, a.D, a.R = B, H, T, D, r
    a.eps = float(eps)
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
        nc = (T + CHUNK - 1) // CHUNK
        if chunk_states.numel() != B * H * nc * 2 * D * J or chunk_states.element_size() != 2 \
                or not chunk_states.is_contiguous():
            raise _lib.HofaError("chunk_states must be a contiguous 16-bit tensor of B*H*ceil(T/64)*2*D*J elements")
        a.chunk_states = chunk_states.data_ptr()
    return a, keep


def chunk_gla_inlier_fwd(Q, K, V, log_gamma, r, chunk_size, log_alpha=None, mix_g=None, gla_scale=None, out=None,
                         states_in=None, requires_grad=False, *, g: Optional[torch.Tensor] = None,
                         eps: float = 1e-5, chunk_states: Optional[torch.Tensor] = None):
    """Chunked GLA over channels ``[r, d_head)``; returns ``(Y, states_out)``.

    Same contract as the reference (src/chunk_gla_inlier.py:153-237):
    ``Y = (1 - mix_g) * gla_scale * RMSNorm(Y_I; eps=1e-5)`` when both
    ``mix_g`` and ``gla_scale`` are given, else ``Y_I``; ``states_out`` is
    ``[B, H, j_pad, d_pad]`` float32 (powers of two, at least 16) holding the
    final state in ``[:, :, :j, :d_head]`` (zeros elsewhere).  ``chunk_size``
    only shapes the reference's reduction order and is not needed here.
    ``g`` (float32 ``[B,H,T,j]``) gives a general per-channel log decay
    instead of ``log_gamma`` (x ``exp(log_alpha)``); ``chunk_states`` (16-bit,
    ``B*H*ceil(T/64)*2*d_head*j``) receives the state entering every chunk as
    transposed hi/lo operand pairs.
    """
    if requires_grad or states_in is not None:
        raise NotImplementedError("per-chunk state export through states_in is not supported; "
                                  "pass chunk_states instead")
    _lib.require_gpu(Q, K, V, log_gamma, log_alpha, mix_g, gla_scale, out, g, chunk_states)
    lib = _lib.load()
    B, H, T, D = Q.shape
    J = D - int(r)
    Y = out if out is not None else torch.empty(B, H, T, D, dtype=Q.dtype, device=Q.device)
    _lib.expect_shape(Y, (B, H, T, D), "out")
    states_out = torch.zeros(B, H, _pow2_at_least_16(J), _pow2_at_least_16(D), dtype=torch.float32, device=Q.device)
    state_view = states_out[:, :, :J, :D]
    a, keep = gla_fwd_args(Q, K, V, log_gamma, r, log_alpha, mix_g, gla_scale, Y, state_view, g, eps, chunk_states)
    nbytes = lib.hofa_gla_fwd_workspace_bytes(ctypes.byref(a))
    if nbytes == 0:
        _lib.check(-1, "chunk_gla_inlier_fwd")
    stream = _lib.stream_handle(Q.device)
    ws = _lib.WORKSPACES.get(Q.device, stream, "gla_fwd", nbytes)
    _lib.check(lib.hofa_gla_fwd(ctypes.byref(a), ws.data_ptr(), ws.numel(), stream), "chunk_gla_inlier_fwd")
    del keep
    return Y, states_out
