"""Outlier-pathway prefill: drop-in for ``src/exact_attention.py``.

``exact_attention`` keeps the signature and meaning of the reference's
``exact_attention_triton(q, k, v, r, sm_scale, mix_g, out=None, split_k=None)``
(src/exact_attention.py:163-188) and runs ``csrc/hofa_attn.hip`` through the
C ABI (``hofa_attn_fwd`` in include/hofa.h).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib


def attn_fwd_args(q, k, v, r, sm_scale, mix_g, out, accumulate, o=None, lse=None, acc=None):
    B, H, T, Dq = q.shape
    D = v.shape[-1]
    r = int(r)
    if not (0 < r <= Dq) or k.shape[-1] < r:
        raise _lib.HofaError(f"r={r} must be in (0, {Dq}] and fit q/k")
    if k.shape[:3] != (B, H, T) or v.shape[:3] != (B, H, T):
        raise _lib.HofaError(f"q/k/v shapes disagree: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    _lib.expect_shape(out, (B, H, T, D), "out")
    a = _lib.AttnFwdArgs()
    a.B, a.H, a.T, a.D, a.R = B, H, T, D, r
    a.sm_scale = float(sm_scale)
    a.accumulate = 1 if accumulate else 0
    a.q, a.k, a.v, a.y = _lib.view(q), _lib.view(k), _lib.view(v), _lib.view(out)
    if mix_g is not None:
        a.mix = _lib.view(mix_g, _lib.per_token_strides(mix_g, B, H, T, "mix_g"))
    if o is not None:
        _lib.expect_shape(o, (B, H, T, D), "o")
        a.o = _lib.view(o)
    if lse is not None:
        if lse.dtype != torch.float32 or not lse.is_contiguous() or lse.numel() != B * H * T:
            raise _lib.HofaError("lse must be a contiguous float32 tensor of B*H*T elements")
        a.lse = lse.data_ptr()
    if acc is not None:
        _lib.expect_shape(acc, (B, H, T, D), "acc")
        if acc.dtype != torch.float32:
            raise _lib.HofaError("acc must be float32")
        a.acc = _lib.view(acc)
    return a


def exact_attention(q, k, v, r: int, sm_scale: float, mix_g: Optional[torch.Tensor], out=None, split_k=None,
                    o: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                    acc: Optional[torch.Tensor] = None):
    """Causal softmax attention on ``q[..., :r] k[..., :r]^T * sm_scale`` against
    full-width ``v``, mixed into ``out``: ``out += mix_g * O``.  Without ``out``
    a fresh tensor holding ``mix_g * O`` is returned (the reference starts from
    zeros, src/exact_attention.py:165-166).  ``split_k`` is accepted for
    signature compatibility and unused, as in the reference.  Optional ``o``
    receives O itself and ``lse`` (float32, B*H*T) the base-2 log-sum-exp of
    the logits scaled by ``sm_scale*log2(e)``.  ``acc`` (float32, the shape of
    ``out``) replaces the prior contents of ``out``: ``out = acc + mix_g * O``,
    rounded once (used with a float32 result of ``chunk_gla_inlier_fwd``).
    """
    _lib.require_gpu(q, k, v, mix_g, out, o, lse, acc)
    lib = _lib.load()
    accumulate = out is not None
    if out is None:
        out = torch.empty(*q.shape[:3], v.shape[-1], dtype=v.dtype, device=v.device)
    a = attn_fwd_args(q, k, v, r, sm_scale, mix_g, out, accumulate, o, lse, acc)
    _lib.check(lib.hofa_attn_fwd(ctypes.byref(a), _lib.stream_handle(q.device)), "exact_attention")
    return out


# Name used by the reference's callers.
exact_attention_triton = exact_attention


def exact_attention_bwd(q, k, v, dout, lse, delta, r: int, sm_scale: float, dq=None, dk=None, dv=None,
                        dv_accumulate: bool = False):
    """Gradients of ``O = softmax(q[..., :r] k[..., :r]^T * sm_scale + causal) v``
    given ``dout`` (dL/dO), the base-2 ``lse`` written by :func:`exact_attention`
    and ``delta = rowsum(dout * O)`` (float32, B*H*T).  Returns ``(dq, dk, dv)``
    with ``dq``/``dk`` of width ``r`` (``[B,H,T,r]``); ``dv_accumulate`` adds
    into a given ``dv``.  The reference has no kernel here: it trains through
    autograd of torch SDPA (src/HybridOutlierFactorizedAttentionTrain.py:258-259).
    """
    _lib.require_gpu(q, k, v, dout, lse, delta, dq, dk, dv)
    lib = _lib.load()
    B, H, T, _ = q.shape
    D = v.shape[-1]
    r = int(r)
    if k.shape[:3] != (B, H, T) or v.shape[:3] != (B, H, T) or tuple(dout.shape) != (B, H, T, D):
        raise _lib.HofaError("q/k/v/dout shapes disagree")
    for name, t in (("lse", lse), ("delta", delta)):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != B * H * T:
            raise _lib.HofaError(f"{name} must be a contiguous float32 tensor of B*H*T elements")
    if dq is None:
        dq = torch.empty(B, H, T, r, dtype=q.dtype, device=q.device)
    if dk is None:
        dk = torch.empty(B, H, T, r, dtype=q.dtype, device=q.device)
    if dv is None:
        dv = torch.empty(B, H, T, D, dtype=v.dtype, device=v.device)
        dv_accumulate = False
    a = _lib.AttnBwdArgs()
    a.B, a.H, a.T, a.D, a.R = B, H, T, D, r
    a.sm_scale = float(sm_scale)
    a.dv_accumulate = 1 if dv_accumulate else 0
    a.q, a.k, a.v, a.dout = _lib.view(q), _lib.view(k), _lib.view(v), _lib.view(dout)
    a.lse, a.delta = lse.data_ptr(), delta.data_ptr()
    a.dq, a.dk, a.dv = _lib.view(dq), _lib.view(dk), _lib.view(dv)
    _lib.check(lib.hofa_attn_bwd(ctypes.byref(a), _lib.stream_handle(q.device)), "exact_attention_bwd")
    return dq, dk, dv
