"""Split-K HOFA decode: drop-in for ``src/hofa_decode_triton.py``.

``fused_hofa_decode`` keeps the reference signature and argument meaning
(src/hofa_decode_triton.py:342-351) and runs the gfx950 kernel of
``csrc/hofa_decode.hip`` through the C ABI (``hofa_decode`` in include/hofa.h).
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib


def _expect(t: torch.Tensor, shape, name: str) -> None:
    if tuple(t.shape) != tuple(shape):
        raise _lib.HofaError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")


def log_alpha_strides(log_alpha: torch.Tensor, H: int, J: int):
    """(tensor, (h, j) element strides) for the accepted ``log_alpha`` layouts.

    ``[1,H,1,J]`` and ``[H,J]`` as in the reference (src/hofa_decode_triton.py:359-366).
    A 1-D tensor is read as ``H`` contiguous rows of ``J`` (length ``H*J``) or
    as one row shared by every head (length ``J``).  The reference's 1-D
    branch (:367-368) steps heads by the whole length, which only addresses
    memory inside the tensor when ``H == 1``; both readings agree there.
    """
    if log_alpha.ndim == 4:
        if log_alpha.shape[1:] != (H, 1, J) or log_alpha.shape[0] != 1:
            raise _lib.HofaError(f"log_alpha: expected [1,{H},1,{J}], got {tuple(log_alpha.shape)}")
        return log_alpha, (log_alpha.stride(1), log_alpha.stride(3))
    if log_alpha.ndim == 2:
        _expect(log_alpha, (H, J), "log_alpha")
        return log_alpha, (log_alpha.stride(0), log_alpha.stride(1))
    if log_alpha.ndim == 1 and log_alpha.numel() in (H * J, J):
        la = log_alpha.contiguous()
        return la, ((J if la.numel() == H * J else 0), 1)
    raise _lib.HofaError(f"log_alpha: unsupported shape {tuple(log_alpha.shape)} for H={H}, J={J}")


def _bh_strides(t: torch.Tensor, B: int, H: int, name: str):
    """(b, h) strides of a per-(batch, head) scalar given as ``[B|1,H]``,
    ``[B|1,H,1]`` or ``[B|1,H,1,1]`` (broadcast strides allowed)."""
    if t.dim() < 2 or t.dim() > 4 or t.shape[0] not in (1, B) or t.shape[1] != H or t.numel() != t.shape[0] * H:
        raise _lib.HofaError(f"{name}: expected a [B={B}, H={H}, 1] tensor, got {tuple(t.shape)}")
    sb = t.stride(0) if t.shape[0] > 1 else 0
    return (sb, t.stride(1))


def decode_args(q, k, v, cache_k, cache_v, state_I_in, state_I_out, log_gamma, mix_g, norm_w, R, seq_len,
                sm_scale, split_k=None, log_alpha=None, seq_len_dev=None, y=None, eps=None):
    """Fill a ``hofa_decode_args_t`` (ctypes) from tensors; returns ``(args, y, keepalive)``."""
    B, H, N, D = q.shape
    R = int(R)
    J = D - R
    # Extents are checked here: the C ABI carries strides only.
    for t, name in ((q, "q"), (k, "k"), (v, "v")):
        _expect(t, (B, H, 1, D), name)
    if cache_k.dim() != 4 or cache_k.shape[:2] != (B, H) or cache_k.shape[3] != R:
        raise _lib.HofaError(f"cache_k: expected [{B},{H},L,{R}], got {tuple(cache_k.shape)}")
    _expect(cache_v, (B, H, cache_k.shape[2], D), "cache_v")
    if seq_len_dev is None and not (1 <= int(seq_len) <= cache_k.shape[2]):
        raise _lib.HofaError(f"seq_len={seq_len} outside [1, {cache_k.shape[2]}]")
    _expect(state_I_in, (B, H, J, D), "state_I_in")
    _expect(state_I_out, (B, H, J, D), "state_I_out")
    _expect(norm_w, (H, D), "norm_w")
    y = torch.empty_like(q) if y is None else y
    _expect(y, (B, H, 1, D), "y")
    if eps is None:
        # src/hofa_decode_triton.py:386
        eps = torch.finfo(torch.float32).eps if q.dtype in (torch.bfloat16, torch.float16, torch.float32) \
            else torch.finfo(q.dtype).eps
    a = _lib.DecodeArgs()
    a.B, a.H, a.D, a.R = B, H, D, R
    a.seq_len = int(seq_len) if seq_len_dev is None else 0
    a.cache_len = int(cache_k.shape[2])
    a.seq_len_dev = None if seq_len_dev is None else seq_len_dev.data_ptr()
    a.sm_scale, a.eps = float(sm_scale), float(eps)
    a.split_k = int(split_k or 0)
    a.q, a.k, a.v = _lib.view(q), _lib.view(k), _lib.view(v)
    a.cache_k, a.cache_v = _lib.view(cache_k), _lib.view(cache_v)
    a.state_in, a.state_out = _lib.view(state_I_in), _lib.view(state_I_out)
    a.log_gamma = _lib.view(log_gamma, _bh_strides(log_gamma, B, H, "log_gamma"))
    a.mix = _lib.view(mix_g, _bh_strides(mix_g, B, H, "mix_g"))
    a.norm_w = _lib.view(norm_w, (norm_w.stride(-2), norm_w.stride(-1)))
    keep = [y]
    if log_alpha is not None:
        la, st = log_alpha_strides(log_alpha, H, J)
        a.log_alpha = _lib.view(la, st)
        keep.append(la)
    a.y = _lib.view(y)
    return a, y, keep


def fused_hofa_decode(q, k, v, cache_k, cache_v, state_I_in, state_I_out, log_gamma, mix_g, norm_w,
                      R: int, seq_len: int, sm_scale: float, split_k: Optional[int] = None,
                      log_alpha: Optional[torch.Tensor] = None, seq_len_dev: Optional[torch.Tensor] = None):
    """One decode token of the hybrid attention; returns ``Y [B,H,1,d_h]``.

    Same contract as the reference (src/hofa_decode_triton.py:342-476):
    q, k, v ``[B,H,1,d_h]`` (q/k RoPE'd), ``cache_k [B,H,L,R]`` and
    ``cache_v [B,H,L,d_h]`` with the new token already at row ``seq_len-1``,
    ``state_I_in`` -> ``state_I_out`` fp32 ``[B,H,J,d_h]``, ``log_gamma`` /
    ``mix_g`` ``[B,H,1]``, ``norm_w [H,d_h]``; writes ``state_I_out``.
    ``seq_len_dev`` (int32 device scalar, optional) replaces ``seq_len`` at
    run time so one captured graph can serve successive positions.
    """
    B, H, N, D = q.shape
    assert N == 1  # src/hofa_decode_triton.py:353
    _lib.require_gpu(q, k, v, cache_k, cache_v, state_I_in, state_I_out, log_gamma, mix_g, norm_w, log_alpha)
    if seq_len_dev is not None and (seq_len_dev.dtype != torch.int32 or seq_len_dev.numel() != 1):
        raise _lib.HofaError("seq_len_dev must be a one-element int32 device tensor")
    lib = _lib.load()
    a, y, keep = decode_args(q, k, v, cache_k, cache_v, state_I_in, state_I_out, log_gamma, mix_g, norm_w, R,
                             seq_len, sm_scale, split_k, log_alpha, seq_len_dev)
    nbytes = lib.hofa_decode_workspace_bytes(ctypes.byref(a))
    if nbytes == 0:
        _lib.check(-1, "fused_hofa_decode")
    stream = _lib.stream_handle(q.device)
    ws = _lib.WORKSPACES.get(q.device, stream, "decode", nbytes)
    rc = lib.hofa_decode(ctypes.byref(a), ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "fused_hofa_decode")
    return y

