"""Host wrappers of the single-token TransformerBlock kernels
(``csrc/hofa_decode_layer.hip``; ``hofa_rows_linear``,
``hofa_decode_prologue`` and ``hofa_decode_advance`` in include/hofa.h).

They take device tensors, enqueue on the current stream and allocate
nothing, so a whole greedy step can be captured in one HIP graph
(``decode_loop.GreedyGraphDecoder``).  Each mirrors a piece of the
reference's per-token path (src/HybridOutlierFactorizedAttention.py:223-451,
src/inference.py:220-239); see the C header for the exact arithmetic.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

_SIXTEEN_BIT = (torch.bfloat16, torch.float16)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """A ``[B, n]`` view of per-row data given as ``[B, n]`` or ``[B, 1, n]``
    with a unit last stride."""
    if t.dim() == 3 and t.shape[1] == 1:
        t = t[:, 0]
    if t.dim() != 2 or t.stride(-1) != 1:
        raise _lib.HofaError(f"{name}: expected [B, n] rows with a unit last stride, got {tuple(t.shape)}")
    return t


def argmax_slots(n: int) -> int:
    """Greedy-key slots per batch row of a row-linear over ``n`` outputs (one per 16-row block)."""
    return (n + 15) // 16


def greedy_from_keys(keys: torch.Tensor, B: int, n: int) -> torch.Tensor:
    """Token index per batch row from the per-block keys (host-side mirror of
    the feedback kernel's reduction, for tests): keys are unsigned 64-bit
    ``value bits << 32 | 0xffffffff - index`` stored as int64."""
    k = keys[:B * argmax_slots(n)].view(B, -1) ^ torch.iinfo(torch.int64).min  # unsigned order as signed
    best = k.max(dim=1).values ^ torch.iinfo(torch.int64).min
    return 0xFFFFFFFF - (best & 0xFFFFFFFF)


def rows_linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, bias: Optional[torch.Tensor] = None,
                ln: Optional[tuple] = None, gelu: bool = False, scale: float = 1.0, scale_cols: int = 0,
                res: Optional[torch.Tensor] = None, argmax: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``out[b] = res[b] + (GELU?)(LN?(x[b]) @ weight.T + bias)`` with ``scale``
    applied to the first ``scale_cols`` outputs; ``ln = (weight, bias, eps)``
    of an ``nn.LayerNorm``.  ``argmax`` (int64, ``B * argmax_slots(N)``
    entries) also receives each 16-row block's greedy key per row (see
    ``greedy_from_keys``).  ``res`` may be ``out``."""
    x2, o2 = _rows(x, "x"), _rows(out, "out")
    B, K = x2.shape
    N = weight.shape[0]
    if weight.shape != (N, K) or not weight.is_contiguous():
        raise _lib.HofaError(f"weight: expected a contiguous [{N}, {K}] matrix, got {tuple(weight.shape)}")
    if o2.shape != (B, N):
        raise _lib.HofaError(f"out: expected [{B}, {N}], got {tuple(o2.shape)}")
    lw, lb = (None, None) if ln is None else (ln[0], ln[1])
    for t, name in ((x2, "x"), (weight, "weight"), (o2, "out"), (bias, "bias"), (res, "res"),
                    (lw, "ln.weight"), (lb, "ln.bias")):
        if t is not None and t.dtype != weight.dtype:
            raise _lib.HofaError(f"{name}: dtype {t.dtype} differs from the weight's {weight.dtype}")
        if t is not None and t is not x2 and t is not o2 and t is not res and not t.is_contiguous():
            raise _lib.HofaError(f"{name}: must be contiguous")
    if weight.dtype not in _SIXTEEN_BIT:
        raise _lib.HofaError(f"rows_linear runs on bf16/f16 weights, got {weight.dtype}")
    _lib.require_gpu(x2, weight, o2, bias, res, argmax, lw, lb)
    a = _lib.RowsLinearArgs()
    a.B, a.K, a.N, a.dtype = B, K, N, _lib.dtype_code(weight)
    a.act, a.scale_cols, a.scale = int(gelu), int(scale_cols), float(scale)
    a.x, a.x_stride = x2.data_ptr(), x2.stride(0)
    if ln is not None:
        lw, lb, eps = ln
        if lw.shape != (K,) or (lb is not None and lb.shape != (K,)):
            raise _lib.HofaError(f"ln: expected [{K}] weight/bias")
        a.ln_w, a.ln_b, a.ln_eps = lw.data_ptr(), _ptr(lb), float(eps)
    a.w = weight.data_ptr()
    if bias is not None:
        if bias.shape != (N,):
            raise _lib.HofaError(f"bias: expected [{N}], got {tuple(bias.shape)}")
        a.bias = bias.data_ptr()
    if res is not None:
        r2 = _rows(res, "res")
        if r2.shape != (B, N):
            raise _lib.HofaError(f"res: expected [{B}, {N}], got {tuple(r2.shape)}")
        a.res, a.res_stride = r2.data_ptr(), r2.stride(0)
    a.y, a.y_stride = o2.data_ptr(), o2.stride(0)
    if argmax is not None:
        if argmax.dtype != torch.int64 or argmax.numel() < B * argmax_slots(N) or not argmax.is_contiguous():
            raise _lib.HofaError(f"argmax: expected a contiguous int64 tensor of at least {B * argmax_slots(N)} "
                                 "elements")
        a.argmax = argmax.data_ptr()
    lib = _lib.load()
    _lib.check(lib.hofa_rows_linear(ctypes.byref(a), _lib.stream_handle(x.device)), "rows_linear")
    return out


def decode_prologue(attn, qkv: torch.Tensor, cache_k: torch.Tensor, cache_v: torch.Tensor, pos: torch.Tensor,
                    log_gamma: torch.Tensor, mix: torch.Tensor) -> None:
    """Gates, RoPE at ``pos`` (int64 device scalar) and cache append of one
    token for the attention module ``attn`` (hybrid path); ``qkv [B, 3*H*D]``
    holds the scaled Q | K | V and gets the rotated Q/K back in place;
    writes ``log_gamma`` and ``mix`` (float32 ``[B, H]``)."""
    a = prologue_args(attn, qkv, cache_k, cache_v, pos, log_gamma, mix)
    lib = _lib.load()
    _lib.check(lib.hofa_decode_prologue(ctypes.byref(a), _lib.stream_handle(qkv.device)), "decode_prologue")


def prologue_args(attn, qkv: torch.Tensor, cache_k: torch.Tensor, cache_v: torch.Tensor, pos: torch.Tensor,
                  log_gamma: torch.Tensor, mix: torch.Tensor):
    """A checked ``hofa_decode_prologue_args_t`` (ctypes) for ``decode_prologue``
    or ``hofa_decode_fused``."""
    B = qkv.shape[0]
    H, D, R = attn.num_heads, attn.d_head, attn.r
    L = cache_k.shape[2]
    _lib.expect_shape(qkv, (B, 3 * H * D), "qkv")
    _lib.expect_shape(cache_k, (B, H, L, R), "cache_k")
    _lib.expect_shape(cache_v, (B, H, L, D), "cache_v")
    _lib.expect_shape(log_gamma, (B, H), "log_gamma")
    _lib.expect_shape(mix, (B, H), "mix")
    if not (cache_k.is_contiguous() and cache_v.is_contiguous() and qkv.stride(1) == 1):
        raise _lib.HofaError("decode_prologue: caches must be contiguous and qkv rows unit-stride")
    if log_gamma.dtype != torch.float32 or mix.dtype != torch.float32 or pos.dtype != torch.int64:
        raise _lib.HofaError("decode_prologue: log_gamma/mix are float32, pos is int64")
    params = [(attn.gate_proj.weight, (H, 2 * D), "gate_proj.weight"), (attn.gate_proj.bias, (H,), "gate_proj.bias")]
    if hasattr(attn, "mix_proj"):
        params += [(attn.mix_proj.weight, (H, 2 * D), "mix_proj.weight"), (attn.mix_proj.bias, (H,), "mix_proj.bias")]
    elif hasattr(attn, "fixed_mix"):
        params += [(attn.fixed_mix, (1, H, 1, 1), "fixed_mix")]
    else:
        raise _lib.HofaError("decode_prologue: the module has neither mix_proj nor fixed_mix")
    for t, shape, name in params:
        if tuple(t.shape) != shape or t.dtype != qkv.dtype or not t.is_contiguous():
            raise _lib.HofaError(f"decode_prologue: {name} must be a contiguous {shape} tensor of {qkv.dtype}, "
                                 f"got {tuple(t.shape)} {t.dtype}")
    rope = (attn.rotary_emb.cos_cached, attn.rotary_emb.sin_cached) if hasattr(attn, "rotary_emb") else (None, None)
    _lib.require_gpu(qkv, cache_k, cache_v, pos, log_gamma, mix, *(t for t, _, _ in params), *rope)
    a = _lib.DecodePrologueArgs()
    a.B, a.H, a.D, a.R = B, H, D, R
    a.dtype, a.cache_len = _lib.dtype_code(qkv), L
    a.qkv, a.qkv_stride = qkv.data_ptr(), qkv.stride(0)
    a.gate_w, a.gate_b = attn.gate_proj.weight.data_ptr(), attn.gate_proj.bias.data_ptr()
    if hasattr(attn, "mix_proj"):
        a.mix_w, a.mix_b = attn.mix_proj.weight.data_ptr(), attn.mix_proj.bias.data_ptr()
    else:
        a.fixed_mix = attn.fixed_mix.data_ptr()
    if hasattr(attn, "rotary_emb"):
        rot = attn.rotary_emb
        cos, sin = rot.cos_cached, rot.sin_cached
        if not (cos.is_contiguous() and sin.is_contiguous() and cos.shape == sin.shape and cos.shape[1] == R
                and cos.dtype == sin.dtype and cos.dtype in (torch.float32, qkv.dtype)):
            raise _lib.HofaError(f"decode_prologue: RoPE tables must be contiguous [rows, {R}] float32 or {qkv.dtype}")
        a.cos, a.sin, a.rope_rows = cos.data_ptr(), sin.data_ptr(), cos.shape[0]
        a.rope_dtype = _lib.dtype_code(cos)
    a.pos = pos.data_ptr()
    a.cache_k, a.cache_v = cache_k.data_ptr(), cache_v.data_ptr()
    a.log_gamma, a.mix = log_gamma.data_ptr(), mix.data_ptr()
    return a


def decode_advance(argmax: torch.Tensor, emb: torch.Tensor, x: torch.Tensor, tok: torch.Tensor, out: torch.Tensor,
                   col: torch.Tensor, pos: torch.Tensor, seq_len: torch.Tensor) -> None:
    """End of a greedy step: tokens from the LM head's per-block keys into
    ``tok [B,1]`` and ``out[:, col]``, their embedding rows into ``x``,
    ``col``/``pos``/``seq_len`` advanced by one."""
    x2 = _rows(x, "x")
    B, Dm = x2.shape
    V = emb.shape[0]
    if emb.shape != (V, Dm) or not emb.is_contiguous() or emb.dtype != x2.dtype:
        raise _lib.HofaError(f"emb: expected a contiguous [{V}, {Dm}] table of x's dtype")
    if tok.numel() != B or not tok.is_contiguous() or tok.dtype != torch.int64 or out.dtype != torch.int64 \
            or out.shape[0] != B or any(t.numel() != 1 for t in (col, pos, seq_len)) \
            or col.dtype != torch.int64 or pos.dtype != torch.int64 or seq_len.dtype != torch.int32 \
            or out.stride(1) != 1 or argmax.dtype != torch.int64 or argmax.numel() < B * argmax_slots(V):
        raise _lib.HofaError("decode_advance: tok [B,1], out [B, cols], argmax [B * ceil(vocab/16)], col and pos "
                             "(one element) must be int64, seq_len a one-element int32")
    _lib.require_gpu(argmax, emb, x2, tok, out, col, pos, seq_len)
    a = _lib.DecodeAdvanceArgs()
    a.B, a.d_model, a.vocab, a.dtype, a.out_cols = B, Dm, V, _lib.dtype_code(emb), out.shape[1]
    a.argmax, a.emb, a.x, a.x_stride = argmax.data_ptr(), emb.data_ptr(), x2.data_ptr(), x2.stride(0)
    a.tok, a.out, a.out_stride = tok.data_ptr(), out.data_ptr(), out.stride(0)
    a.col, a.pos, a.seq_len = col.data_ptr(), pos.data_ptr(), seq_len.data_ptr()
    lib = _lib.load()
    _lib.check(lib.hofa_decode_advance(ctypes.byref(a), _lib.stream_handle(x.device)), "decode_advance")
