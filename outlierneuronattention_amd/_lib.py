"""ctypes binding to ``libhofa.so`` (the C ABI declared in ``include/hofa.h``).

torch is imported first on purpose: its bundled HIP runtime is then the one
the library binds to (same SONAME), so torch's streams and allocations are
valid inside the library.  The library is required: there is no fallback, and
every op raises if it is missing or was built for another GPU.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhofa.so")

HOFA_F32, HOFA_BF16, HOFA_F16 = 0, 1, 2
DECODE_STATIC_SCRATCH_BYTES = 8 << 20  # HOFA_DECODE_STATIC_SCRATCH_BYTES of include/hofa.h
_DTYPE_CODE = {torch.float32: HOFA_F32, torch.bfloat16: HOFA_BF16, torch.float16: HOFA_F16}
_ERRORS = {-1: "invalid argument", -2: "unsupported configuration", -3: "launch failure", -4: "workspace"}


class HofaError(RuntimeError):
    """Raised when the HIP library rejects a call or a launch fails."""


class View(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("stride", ctypes.c_int64 * 4)]


class DecodeArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("D", ctypes.c_int32), ("R", ctypes.c_int32),
                ("seq_len", ctypes.c_int32), ("cache_len", ctypes.c_int32),
                ("seq_len_dev", ctypes.c_void_p),
                ("sm_scale", ctypes.c_float), ("eps", ctypes.c_float),
                ("split_k", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("q", View), ("k", View), ("v", View),
                ("cache_k", View), ("cache_v", View),
                ("state_in", View), ("state_out", View),
                ("log_gamma", View), ("mix", View), ("norm_w", View), ("log_alpha", View),
                ("y", View)]


class AttnFwdArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("T", ctypes.c_int32), ("D", ctypes.c_int32),
                ("R", ctypes.c_int32), ("sm_scale", ctypes.c_float), ("accumulate", ctypes.c_int32),
                ("reserved", ctypes.c_int32),
                ("q", View), ("k", View), ("v", View), ("mix", View), ("y", View), ("o", View),
                ("lse", ctypes.c_void_p), ("acc", View)]


class GlaFwdArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("T", ctypes.c_int32), ("D", ctypes.c_int32),
                ("R", ctypes.c_int32), ("eps", ctypes.c_float), ("fuse_norm_gate", ctypes.c_int32),
                ("state_pad_rows", ctypes.c_int32),
                ("q", View), ("k", View), ("v", View),
                ("log_gamma", View), ("log_alpha", View), ("g", View),
                ("mix", View), ("gla_scale", View),
                ("y", View), ("state_out", View),
                ("chunk_states", ctypes.c_void_p),
                ("n_out", View), ("rstd", ctypes.c_void_p),
                ("round_operands", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class AttnBwdArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("T", ctypes.c_int32), ("D", ctypes.c_int32),
                ("R", ctypes.c_int32), ("sm_scale", ctypes.c_float), ("dv_accumulate", ctypes.c_int32),
                ("reserved", ctypes.c_int32),
                ("q", View), ("k", View), ("v", View), ("dout", View),
                ("lse", ctypes.c_void_p), ("delta", ctypes.c_void_p),
                ("dq", View), ("dk", View), ("dv", View)]


class GlaBwdArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("T", ctypes.c_int32), ("D", ctypes.c_int32),
                ("R", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("q", View), ("k", View), ("v", View),
                ("log_gamma", View), ("log_alpha", View), ("g", View),
                ("mix", View), ("gla_scale", View),
                ("n", View), ("o", View),
                ("rstd", ctypes.c_void_p), ("chunk_states", ctypes.c_void_p),
                ("dy", View),
                ("dq", View), ("dk", View), ("dv", View),
                ("d_log_gamma", View), ("d_g", View), ("d_log_alpha", View), ("d_mix", View),
                ("d_gla_scale", View),
                ("dout_attn", View), ("delta", ctypes.c_void_p)]


class RowsLinearArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("K", ctypes.c_int32), ("N", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("act", ctypes.c_int32), ("scale_cols", ctypes.c_int32),
                ("scale", ctypes.c_float), ("ln_eps", ctypes.c_float),
                ("x", ctypes.c_void_p), ("x_stride", ctypes.c_int64),
                ("ln_w", ctypes.c_void_p), ("ln_b", ctypes.c_void_p),
                ("w", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("res", ctypes.c_void_p), ("res_stride", ctypes.c_int64),
                ("y", ctypes.c_void_p), ("y_stride", ctypes.c_int64),
                ("argmax", ctypes.c_void_p)]


class DecodePrologueArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("D", ctypes.c_int32), ("R", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("cache_len", ctypes.c_int32), ("rope_rows", ctypes.c_int32),
                ("rope_dtype", ctypes.c_int32),
                ("qkv", ctypes.c_void_p), ("qkv_stride", ctypes.c_int64),
                ("gate_w", ctypes.c_void_p), ("gate_b", ctypes.c_void_p),
                ("mix_w", ctypes.c_void_p), ("mix_b", ctypes.c_void_p),
                ("fixed_mix", ctypes.c_void_p),
                ("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p),
                ("pos", ctypes.c_void_p),
                ("cache_k", ctypes.c_void_p), ("cache_v", ctypes.c_void_p),
                ("log_gamma", ctypes.c_void_p), ("mix", ctypes.c_void_p)]


class DecodeAdvanceArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("d_model", ctypes.c_int32), ("vocab", ctypes.c_int32),
                ("dtype", ctypes.c_int32), ("out_cols", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("argmax", ctypes.c_void_p), ("emb", ctypes.c_void_p),
                ("x", ctypes.c_void_p), ("x_stride", ctypes.c_int64),
                ("tok", ctypes.c_void_p), ("out", ctypes.c_void_p), ("out_stride", ctypes.c_int64),
                ("col", ctypes.c_void_p), ("pos", ctypes.c_void_p), ("seq_len", ctypes.c_void_p)]


# (name, restype, argtypes) of every entry point declared in include/hofa.h
EXPORTS = [
    ("hofa_decode_workspace_bytes", ctypes.c_size_t, [ctypes.POINTER(DecodeArgs)]),
    ("hofa_decode_plan", ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_int32),
                                        ctypes.POINTER(ctypes.c_int32)]),
    ("hofa_decode", ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("hofa_decode_static", ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]),
    ("hofa_attn_fwd", ctypes.c_int, [ctypes.POINTER(AttnFwdArgs), ctypes.c_void_p]),
    ("hofa_gla_fwd_workspace_bytes", ctypes.c_size_t, [ctypes.POINTER(GlaFwdArgs)]),
    ("hofa_gla_fwd", ctypes.c_int, [ctypes.POINTER(GlaFwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("hofa_attn_bwd", ctypes.c_int, [ctypes.POINTER(AttnBwdArgs), ctypes.c_void_p]),
    ("hofa_gla_bwd_workspace_bytes", ctypes.c_size_t, [ctypes.POINTER(GlaBwdArgs)]),
    ("hofa_gla_bwd", ctypes.c_int, [ctypes.POINTER(GlaBwdArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("hofa_rows_linear", ctypes.c_int, [ctypes.POINTER(RowsLinearArgs), ctypes.c_void_p]),
    ("hofa_decode_prologue", ctypes.c_int, [ctypes.POINTER(DecodePrologueArgs), ctypes.c_void_p]),
    ("hofa_decode_advance", ctypes.c_int, [ctypes.POINTER(DecodeAdvanceArgs), ctypes.c_void_p]),
    ("hofa_decode_fused_workspace_bytes", ctypes.c_size_t, [ctypes.POINTER(DecodeArgs)]),
    ("hofa_decode_fused", ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.POINTER(DecodePrologueArgs),
                                         ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    ("hofa_last_error", ctypes.c_char_p, []),
    ("hofa_version", ctypes.c_int, []),
]

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise HofaError(f"HOFA HIP library not found at {path}; build it with "
                                "`python -m outlierneuronattention_amd.build_lib`")
            lib = ctypes.CDLL(path)
            for name, res, args in EXPORTS:
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().hofa_last_error().decode(errors="replace")
        raise HofaError(f"{what} failed ({_ERRORS.get(rc, rc)}): {msg}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise HofaError(f"unsupported dtype {t.dtype}") from None


def view(t: torch.Tensor | None, strides=None) -> View:
    """A ``hofa_view_t`` of ``t``; ``strides`` overrides ``t.stride()`` (element units)."""
    v = View()
    if t is None:
        return v
    v.data = t.data_ptr()
    v.dtype = dtype_code(t)
    st = list(t.stride() if strides is None else strides)
    for i, s in enumerate(st[:4]):
        v.stride[i] = int(s)
    return v


def expect_shape(t: torch.Tensor, shape, name: str) -> None:
    if tuple(t.shape) != tuple(shape):
        raise HofaError(f"{name}: expected shape {tuple(shape)}, got {tuple(t.shape)}")


def per_token_strides(t: torch.Tensor, B: int, H: int, T: int, name: str):
    """(b, h, t) strides of a per-(batch, head, token) scalar given as
    ``[B|1, H|1, T]`` or ``[B|1, H|1, T, 1]`` (broadcast dims get stride 0)."""
    if t.dim() == 4:
        if t.shape[3] != 1:
            raise HofaError(f"{name}: expected a trailing dim of 1, got {tuple(t.shape)}")
    elif t.dim() != 3:
        raise HofaError(f"{name}: expected [B,H,T] or [B,H,T,1], got {tuple(t.shape)}")
    if t.shape[0] not in (1, B) or t.shape[1] not in (1, H) or t.shape[2] != T:
        raise HofaError(f"{name}: expected [{B},{H},{T}], got {tuple(t.shape)}")
    return tuple(t.stride(i) if t.shape[i] > 1 else 0 for i in range(3))


def per_head_strides(t: torch.Tensor, H: int, W: int, name: str):
    """(h, w) strides of a per-head row given as ``[1,H,1,W]``, ``[H,W]`` or
    ``[H*W]`` (contiguous)."""
    if t.dim() == 4 and t.shape[0] == 1 and t.shape[1] == H and t.shape[2] == 1 and t.shape[3] == W:
        return t, (t.stride(1), t.stride(3))
    if t.dim() == 2 and tuple(t.shape) == (H, W):
        return t, (t.stride(0), t.stride(1))
    if t.dim() == 1 and t.numel() == H * W:
        t = t.contiguous()
        return t, (W, 1)
    raise HofaError(f"{name}: expected [1,{H},1,{W}], [{H},{W}] or [{H * W}], got {tuple(t.shape)}")


def require_gpu(*tensors: torch.Tensor) -> None:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise HofaError(f"HOFA ops run on the GPU only; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise HofaError(f"tensors on different devices: {dev} and {t.device}")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class WorkspaceCache:
    """Scratch buffers keyed by (device, stream, purpose).

    One buffer per stream keeps concurrently running streams from sharing
    scratch.  A buffer only grows, and a superseded buffer is never freed: a
    HIP graph captured earlier on the stream keeps the old address in its
    kernel arguments, so freeing it would let the allocator hand that memory
    to another tensor that the graph's replays then overwrite.  Growth is at
    least twofold, so the retired buffers together stay below the size of the
    live one.  Allocate (warm up) before graph capture.
    """

    def __init__(self):
        self._bufs: dict = {}
        self._retired: list = []

    def get(self, device: torch.device, stream: int, tag: str, nbytes: int) -> torch.Tensor:
        key = (device.index, stream, tag)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            size = max(nbytes, 256)
            if buf is not None:
                self._retired.append(buf)
                size = max(size, 2 * buf.numel())
            buf = torch.empty(size, dtype=torch.uint8, device=device)
            self._bufs[key] = buf
        return buf

    def retired_bytes(self) -> int:
        return sum(b.numel() for b in self._retired)


WORKSPACES = WorkspaceCache()
