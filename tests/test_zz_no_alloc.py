"""hofa_decode_static: the allocation-free decode entry point, called through
the C ABI and checked against hofa_decode with a caller workspace (same
kernels and split plan, so the results are bitwise equal) on two calls in a
row, the second smaller, and against the float64 oracle."""
import ctypes

import pytest
import torch

from outlierneuronattention_amd import _lib
from outlierneuronattention_amd.hofa_decode import decode_args

from .test_decode_gpu import check, make_case

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _call(g, R, seq_len, sm, static):
    lib = _lib.load()
    s_out = torch.empty_like(g["state_in"])
    a, y, keep = decode_args(g["q"], g["k"], g["v"], g["cache_k"], g["cache_v"], g["state_in"], s_out,
                             g["log_gamma"], g["mix"], g["norm_w"], R, seq_len, sm, log_alpha=g["log_alpha"])
    stream = _lib.stream_handle(g["q"].device)
    if static:
        rc = lib.hofa_decode_static(ctypes.byref(a), stream)
    else:
        nbytes = lib.hofa_decode_workspace_bytes(ctypes.byref(a))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        keep.append(ws)
        rc = lib.hofa_decode(ctypes.byref(a), ws.data_ptr(), nbytes, stream)
    _lib.check(rc, "hofa_decode_static" if static else "hofa_decode")
    torch.cuda.synchronize()
    return y, s_out


@pytest.mark.parametrize("first,second", [
    ((4, 16, 32768, 32768, 64, 16, True), (1, 4, 3000, 2500, 64, 16, False)),
    ((2, 8, 9000, 8999, 128, 32, True), (1, 2, 700, 1, 64, 16, True)),
])
def test_static_decode_matches_workspace_decode(first, second):
    for i, (B, H, L, seq, D, R, alpha) in enumerate((first, second)):
        print(f"hofa_decode_static call {i}: B={B} H={H} L={L} seq={seq} D={D} R={R} alpha={alpha}", flush=True)
        g, sm, y_ref, s_ref = make_case(B, H, L, seq, D, R, torch.bfloat16, alpha=alpha, seed=40 + i)
        y_s, st_s = _call(g, R, seq, sm, static=True)
        y_w, st_w = _call(g, R, seq, sm, static=False)
        assert torch.equal(y_s, y_w) and torch.equal(st_s, st_w)
        check(y_s, st_s, y_ref, s_ref, torch.bfloat16)


def test_static_decode_rejects_oversized_plans():
    """A plan whose partials exceed the static array is refused before any launch."""
    lib = _lib.load()
    from .test_capi import _decode_args
    a = _decode_args(B=8, H=64, D=128, R=16, L=1 << 16)
    a.split_k = 64  # 512 heads x 64 partials of 130 floats: about 17 MB
    nbytes = lib.hofa_decode_workspace_bytes(ctypes.byref(a))
    assert nbytes > _lib.DECODE_STATIC_SCRATCH_BYTES
    rc = lib.hofa_decode_static(ctypes.byref(a), None)
    assert rc == -4
    assert b"static" in lib.hofa_last_error()
