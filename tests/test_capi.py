"""The C ABI library: it loads, exports every declared entry point, and its
host-side argument checks reject bad calls before touching a GPU (CPU only)."""
import ctypes
import os
import re

import pytest
import torch

from outlierneuronattention_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    src = open(os.path.join(ROOT, "include", "hofa.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(hofa_[a-z_0-9]+)\s*\(", src, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert "hofa_decode" in names and len(names) >= 5
    for n in names:
        assert hasattr(lib, n), n
    bound = {e[0] for e in _lib.EXPORTS}
    assert set(names) == bound, set(names) ^ bound


def test_version():
    assert _lib.load().hofa_version() >= 1


def _fake_view(dtype=_lib.HOFA_BF16, strides=(0, 0, 0, 1), addr=4096):
    v = _lib.View()
    v.data, v.dtype = addr, dtype
    for i, s in enumerate(strides):
        v.stride[i] = s
    return v


def _decode_args(B=1, H=2, D=64, R=16, L=256, dt=_lib.HOFA_BF16):
    a = _lib.DecodeArgs()
    a.B, a.H, a.D, a.R, a.seq_len, a.cache_len = B, H, D, R, L, L
    a.sm_scale, a.eps = 2.0, 1e-7
    J = D - R
    a.q = a.k = a.v = a.y = _fake_view(dt, (H * D, D, D, 1))
    a.cache_k = _fake_view(dt, (H * L * R, L * R, R, 1), 8192)
    a.cache_v = _fake_view(dt, (H * L * D, L * D, D, 1), 16384)
    a.state_in = _fake_view(_lib.HOFA_F32, (H * J * D, J * D, D, 1), 32768)
    a.state_out = _fake_view(_lib.HOFA_F32, (H * J * D, J * D, D, 1), 65536)
    a.log_gamma = a.mix = _fake_view(_lib.HOFA_F32, (H, 1, 0, 0))
    a.norm_w = _fake_view(_lib.HOFA_F32, (D, 1, 0, 0))
    return a


def _expect_error(a, code, text):
    lib = _lib.load()
    rc = lib.hofa_decode(ctypes.byref(a), None, 0, None)
    assert rc == code, (rc, lib.hofa_last_error())
    assert text in lib.hofa_last_error().decode()
    assert lib.hofa_decode_workspace_bytes(ctypes.byref(a)) == 0


@pytest.mark.parametrize("field,value,code,text", [
    ("D", 96, -2, "head dim"),
    ("R", 8, -2, "outlier dims"),
    ("R", 64, -2, "outlier dims"),
    ("seq_len", 0, -1, "must be >= 1"),
    ("split_k", 1000, -1, "split_k"),
])
def test_decode_rejects_bad_scalars(field, value, code, text):
    a = _decode_args()
    setattr(a, field, value)
    _expect_error(a, code, text)


def test_decode_rejects_layouts():
    a = _decode_args()
    a.cache_v = _fake_view(_lib.HOFA_BF16, (0, 0, 64, 2), 16384)
    _expect_error(a, -1, "contiguous in the last dim")
    a = _decode_args()
    a.cache_k = _fake_view(_lib.HOFA_BF16, (0, 0, 12, 1), 8192)
    _expect_error(a, -1, "16-byte aligned")
    a = _decode_args()
    a.state_out = a.state_in
    _expect_error(a, -1, "alias")
    a = _decode_args()
    a.cache_v = _fake_view(_lib.HOFA_F16, (0, 0, 64, 1), 16384)
    _expect_error(a, -1, "share one dtype")
    a = _decode_args()
    a.state_in = _fake_view(_lib.HOFA_BF16, (0, 0, 64, 1), 32768)
    _expect_error(a, -1, "float32")


def test_decode_workspace_needs_room():
    lib = _lib.load()
    a = _decode_args(L=4096)
    n = lib.hofa_decode_workspace_bytes(ctypes.byref(a))
    assert n > 0
    rc = lib.hofa_decode(ctypes.byref(a), ctypes.c_void_p(1 << 20), n - 4, None)
    assert rc == -4 and "workspace" in lib.hofa_last_error().decode()


def test_python_wrapper_requires_gpu_tensors():
    from outlierneuronattention_amd import fused_hofa_decode
    q = torch.zeros(1, 2, 1, 64)
    with pytest.raises(_lib.HofaError, match="GPU only"):
        fused_hofa_decode(q, q, q, torch.zeros(1, 2, 8, 16), torch.zeros(1, 2, 8, 64), torch.zeros(1, 2, 48, 64),
                          torch.zeros(1, 2, 48, 64), torch.zeros(1, 2, 1), torch.zeros(1, 2, 1), torch.ones(2, 64),
                          16, 8, 2.0)
    with pytest.raises(AssertionError):  # N == 1 check mirrors src/hofa_decode_triton.py:353
        q2 = torch.zeros(1, 2, 2, 64)
        fused_hofa_decode(q2, q2, q2, None, None, None, None, None, None, None, 16, 8, 2.0)


def test_decode_wrapper_checks_extents_on_host():
    """Extents never reach the C ABI (strides only), so the wrapper must refuse them."""
    from outlierneuronattention_amd.hofa_decode import decode_args, log_alpha_strides
    B, H, L, D, R = 2, 3, 64, 64, 16
    J = D - R
    q = torch.zeros(B, H, 1, D)
    ck, cv = torch.zeros(B, H, L, R), torch.zeros(B, H, L, D)
    s = torch.zeros(B, H, J, D)
    lg, mix, nw = torch.zeros(B, H, 1), torch.zeros(B, H, 1), torch.ones(H, D)
    a, y, _ = decode_args(q, q, q, ck, cv, s, s.clone(), lg, mix, nw, R, L, 2.0)
    assert a.B == B and a.cache_len == L and y.shape == q.shape
    bad = [
        dict(cache_v=torch.zeros(B, H, L - 1, D)),
        dict(cache_k=torch.zeros(B, H, L, 32)),
        dict(state_I_in=torch.zeros(B, H, D, D)),
        dict(norm_w=torch.ones(1, D)),
        dict(log_gamma=torch.zeros(B, H + 1, 1)),
        dict(mix_g=torch.zeros(B, H, 2)),
        dict(seq_len=L + 1),
        dict(seq_len=0),
    ]
    base = dict(q=q, k=q, v=q, cache_k=ck, cache_v=cv, state_I_in=s, state_I_out=s.clone(), log_gamma=lg,
                mix_g=mix, norm_w=nw, R=R, seq_len=L, sm_scale=2.0)
    for b in bad:
        kw = dict(base, **b)
        with pytest.raises(_lib.HofaError):
            decode_args(**kw)
    # log_alpha layouts: (h, j) strides and 1-D readings
    la4 = torch.zeros(1, H, 1, J)
    assert log_alpha_strides(la4, H, J)[1] == (J, 1)
    assert log_alpha_strides(torch.zeros(H, J), H, J)[1] == (J, 1)
    assert log_alpha_strides(torch.zeros(H * J), H, J)[1] == (J, 1)
    assert log_alpha_strides(torch.zeros(J), H, J)[1] == (0, 1)
    for shape in [(1, H, 1, J + 1), (H, J - 1), (H * J + 1,)]:
        with pytest.raises(_lib.HofaError):
            log_alpha_strides(torch.zeros(shape), H, J)


# ---------------------------------------------------------------- single-token block entry points
def _rows_args(B=2, K=1024, N=512, dt=_lib.HOFA_BF16):
    a = _lib.RowsLinearArgs()
    a.B, a.K, a.N, a.dtype = B, K, N, dt
    a.x, a.x_stride = 4096, K
    a.w = 8192
    a.y, a.y_stride = 16384, N
    return a


@pytest.mark.parametrize("field,value,code,text", [
    ("B", 5, -2, "B=5"),
    ("B", 0, -2, "B=0"),
    ("K", 1020, -2, "multiple of 8"),
    ("K", 8192, -2, "at most 4096"),
    ("N", 0, -1, "N=0"),
    ("dtype", _lib.HOFA_F32, -2, "bf16 or f16"),
    ("act", 2, -1, "act=2"),
    ("w", None, -1, "NULL"),
    ("y_stride", 100, -1, "row strides"),
])
def test_rows_linear_rejects_bad_arguments(field, value, code, text):
    lib = _lib.load()
    a = _rows_args()
    setattr(a, field, value)
    rc = lib.hofa_rows_linear(ctypes.byref(a), None)
    assert rc == code, (rc, lib.hofa_last_error())
    assert text in lib.hofa_last_error().decode()


def test_rows_linear_rejects_misaligned_rows_and_orphan_ln_bias():
    lib = _lib.load()
    a = _rows_args()
    a.w = 8194
    assert lib.hofa_rows_linear(ctypes.byref(a), None) == -1 and "aligned" in lib.hofa_last_error().decode()
    a = _rows_args()
    a.ln_b = 1 << 16
    assert lib.hofa_rows_linear(ctypes.byref(a), None) == -1 and "ln_b" in lib.hofa_last_error().decode()


def _prologue_args(D=64, R=16):
    a = _lib.DecodePrologueArgs()
    a.B, a.H, a.D, a.R, a.dtype, a.cache_len = 1, 4, D, R, _lib.HOFA_BF16, 32
    a.qkv, a.qkv_stride = 4096, 3 * 4 * D
    a.gate_w = a.gate_b = a.mix_w = a.mix_b = 8192
    a.pos = a.cache_k = a.cache_v = a.log_gamma = a.mix = 16384
    return a


@pytest.mark.parametrize("field,value,code,text", [
    ("D", 96, -2, "D=96"),
    ("R", 15, -2, "R=15"),
    ("R", 64, -2, "R=64"),
    ("dtype", _lib.HOFA_F32, -2, "bf16 or f16"),
    ("qkv_stride", 10, -1, "qkv_stride"),
    ("pos", None, -1, "NULL"),
])
def test_decode_prologue_rejects_bad_arguments(field, value, code, text):
    lib = _lib.load()
    a = _prologue_args()
    setattr(a, field, value)
    rc = lib.hofa_decode_prologue(ctypes.byref(a), None)
    assert rc == code, (rc, lib.hofa_last_error())
    assert text in lib.hofa_last_error().decode()


def test_decode_prologue_needs_a_mix_source_and_paired_tables():
    lib = _lib.load()
    a = _prologue_args()
    a.mix_w = a.mix_b = None
    assert lib.hofa_decode_prologue(ctypes.byref(a), None) == -1 and "fixed_mix" in lib.hofa_last_error().decode()
    a = _prologue_args()
    a.cos, a.rope_rows = 1 << 16, 8
    assert lib.hofa_decode_prologue(ctypes.byref(a), None) == -1 and "cos and sin" in lib.hofa_last_error().decode()
    a = _prologue_args()
    a.cos = a.sin = 1 << 16
    a.rope_rows, a.rope_dtype = 8, _lib.HOFA_F16
    assert lib.hofa_decode_prologue(ctypes.byref(a), None) == -1 and "rope_dtype" in lib.hofa_last_error().decode()


def test_decode_advance_rejects_bad_arguments():
    lib = _lib.load()
    a = _lib.DecodeAdvanceArgs()
    a.B, a.d_model, a.vocab, a.dtype, a.out_cols = 5, 64, 100, _lib.HOFA_BF16, 8
    a.argmax = a.emb = a.x = a.tok = a.out = a.col = a.pos = a.seq_len = 4096
    assert lib.hofa_decode_advance(ctypes.byref(a), None) == -2 and "B=5" in lib.hofa_last_error().decode()
    a.B, a.out_cols = 2, 0
    assert lib.hofa_decode_advance(ctypes.byref(a), None) == -1 and "out_cols=0" in lib.hofa_last_error().decode()
    a.out_cols, a.tok = 8, None
    assert lib.hofa_decode_advance(ctypes.byref(a), None) == -1 and "NULL" in lib.hofa_last_error().decode()


def test_decode_layer_wrappers_require_gpu_tensors():
    from outlierneuronattention_amd.decode_layer import rows_linear
    w = torch.zeros(8, 16, dtype=torch.bfloat16)
    with pytest.raises(_lib.HofaError, match="GPU only"):
        rows_linear(torch.zeros(1, 16, dtype=torch.bfloat16), w, torch.zeros(1, 8, dtype=torch.bfloat16))
    with pytest.raises(_lib.HofaError, match="bf16/f16"):
        rows_linear(torch.zeros(1, 16), w.float(), torch.zeros(1, 8))


def test_greedy_key_encoding_orders_values_and_breaks_ties_to_the_first_index():
    """The LM head's per-block keys: order-preserving float bits << 32 |
    0xffffffff - index (restated here for float32 values), reduced per row."""
    import struct
    from outlierneuronattention_amd.decode_layer import argmax_slots, greedy_from_keys

    def key(v, n):
        b = struct.unpack("<I", struct.pack("<f", v))[0]
        k = (~b & 0xFFFFFFFF) if b & 0x80000000 else (b | 0x80000000)
        u = (k << 32) | (0xFFFFFFFF - n)
        return u - (1 << 64) if u >= 1 << 63 else u  # stored as int64

    N = 40  # three 16-row blocks per row
    rows = [[-3.0] * N, [0.5] * N]
    rows[0][37] = -0.25                    # the maximum among negatives
    rows[1][5], rows[1][21] = 2.0, 2.0     # a tie across blocks: the first index wins
    keys = torch.zeros(2 * argmax_slots(N), dtype=torch.int64)
    for b, vals in enumerate(rows):
        for blk in range(argmax_slots(N)):
            best = max(key(vals[n], n) + (1 << 64 if key(vals[n], n) < 0 else 0)
                       for n in range(16 * blk, min(N, 16 * blk + 16)))
            keys[b * argmax_slots(N) + blk] = best - (1 << 64) if best >= 1 << 63 else best
    assert greedy_from_keys(keys, 2, N).tolist() == [37, 5]


def test_decode_prologue_wrapper_checks_module_parameters():
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.decode_layer import decode_prologue, rows_linear
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import HybridOutlierFactorizedAttention
    a = HybridOutlierFactorizedAttention(ModelConfig(d_model=128, num_heads=2, num_layers=1, r=16, device="cpu"))
    B, H, D = 1, 2, 64
    qkv = torch.zeros(B, 3 * H * D, dtype=torch.bfloat16)
    ck, cv = torch.zeros(B, H, 8, 16, dtype=torch.bfloat16), torch.zeros(B, H, 8, D, dtype=torch.bfloat16)
    pos, lg, mix = torch.zeros(1, dtype=torch.int64), torch.zeros(B, H), torch.zeros(B, H)
    with pytest.raises(_lib.HofaError, match="gate_proj.weight"):  # float32 module, bf16 activations
        decode_prologue(a, qkv, ck, cv, pos, lg, mix)
    a = a.to(torch.bfloat16)
    with pytest.raises(_lib.HofaError, match="GPU only"):
        decode_prologue(a, qkv, ck, cv, pos, lg, mix)
    w = torch.zeros(8, 16, dtype=torch.bfloat16)
    with pytest.raises(_lib.HofaError, match="ln.weight"):
        rows_linear(torch.zeros(1, 16, dtype=torch.bfloat16), w, torch.zeros(1, 8, dtype=torch.bfloat16),
                    ln=(torch.ones(16), None, 1e-5))


def test_decode_fused_rejects_mismatched_prologue():
    lib = _lib.load()
    a = _decode_args(B=1, H=4, D=64, R=16)
    p = _prologue_args(D=64, R=16)
    p.H = 2
    assert lib.hofa_decode_fused(ctypes.byref(a), ctypes.byref(p), None, 0, None) == -1
    assert "must match" in lib.hofa_last_error().decode()
    p = _prologue_args(D=64, R=16)
    p.mix_w = p.mix_b = None
    assert lib.hofa_decode_fused(ctypes.byref(a), ctypes.byref(p), None, 0, None) == -1
    assert "fixed_mix" in lib.hofa_last_error().decode()
    a32 = _decode_args(B=1, H=4, D=64, R=16, dt=_lib.HOFA_F32)
    p32 = _prologue_args(D=64, R=16)
    p32.dtype = _lib.HOFA_F32
    assert lib.hofa_decode_fused(ctypes.byref(a32), ctypes.byref(p32), None, 0, None) == -2
    assert lib.hofa_decode_fused(ctypes.byref(a), None, None, 0, None) == -1
    n = lib.hofa_decode_fused_workspace_bytes(ctypes.byref(a))
    assert n > lib.hofa_decode_workspace_bytes(ctypes.byref(a))  # one more partial per head
