"""GPU parity of the prefill kernels (outlier attention, inlier GLA) against
the CPU oracle.

Tolerances:
* bf16/f16 outputs vs the float64 oracle on the same rounded inputs: max-abs
  <= 2e-2 (outputs are O(1)); f32 inputs (bf16 matrix operands): 3e-2.
* GLA final state (fp32 accumulation of bf16 products): relative L2 <= 1e-3
  against the float64 oracle on the same rounded inputs.
* base-2 log-sum-exp of the attention rows: f32 inputs max-abs <= 1e-3 (f32
  row sums); bf16/f16 inputs max-abs <= 6e-3: their row sum is taken on the
  matrix core over the same 16-bit rounded probabilities that form O (so O is
  normalised consistently), and each rounded probability carries a relative
  error of at most 2^-8, i.e. log2(1 + 2^-8) = 5.6e-3 on the sum.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import hofa_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
LOG2E = 1.0 / math.log(2.0)


def _qkv(B, H, T, D, dtype, seed, scale=1.0):
    """Q/K/V as [B,H,T,D] views of [B,T,H,3D] memory (the module's layout)."""
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, T, H, 3 * D, generator=gen) * scale).to(DEV, dtype)
    return tuple(x[..., i * D:(i + 1) * D].transpose(1, 2) for i in range(3))


def _c(t):
    return t.detach().cpu().double()


ATTN_CASES = [
    # B, H, T, D, R, dtype
    (2, 3, 200, 64, 16, torch.bfloat16),
    (1, 2, 1000, 64, 32, torch.bfloat16),
    (1, 2, 64, 64, 16, torch.bfloat16),
    (2, 1, 1, 64, 16, torch.bfloat16),
    (1, 2, 129, 64, 64, torch.bfloat16),
    (1, 2, 333, 128, 16, torch.bfloat16),
    (1, 1, 190, 128, 64, torch.bfloat16),
    (2, 2, 257, 64, 16, torch.float16),
    (1, 2, 300, 64, 16, torch.float32),
    (1, 8, 512, 64, 16, torch.bfloat16),  # 8 heads: XCD-grouped block order
]


@pytest.mark.parametrize("B,H,T,D,R,dtype", ATTN_CASES)
def test_exact_attention_matches_oracle(B, H, T, D, R, dtype):
    print(f"attn B={B} H={H} T={T} D={D} R={R} {dtype}", flush=True)
    from outlierneuronattention_amd.exact_attention import exact_attention
    q, k, v = _qkv(B, H, T, D, dtype, seed=T + R)
    gen = torch.Generator().manual_seed(1)
    mix = torch.sigmoid(torch.randn(B, H, T, 1, generator=gen)).to(DEV, dtype)
    sm = math.sqrt(D / R)
    prior = torch.randn(B, H, T, D, generator=gen).to(DEV, dtype)
    out = prior.clone()
    o = torch.empty(B, H, T, D, dtype=dtype, device=DEV)
    lse = torch.empty(B * H * T, dtype=torch.float32, device=DEV)
    exact_attention(q, k, v, R, sm, mix, out=out, o=o, lse=lse)
    torch.cuda.synchronize()
    O, L = ref.outlier_attention(_c(q)[..., :R], _c(k)[..., :R], _c(v), sm, return_lse=True)
    tol = 3e-2 if dtype == torch.float32 else 2e-2
    assert (_c(o) - O).abs().max().item() <= tol
    expect = _c(prior) + _c(mix) * O
    assert (_c(out) - expect).abs().max().item() <= tol
    lse_tol = 1e-3 if dtype == torch.float32 else 6e-3
    assert (lse.cpu().double().view(B, H, T) - L * LOG2E).abs().max().item() <= lse_tol
    # without `out`: a fresh mix*O
    fresh = exact_attention(q, k, v, R, sm, mix)
    torch.cuda.synchronize()
    assert (_c(fresh) - _c(mix) * O).abs().max().item() <= tol


def _gla_inputs(B, H, T, D, R, dtype, mode, seed, strength=1.0):
    q, k, v = _qkv(B, H, T, D, dtype, seed)
    J = D - R
    gen = torch.Generator().manual_seed(seed + 1)
    lg = F.logsigmoid(torch.randn(B, H, T, generator=gen) - 1.0) * strength
    la = 0.5 * torch.randn(1, H, 1, J, generator=gen) if mode == "alpha" else None
    g = (torch.clamp(F.logsigmoid(torch.randn(B, H, T, J, generator=gen)) / 16, -5, 0) * strength
         if mode == "general" else None)
    mix = torch.sigmoid(torch.randn(B, H, T, 1, generator=gen))
    gs = 1 + 0.2 * torch.randn(1, H, 1, D, generator=gen)
    return q, k, v, lg, la, g, mix, gs


GLA_CASES = [
    # B, H, T, D, R, dtype, decay mode
    (2, 3, 200, 64, 16, torch.bfloat16, "scalar"),
    (2, 3, 200, 64, 16, torch.bfloat16, "alpha"),
    (1, 2, 300, 64, 16, torch.bfloat16, "general"),
    (1, 2, 64, 64, 16, torch.bfloat16, "alpha"),
    (2, 1, 5, 64, 16, torch.bfloat16, "alpha"),
    (1, 2, 257, 64, 32, torch.bfloat16, "alpha"),
    (1, 2, 150, 64, 0, torch.bfloat16, "scalar"),
    (1, 2, 200, 128, 16, torch.bfloat16, "alpha"),
    (1, 1, 130, 128, 64, torch.bfloat16, "general"),
    (1, 2, 190, 64, 16, torch.float16, "alpha"),
    (1, 2, 190, 64, 16, torch.float32, "alpha"),
]


def _check_gla(B, H, T, D, R, dtype, mode, strength=1.0, seed=0, round_operands=False):
    """round_operands: operands and state rounded to bf16 once (16-bit inputs),
    as the reference kernel does; else hi/lo operand pairs (the default)."""
    from outlierneuronattention_amd.chunk_gla_inlier import chunk_gla_inlier_fwd
    q, k, v, lg, la, g, mix, gs = _gla_inputs(B, H, T, D, R, dtype, mode, seed, strength)
    J = D - R
    kw = dict(log_alpha=None if la is None else la.to(DEV), mix_g=mix.to(DEV, dtype), gla_scale=gs.to(DEV),
              round_operands=round_operands)
    if g is not None:
        kw["g"] = g.to(DEV)
    Y, states = chunk_gla_inlier_fwd(q, k, v, lg.to(DEV), R, 64, **kw)
    Yraw, _ = chunk_gla_inlier_fwd(q, k, v, lg.to(DEV), R, 64, log_alpha=kw["log_alpha"], g=kw.get("g"),
                                   round_operands=round_operands)
    torch.cuda.synchronize()
    gd = g.double() if g is not None else ref.decay_from_gates(lg.double(), J, None if la is None else la.double())
    y_i, S = ref.gla_chunked(_c(q)[..., R:], _c(k)[..., R:], _c(v), gd, chunk=64)
    y_fused = (1 - _c(kw["mix_g"])) * gs.double() * ref.rmsnorm(y_i, 1e-5)
    rounded = dtype != torch.float32 and round_operands
    # hi/lo operands track fp32: the state within 1e-3, outputs within the bf16 bar.  Operands
    # rounded to bf16 once (the reference's .to(dtype) before each tl.dot) leave ~2^-9 relative per
    # product term, which RMSNorm magnifies on tokens of small norm.
    tol = 3e-2 if dtype == torch.float32 else (6e-2 if rounded else 2e-2)
    state_tol = 6e-3 if rounded else 1e-3
    scale = max(1.0, y_i.abs().max().item())
    err_raw = ((_c(Yraw) - y_i).abs().max() / scale).item()
    err = (_c(Y) - y_fused).abs().max().item()
    s = states[:, :, :J, :D].cpu().double()
    rel = ((s - S).norm() / S.norm()).item()
    print(f"  rounded={rounded}: raw rel-max {err_raw:.3e}, fused max-abs {err:.3e}, state rel {rel:.3e}", flush=True)
    assert err_raw <= tol, f"raw Y_I rel-max err {err_raw}"
    assert err <= tol, f"fused Y err {err}"
    assert states.shape == (B, H, max(16, 1 << (J - 1).bit_length()), max(16, 1 << (D - 1).bit_length()))
    assert rel <= state_tol, f"state rel err {rel}"
    assert torch.count_nonzero(states[:, :, J:, :]) == 0


@pytest.mark.parametrize("B,H,T,D,R,dtype,mode", GLA_CASES)
def test_chunk_gla_matches_oracle(B, H, T, D, R, dtype, mode):
    print(f"gla B={B} H={H} T={T} D={D} R={R} {dtype} {mode}", flush=True)
    _check_gla(B, H, T, D, R, dtype, mode)


@pytest.mark.parametrize("B,H,T,D,R,dtype,mode", [c for c in GLA_CASES if c[5] != torch.float32][:3] +
                         [(1, 2, 200, 128, 16, torch.bfloat16, "alpha"), (1, 2, 190, 64, 16, torch.float16, "alpha")])
def test_chunk_gla_rounded_operands(B, H, T, D, R, dtype, mode):
    """round_operands=True: operands rounded to bf16 once, the reference kernel's numerics."""
    print(f"gla rounded B={B} H={H} T={T} D={D} R={R} {dtype} {mode}", flush=True)
    _check_gla(B, H, T, D, R, dtype, mode, round_operands=True)


@pytest.mark.parametrize("mode", ["scalar", "alpha", "general"])
def test_chunk_gla_strong_decay_falls_back_exactly(mode):
    """Decays of tens of nats per token exceed the factored form's range; the
    element-wise path must still match."""
    print(f"gla strong decay {mode}", flush=True)
    _check_gla(1, 2, 200, 64, 16, torch.bfloat16, mode, strength=40.0 if mode != "general" else 400.0, seed=3)
