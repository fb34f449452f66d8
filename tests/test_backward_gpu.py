"""Backward parity on the GPU: gradients of the HOFA core (``hofa_core``:
the inlier GLA + RMSNorm/gate epilogue backward, then the outlier attention
backward) against float64 autograd of the oracle on the CPU, on the same
inputs rounded to the kernel dtype.

The reference has no backward kernel of its own: it trains through autograd
of SDPA + fla ``chunk_gla`` + torch ops (src/HybridOutlierFactorizedAttentionTrain.py:241-294),
so autograd of the restated forward is the parity target.

Tolerances (max-abs error / max-abs of the reference gradient):
* float32 inputs: gradients that only pass through the GLA/epilogue kernels
  (d q[..., r:], d k[..., r:], d log_gamma, d log_alpha, d gla_scale, d mix)
  5e-3 -- their products use hi/lo split operands; gradients through the
  attention backward (d q_o, d k_o, d v) 2e-2 -- its dV/dK/dQ products take
  bf16 operands (P, dS, dO) as flash-attention backward passes do;
* bfloat16 inputs: 2e-2 on every gradient (outputs are rounded to bf16).
"""
import math

import pytest
import torch

from oracle.hofa_ref import FP32_EPS, decay_from_gates, gla_chunked, outlier_attention, rmsnorm

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ["q_o", "k_o", "q", "k", "v", "log_gamma", "log_alpha", "mix", "gla_scale"]


def _inputs(B, H, T, D, R, alpha, mix, decay, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=gen)
    J = D - R
    x = {
        "q_o": rn(B, H, T, R) if R else None,
        "k_o": rn(B, H, T, R) if R else None,
        "q": rn(B, H, T, D) * 0.5, "k": rn(B, H, T, D) * 0.5, "v": rn(B, H, T, D),
        "log_gamma": torch.nn.functional.logsigmoid(rn(B, H, T) + 2.0) * decay,
        "log_alpha": rn(1, H, 1, J) * 0.5 if alpha else None,
        "mix": torch.sigmoid(rn(B, H, T)) if mix else None,
        "gla_scale": 1.0 + 0.3 * rn(1, H, 1, D),
    }
    dy = rn(B, H, T, D)
    # round once to the kernel dtype; both sides start from these values
    for k_, t in x.items():
        if t is not None and k_ not in ("log_alpha", "gla_scale"):
            x[k_] = t.to(dtype).float()
    return x, dy.to(dtype).float()


def _oracle_grads(x, dy, R, sm):
    leaves = {k: (t.double().requires_grad_() if t is not None else None) for k, t in x.items()}
    q, k, v = leaves["q"], leaves["k"], leaves["v"]
    J = q.shape[-1] - R
    g = decay_from_gates(leaves["log_gamma"], J, leaves["log_alpha"])
    yi, _ = gla_chunked(q[..., R:], k[..., R:], v, g)
    yn = rmsnorm(yi, FP32_EPS) * leaves["gla_scale"]
    if leaves["mix"] is not None:
        m = leaves["mix"].unsqueeze(-1)
        y = (1 - m) * yn + m * outlier_attention(leaves["q_o"], leaves["k_o"], v, sm)
    else:
        y = yn
    y.backward(dy.double())
    return {k: t.grad for k, t in leaves.items() if t is not None}


def _gpu_grads(x, dy, R, sm, dtype):
    from outlierneuronattention_amd.autograd import hofa_core
    dev = {}
    for k, t in x.items():
        if t is None:
            dev[k] = None
            continue
        keep32 = k in ("log_alpha", "gla_scale")
        dev[k] = t.to(DEV, torch.float32 if keep32 else dtype).requires_grad_()
    y = hofa_core(dev["q_o"], dev["k_o"], dev["q"], dev["k"], dev["v"], dev["log_gamma"], dev["log_alpha"],
                  dev["mix"], dev["gla_scale"], R, sm)
    y.backward(dy.to(DEV, dtype))
    torch.cuda.synchronize()
    return {k: t.grad for k, t in dev.items() if t is not None}


def _check(out, ref, tol, what):
    ref = ref.double()
    out = out.detach().double().cpu()
    assert torch.isfinite(out).all(), f"{what}: non-finite gradient"
    scale = ref.abs().max().item()
    err = (out - ref).abs().max().item()
    assert err <= tol * scale, f"{what}: max err {err:.3e} > {tol} x {scale:.3e}"


CASES = [
    # B, H, T, D, R, alpha, mix, decay, dtype
    (2, 3, 200, 64, 16, True, True, 1.0, torch.float32),
    (2, 3, 200, 64, 16, True, True, 1.0, torch.bfloat16),
    (1, 2, 64, 64, 16, False, True, 1.0, torch.float32),
    (1, 2, 37, 64, 32, True, True, 1.0, torch.float32),
    (1, 2, 300, 64, 32, False, True, 0.3, torch.bfloat16),
    (1, 2, 150, 128, 64, True, True, 1.0, torch.float32),
    (1, 2, 150, 128, 32, True, True, 1.0, torch.bfloat16),
    (1, 2, 130, 64, 0, True, False, 1.0, torch.float32),      # pure GLA (r = 0)
    (1, 2, 130, 128, 16, False, True, 1.0, torch.float16),
    (1, 2, 160, 64, 16, True, True, 4.0, torch.float32),      # strong decay: element-wise chunk path
    (1, 2, 160, 64, 16, True, True, 4.0, torch.bfloat16),
    (1, 1, 4200, 64, 16, True, True, 1.0, torch.bfloat16),  # 66 chunks: the per-head suffix runs in two passes
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}D{c[3]}R{c[4]}"
                         f"{'a' if c[5] else ''}{'m' if c[6] else ''}x{c[7]}-{str(c[8])[6:]}")
def test_hofa_core_backward_matches_oracle(case):
    B, H, T, D, R, alpha, mix, decay, dtype = case
    print(f"backward {case}", flush=True)
    sm = math.sqrt(D / R) if R else 1.0
    x, dy = _inputs(B, H, T, D, R, alpha, mix, decay, dtype, seed=T + D + R)
    ref = _oracle_grads(x, dy, R, sm)
    out = _gpu_grads(x, dy, R, sm, dtype)
    f32 = dtype == torch.float32
    for name in NAMES:
        if name not in ref:
            continue
        if name in ("q", "k"):  # the GLA part; channels [0, R) get no gradient from the core
            _check(out[name][..., R:], ref[name][..., R:], 5e-3 if f32 else 2e-2, f"d{name}[r:]")
            assert out[name][..., :R].abs().max().item() == 0.0 if R else True
            continue
        attn_path = name in ("q_o", "k_o", "v")
        tol = (2e-2 if attn_path else 5e-3) if f32 else 2e-2
        _check(out[name], ref[name], tol, f"d{name}")


@pytest.mark.parametrize("T", [190, 4200])
def test_gla_backward_general_decay_matches_oracle(T):
    """General per-channel decay g (fla-style), through chunk_gla_inlier_bwd directly;
    T = 4200 spans 66 chunks (more than one pass of the per-head suffix)."""
    from outlierneuronattention_amd.chunk_gla_inlier import (chunk_gla_inlier_bwd, chunk_gla_inlier_fwd,
                                                              chunk_states_numel)
    print(f"general-decay backward T={T}", flush=True)
    B, H, D, R = 1, 2, 64, 16
    J = D - R
    gen = torch.Generator().manual_seed(7)
    q, k, v = (torch.randn(B, H, T, D, generator=gen) * 0.5 for _ in range(3))
    g = torch.clamp(torch.nn.functional.logsigmoid(torch.randn(B, H, T, J, generator=gen)) / 4, -5, 0)
    mix = torch.sigmoid(torch.randn(B, H, T, generator=gen))
    gs = 1 + 0.3 * torch.randn(1, H, 1, D, generator=gen)
    dy = torch.randn(B, H, T, D, generator=gen)
    leaves = [t.double().requires_grad_() for t in (q, k, v, g, mix, gs)]
    yi, _ = gla_chunked(leaves[0][..., R:], leaves[1][..., R:], leaves[2], leaves[3])
    y = (1 - leaves[4].unsqueeze(-1)) * rmsnorm(yi, FP32_EPS) * leaves[5]
    y.backward(dy.double())
    ref = [t.grad for t in leaves]

    dq_, dk_, dv_, dg_, dm_, dgs_ = (t.to(DEV) for t in (q, k, v, g, mix, gs))
    Qd, Kd, Vd, gd, md, gsd = dq_, dk_, dv_, dg_, dm_, dgs_
    n = torch.empty(B, H, T, D, device=DEV)
    rstd = torch.empty(B * H * T, device=DEV)
    cs = torch.empty(chunk_states_numel(B, H, T, D, J), dtype=torch.int16, device=DEV)
    y_out = torch.empty(B, H, T, D, device=DEV)
    chunk_gla_inlier_fwd(Qd, Kd, Vd, None, R, 64, mix_g=md, gla_scale=gsd, out=y_out, g=gd, eps=FP32_EPS,
                         chunk_states=cs, n_out=n, rstd=rstd)
    out = chunk_gla_inlier_bwd(Qd, Kd, Vd, None, R, dy.to(DEV), n, rstd, cs, gsd, mix_g=md, g=gd)
    torch.cuda.synchronize()
    _check(out["dq"][..., R:], ref[0][..., R:], 5e-3, "dq")
    _check(out["dk"][..., R:], ref[1][..., R:], 5e-3, "dk")
    _check(out["dv"], ref[2], 5e-3, "dv")
    _check(out["d_g"], ref[3], 5e-3, "dg")
    _check(out["d_mix"], ref[4], 5e-3, "dmix")
    _check(out["d_gla_scale"].view(1, H, 1, D), ref[5], 5e-3, "dgla_scale")


def test_attention_backward_alone_matches_torch():
    """exact_attention_bwd vs autograd of the oracle softmax attention (no GLA)."""
    from outlierneuronattention_amd.exact_attention import exact_attention, exact_attention_bwd
    B, H, T, D, R = 2, 2, 333, 64, 16
    gen = torch.Generator().manual_seed(3)
    q, k = (torch.randn(B, H, T, R, generator=gen).bfloat16().float() for _ in range(2))
    v = torch.randn(B, H, T, D, generator=gen).bfloat16().float()
    do = torch.randn(B, H, T, D, generator=gen).bfloat16().float()
    sm = 2.0
    leaves = [t.double().requires_grad_() for t in (q, k, v)]
    outlier_attention(*leaves, sm).backward(do.double())
    qd, kd, vd, dod = (t.to(DEV, torch.bfloat16) for t in (q, k, v, do))
    o = torch.empty(B, H, T, D, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(B * H * T, device=DEV)
    exact_attention(qd, kd, vd, R, sm, None, o=o, lse=lse)
    delta = (dod.float() * o.float()).sum(-1).reshape(-1).contiguous()
    dq, dk, dv = exact_attention_bwd(qd, kd, vd, dod, lse, delta, R, sm)
    torch.cuda.synchronize()
    for out, ref, name in ((dq, leaves[0].grad, "dq"), (dk, leaves[1].grad, "dk"), (dv, leaves[2].grad, "dv")):
        _check(out, ref, 2e-2, name)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hofa_core_backward_shared_outlier_channels(dtype):
    """``q_o = k_o = None``: the outlier channels are q[..., :r], k[..., :r]
    (no RoPE); the attention gradient is written into dq/dk[..., :r] in place."""
    from outlierneuronattention_amd.autograd import hofa_core
    B, H, T, D, R = 2, 2, 180, 64, 16
    x, dy = _inputs(B, H, T, D, R, True, True, 1.0, dtype, seed=99)
    sm = math.sqrt(D / R)
    leaves = {k: (t.double().requires_grad_() if t is not None else None) for k, t in x.items()}
    q, k, v = leaves["q"], leaves["k"], leaves["v"]
    g = decay_from_gates(leaves["log_gamma"], D - R, leaves["log_alpha"])
    yi, _ = gla_chunked(q[..., R:], k[..., R:], v, g)
    m = leaves["mix"].unsqueeze(-1)
    y = (1 - m) * rmsnorm(yi, FP32_EPS) * leaves["gla_scale"] + m * outlier_attention(q[..., :R], k[..., :R], v, sm)
    y.backward(dy.double())
    dev = {kk: (t.to(DEV, torch.float32 if kk in ("log_alpha", "gla_scale") else dtype).requires_grad_()
                if t is not None else None) for kk, t in x.items()}
    out = hofa_core(None, None, dev["q"], dev["k"], dev["v"], dev["log_gamma"], dev["log_alpha"], dev["mix"],
                    dev["gla_scale"], R, sm)
    out.backward(dy.to(DEV, dtype))
    torch.cuda.synchronize()
    tol = 2e-2
    for name in ("q", "k", "v", "log_gamma", "log_alpha", "mix", "gla_scale"):
        _check(dev[name].grad, leaves[name].grad, tol, f"d{name}")
