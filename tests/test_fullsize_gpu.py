"""Parity at the BASELINE shapes themselves (cfg2 prefill, cfg4 training
step), against the float64 oracle on the same rounded inputs.

The GPU runs the whole configuration; the oracle recomputes a few
(batch, head) slices over all of T (heads and batches are independent, so a
slice of the full run must equal the oracle on that slice).  The slices
include the last head, so the XCD-grouped block order at 64 / 96 heads and
the per-head offsets at full T are covered, as are the 64-chunk (cfg2) and
32-chunk (cfg4) scans.

Tolerances (stated here, as in test_prefill_gpu.py / test_backward_gpu.py):
* cfg2 output y (bf16): max-abs <= 2e-2; GLA final state: relative L2 <= 1e-3.
  (One rounding of y: the GLA part reaches the attention kernel in float32.
  Rounding it to bf16 first, as the reference's two-kernel order does, alone
  costs up to one bf16 ulp of |y| ~ 4.6, i.e. 2.7e-2 at this shape.)
* cfg4 output y (bf16): max-abs <= 2e-2; every gradient: max-abs <= 2e-2 x
  the largest |gradient| of the oracle on the slice.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import hofa_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _c(t):
    return t.detach().cpu().double()


def test_cfg2_prefill_full_size():
    """cfg2: B=4, T=4096, H=16, d_h=64, r=16, general per-channel decay, bf16."""
    from outlierneuronattention_amd.prefill import prefill_fwd
    B, T, H, D, R = 4, 4096, 16, 64, 16
    J = D - R
    sm = math.sqrt(D / R)
    print(f"cfg2 full size B={B} T={T} H={H}", flush=True)
    gen = torch.Generator().manual_seed(2024)
    x = torch.randn(B, T, H, 3 * D, generator=gen).to(DEV, torch.bfloat16)
    q, k, v = (x[..., i * D:(i + 1) * D].transpose(1, 2) for i in range(3))
    g = torch.clamp(F.logsigmoid(torch.randn(B, H, T, J, generator=gen)) / 16, -5, 0).to(DEV)
    mix = torch.sigmoid(torch.randn(B, H, T, generator=gen)).to(DEV, torch.bfloat16)
    gs = (1 + 0.2 * torch.randn(1, H, 1, D, generator=gen)).to(DEV)
    lg = torch.zeros(B, H, T, device=DEV)
    # the inference module's prefill core (bench.py times the same call): GLA in float32, then the
    # attention adds mix * O and rounds once
    y, states = prefill_fwd(q, k, v, lg, R, sm, mix, gs, g=g, eps=1e-5)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (1, 7), (2, 8), (3, 15)):
        qs, ks, vs = _c(q[b:b + 1, h:h + 1]), _c(k[b:b + 1, h:h + 1]), _c(v[b:b + 1, h:h + 1])
        y_i, S = ref.gla_chunked(qs[..., R:], ks[..., R:], vs, _c(g[b:b + 1, h:h + 1]), chunk=64)
        m = _c(mix[b:b + 1, h:h + 1]).unsqueeze(-1)
        y_ref = (1 - m) * _c(gs[:, h:h + 1]) * ref.rmsnorm(y_i, 1e-5) + m * ref.outlier_attention(
            qs[..., :R], ks[..., :R], vs, sm)
        err = (_c(y[b:b + 1, h:h + 1]) - y_ref).abs().max().item()
        srel = ((_c(states[b, h, :J, :D]) - S[0, 0]).norm() / S.norm()).item()
        print(f"  slice b={b} h={h}: y max-abs {err:.3e}, state rel {srel:.3e}", flush=True)
        assert err <= 2e-2, (b, h, err)
        assert srel <= 1e-3, (b, h, srel)


def test_cfg4_train_step_full_size():
    """cfg4: B=8, T=2048, H=12, d_h=64, r=16, learnable per-channel decay,
    bf16 operands with fp32 decay/gate/scale parameters; every gradient."""
    from outlierneuronattention_amd.autograd import hofa_core
    B, T, H, D, R = 8, 2048, 12, 64, 16
    J = D - R
    sm = math.sqrt(D / R)
    print(f"cfg4 full size B={B} T={T} H={H}", flush=True)
    gen = torch.Generator().manual_seed(4048)
    x = torch.randn(B, T, H, 3 * D, generator=gen).to(torch.bfloat16)
    q, k, v = (x[..., i * D:(i + 1) * D].transpose(1, 2).contiguous() for i in range(3))
    lg = F.logsigmoid(torch.randn(B, H, T, generator=gen) + 3.0)
    la = torch.log(-F.logsigmoid(2 + 4 * torch.rand(1, H, 1, J, generator=gen)))
    mix = torch.sigmoid(torch.randn(B, H, T, generator=gen))
    gs = 1 + 0.3 * torch.randn(1, H, 1, D, generator=gen)
    dy = torch.randn(B, H, T, D, generator=gen).to(torch.bfloat16)
    leaves = {n: t.to(DEV).requires_grad_() for n, t in
              dict(q=q, k=k, v=v, lg=lg, la=la, mix=mix, gs=gs).items()}
    y = hofa_core(None, None, leaves["q"], leaves["k"], leaves["v"], leaves["lg"], leaves["la"], leaves["mix"],
                  leaves["gs"], R, sm)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    heads = [0, 11]
    grads = {n: _c(t.grad) for n, t in leaves.items()}
    # oracle per batch row on the selected heads; the per-head parameters
    # (log_alpha, gla_scale) accumulate over the batch rows
    acc_la = torch.zeros(1, len(heads), 1, J, dtype=torch.float64)
    acc_gs = torch.zeros(1, len(heads), 1, D, dtype=torch.float64)
    worst = {}

    def check(name, got, want, tol=2e-2, relative=True):
        err = (got - want).abs().max().item()
        if relative:
            err /= max(want.abs().max().item(), 1e-30)
        worst[name] = max(worst.get(name, 0.0), err)
        assert err <= tol, (name, err)

    la_h = _c(la[:, heads]).requires_grad_()
    gs_h = _c(gs[:, heads]).requires_grad_()
    for b in range(B):
        sl = dict(q=_c(q[b:b + 1, heads]), k=_c(k[b:b + 1, heads]), v=_c(v[b:b + 1, heads]),
                  lg=_c(lg[b:b + 1, heads]), mix=_c(mix[b:b + 1, heads]))
        for t in sl.values():
            t.requires_grad_()
        gdec = ref.decay_from_gates(sl["lg"], J, la_h)
        y_i, _ = ref.gla_chunked(sl["q"][..., R:], sl["k"][..., R:], sl["v"], gdec, chunk=64)
        m = sl["mix"].unsqueeze(-1)
        y_ref = (1 - m) * gs_h * ref.rmsnorm(y_i) + m * ref.outlier_attention(sl["q"][..., :R], sl["k"][..., :R],
                                                                                sl["v"], sm)
        check("y", _c(y[b:b + 1, heads]), y_ref.detach(), relative=False)
        y_ref.backward(_c(dy[b:b + 1, heads]))
        for n in ("q", "k", "v", "lg", "mix"):
            check("d" + n, grads[n][b:b + 1, heads], sl[n].grad)
        del y_ref, y_i, gdec
    check("dla", grads["la"][:, heads], la_h.grad)
    check("dgs", grads["gs"][:, heads], gs_h.grad)
    print("  worst relative max-abs errors: " + ", ".join(f"{n} {e:.2e}" for n, e in worst.items()), flush=True)
