"""Pins for the CPU oracle (oracle/hofa_ref.py); CPU only.

Every oracle function is checked against something other than its own
formula: golden vectors written by the reference itself, a library routine,
an independent formulation, or an invariant.  ``test_planted_mistakes_are_caught``
plants plausible mistakes in the oracle and requires the golden check to fail.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import hofa_ref as ref
from tests.golden_util import golden_cases, load_golden


def _ref_for(case, dtype=torch.float64):
    g = load_golden(case)
    m = ref.HOFARef(g["params"], g["d_model"], g["H"], g["r"], dtype=dtype, chunk=8)
    return g, m


def _run_steps(m, x):
    outs, cache, state = [], None, None
    for t in range(x.shape[1]):
        y, cache, state = m.forward_step(x[:, t:t + 1], cache, state)
        outs.append(y)
    return torch.cat(outs, 1), cache, state


@pytest.mark.parametrize("case", golden_cases())
def test_decode_steps_match_reference_golden(case):
    g, m = _ref_for(case)
    y, cache, state = _run_steps(m, g["x"])
    j = m.j
    torch.testing.assert_close(y.float(), g["y"], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(state.float(), g["state"][:, :, :j, :], rtol=1e-4, atol=1e-5)
    # the reference keeps a zero-padded [d_h, d_h] state (Train :411-433)
    assert torch.count_nonzero(g["state"][:, :, j:, :]) == 0
    torch.testing.assert_close(cache[0].float(), g["cache_k"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(cache[1].float(), g["cache_v"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("case", golden_cases())
@pytest.mark.parametrize("chunk", [4, 8, 64])
def test_prefill_matches_reference_decode_golden(case, chunk):
    """A prefill over N tokens equals N decode steps from an empty cache."""
    g, m = _ref_for(case)
    m.chunk = chunk
    y, (kc, vc), S = m.forward(g["x"], return_state=True)
    torch.testing.assert_close(y.float(), g["y"], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(S.float(), g["state"][:, :, :m.j, :], rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(kc.float(), g["cache_k"], rtol=1e-5, atol=1e-6)


def _rand_gla(B=2, H=3, T=37, J=5, D=7, strength=0.5, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, J, generator=gen, dtype=torch.float64)
    k = torch.randn(B, H, T, J, generator=gen, dtype=torch.float64)
    v = torch.randn(B, H, T, D, generator=gen, dtype=torch.float64)
    g = F.logsigmoid(torch.randn(B, H, T, J, generator=gen, dtype=torch.float64)) * strength
    return q, k, v, g


def test_gla_three_formulations_agree():
    q, k, v, g = _rand_gla()
    y_rec, S_rec = ref.gla_recurrent(q, k, v, g)
    y_quad = ref.gla_quadratic(q, k, v, g)
    torch.testing.assert_close(y_rec, y_quad, rtol=1e-10, atol=1e-10)
    for c in (1, 4, 16, 64):
        y_ch, S_ch = ref.gla_chunked(q, k, v, g, chunk=c)
        torch.testing.assert_close(y_ch, y_rec, rtol=1e-10, atol=1e-10)
        torch.testing.assert_close(S_ch, S_rec, rtol=1e-10, atol=1e-10)


def test_gla_initial_state_and_split():
    """Running [0,T) equals running [0,t) then [t,T) from the carried state."""
    q, k, v, g = _rand_gla(T=40)
    y_all, S_all = ref.gla_chunked(q, k, v, g, chunk=8)
    y1, S1 = ref.gla_chunked(q[:, :, :13], k[:, :, :13], v[:, :, :13], g[:, :, :13], chunk=8)
    y2, S2 = ref.gla_recurrent(q[:, :, 13:], k[:, :, 13:], v[:, :, 13:], g[:, :, 13:], S0=S1)
    torch.testing.assert_close(torch.cat([y1, y2], 2), y_all, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(S2, S_all, rtol=1e-10, atol=1e-10)


def test_gla_no_decay_is_causal_linear_attention():
    """g = 0 reduces to un-normalised causal linear attention ``tril(QK^T) V``."""
    q, k, v, _ = _rand_gla()
    g = torch.zeros_like(q)
    y, _ = ref.gla_chunked(q, k, v, g, chunk=8)
    A = torch.matmul(q, k.transpose(-1, -2)).tril()
    torch.testing.assert_close(y, torch.matmul(A, v), rtol=1e-10, atol=1e-10)


def test_gla_strong_decay_is_stable():
    """Decay of -30 per token: every history term vanishes; y_t -> (q_t.k_t) v_t."""
    q, k, v, _ = _rand_gla(T=70)
    g = torch.full_like(q, -30.0)
    y, S = ref.gla_chunked(q, k, v, g, chunk=64)
    assert torch.isfinite(y).all() and torch.isfinite(S).all()
    torch.testing.assert_close(y, (q * k).sum(-1, keepdim=True) * v, rtol=1e-9, atol=1e-9)


def test_outlier_attention_matches_sdpa():
    gen = torch.Generator().manual_seed(1)
    q = torch.randn(2, 3, 33, 16, generator=gen, dtype=torch.float64)
    k = torch.randn(2, 3, 33, 16, generator=gen, dtype=torch.float64)
    v = torch.randn(2, 3, 33, 64, generator=gen, dtype=torch.float64)
    out = ref.outlier_attention(q, k, v, 2.0)
    expect = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=2.0)
    torch.testing.assert_close(out, expect, rtol=1e-10, atol=1e-10)
    # non-causal with more keys than queries (decode-style rows)
    out2 = ref.outlier_attention(q[:, :, -1:], k, v, 2.0, causal=False)
    torch.testing.assert_close(out2, out[:, :, -1:], rtol=1e-10, atol=1e-10)


def test_rope_is_a_rotation_and_composes():
    r, n = 16, 50
    cos, sin = ref.rope_tables(r, n)
    cos, sin = cos.double(), sin.double()
    x = torch.randn(3, r, dtype=torch.float64)
    # position 0 is the identity; norms are preserved
    torch.testing.assert_close(ref.apply_rope(x, cos[0], sin[0]), x)
    y = ref.apply_rope(x, cos[7], sin[7])
    torch.testing.assert_close(y.norm(dim=-1), x.norm(dim=-1))
    # rotating by a then by b equals rotating by a+b
    z = ref.apply_rope(ref.apply_rope(x, cos[7], sin[7]), cos[11], sin[11])
    torch.testing.assert_close(z, ref.apply_rope(x, cos[18], sin[18]), rtol=1e-6, atol=1e-6)
    # relative-position property of the dot product
    a, b = torch.randn(r, dtype=torch.float64), torch.randn(r, dtype=torch.float64)
    d1 = (ref.apply_rope(a, cos[20], sin[20]) * ref.apply_rope(b, cos[5], sin[5])).sum()
    d2 = (ref.apply_rope(a, cos[30], sin[30]) * ref.apply_rope(b, cos[15], sin[15])).sum()
    torch.testing.assert_close(d1, d2, rtol=1e-5, atol=1e-5)


def test_decode_step_equals_last_prefill_row():
    """decode(step N) == last row of the attention core over N+1 tokens."""
    gen = torch.Generator().manual_seed(3)
    B, H, N, d, r = 2, 2, 29, 64, 16
    j = d - r
    q = torch.randn(B, H, N + 1, d, generator=gen, dtype=torch.float64)
    k = torch.randn(B, H, N + 1, d, generator=gen, dtype=torch.float64)
    v = torch.randn(B, H, N + 1, d, generator=gen, dtype=torch.float64)
    lg = F.logsigmoid(torch.randn(B, H, N + 1, generator=gen, dtype=torch.float64))
    la = torch.randn(H, j, generator=gen, dtype=torch.float64) * 0.5
    mix = torch.sigmoid(torch.randn(B, H, N + 1, generator=gen, dtype=torch.float64))
    gs = 1 + 0.2 * torch.randn(1, H, 1, d, generator=gen, dtype=torch.float64)
    g = ref.decay_from_gates(lg, j, la)
    Y, S = ref.hofa_core(q, k, v, g, mix, gs, r, 2.0, chunk=8)
    _, S_prev = ref.hofa_core(q[:, :, :N], k[:, :, :N], v[:, :, :N], g[:, :, :N], mix[:, :, :N], gs, r, 2.0)
    y_dec, S_dec = ref.decode_step(q[:, :, N], k[:, :, N], v[:, :, N], k[..., :r], v, N + 1, S_prev,
                                   lg[:, :, N], mix[:, :, N], gs.reshape(H, d), r, 2.0, log_alpha=la)
    torch.testing.assert_close(y_dec, Y[:, :, N], rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(S_dec, S, rtol=1e-9, atol=1e-9)


def test_rmsnorm_matches_torch_module():
    y = torch.randn(4, 64)
    torch.testing.assert_close(ref.rmsnorm(y), torch.nn.RMSNorm(64, elementwise_affine=False)(y))


MUTATIONS = ["swap_gate_halves", "rotate_half_sign", "exclusive_state", "sm_scale_no_sqrt", "blend_swapped",
             "alpha_not_exp"]


@pytest.mark.parametrize("mutation", MUTATIONS)
def test_planted_mistakes_are_caught(mutation, monkeypatch):
    """Each plausible slip, planted in the oracle, must break the golden match."""
    case = "r16_alpha"
    g, m = _ref_for(case)
    if mutation == "swap_gate_halves":
        orig = ref.compute_gates
        monkeypatch.setattr(ref, "compute_gates", lambda Q, K, *a, **kw: orig(K, Q, *a, **kw))
    elif mutation == "rotate_half_sign":
        monkeypatch.setattr(ref, "rotate_half", lambda x: -torch.cat((-x[..., x.shape[-1] // 2:],
                                                                       x[..., :x.shape[-1] // 2]), -1))
    elif mutation == "exclusive_state":
        orig_ds = ref.decode_step

        def bad(q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm, eps=ref.FP32_EPS, log_alpha=None):
            y, S = orig_ds(q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm, eps, log_alpha)
            y2, _ = orig_ds(q, k * 0, v, ck, cv, L, S0, lg, mix, nw, r, sm, eps, log_alpha)
            return y2, S
        monkeypatch.setattr(ref, "decode_step", bad)
    elif mutation == "sm_scale_no_sqrt":
        orig_ds = ref.decode_step
        monkeypatch.setattr(ref, "decode_step",
                            lambda q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm, **kw:
                            orig_ds(q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm * sm, **kw))
    elif mutation == "blend_swapped":
        orig_ds = ref.decode_step
        monkeypatch.setattr(ref, "decode_step",
                            lambda q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm, **kw:
                            orig_ds(q, k, v, ck, cv, L, S0, lg, 1 - mix, nw, r, sm, **kw))
    elif mutation == "alpha_not_exp":
        orig_ds = ref.decode_step
        monkeypatch.setattr(ref, "decode_step",
                            lambda q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm, eps=ref.FP32_EPS, log_alpha=None:
                            orig_ds(q, k, v, ck, cv, L, S0, lg, mix, nw, r, sm, eps,
                                    None if log_alpha is None else torch.log(log_alpha.abs() + 1e-3)))
    y, _, _ = _run_steps(m, g["x"])
    assert not torch.allclose(y.float(), g["y"], rtol=1e-3, atol=1e-3), mutation


def test_core_backward_matches_finite_differences():
    """The backward target of the GPU kernels is autograd of ``hofa_core``; pin
    it against central finite differences (torch.autograd.gradcheck, float64)
    on a tiny shape that spans two chunks, with per-channel decay and a mix."""
    torch.manual_seed(11)
    B, H, T, D, r = 1, 1, 6, 8, 2
    J = D - r
    q = torch.randn(B, H, T, D, dtype=torch.float64, requires_grad=True)
    k = torch.randn(B, H, T, D, dtype=torch.float64, requires_grad=True)
    v = torch.randn(B, H, T, D, dtype=torch.float64, requires_grad=True)
    g = (torch.nn.functional.logsigmoid(torch.randn(B, H, T, J, dtype=torch.float64)) * 0.5).requires_grad_()
    mix = torch.sigmoid(torch.randn(B, H, T, dtype=torch.float64)).requires_grad_()
    gs = (1 + 0.3 * torch.randn(1, H, 1, D, dtype=torch.float64)).requires_grad_()

    def f(q, k, v, g, mix, gs):
        return ref.hofa_core(q, k, v, g, mix, gs, r, 1.3, eps=1e-6, chunk=4)[0]

    assert torch.autograd.gradcheck(f, (q, k, v, g, mix, gs), eps=1e-6, atol=1e-7, rtol=1e-5)


# ---------------------------------------------------------------- language-model stack
def _lm_golden(name):
    import numpy as np
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"hofa_lm_{name}.npz"))
    d_model, H, layers, vocab, B, N, alpha = (int(v) for v in z["meta"])
    params = {k[len("param."):]: torch.from_numpy(z[k].copy()) for k in z.files if k.startswith("param.")}
    return dict(d_model=d_model, H=H, r_list=[int(v) for v in z["r_list"]], params=params,
                ids=torch.from_numpy(z["ids"].copy()), logits=torch.from_numpy(z["logits"].copy()))


LM_CASES = ["2l_r16", "3l_rlist_alpha"]


@pytest.mark.parametrize("name", LM_CASES)
def test_lm_matches_reference_golden(name):
    """SubwordLMRef against logits written by the reference's own SubwordLM."""
    g = _lm_golden(name)
    m = ref.SubwordLMRef(g["params"], g["d_model"], g["H"], g["r_list"])
    logits = m.forward(g["ids"])
    torch.testing.assert_close(logits.float(), g["logits"], rtol=1e-4, atol=1e-4)


def test_layer_norm_and_gelu_match_torch_modules():
    x = torch.randn(3, 5, 64, dtype=torch.float64) * 3 + 7
    ln = torch.nn.LayerNorm(64).double()
    with torch.no_grad():
        ln.weight.normal_()
        ln.bias.normal_()
    torch.testing.assert_close(ref.layer_norm(x, ln.weight, ln.bias), ln(x).detach())
    torch.testing.assert_close(ref.gelu(x - 7), torch.nn.GELU()(x - 7))


def test_lm_decode_steps_equal_last_prefill_rows():
    """forward_step over cached prefill state == last row of a longer prefill
    (the reference's own check, benchmarks/validate_kernels.py:312-337)."""
    g = _lm_golden("3l_rlist_alpha")
    m = ref.SubwordLMRef(g["params"], g["d_model"], g["H"], g["r_list"])
    ids = g["ids"]
    n0 = ids.shape[1] - 4
    _, caches, states = m.forward(ids[:, :n0], return_state=True)
    for t in range(n0, ids.shape[1]):
        step, caches, states = m.forward_step(ids[:, t:t + 1], caches, states)
        full = m.forward(ids[:, :t + 1], last_only=True)
        torch.testing.assert_close(step, full, rtol=1e-9, atol=1e-9)


LM_MUTATIONS = ["post_ln", "untied_head_transpose", "relu_mlp", "ln_eps_zero_mean"]


@pytest.mark.parametrize("mutation", LM_MUTATIONS)
def test_lm_planted_mistakes_are_caught(mutation, monkeypatch):
    g = _lm_golden("2l_r16")
    m = ref.SubwordLMRef(g["params"], g["d_model"], g["H"], g["r_list"])
    if mutation == "post_ln":  # normalise after the residual add instead of before the sublayer
        def fwd(ids):
            x = m.emb[ids]
            for attn, t in m.layers:
                x = ref.layer_norm(x + attn.forward(x, eps=m.attn_eps), t["ln_1.weight"], t["ln_1.bias"])
                x = ref.layer_norm(x + m._mlp(t, x), t["ln_2.weight"], t["ln_2.bias"])
            return m._head(x)
        out = fwd(g["ids"])
    else:
        if mutation == "untied_head_transpose":
            monkeypatch.setattr(m, "_head", lambda x: ref.layer_norm(x, *m.lnf) @ m.emb[:, torch.randperm(
                m.emb.shape[1], generator=torch.Generator().manual_seed(0))].T)
        elif mutation == "relu_mlp":  # (erf vs tanh GELU differ by ~2e-5 here; nn.GELU pins the erf form)
            monkeypatch.setattr(ref, "gelu", F.relu)
        elif mutation == "ln_eps_zero_mean":  # RMS-style normalisation without the mean
            monkeypatch.setattr(ref, "layer_norm",
                                lambda x, w, b, eps=1e-5: x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w + b)
        out = m.forward(g["ids"])
    assert not torch.allclose(out.float(), g["logits"], rtol=1e-3, atol=1e-3), mutation
