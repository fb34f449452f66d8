"""YaRN context extension of the rotary tables (src/yarn.py:17-86).

CPU: the frequencies against the published YaRN ("NTK-by-parts") formulas
written out here, the patched tables and mscale, and that tables regrown
after a patch use the patched frequencies (src/modules/modules.py:19-26).
GPU: a bf16 language model with YaRN-patched bf16 tables decodes through the
fused greedy graph step (in-kernel RoPE from the 16-bit tables) within the
LM bar of tests/test_lm_gpu.py (logits max-abs <= 2e-2 x the largest |logit|)
of the float64 LM oracle given the same tables.
"""
import math

import pytest
import torch

from outlierneuronattention_amd.yarn import patch_model_yarn, yarn_find_correction_dim, yarn_inv_freq

DIM, BASE, L0 = 16, 10000.0, 1024


def _published(scale, mode, beta_fast=32.0, beta_slow=1.0):
    """theta_i = base^(-2i/dim); d(beta) = dim ln(L / (2 pi beta)) / (2 ln base);
    ramp_i = clamp((i - floor d(beta_fast)) / (ceil d(beta_slow) - floor d(beta_fast)), 0, 1)."""
    n = DIM // 2
    theta = [BASE ** (-2 * i / DIM) for i in range(n)]
    d = lambda beta: DIM * math.log(L0 / (2 * math.pi * beta)) / (2 * math.log(BASE))  # noqa: E731
    lo, hi = max(0, math.floor(d(beta_fast))), min(n - 1, math.ceil(d(beta_slow)))
    hi = hi if hi > lo else lo + 1e-3
    out = []
    for i in range(n):
        ramp = min(1.0, max(0.0, (i - lo) / (hi - lo)))
        if mode == "geometric":
            out.append(theta[i] * scale ** (-ramp))
        else:
            out.append(ramp * theta[i] / scale + (1 - ramp) * theta[i])
    return torch.tensor(out, dtype=torch.float64)


@pytest.mark.parametrize("mode", ["geometric", "arithmetic"])
@pytest.mark.parametrize("scale", [4.0, 16.0])
def test_frequencies_follow_the_published_formula(mode, scale):
    got = yarn_inv_freq(DIM, BASE, scale, L0, mode=mode)
    assert got.dtype == torch.float32
    torch.testing.assert_close(got.double(), _published(scale, mode), rtol=1e-6, atol=0)
    # the fastest pairs keep their frequency, the slowest are interpolated by the full scale
    assert got[0].item() == pytest.approx(1.0)
    assert got[-1].item() == pytest.approx(BASE ** (-2 * (DIM // 2 - 1) / DIM) / scale, rel=1e-5)


def test_correction_dim_closed_form():
    assert yarn_find_correction_dim(32.0, DIM, BASE, L0) == pytest.approx(
        DIM * math.log(L0 / (64 * math.pi)) / (2 * math.log(BASE)))


def _lm(cls="infer"):
    from outlierneuronattention_amd.config import ModelConfig
    if cls == "infer":
        from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    else:
        from outlierneuronattention_amd.HybridOutlierFactorizedAttentionTrain import SubwordLM
    torch.manual_seed(0)
    return SubwordLM(100, ModelConfig(d_model=64, num_heads=4, num_layers=2, r=DIM, device="cpu"))


@pytest.mark.parametrize("cls", ["infer", "train"])
def test_patch_writes_scaled_16bit_tables(cls):
    m = _lm(cls)
    assert patch_model_yarn(m, target_seq_len=8192, original_seq_len=L0) == 2
    s = 8192 / L0
    ms = 1 + 0.1 * math.log(s)
    inv = _published(s, "geometric")
    for layer in m.layers:
        rot = layer.attn.rotary_emb
        assert rot.cos_cached.dtype == torch.bfloat16 and rot.cos_cached.shape == (131072, DIM)
        pos = torch.tensor([0.0, 1.0, 777.0, 8191.0], dtype=torch.float64)
        ang = torch.outer(pos, inv)
        want_c = (torch.cat([ang, ang], -1).cos() * ms)
        want_s = (torch.cat([ang, ang], -1).sin() * ms)
        got_c = rot.cos_cached[pos.long()].double()
        got_s = rot.sin_cached[pos.long()].double()
        # one bf16 rounding (2^-8 relative) plus the float32 angle at position 8191
        assert (got_c - want_c).abs().max().item() <= 1e-2 and (got_s - want_s).abs().max().item() <= 1e-2


def test_no_extension_keeps_frequencies_and_regrowth_uses_patched_ones():
    m = _lm()
    patch_model_yarn(m, target_seq_len=512, original_seq_len=L0, dtype=torch.float32)
    rot = m.layers[0].attn.rotary_emb
    torch.testing.assert_close(rot.inv_freq.double(), _published(1.0, "geometric"), rtol=1e-6, atol=0)
    patch_model_yarn(m, target_seq_len=4096, original_seq_len=L0, dtype=torch.float32, mscale=1.0)
    inv = rot.inv_freq.clone()
    cos, _ = rot(200000)  # past the table: regrown in float32 from the patched inv_freq
    assert cos.shape == (200000, DIM) and cos.dtype == torch.float32
    ang = 199999.0 * inv.double()
    torch.testing.assert_close(cos[-1].double(), torch.cat([ang, ang]).cos(), rtol=0, atol=2e-2)


@pytest.mark.gpu
def test_fused_decoder_with_yarn_tables_matches_lm_oracle():
    from oracle import hofa_ref as ref
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    V, B, N, steps = 4096, 2, 300, 4
    torch.manual_seed(5)
    with torch.device("cuda"):
        m = SubwordLM(V, ModelConfig(d_model=512, num_heads=8, num_layers=2, r=16, device="cuda"))
    with torch.no_grad():
        for layer in m.layers:
            layer.attn.gate_proj.weight.normal_(0, 0.1)
            layer.attn.mix_proj.weight.normal_(0, 0.1)
            layer.attn.W_q.weight.mul_(2.0)
            layer.attn.W_k.weight.mul_(2.0)
    m = m.to(torch.bfloat16).eval()
    assert patch_model_yarn(m, target_seq_len=4 * 2048, original_seq_len=2048) == 2  # bf16 tables, mscale 1.139
    ids = torch.randint(0, V, (B, N), generator=torch.Generator().manual_seed(1)).to("cuda")
    print(f"YaRN fused decode: B={B} prompt={N} steps={steps}", flush=True)
    dec = GreedyGraphDecoder(m, B, N + steps + 2, fused=True)
    got = [dec.prefill(ids).float().cpu()]
    toks = [dec.tok.clone().cpu()]
    for _ in range(steps):
        toks.append(dec.decode(1).clone().cpu())
        got.append(dec.logits.float().cpu())
    torch.cuda.synchronize()
    sd = {k: v.detach().cpu() for k, v in m.state_dict().items()}
    tabs = [(layer.attn.rotary_emb.cos_cached.cpu(), layer.attn.rotary_emb.sin_cached.cpu()) for layer in m.layers]
    o = ref.SubwordLMRef(sd, 512, 8, [16, 16], act_dtype=torch.bfloat16, rope_tables=tabs)
    with torch.no_grad():
        want, caches, states = o.forward(ids.cpu(), return_state=True, last_only=True)
        wants = [want]
        for i in range(steps):
            want, caches, states = o.forward_step(toks[i], caches, states)
            wants.append(want)
    for i, (g, w) in enumerate(zip(got, wants)):
        scale = w.abs().max().item()
        err = (g.double() - w).abs().max().item()
        print(f"  step {i}: max-abs {err:.3e} of {scale:.3e}", flush=True)
        assert err <= 2e-2 * scale, (i, err, scale)
