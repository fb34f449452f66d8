"""Fused single-token TransformerBlock kernels (csrc/hofa_decode_layer.hip).

* ``rows_linear`` against a float32 torch chain that rounds to the 16-bit
  type wherever the module's own ops do (nn.LayerNorm output, nn.Linear
  output, GELU, the ``/ d_h**0.25`` scale, the residual add), to 1e-2
  relative to the largest output (a different fp32 summation order may move
  a value across one bf16 rounding step); the greedy key must name the first
  maximum of the kernel's own output exactly (first index on ties).
* ``decode_prologue`` against the module's torch ops for gates, RoPE at the
  device position and the cache append (1e-2 relative: 16-bit logits).
* the fused greedy decoder against the module-op decoder (``fused=False``)
  on a bf16 SubwordLM: per-step logits within 3e-2 of the largest logit,
  and identical tokens (the test model's logit gaps are far above that).
"""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _r(t, dt):
    return t.to(dt).float()


def _ref_linear(x, w, bias, ln, gelu, scale, scale_cols, res, dt):
    xf = x.float()
    if ln is not None:
        lw, lb, eps = ln
        xf = _r(F.layer_norm(xf, (xf.shape[-1],), lw.float(), lb.float(), eps), dt)
    t = xf @ w.float().T
    if bias is not None:
        t = t + bias.float()
    t = _r(t, dt)
    if gelu:
        t = _r(F.gelu(t), dt)
    if scale_cols:
        t[:, :scale_cols] = _r(t[:, :scale_cols] * scale, dt)
    if res is not None:
        t = _r(res.float() + t, dt)
    return t


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,K,N,ln,gelu,bias,res,scale_cols", [
    (1, 1024, 3072, True, False, False, False, 2048),
    (4, 1024, 1024, False, False, False, True, 0),
    (3, 1024, 4096, True, True, True, False, 0),
    (2, 4096, 1000, False, False, True, True, 0),
    (4, 256, 20011, True, False, False, False, 0),
])
def test_rows_linear_matches_module_chain(dt, B, K, N, ln, gelu, bias, res, scale_cols):
    from outlierneuronattention_amd.decode_layer import argmax_slots, greedy_from_keys, rows_linear
    g = torch.Generator().manual_seed(B * 7 + K + N)
    x = (torch.randn(B, K, generator=g) * 2 + 0.5).to(DEV, dt)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(DEV, dt)
    bb = (0.1 * torch.randn(N, generator=g)).to(DEV, dt) if bias else None
    lnp = ((1 + 0.2 * torch.randn(K, generator=g)).to(DEV, dt), (0.1 * torch.randn(K, generator=g)).to(DEV, dt),
           1e-5) if ln else None
    rr = torch.randn(B, N, generator=g).to(DEV, dt) if res else None
    scale = 1.0 / 64 ** 0.25
    ref = _ref_linear(x, w, bb, lnp, gelu, scale, scale_cols, rr, dt)
    out = torch.empty(B, N, device=DEV, dtype=dt)
    keys = torch.full((B * argmax_slots(N),), -1, dtype=torch.int64, device=DEV)  # every slot gets written
    print(f"rows_linear dt={dt} B={B} K={K} N={N}", flush=True)
    rows_linear(x, w, out, bias=bb, ln=lnp, gelu=gelu, scale=scale, scale_cols=scale_cols,
                res=None if rr is None else rr.clone(), argmax=keys)
    torch.cuda.synchronize()
    err = (out.float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), err
    idx = greedy_from_keys(keys, B, N)
    assert torch.equal(idx, out.float().argmax(-1)), (idx, out.float().argmax(-1))


@pytest.mark.parametrize("dt,offset", [(torch.float16, 200.0), (torch.bfloat16, 200.0), (torch.float16, -60.0)])
def test_rows_linear_layernorm_large_offset(dt, offset):
    """Rows whose mean is far above their spread: the LayerNorm variance is a
    sum of squared deviations (two passes), so nothing cancels."""
    from outlierneuronattention_amd.decode_layer import rows_linear
    g = torch.Generator().manual_seed(11)
    B, K, N = 4, 1024, 1024
    x = (torch.randn(B, K, generator=g) + offset).to(DEV, dt)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(DEV, dt)
    lnp = (torch.ones(K).to(DEV, dt), torch.zeros(K).to(DEV, dt), 1e-5)
    ref = _ref_linear(x, w, None, lnp, False, 1.0, 0, None, dt)
    out = torch.empty(B, N, device=DEV, dtype=dt)
    print(f"rows_linear LN offset={offset} dt={dt}", flush=True)
    rows_linear(x, w, out, ln=lnp)
    torch.cuda.synchronize()
    err = (out.float() - ref).abs().max().item()
    assert err <= 1e-2 * ref.abs().max().item(), err


def test_rows_linear_in_place_residual_and_errors():
    from outlierneuronattention_amd import _lib
    from outlierneuronattention_amd.decode_layer import rows_linear
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 512, generator=g).to(DEV, torch.bfloat16)
    w = (torch.randn(512, 512, generator=g) / 20).to(DEV, torch.bfloat16)
    y = torch.randn(2, 512, generator=g).to(DEV, torch.bfloat16)
    ref = _ref_linear(x, w, None, None, False, 1.0, 0, y, torch.bfloat16)
    rows_linear(x, w, y, res=y)
    torch.cuda.synchronize()
    assert (y.float() - ref).abs().max().item() <= 1e-2 * ref.abs().max().item()
    with pytest.raises(_lib.HofaError):
        rows_linear(torch.zeros(5, 512, device=DEV, dtype=torch.bfloat16), w, torch.zeros(5, 512, device=DEV,
                                                                                           dtype=torch.bfloat16))
    with pytest.raises(_lib.HofaError):
        rows_linear(x.float(), w.float(), torch.zeros(2, 512, device=DEV))


def _attn_module(fixed=False, seed=0):
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import HybridOutlierFactorizedAttention
    torch.manual_seed(seed)
    cfg = ModelConfig(d_model=256, num_heads=4, num_layers=1, r=16, fixed_blend_weight=fixed, device=DEV)
    a = HybridOutlierFactorizedAttention(cfg)
    with torch.no_grad():
        a.gate_proj.weight.normal_(0, 0.3)
        if fixed:
            a.fixed_mix.normal_(0, 1.0)
        else:
            a.mix_proj.weight.normal_(0, 0.3)
            a.mix_proj.bias.normal_(0, 0.5)
    return a.to(DEV, torch.bfloat16)


@pytest.mark.parametrize("fixed", [False, True])
def test_decode_prologue_matches_module_ops(fixed):
    from outlierneuronattention_amd.decode_layer import decode_prologue
    from outlierneuronattention_amd.modules import apply_rotary_pos_emb
    a = _attn_module(fixed)
    B, H, D, R, L = 3, 4, 64, 16, 40
    g = torch.Generator().manual_seed(9)
    qkv = torch.randn(B, 3 * H * D, generator=g).to(DEV, torch.bfloat16)
    ck = torch.zeros(B, H, L, R, device=DEV, dtype=torch.bfloat16)
    cv = torch.zeros(B, H, L, D, device=DEV, dtype=torch.bfloat16)
    pos = torch.tensor([17], dtype=torch.int64, device=DEV)
    lg = torch.zeros(B, H, device=DEV)
    mix = torch.zeros(B, H, device=DEV)
    Q = qkv[:, :H * D].view(B, H, 1, D).clone()
    K = qkv[:, H * D:2 * H * D].view(B, H, 1, D).clone()
    V = qkv[:, 2 * H * D:].view(B, H, 1, D).clone()
    with torch.no_grad():
        gl, mg = a._compute_gates_optimized(Q, K)
        lg_ref = F.logsigmoid(-gl).squeeze(-1).squeeze(-1).float()
        mix_ref = mg.squeeze(-1).squeeze(-1).float()
        cos, sin = a.rotary_emb.cos_cached[17:18], a.rotary_emb.sin_cached[17:18]
        qo, ko = apply_rotary_pos_emb(Q[..., :R], K[..., :R], cos, sin)
    decode_prologue(a, qkv, ck, cv, pos, lg, mix)
    torch.cuda.synchronize()
    assert (lg - lg_ref).abs().max().item() <= 1e-2 * max(1.0, lg_ref.abs().max().item())
    assert (mix - mix_ref).abs().max().item() <= 1e-2
    q_new = qkv[:, :H * D].view(B, H, 1, D)
    k_new = qkv[:, H * D:2 * H * D].view(B, H, 1, D)
    assert (q_new[..., :R].float() - qo.float()).abs().max().item() <= 2e-2
    assert (k_new[..., :R].float() - ko.float()).abs().max().item() <= 2e-2
    assert torch.equal(q_new[..., R:], Q[..., R:]) and torch.equal(k_new[..., R:], K[..., R:])
    assert torch.equal(ck[:, :, 17], k_new[:, :, 0, :R]) and torch.equal(cv[:, :, 17], V[:, :, 0])
    assert ck[:, :, :17].abs().sum().item() == 0 and cv[:, :, 18:].abs().sum().item() == 0


def _lm(seed, layers=2, alpha=False):
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    cfg = ModelConfig(d_model=256, num_heads=4, num_layers=layers, r=16, learnable_alpha=alpha, device=DEV)
    torch.manual_seed(seed)
    m = SubwordLM(512, cfg)
    with torch.no_grad():
        for layer in m.layers:
            at = layer.attn
            at.gate_proj.weight.normal_(0, 0.3)
            at.mix_proj.weight.normal_(0, 0.3)
            at.gla_scale.uniform_(0.5, 1.5)
            if alpha:
                at.log_alpha.normal_(0, 0.5)
        m.lm_head.weight.mul_(8.0)  # well-separated greedy choices
    return m.to(DEV, torch.bfloat16).eval()


@pytest.mark.parametrize("B,alpha,pro", [(1, False, True), (4, True, True), (2, False, False)])
def test_fused_graph_decoder_matches_module_op_decoder(B, alpha, pro):
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    m = _lm(seed=4 + B, alpha=alpha)
    N, steps = 45, 12
    ids = torch.randint(0, 512, (B, N), generator=torch.Generator().manual_seed(B)).to(DEV)
    ref = GreedyGraphDecoder(m, B, N + steps + 2, fused=False)
    fus = GreedyGraphDecoder(m, B, N + steps + 2, fused=True, prologue_in_decode=pro)
    assert fus.fused and not ref.fused
    ref.prefill(ids)
    fus.prefill(ids)
    for s in range(steps):  # one step at a time: the first is eager, then graph replays
        tr = ref.decode(1).clone()
        tf = fus.decode(1).clone()
        torch.cuda.synchronize()
        scale = ref.logits.float().abs().max().item()
        err = (fus.logits.float() - ref.logits.float()).abs().max().item()
        print(f"B={B} step {s}: tokens {tf.tolist()} vs {tr.tolist()}, logit err {err:.3e} of {scale:.3e}")
        assert err <= 3e-2 * scale
        assert torch.equal(tf, tr)
    assert int(fus.pos.item()) == N + steps and int(fus.seq_len.item()) == N + steps + 1
    for i in range(len(m.layers)):
        for c_f, c_r in zip(fus.caches[i], ref.caches[i]):
            d = (c_f[:, :, :N + steps].float() - c_r[:, :, :N + steps].float()).abs().max().item()
            assert d <= 3e-2 * max(1.0, c_r.float().abs().max().item())


@pytest.mark.parametrize("variant", ["per_layer_r_dh128", "fixed_blend_dh128"])
def test_fused_decoder_variants_match_module_op_decoder(variant):
    """The reference's 350M-style schedule varies r per layer at d_h = 128
    (training/training_config.py:407-422: r = [64, 32, 32] + [16]*18 + [32, 32, 64]);
    a three-layer U-shape r = [64, 16, 32] and the fixed-blend ablation
    (src/HybridOutlierFactorizedAttention.py:40-41) decode through the fused
    step exactly as through the module's own ops (tolerances as above)."""
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    fixed = variant == "fixed_blend_dh128"
    r = [32, 32] if fixed else [64, 16, 32]
    cfg = ModelConfig(d_model=256, num_heads=2, num_layers=len(r), r=r, fixed_blend_weight=fixed, device=DEV)
    torch.manual_seed(17)
    m = SubwordLM(512, cfg)
    with torch.no_grad():
        for layer in m.layers:
            at = layer.attn
            at.gate_proj.weight.normal_(0, 0.3)
            if fixed:
                at.fixed_mix.normal_(0, 1.0)
            else:
                at.mix_proj.weight.normal_(0, 0.3)
            at.gla_scale.uniform_(0.5, 1.5)
        m.lm_head.weight.mul_(8.0)
    m = m.to(DEV, torch.bfloat16).eval()
    assert [layer.attn.d_head for layer in m.layers] == [128] * len(r)
    B, N, steps = 2, 70, 8
    ids = torch.randint(0, 512, (B, N), generator=torch.Generator().manual_seed(5)).to(DEV)
    ref = GreedyGraphDecoder(m, B, N + steps + 2, fused=False)
    fus = GreedyGraphDecoder(m, B, N + steps + 2, fused=True)
    ref.prefill(ids)
    fus.prefill(ids)
    for s in range(steps):
        tr = ref.decode(1).clone()
        tf = fus.decode(1).clone()
        torch.cuda.synchronize()
        scale = ref.logits.float().abs().max().item()
        err = (fus.logits.float() - ref.logits.float()).abs().max().item()
        print(f"{variant} step {s}: tokens {tf.tolist()} vs {tr.tolist()}, logit err {err:.3e} of {scale:.3e}")
        assert err <= 3e-2 * scale
        assert torch.equal(tf, tr)


def test_prologue_in_decode_matches_prologue_launch():
    """hofa_decode_fused (gates, RoPE and cache append inside the decode
    launch, the new token as an extra split partial) against
    hofa_decode_prologue + hofa_decode on the same step: identical caches,
    GLA state within 1e-6 relative, outputs within 1e-2 of the largest (the
    token's score is summed in another order), at a length spanning many
    splits, with the gate's mix projection and with the fixed blend."""
    import ctypes
    from outlierneuronattention_amd import _lib
    from outlierneuronattention_amd.decode_layer import decode_prologue, prologue_args
    from outlierneuronattention_amd.hofa_decode import decode_args
    for fixed in (False, True):
        a = _attn_module(fixed, seed=3)
        B, H, D, R, L = 2, 4, 64, 16, 3000
        g = torch.Generator().manual_seed(21)
        pos = torch.tensor([2047], dtype=torch.int64, device=DEV)
        seq = torch.tensor([2048], dtype=torch.int32, device=DEV)
        qkv0 = torch.randn(B, 3 * H * D, generator=g).to(DEV, torch.bfloat16)
        ck0 = torch.randn(B, H, L, R, generator=g).to(DEV, torch.bfloat16)
        cv0 = torch.randn(B, H, L, D, generator=g).to(DEV, torch.bfloat16)
        s_in = (0.1 * torch.randn(B, H, D - R, D, generator=g)).to(DEV)
        nw = a.gla_scale.view(H, D)
        outs = []
        for fused in (False, True):
            print(f"prologue-in-decode fixed={fixed} fused={fused}", flush=True)
            qkv, ck, cv = qkv0.clone(), ck0.clone(), cv0.clone()
            lg, mix = torch.zeros(B, H, device=DEV), torch.zeros(B, H, device=DEV)
            s_out = torch.empty_like(s_in)
            y = torch.empty(B, H, 1, D, device=DEV, dtype=torch.bfloat16)
            q = qkv[:, :H * D].view(B, H, 1, D)
            k = qkv[:, H * D:2 * H * D].view(B, H, 1, D)
            v = qkv[:, 2 * H * D:].view(B, H, 1, D)
            lib = _lib.load()
            if not fused:
                decode_prologue(a, qkv, ck, cv, pos, lg, mix)
            args, _, keep = decode_args(q, k, v, ck, cv, s_in, s_out, lg, mix, nw, R, L, (D / R) ** 0.5,
                                        seq_len_dev=seq, y=y)
            stream = _lib.stream_handle(q.device)
            if fused:
                pro = prologue_args(a, qkv, ck, cv, pos, lg, mix)
                n = lib.hofa_decode_fused_workspace_bytes(ctypes.byref(args))
                ws = torch.empty(n, dtype=torch.uint8, device=DEV)
                rc = lib.hofa_decode_fused(ctypes.byref(args), ctypes.byref(pro), ws.data_ptr(), n, stream)
            else:
                n = lib.hofa_decode_workspace_bytes(ctypes.byref(args))
                ws = torch.empty(n, dtype=torch.uint8, device=DEV)
                rc = lib.hofa_decode(ctypes.byref(args), ws.data_ptr(), n, stream)
            _lib.check(rc, "decode")
            torch.cuda.synchronize()
            outs.append((y.float(), s_out, ck, cv))
        (y0, s0, ck_a, cv_a), (y1, s1, ck_b, cv_b) = outs
        print(f"fixed={fixed}: y err {(y0 - y1).abs().max().item():.3e}, state err {(s0 - s1).abs().max().item():.3e}")
        assert torch.equal(ck_a, ck_b) and torch.equal(cv_a, cv_b)
        assert (s0 - s1).abs().max().item() <= 1e-6 * s0.abs().max().item()
        assert (y0 - y1).abs().max().item() <= 1e-2 * y0.abs().max().item()
