"""The non-hybrid configurations of both module classes on the GPU against
the float64 oracle (``HOFARef.forward_variant``):

* ``r = 0`` (pure normalized GLA on every head),
* ``r = d_h`` (causal softmax attention on every head, RoPE on all channels),
* the width split (``mha_heads_for_width_split`` attention heads + GLA heads).

Tolerances, relative to the largest |output| of the case (float32 modules):
prefill 5e-3 (the attention kernel feeds bf16 probabilities to the PV
product), decode 5e-3 against the oracle's prefill over the grown sequence
(decode == last prefill row), and 2e-2 for the input gradient of the Train
width split against float64 autograd of the oracle.
"""
import pytest
import torch

from oracle import hofa_ref as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
B, H, DH = 2, 4, 64
D = H * DH

CASES = [  # (name, r, mha_heads)
    ("r0", 0, 0),
    ("rdh", DH, 0),
    ("split", 0, 2),
]


def _cfg(r, m, alpha):
    from outlierneuronattention_amd.config import ModelConfig
    return ModelConfig(d_model=D, num_heads=H, num_layers=2, r=r, mha_heads_for_width_split=m,
                       learnable_alpha=alpha, device=DEV)


def _module(cls_name, r, m, alpha, seed=0):
    if cls_name == "train":
        from outlierneuronattention_amd.HybridOutlierFactorizedAttentionTrain import HybridOutlierFactorizedAttention
    else:
        from outlierneuronattention_amd.HybridOutlierFactorizedAttention import HybridOutlierFactorizedAttention
    torch.manual_seed(seed)
    mod = HybridOutlierFactorizedAttention(_cfg(r, m, alpha)).to(DEV)
    with torch.no_grad():
        for name, p in mod.named_parameters():
            if name.startswith("W_") or name == "out_proj.weight":
                p.normal_(0, D ** -0.5)
            elif name == "gate_proj.weight":
                p.normal_(0, 0.3)
            elif name == "gla_scale":
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
            elif name == "log_alpha":
                p.normal_(0, 0.5)
    return mod


def _oracle(mod, r):
    st = {k: v.detach().cpu() for k, v in mod.state_dict().items()}
    return ref.HOFARef(st, D, H, r, dtype=torch.float64)


def _want(mod, r, m, x, cls_name, alpha):
    mha = H if r == DH else m
    use_alpha = alpha and cls_name == "train"  # the inference class's GLA-only paths take no alpha
    out, _ = _oracle(mod, r).forward_variant(x.detach().cpu().double(), mha_heads=mha, scale=1.0,
                                             use_alpha=use_alpha)
    return out


def _close(got, want, tol, what):
    want = want.to(got.device).float()
    scale = want.abs().max().item()
    err = (got.float() - want).abs().max().item()
    assert err <= tol * scale, f"{what}: max-abs {err:.3e} > {tol} x {scale:.3e}"


@pytest.mark.parametrize("cls_name", ["infer", "train"])
@pytest.mark.parametrize("alpha", [False, True])
@pytest.mark.parametrize("name,r,m", CASES)
def test_variant_prefill_matches_oracle(cls_name, alpha, name, r, m):
    mod = _module(cls_name, r, m, alpha).eval()
    x = torch.randn(B, 150, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(1))
    with torch.no_grad():
        got = mod(x)
    _close(got, _want(mod, r, m, x, cls_name, alpha), 5e-3, f"{cls_name} {name} prefill")


@pytest.mark.parametrize("name,r,m", CASES)
def test_inference_variant_decode_equals_prefill_rows(name, r, m):
    mod = _module("infer", r, m, False).eval()
    n0, steps = 120, 4
    x = torch.randn(B, n0 + steps, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(2))
    with torch.no_grad():
        _, cache_O, state = mod(x[:, :n0], return_state=True)
        for i in range(steps):
            out, cache_O, state = mod.forward_step(x[:, n0 + i:n0 + i + 1], cache_O, state)
            want = _want(mod, r, m, x[:, :n0 + i + 1], "infer", False)[:, -1:]
            _close(out, want, 5e-3, f"infer {name} decode step {i}")


@pytest.mark.parametrize("name,r", [("r0", 0), ("rdh", DH)])
@pytest.mark.parametrize("alpha", [False, True])
def test_train_variant_decode_equals_prefill_rows(name, r, alpha):
    mod = _module("train", r, 0, alpha).eval()
    n = 24
    x = torch.randn(B, n, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(3))
    cache_O = state = None
    with torch.no_grad():
        for i in range(n):
            out, cache_O, state = mod.forward_step(x[:, i:i + 1], cache_O, state)
            if i % 6 == 5 or i == n - 1:
                want = _want(mod, r, 0 if r == 0 else H, x[:, :i + 1], "train", alpha)[:, -1:]
                _close(out, want, 5e-3, f"train {name} decode step {i}")


def test_train_width_split_decode_follows_the_reference_r0_branch():
    """The reference's Train ``forward_step`` has no width-split branch: with
    ``r = 0`` it takes its pure-GLA branch over every head (:342-359), and so
    does this class."""
    mod = _module("train", 0, 2, True).eval()
    x = torch.randn(B, 12, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(6))
    cache_O = state = None
    with torch.no_grad():
        for i in range(12):
            out, cache_O, state = mod.forward_step(x[:, i:i + 1], cache_O, state)
    _close(out, _want(mod, 0, 0, x, "train", True)[:, -1:], 5e-3, "train width split decode")


@pytest.mark.parametrize("alpha", [False, True])
def test_train_width_split_input_gradient_matches_oracle(alpha):
    mod = _module("train", 0, 2, alpha)
    x = torch.randn(B, 130, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(4), requires_grad=True)
    dy = torch.randn(B, 130, D, device=DEV, generator=torch.Generator(device=DEV).manual_seed(5))
    (mod(x) * dy).sum().backward()
    xr = x.detach().cpu().double().requires_grad_(True)
    out, _ = _oracle(mod, 0).forward_variant(xr, mha_heads=2, use_alpha=alpha)
    (out * dy.cpu().double()).sum().backward()
    _close(x.grad, xr.grad, 2e-2, "train width split dx")
