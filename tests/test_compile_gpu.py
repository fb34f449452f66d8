"""The Train model under ``torch.compile`` (the reference trains with
``torch.compile(model, dynamic=True)``, training/train.py:157, and bf16
autocast, :200): the attention core is the ``hofa::prefill_fwd`` /
``hofa::prefill_bwd`` operator pair, so Dynamo traces forward and backward
with no graph break (``fullgraph=True``) and the compiled step matches eager.

Backend ``aot_eager`` (Dynamo + AOTAutograd, the graph run op by op) checks
the tracing and the operators' fake and autograd registrations without code
generation.  Tolerance: the compiled and eager steps run the same kernels;
the loss agrees to 1e-4 relative and every gradient to 1e-3 of its largest
entry (autocast may place casts differently in the traced graph).
"""
import copy

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(alpha: bool, r):
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.HybridOutlierFactorizedAttentionTrain import SubwordLM
    torch.manual_seed(3)
    cfg = ModelConfig(d_model=256, num_heads=4, num_layers=2, r=r, learnable_alpha=alpha, device=DEV)
    m = SubwordLM(512, cfg).to(DEV)
    # non-trivial gates so every gradient path carries signal
    with torch.no_grad():
        for layer in m.layers:
            layer.attn.gate_proj.weight.normal_(0, 0.1)
            if hasattr(layer.attn, "mix_proj"):
                layer.attn.mix_proj.weight.normal_(0, 0.1)
            if alpha:
                layer.attn.log_alpha.normal_(0, 0.5)
    return m


def _step(model, x, y):
    model.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, loss = model(x, y)
    loss.backward()
    return loss.detach().float(), {n: p.grad.detach().float().clone() for n, p in model.named_parameters()
                                   if p.grad is not None}


@pytest.mark.parametrize("alpha,r", [(True, 16), (False, [16, 0])])
def test_compiled_train_step_matches_eager(alpha, r):
    torch._dynamo.reset()
    eager = _model(alpha, r)
    comp_model = copy.deepcopy(eager)
    compiled = torch.compile(comp_model, dynamic=True, fullgraph=True, backend="aot_eager")
    for T in (128, 200):  # the second length reuses the dynamic graph
        g = torch.Generator(device=DEV).manual_seed(T)
        x = torch.randint(0, 512, (2, T), device=DEV, generator=g)
        y = torch.randint(0, 512, (2, T), device=DEV, generator=g)
        le, ge = _step(eager, x, y)
        lc, gc = _step(compiled, x, y)
        assert abs(le.item() - lc.item()) <= 1e-4 * abs(le.item()), (T, le.item(), lc.item())
        assert ge.keys() == {k.replace("_orig_mod.", "") for k in gc.keys()} or ge.keys() == gc.keys()
        for name, a in ge.items():
            b = gc.get(name, gc.get("_orig_mod." + name))
            scale = a.abs().max().item() + 1e-30
            err = (a - b).abs().max().item()
            assert err <= 1e-3 * scale, f"T={T} {name}: {err:.3e} vs max {scale:.3e}"
