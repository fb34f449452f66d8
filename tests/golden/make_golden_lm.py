"""Write golden logits from the reference's own language-model stack.

Run in the build container only (needs the reference checkout):

    python tests/golden/make_golden_lm.py /root/reference

It builds the reference's Train ``SubwordLM`` (src/HybridOutlierFactorizedAttentionTrain.py:469-502,
``TransformerBlock`` :441-466) on the CPU and runs its own ``forward``: token
embedding, per-layer ``x + attn(ln_1(x))`` and ``x + mlp(ln_2(x))``,
``ln_f`` and the tied LM head.  The Train attention's ``forward`` needs fla,
which is absent here, so each layer's attention is driven through the same
module's pure-torch ``forward_step`` (:298-438) token by token from an empty
cache -- a prefill of N tokens equals N decode steps.  Everything else is the
reference's own code, so the vectors pin the block composition, the MLP, the
tied head and the per-layer r list.

Output: ``tests/golden/hofa_lm_<case>.npz`` (weights, ids, logits as plain
arrays; load with ``numpy.load`` (no pickle)).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

CASES = {
    # name: (d_model, H, r (int or per-layer list), vocab, B, N, learnable_alpha)
    "2l_r16": (128, 2, 16, 97, 2, 18, False),
    "3l_rlist_alpha": (128, 2, [16, 32, 16], 89, 1, 14, True),
}


def _stepwise(attn):
    def forward(x):
        cache, state, outs = None, None, []
        for t in range(x.shape[1]):
            y, cache, state = attn.forward_step(x[:, t:t + 1], cache, state)
            outs.append(y)
        return torch.cat(outs, 1)
    return forward


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from src.config import ModelConfig  # noqa: E402
    from src.HybridOutlierFactorizedAttentionTrain import SubwordLM  # noqa: E402

    out_dir = os.path.dirname(os.path.abspath(__file__))
    for name, (d_model, H, r, vocab, B, N, alpha) in CASES.items():
        layers = len(r) if isinstance(r, list) else 2
        cfg = ModelConfig(d_model=d_model, num_heads=H, num_layers=layers, r=r, learnable_alpha=alpha,
                          device="cpu")
        torch.manual_seed(42)
        m = SubwordLM(vocab, cfg).eval()
        g = torch.Generator().manual_seed(9)
        with torch.no_grad():
            for pname, p in m.named_parameters():
                if ".gate_proj" in pname or ".mix_proj" in pname:
                    p.copy_(torch.randn(p.shape, generator=g) * 0.2 + (p if pname.endswith("bias") else 0))
                elif pname.endswith("log_alpha"):
                    p.copy_(torch.randn(p.shape, generator=g) * 0.5)
                elif pname.endswith("gla_scale"):
                    p.copy_(1.0 + 0.3 * torch.randn(p.shape, generator=g))
                elif pname.endswith(("W_q.weight", "W_k.weight", "W_v.weight")):
                    p.mul_(8.0)  # larger Q/K/V so the softmax is not flat
                elif pname.startswith("layers.") and (".ln_" in pname or pname.endswith(".bias")):
                    p.add_(0.1 * torch.randn(p.shape, generator=g))  # non-trivial LayerNorm and MLP biases
                elif pname.startswith("ln_f"):
                    p.add_(0.1 * torch.randn(p.shape, generator=g))
        for layer in m.layers:
            layer.attn.forward = _stepwise(layer.attn)
        ids = torch.randint(0, vocab, (B, N), generator=g)
        with torch.no_grad():
            logits, _ = m(ids)
        arrays = {f"param.{k}": v.detach().numpy() for k, v in m.state_dict().items()}
        r_list = r if isinstance(r, list) else [r] * layers
        arrays.update({"ids": ids.numpy(), "logits": logits.numpy(),
                       "r_list": np.array(r_list, dtype=np.int64),
                       "meta": np.array([d_model, H, layers, vocab, B, N, int(alpha)], dtype=np.int64)})
        path = os.path.join(out_dir, f"hofa_lm_{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path}: logits{tuple(logits.shape)}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
