"""Write golden vectors from the reference's own PyTorch decode path.

Run in the build container only (needs the reference checkout):

    python tests/golden/make_golden.py /root/reference

It imports ``HybridOutlierFactorizedAttention`` from the reference's
``src/HybridOutlierFactorizedAttentionTrain.py`` (pure torch, CPU) and drives
``forward_step`` (:298-438) token by token from an empty cache.  Its outputs
pin the conventions no closed form fixes: which half of ``gate_proj`` /
``mix_proj`` multiplies Q, the RoPE half-split and position, ``sm_scale``,
the alpha padding, the zero-padded ``[d_h, d_h]`` state and the blend.  Since a
prefill of N tokens equals N decode steps from an empty cache, the same
vectors also pin the prefill composition.

Output: ``tests/golden/hofa_train_step_<case>.npz`` (inputs, weights and
outputs as plain arrays; load with ``numpy.load`` (no pickle)).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

CASES = {
    # name: (d_model, H, r, learnable_alpha, fixed_blend_weight, B, N)
    "r16_mix": (128, 2, 16, False, False, 2, 24),
    "r16_alpha": (128, 2, 16, True, False, 2, 24),
    "r16_fixed": (128, 2, 16, False, True, 2, 20),
    "r32_alpha_dh64": (128, 2, 32, True, False, 2, 20),
    "r16_dh128": (128, 1, 16, True, False, 2, 16),
}


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from src.config import ModelConfig  # noqa: E402
    from src.HybridOutlierFactorizedAttentionTrain import HybridOutlierFactorizedAttention  # noqa: E402

    out_dir = os.path.dirname(os.path.abspath(__file__))
    for name, (d_model, H, r, alpha, fixed, B, N) in CASES.items():
        cfg = ModelConfig(d_model=d_model, num_heads=H, num_layers=2, r=r, learnable_alpha=alpha,
                          fixed_blend_weight=fixed, device="cpu")
        torch.manual_seed(42)
        m = HybridOutlierFactorizedAttention(cfg).eval()
        # The reference initialises the gate weights to zero; perturb every
        # parameter so each convention leaves a visible trace in the outputs.
        g = torch.Generator().manual_seed(7)
        with torch.no_grad():
            for pname, p in m.named_parameters():
                if pname.startswith(("gate_proj", "mix_proj")):
                    p.copy_(torch.randn(p.shape, generator=g) * 0.2 + (p if pname.endswith("bias") else 0))
                elif pname == "log_alpha":
                    p.copy_(torch.randn(p.shape, generator=g) * 0.5)
                elif pname == "gla_scale":
                    p.copy_(1.0 + 0.3 * torch.randn(p.shape, generator=g))
                elif pname == "fixed_mix":
                    p.copy_(torch.randn(p.shape, generator=g))
                elif pname.startswith(("W_q", "W_k", "W_v")):
                    p.mul_(8.0)  # larger Q/K/V so the softmax is not flat
        x = torch.randn(B, N, d_model, generator=g)
        outs = []
        cache, state = None, None
        with torch.no_grad():
            for t in range(N):
                y, cache, state = m.forward_step(x[:, t:t + 1], cache, state)
                outs.append(y)
        y = torch.cat(outs, 1)
        arrays = {f"param.{k}": v.detach().numpy() for k, v in m.state_dict().items()}
        arrays.update({
            "x": x.numpy(), "y": y.numpy(), "cache_k": cache[0].numpy(), "cache_v": cache[1].numpy(),
            "state": state.numpy(),
            "meta": np.array([d_model, H, r, int(alpha), int(fixed), B, N], dtype=np.int64),
        })
        path = os.path.join(out_dir, f"hofa_train_step_{name}.npz")
        np.savez_compressed(path, **arrays)
        print(f"wrote {path}: y{tuple(y.shape)} state{tuple(state.shape)}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
