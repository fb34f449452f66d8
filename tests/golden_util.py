"""Loading helpers for the golden fixtures written by tests/golden/make_golden.py."""
import glob
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden_cases():
    return sorted(os.path.basename(p)[len("hofa_train_step_"):-4]
                  for p in glob.glob(os.path.join(GOLDEN, "hofa_train_step_*.npz")))


def load_golden(name):
    z = np.load(os.path.join(GOLDEN, f"hofa_train_step_{name}.npz"))
    d_model, H, r, alpha, fixed, B, N = (int(v) for v in z["meta"])
    params = {k[len("param."):]: torch.from_numpy(z[k].copy()) for k in z.files if k.startswith("param.")}
    return dict(d_model=d_model, H=H, r=r, alpha=bool(alpha), fixed=bool(fixed), B=B, N=N,
                params=params, x=torch.from_numpy(z["x"].copy()), y=torch.from_numpy(z["y"].copy()),
                cache_k=torch.from_numpy(z["cache_k"].copy()), cache_v=torch.from_numpy(z["cache_v"].copy()),
                state=torch.from_numpy(z["state"].copy()))
