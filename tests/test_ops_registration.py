"""The ``torch.library`` operators of the attention core, on the CPU: their
fake implementations give the shapes, dtypes and strides of the real ones
(the GPU tests run both and compare), so ``torch.compile`` can trace the
Train module through them without running a kernel."""
import math

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import outlierneuronattention_amd.autograd  # noqa: F401  (registers hofa::*)
from outlierneuronattention_amd.chunk_gla_inlier import chunk_states_numel


def _inputs(B, T, H, D, dt=torch.bfloat16, alpha=True, mix=True):
    mk = lambda *s: torch.empty(*s, dtype=dt)  # noqa: E731
    q, k, v = (mk(B, T, H, D).transpose(1, 2) for _ in range(3))
    lg = torch.empty(B, H, T, dtype=dt)
    la = torch.empty(1, H, 1, D - 16) if alpha else None
    m = torch.empty(B, H, T, dtype=dt) if mix else None
    gs = torch.empty(1, H, 1, D)
    return q, k, v, lg, la, m, gs


@pytest.mark.parametrize("save", [False, True])
@pytest.mark.parametrize("T", [100, 4096])
def test_prefill_fwd_fake_shapes(save, T):
    B, H, D, r = 2, 3, 64, 16
    with FakeTensorMode():
        q, k, v, lg, la, m, gs = _inputs(B, T, H, D)
        q_o, k_o = q[..., :r].contiguous(), k[..., :r].contiguous()
        y, states, n, rstd, cs, o, lse = torch.ops.hofa.prefill_fwd(q, k, v, lg, la, m, gs, q_o, k_o, r,
                                                                     math.sqrt(D / r), save)
    assert y.shape == (B, H, T, D) and y.dtype == torch.bfloat16 and y.is_contiguous()
    assert states.shape == (B, H, 64, 64) and states.dtype == torch.float32
    if save:
        assert n.shape == (B, H, T, D) and rstd.shape == (B * H * T,) and rstd.dtype == torch.float32
        assert cs.numel() == chunk_states_numel(B, H, T, D, D - r) and cs.dtype == torch.int16
        assert o.shape == (B, H, T, D) and lse.shape == (B * H * T,)
    else:
        assert n.numel() == rstd.numel() == cs.numel() == o.numel() == lse.numel() == 0


def test_prefill_bwd_fake_shapes():
    B, T, H, D, r = 2, 130, 3, 64, 16
    with FakeTensorMode():
        q, k, v, lg, la, m, gs = _inputs(B, T, H, D)
        dy = torch.empty(B, H, T, D, dtype=torch.bfloat16)
        n = torch.empty(B, H, T, D, dtype=torch.bfloat16)
        rstd = torch.empty(B * H * T)
        cs = torch.empty(chunk_states_numel(B, H, T, D, D - r), dtype=torch.int16)
        o = torch.empty(B, H, T, D, dtype=torch.bfloat16)
        lse = torch.empty(B * H * T)
        out = torch.ops.hofa.prefill_bwd(dy, None, None, q, k, v, lg, la, m, gs, n, rstd, cs, o, lse, r, 2.0)
    dq_o, dk_o, dq, dk, dv, d_lg, d_la, d_mix, d_gs = out
    assert dq_o.numel() == 0 and dk_o.numel() == 0
    assert dq.shape == q.shape and dq.stride() == q.stride() and dk.stride() == k.stride()
    assert dv.shape == (B, H, T, D) and dv.is_contiguous()
    assert d_lg.shape == (B, H, T) and d_la.shape == (H, D - r) and d_mix.shape == (B, H, T)
    assert d_gs.shape == (H, D) and all(t.dtype == torch.float32 for t in (d_lg, d_la, d_mix, d_gs))


def test_ops_are_registered_with_autograd_and_fake():
    import re
    for name in ("prefill_fwd", "prefill_bwd", "decode_step"):
        op = getattr(torch.ops.hofa, name).default
        for key in ("Meta", "Autograd"):
            assert torch._C._dispatch_has_kernel_for_dispatch_key(op.name(), key), (name, key)
    # decode writes state_out in place and says so in its schema
    schema = str(torch.ops.hofa.decode_step.default._schema)
    assert re.search(r"Tensor\(a\d*!\) state_out", schema), schema
    assert "!" not in str(torch.ops.hofa.prefill_fwd.default._schema)
