"""The attention core's training step (forward and backward through the
``hofa::prefill_fwd`` / ``hofa::prefill_bwd`` operators) captured in one HIP
graph and replayed.

Every replay, with eager steps and synchronisations between the replays,
must reproduce the eager output and gradients bit for bit: the kernels use no
atomics, and the captured launches are the eager ones.  Before each replay
the static output and gradient tensors are overwritten with NaN, so a
replay that skips writing any of them fails.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B=2, H=4, T=600, D=64, R=16, seed=5):
    J = D - R
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, H, 3 * D, generator=gen).to(DEV, torch.bfloat16)
    q, k, v = (x[..., i * D:(i + 1) * D].transpose(1, 2).contiguous() for i in range(3))
    lg = (-torch.rand(B, H, T, generator=gen)).to(DEV)
    la = (0.5 * torch.randn(1, H, 1, J, generator=gen)).to(DEV)
    mix = torch.sigmoid(torch.randn(B, H, T, generator=gen)).to(DEV)
    gs = (1 + 0.1 * torch.randn(1, H, 1, D, generator=gen)).to(DEV)
    dy = torch.randn(B, H, T, D, generator=gen).to(DEV, torch.bfloat16)
    leaves = dict(q=q, k=k, v=v, lg=lg, la=la, mix=mix, gs=gs)
    for t in leaves.values():
        t.requires_grad_()
    return leaves, dy, R, math.sqrt(D / R)


def test_captured_train_step_replays_match_eager():
    from outlierneuronattention_amd.autograd import hofa_core
    leaves, dy, R, sm = _inputs()
    print("graph-captured train step: B=2 H=4 T=600 d_h=64 r=16", flush=True)

    def step():
        for t in leaves.values():
            t.grad = None
        y = hofa_core(None, None, leaves["q"], leaves["k"], leaves["v"], leaves["lg"], leaves["la"], leaves["mix"],
                      leaves["gs"], R, sm)
        y.backward(dy)
        return y

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            y_e = step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref_y = y_e.detach().clone()
    ref = {n: t.grad.detach().clone() for n, t in leaves.items()}

    graph = torch.cuda.CUDAGraph()
    for t in leaves.values():
        t.grad = None
    with torch.cuda.graph(graph):
        y_g = hofa_core(None, None, leaves["q"], leaves["k"], leaves["v"], leaves["lg"], leaves["la"],
                        leaves["mix"], leaves["gs"], R, sm)
        y_g.backward(dy)
    static = {n: t.grad for n, t in leaves.items()}
    assert all(g is not None for g in static.values())

    for i in range(3):
        with torch.no_grad():
            y_g.fill_(float("nan"))
            for g in static.values():
                g.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_g, ref_y), f"replay {i}: output"
        for n, g in static.items():
            assert torch.equal(g, ref[n]), f"replay {i}: d{n}"
        # the program's own eager work between replays (same kernels, its own workspaces)
        y_e = step()
        torch.cuda.synchronize()
        assert torch.equal(y_e, ref_y), f"eager step after replay {i}"
        for n, t in leaves.items():
            assert torch.equal(t.grad, ref[n]), f"eager step after replay {i}: d{n}"
