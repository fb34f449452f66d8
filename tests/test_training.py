"""Training integration (loader, chunked cross entropy, optimizer step).

CPU: the uint16 token loader and the learning-rate schedule.  GPU: the
chunked cross entropy gives the direct cross entropy's loss and gradients
(training/train_cpt.py:137-176 states they are identical), and compiled
optimizer steps on a fixed batch lower its loss.
"""
import math

import numpy as np
import pytest
import torch

from outlierneuronattention_amd.training import FastTokenLoader, adjust_learning_rate


def test_token_loader_batches_and_wraps(tmp_path):
    toks = np.arange(1000, dtype=np.uint16) * 7 % 50257
    path = tmp_path / "train.bin"
    toks.tofile(path)
    ld = FastTokenLoader(str(path), global_batch_size=3, seq_len=99, start_idx=100)
    x, y, nxt = ld.get_batch()
    assert x.dtype == torch.int64 and x.shape == (3, 99) and y.shape == (3, 99)
    rows = torch.from_numpy(toks[100:400].astype(np.int64)).view(3, 100)
    assert torch.equal(x, rows[:, :-1]) and torch.equal(y, rows[:, 1:]) and nxt == 400
    ld.get_batch(), ld.get_batch()          # 400..700, 700..1000
    x, _, nxt = ld.get_batch()              # 1000 + 300 > 1000: wraps to 0
    assert nxt == 300 and torch.equal(x[0], torch.from_numpy(toks[0:99].astype(np.int64)))


def test_token_loader_rejects_short_files(tmp_path):
    path = tmp_path / "tiny.bin"
    np.zeros(10, dtype=np.uint16).tofile(path)
    with pytest.raises(ValueError):
        FastTokenLoader(str(path), 2, 8)


def test_learning_rate_schedule():
    opt = torch.optim.SGD([torch.nn.Parameter(torch.zeros(1))], lr=0.0)
    opt.param_groups[0]["lr_multiplier"] = 2.0
    assert adjust_learning_rate(opt, 5, 110, 1e-3, 10) == pytest.approx(5e-4)
    assert opt.param_groups[0]["lr"] == pytest.approx(1e-3)
    assert adjust_learning_rate(opt, 10, 110, 1e-3, 10) == pytest.approx(1e-3)
    assert adjust_learning_rate(opt, 60, 110, 1e-3, 10) == pytest.approx(0.5e-3)
    assert adjust_learning_rate(opt, 110, 110, 1e-3, 10) == pytest.approx(0.0, abs=1e-12)
    assert adjust_learning_rate(opt, 35, 110, 1e-3, 10) == pytest.approx(1e-3 * 0.5 * (1 + math.cos(math.pi / 4)))


def _lm(seed=5):
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.HybridOutlierFactorizedAttentionTrain import SubwordLM
    torch.manual_seed(seed)
    cfg = ModelConfig(d_model=256, num_heads=4, num_layers=2, r=16, learnable_alpha=True, device="cuda")
    return SubwordLM(1000, cfg).to("cuda")


@pytest.mark.gpu
def test_chunked_cross_entropy_matches_direct():
    from outlierneuronattention_amd.training import forward_and_backward_chunked
    m = _lm()
    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randint(0, 1000, (2, 300), device="cuda", generator=g)
    y = torch.randint(0, 1000, (2, 300), device="cuda", generator=g)
    m.zero_grad()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, loss = m(x, y)
    (loss / 2).backward()
    direct = {n: p.grad.float().clone() for n, p in m.named_parameters()}
    m.zero_grad()
    l2 = forward_and_backward_chunked(m, x, y, grad_accum_steps=2, chunk_size=128, checkpointing_interval=1)
    assert abs(l2 - loss.item()) <= 1e-3 * loss.item(), (l2, loss.item())
    for n, p in m.named_parameters():
        scale = direct[n].abs().max().item() + 1e-30
        err = (p.grad.float() - direct[n]).abs().max().item()
        assert err <= 2e-2 * scale, f"{n}: {err:.3e} vs {scale:.3e}"


@pytest.mark.gpu
def test_compiled_train_steps_fit_a_batch():
    from outlierneuronattention_amd.training import train_step
    torch._dynamo.reset()
    m = _lm()
    opt = torch.optim.AdamW(m.parameters(), lr=3e-3, weight_decay=0.1)
    comp = torch.compile(m, dynamic=True, backend="aot_eager")
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randint(0, 1000, (4, 128), device="cuda", generator=g)
    y = torch.randint(0, 1000, (4, 128), device="cuda", generator=g)
    losses = [train_step(comp, opt, x, y, micro_batch_size=2) for _ in range(8)]
    assert all(math.isfinite(v) for v in losses)
    assert losses[-1] < losses[0] - 0.5, losses
