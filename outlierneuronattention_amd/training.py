"""Training integration around the HOFA core: the callers of the Train model
that the reference's training scripts provide.

* :class:`FastTokenLoader` reads the reference's token cache format, a flat
  little-endian uint16 file, through a memory map (training/data_utils.py:5-33):
  every batch takes ``global_batch_size * (seq_len + 1)`` consecutive tokens
  from a running index, wraps to the start of the file when the next batch
  would run past its end, and splits rows into inputs ``x = row[:-1]`` and
  targets ``y = row[1:]``.
* :func:`forward_and_backward_chunked` is the chunked cross entropy of
  training/train_cpt.py:137-176: the trunk runs once under bf16 autocast, the
  tied LM head and the loss run over ``chunk_size`` tokens at a time, each
  chunk's gradient with respect to the final hidden state is collected, and one
  backward pass through the trunk follows.  The loss and gradients equal those
  of the direct cross entropy while only one chunk's logits are alive at once.
* :func:`train_step` is one optimizer step of training/train.py:175-223:
  micro-batches sliced from the global batch, bf16 autocast, gradient
  accumulation, clipping and the update; :func:`adjust_learning_rate` is the
  linear-warmup cosine schedule it uses (src/modules/benchmark_utils.py:151-159).

The model may be wrapped by ``torch.compile`` (the reference compiles with
``dynamic=True``, training/train.py:157): the attention core is the
``hofa::prefill_fwd`` / ``hofa::prefill_bwd`` operator pair.
"""
from __future__ import annotations

import math
import os
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F


class FastTokenLoader:
    """Batches of ``(x, y)`` token ids from a uint16 cache file."""

    def __init__(self, cache_path: str, global_batch_size: int, seq_len: int, start_idx: int = 0):
        self.cache_path = cache_path
        self.global_batch_size = int(global_batch_size)
        self.seq_len = int(seq_len)
        self.tokens_per_batch = self.global_batch_size * (self.seq_len + 1)
        self.total_tokens = os.path.getsize(cache_path) // 2
        if self.total_tokens < self.tokens_per_batch:
            raise ValueError(f"{cache_path}: {self.total_tokens} tokens, one batch needs {self.tokens_per_batch}")
        self.mmap = np.memmap(cache_path, dtype=np.uint16, mode="r", shape=(self.total_tokens,))
        self.current_idx = int(start_idx)

    def get_batch(self) -> Tuple[torch.Tensor, torch.Tensor, int]:
        """``(x [B, N], y [B, N], next index)``; int64, in pinned host memory
        when a GPU is present so the copy to the device can be asynchronous."""
        if self.current_idx + self.tokens_per_batch > self.total_tokens:
            self.current_idx = 0
        chunk = np.asarray(self.mmap[self.current_idx:self.current_idx + self.tokens_per_batch], dtype=np.int64)
        data = torch.from_numpy(chunk)
        if torch.cuda.is_available():
            data = data.pin_memory()
        data = data.view(self.global_batch_size, self.seq_len + 1)
        self.current_idx += self.tokens_per_batch
        return data[:, :-1].contiguous(), data[:, 1:].contiguous(), self.current_idx


def _trunk(model, x: torch.Tensor, checkpointing_interval: Optional[int]) -> torch.Tensor:
    h = model.token_emb(x)
    for i, layer in enumerate(model.layers):
        if checkpointing_interval is not None and i % checkpointing_interval == 0:
            h = torch.utils.checkpoint.checkpoint(layer, h, use_reentrant=False)
        else:
            h = layer(h)
    return model.ln_f(h)


def forward_and_backward_chunked(model, x: torch.Tensor, targets: torch.Tensor, grad_accum_steps: int = 1,
                                 chunk_size: int = 4096, checkpointing_interval: Optional[int] = None) -> float:
    """Loss (mean cross entropy over the batch's tokens) of ``model`` on
    ``(x, targets)``, with every parameter's gradient accumulated as by
    ``(loss / grad_accum_steps).backward()``; the logits exist one chunk of
    ``chunk_size`` tokens at a time.  ``model`` is a Train ``SubwordLM``."""
    B, N = x.shape
    total = B * N
    with torch.autocast("cuda", dtype=torch.bfloat16):
        h = _trunk(model, x, checkpointing_interval)
        h_flat = h.reshape(total, -1)
        y_flat = targets.reshape(total)
        grad_h = torch.empty_like(h_flat)
        loss_sum = torch.zeros((), dtype=torch.float32, device=x.device)
        for i in range(0, total, chunk_size):
            end = min(i + chunk_size, total)
            sub_h = h_flat[i:end].detach().requires_grad_(True)
            logits = model.lm_head(sub_h)
            sub = F.cross_entropy(logits.float(), y_flat[i:end], reduction="sum") / total
            loss_sum += sub.detach()
            (sub / grad_accum_steps).backward()
            grad_h[i:end] = sub_h.grad
    h_flat.backward(grad_h)
    return float(loss_sum)


def adjust_learning_rate(optimizer, step: int, total_steps: int, base_lr: float, warmup_steps: int) -> float:
    """Linear warmup to ``base_lr``, then a half cosine to zero; a param
    group's ``lr_multiplier`` scales its rate."""
    if step < warmup_steps:
        lr = base_lr * (step / warmup_steps)
    else:
        progress = (step - warmup_steps) / max(1, total_steps - warmup_steps)
        lr = base_lr * 0.5 * (1.0 + math.cos(math.pi * progress))
    for group in optimizer.param_groups:
        group["lr"] = lr * group.get("lr_multiplier", 1.0)
    return lr


def train_step(model, optimizer, x_global: torch.Tensor, y_global: torch.Tensor, micro_batch_size: int,
               grad_clip_norm: float = 1.0, mixed_precision: bool = True) -> float:
    """One optimizer step over a global batch split into micro-batches of
    ``micro_batch_size`` rows; returns the mean loss."""
    optimizer.zero_grad(set_to_none=True)
    steps = x_global.shape[0] // micro_batch_size
    if steps * micro_batch_size != x_global.shape[0]:
        raise ValueError(f"global batch {x_global.shape[0]} is not a multiple of {micro_batch_size}")
    total = torch.zeros((), dtype=torch.float32, device=x_global.device)
    for m in range(steps):
        x = x_global[m * micro_batch_size:(m + 1) * micro_batch_size]
        y = y_global[m * micro_batch_size:(m + 1) * micro_batch_size]
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=mixed_precision):
            _, loss = model(x, targets=y)
            loss = loss / steps
        loss.backward()
        total += loss.detach().float()
    if grad_clip_norm > 0:
        torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip_norm)
    optimizer.step()
    return float(total)
