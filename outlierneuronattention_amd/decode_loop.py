"""Greedy multi-step decoding of ``SubwordLM`` inside captured HIP graphs.

The reference's generation loop (src/inference.py:150-239) prefills the
prompt with ``model(context, return_state=True)``, pre-allocates the outlier
caches to ``prompt + max_new_tokens`` rows (:155-168) and then calls
``forward_step`` once per token with a Python ``cache_seq_len``.  Its graph
benchmark (benchmarks/profile_full_decode.py:54-75) captures one
``forward_step`` and replays it: the RoPE row, the cache slot and the
attended length are Python integers frozen into the capture, so every replay
recomputes the same position.

Here the decode position lives in device memory, so one capture serves every
step:

* ``pos`` (int64, one element) indexes the RoPE tables (``index_select``) and
  the cache slot of the new token (``index_copy_``);
* ``seq_len`` (int32, one element) is ``pos + 1`` and is read by the decode
  kernel at run time (``fused_hofa_decode(..., seq_len_dev=...)``);
* the greedy token (``argmax`` of the last logits) is written to the static
  input of the next step and appended to the output at a device-side column;
* both counters advance inside the graph.

The GLA state is ping-pong as in the reference (``forward_step`` returns
``(state_out, state_in)``, src/HybridOutlierFactorizedAttention.py:422): two
graphs are captured, one reading buffer A and writing B, the other the
reverse, and replays alternate between them.

Only the hybrid attention path (0 < r < d_head, no width-split heads) is
supported, which is the configuration the reference's graph benchmark runs.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .HybridOutlierFactorizedAttention import SubwordLM
from .hofa_decode import fused_hofa_decode
from .modules import apply_rotary_pos_emb


def _attn_step(attn, x, cache_k, cache_v, s_in, s_out, pos, seq_len):
    """One token through one attention module with a device-side position.

    Same arithmetic as the module's hybrid ``forward_step``
    (src/HybridOutlierFactorizedAttention.py:223-422): projections, gates on
    the pre-RoPE Q/K, RoPE of the outlier channels at row ``pos``, cache
    append, then the fused decode kernel over ``seq_len`` rows."""
    Q, K, V = attn._project(x)
    gate_logits, mix_g = attn._compute_gates_optimized(Q, K)
    log_gamma = F.logsigmoid(-gate_logits).squeeze(-1)
    r = attn.r
    if hasattr(attn, "rotary_emb"):
        cos = attn.rotary_emb.cos_cached.index_select(0, pos)
        sin = attn.rotary_emb.sin_cached.index_select(0, pos)
        Q_O, K_O = apply_rotary_pos_emb(Q[..., :r], K[..., :r], cos, sin)
        Q[..., :r] = Q_O
        K[..., :r] = K_O
    cache_k.index_copy_(2, pos, K[..., :r])
    cache_v.index_copy_(2, pos, V)
    Y = fused_hofa_decode(Q, K, V, cache_k, cache_v, s_in, s_out, log_gamma, mix_g.squeeze(-1),
                          attn.gla_scale.view(attn.num_heads, attn.d_head), r, cache_k.shape[2],
                          (attn.d_head / r) ** 0.5,
                          log_alpha=attn.log_alpha if attn.learnable_alpha else None, seq_len_dev=seq_len)
    return attn._merge(Y, x.dtype)


class GreedyGraphDecoder:
    """Prefill a batch of prompts, then decode greedily from captured graphs.

    ``capacity`` is the cache length in rows (prompt + new tokens); caches and
    states are allocated once, in the dtype of the model's parameters.
    """

    def __init__(self, model: SubwordLM, batch: int, capacity: int):
        for layer in model.layers:
            a = layer.attn
            if not (0 < a.r < a.d_head) or a.forced_mha_heads > 0:
                raise NotImplementedError("GreedyGraphDecoder supports the hybrid path (0 < r < d_head) only")
            if hasattr(a, "rotary_emb"):
                a.rotary_emb(capacity)  # grow the tables before any capture
        p = next(model.parameters())
        self.model, self.B, self.capacity = model, batch, capacity
        self.device, self.dtype = p.device, p.dtype
        dev = self.device
        self.caches, self.states = [], []
        for layer in model.layers:
            a = layer.attn
            self.caches.append((torch.zeros(batch, a.num_heads, capacity, a.r, device=dev, dtype=self.dtype),
                                torch.zeros(batch, a.num_heads, capacity, a.d_head, device=dev, dtype=self.dtype)))
            self.states.append(tuple(torch.zeros(batch, a.num_heads, a.j, a.d_head, device=dev, dtype=torch.float32)
                                     for _ in range(2)))
        self.pos = torch.zeros(1, dtype=torch.int64, device=dev)
        self.seq_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.col = torch.zeros(1, dtype=torch.int64, device=dev)
        self.tok = torch.zeros(batch, 1, dtype=torch.int64, device=dev)
        self.out = torch.zeros(batch, capacity, dtype=torch.int64, device=dev)  # generated tokens by column
        self.logits = None
        self.graphs = None
        self.stream = torch.cuda.Stream(device=dev)
        self.n_prompt = 0
        self.n_done = 0
        self.parity = 0  # which state buffer holds the current state

    # ------------------------------------------------------------------ prefill
    @torch.no_grad()
    def prefill(self, ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt ``ids [B, N]``; returns the logits of its last row
        ``[B, 1, vocab]`` and sets the first greedy token."""
        B, N = ids.shape
        if B != self.B or N + 1 > self.capacity:
            raise ValueError(f"prompt {tuple(ids.shape)} does not fit batch {self.B} / capacity {self.capacity}")
        m = self.model
        x = m.token_emb(ids)
        for i, layer in enumerate(m.layers):
            x, (k_c, v_c), (s, _) = layer(x, return_state=True)
            self.caches[i][0][:, :, :N].copy_(k_c)
            self.caches[i][1][:, :, :N].copy_(v_c)
            self.states[i][0].copy_(s)
            del k_c, v_c, s
        logits = m.lm_head(m.ln_f(x[:, -1:]))
        self.n_prompt = N
        self.n_done = 0
        self.parity = 0
        self.pos.fill_(N)
        self.seq_len.fill_(N + 1)
        self.col.zero_()
        self.tok.copy_(logits.argmax(-1))
        self.logits = torch.empty_like(logits)
        self.logits.copy_(logits)
        self.graphs = None
        return logits

    # ------------------------------------------------------------------ decode
    def _step(self, parity: int):
        """One greedy token; graph-capturable (no host reads, no allocation
        outside the capture pool)."""
        m = self.model
        x = m.token_emb(self.tok)
        for i, layer in enumerate(m.layers):
            s_in, s_out = self.states[i][parity], self.states[i][1 - parity]
            a = _attn_step(layer.attn, layer.ln_1(x), self.caches[i][0], self.caches[i][1], s_in, s_out,
                           self.pos, self.seq_len)
            x = x + a
            x = x + layer.mlp(layer.ln_2(x))
        logits = m.lm_head(m.ln_f(x))
        self.logits.copy_(logits)
        nxt = logits.argmax(-1)
        self.tok.copy_(nxt)
        self.out.index_copy_(1, self.col, nxt)
        self.pos.add_(1)
        self.seq_len.add_(1)
        self.col.add_(1)

    @torch.no_grad()
    def decode(self, steps: int, graphs: bool = True) -> torch.Tensor:
        """``steps`` greedy tokens (each one ``forward_step`` of the reference's
        loop, consuming the previous greedy token); returns them as
        ``[B, steps]``.  Before the graphs exist, one step runs eagerly on the
        decode stream (it sets up the kernel workspaces) and the graphs are
        captured after it; every later step is a graph replay."""
        if self.n_prompt == 0:
            raise RuntimeError("call prefill() first")
        if self.n_prompt + self.n_done + steps > self.capacity:
            raise ValueError(f"{self.n_prompt} + {self.n_done} + {steps} tokens exceed the cache capacity "
                             f"{self.capacity}")
        c0 = self.n_done
        self.n_done += steps
        s = self.stream
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            for _ in range(steps):
                if not graphs or self.graphs is None:
                    self._step(self.parity)
                    if graphs:
                        self._capture()
                else:
                    self.graphs[self.parity].replay()
                self.parity ^= 1
        torch.cuda.current_stream(self.device).wait_stream(s)
        return self.out[:, c0:c0 + steps]

    def _capture(self):
        """Graphs for both state parities, sharing one memory pool."""
        g0, g1 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
        with torch.cuda.graph(g0, stream=self.stream):
            self._step(0)
        with torch.cuda.graph(g1, stream=self.stream, pool=g0.pool()):
            self._step(1)
        self.graphs = (g0, g1)
