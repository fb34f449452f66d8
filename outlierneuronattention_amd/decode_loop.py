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

For 16-bit models (bf16/f16, batch <= 4, d_model <= 1024) the step is the
fused one (``fused=True``, the default there): per layer a LayerNorm+QKV
row-linear, the gate/RoPE/cache-append prologue, the split-K decode, the
out-projection with its residual, LayerNorm+fc1+GELU and fc2 with its
residual (``decode_layer``), then LayerNorm+LM head with a device argmax and
one kernel that feeds the token back -- about seven launches per layer.
``fused=False`` keeps the module's own torch ops around the decode kernel.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F

from . import _lib
from .decode_layer import argmax_slots, decode_advance, decode_prologue, prologue_args, rows_linear
from .HybridOutlierFactorizedAttention import SubwordLM
from .hofa_decode import decode_args, fused_hofa_decode
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

    def __init__(self, model: SubwordLM, batch: int, capacity: int, fused: bool | None = None,
                 prologue_in_decode: bool = True):
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
        d = model.ln_f.normalized_shape[0]
        can_fuse = self.dtype in (torch.bfloat16, torch.float16) and batch <= 4 and 4 * d <= 4096
        if fused and not can_fuse:
            raise NotImplementedError("the fused decode step needs bf16/f16 weights, batch <= 4 and d_model <= 1024")
        self.fused = can_fuse if fused is None else bool(fused)
        # fused step: gates/RoPE/cache append inside the decode launch (hofa_decode_fused), or as
        # a launch of their own before it (hofa_decode_prologue + hofa_decode)
        self.prologue_in_decode = bool(prologue_in_decode)
        if self.fused:
            self._init_fused(d)

    def _init_fused(self, d: int):
        """Buffers of the fused step and a concatenated [3d, d] Q|K|V weight per layer."""
        dev, dt, B = self.device, self.dtype, self.B
        m = self.model
        self.w_qkv = [torch.cat([layer.attn.W_q.weight, layer.attn.W_k.weight, layer.attn.W_v.weight]).contiguous()
                      for layer in m.layers]
        H = m.layers[0].attn.num_heads
        self.x = torch.zeros(B, d, device=dev, dtype=dt)          # residual stream of the current token
        self.qkv = torch.zeros(B, 3 * d, device=dev, dtype=dt)
        self.y_attn = torch.zeros(B, H, 1, d // H, device=dev, dtype=dt)
        self.h_mlp = torch.zeros(B, 4 * d, device=dev, dtype=dt)
        self.lg = torch.zeros(B, H, device=dev, dtype=torch.float32)
        self.mix = torch.zeros(B, H, device=dev, dtype=torch.float32)
        V = m.lm_head.weight.shape[0]
        self.keys = torch.zeros(B * argmax_slots(V), dtype=torch.int64, device=dev)  # per-block greedy keys
        self.ws = None

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
        if self.fused:
            self.x.copy_(m.token_emb(self.tok)[:, 0])
        self.graphs = None
        return logits

    # ------------------------------------------------------------------ decode
    def _step(self, parity: int):
        """One greedy token; graph-capturable (no host reads, no allocation
        outside the capture pool)."""
        if self.fused:
            return self._step_fused(parity)
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

    def _step_fused(self, parity: int):
        """The fused greedy step: seven launches per layer, then the LM head
        with argmax and the feedback kernel; allocates nothing.  With
        prologue_in_decode the gates/RoPE/cache append run inside the decode
        launch (six launches per layer)."""
        m, B = self.model, self.B
        x = self.x
        for i, layer in enumerate(m.layers):
            a = layer.attn
            H, D = a.num_heads, a.d_head
            HD = H * D
            rows_linear(x, self.w_qkv[i], self.qkv, ln=(layer.ln_1.weight, layer.ln_1.bias, layer.ln_1.eps),
                        scale=1.0 / D ** 0.25, scale_cols=2 * HD)
            ck, cv = self.caches[i]
            if not self.prologue_in_decode:
                decode_prologue(a, self.qkv, ck, cv, self.pos, self.lg, self.mix)
            q = self.qkv[:, :HD].view(B, H, 1, D)
            k = self.qkv[:, HD:2 * HD].view(B, H, 1, D)
            v = self.qkv[:, 2 * HD:].view(B, H, 1, D)
            s_in, s_out = self.states[i][parity], self.states[i][1 - parity]
            args, _, keep = decode_args(q, k, v, ck, cv, s_in, s_out, self.lg, self.mix, a.gla_scale.view(H, D),
                                        a.r, ck.shape[2], (D / a.r) ** 0.5,
                                        log_alpha=a.log_alpha if a.learnable_alpha else None,
                                        seq_len_dev=self.seq_len, y=self.y_attn)
            lib = _lib.load()
            pro = prologue_args(a, self.qkv, ck, cv, self.pos, self.lg, self.mix) if self.prologue_in_decode else None
            nbytes = (lib.hofa_decode_fused_workspace_bytes if pro is not None
                      else lib.hofa_decode_workspace_bytes)(ctypes.byref(args))
            if nbytes == 0:
                _lib.check(-1, "decode step")
            if self.ws is None or self.ws.numel() < nbytes:
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError("decode workspace must be sized before graph capture")
                self.ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            stream = _lib.stream_handle(self.device)
            if pro is not None:
                rc = lib.hofa_decode_fused(ctypes.byref(args), ctypes.byref(pro), self.ws.data_ptr(), self.ws.numel(),
                                           stream)
            else:
                rc = lib.hofa_decode(ctypes.byref(args), self.ws.data_ptr(), self.ws.numel(), stream)
            _lib.check(rc, "decode step")
            del keep
            rows_linear(self.y_attn.view(B, HD), a.out_proj.weight, x, res=x)
            fc1, fc2 = layer.mlp[0], layer.mlp[2]
            rows_linear(x, fc1.weight, self.h_mlp, bias=fc1.bias, ln=(layer.ln_2.weight, layer.ln_2.bias,
                                                                      layer.ln_2.eps), gelu=True)
            rows_linear(self.h_mlp, fc2.weight, x, bias=fc2.bias, res=x)
        rows_linear(x, m.lm_head.weight, self.logits[:, 0], ln=(m.ln_f.weight, m.ln_f.bias, m.ln_f.eps),
                    argmax=self.keys)
        decode_advance(self.keys, m.lm_head.weight, x, self.tok, self.out, self.col, self.pos, self.seq_len)

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
