"""Inference HOFA module: drop-in for ``src/HybridOutlierFactorizedAttention.py``.

Same constructor, parameter names and shapes, ``forward`` / ``forward_step``
signatures, return values and cache / state layout as the reference class
(src/HybridOutlierFactorizedAttention.py:11-422), plus ``TransformerBlock`` and
``SubwordLM`` (:425-513).  The hybrid path (0 < r < d_head) runs on the gfx950
kernels of this package:

* prefill: ``chunk_gla_inlier_fwd`` computes ``(1 - mix) * gla_scale *
  RMSNorm(GLA)`` and ``exact_attention`` adds ``mix * softmax-attention``
  (the reference's two-kernel order, :201-208), the GLA part passed on in
  float32 so the output is rounded once (``prefill.prefill_fwd``);
* decode: ``fused_hofa_decode`` (split-K cache streaming + state update).

Projections, gate einsums and RoPE are PyTorch GEMM/elementwise work as in
the reference.  The special cases r == 0, r == d_head and the width-split
ablation keep the reference's arithmetic; where the attention kernel covers
them (head dim 64/128, QK width 16/32/64) it is used, otherwise PyTorch SDPA
as in the reference.
"""
from __future__ import annotations

import copy
import warnings

import torch
import torch.nn as nn
import torch.nn.functional as F

from .chunk_gla_inlier import chunk_gla_inlier_fwd
from .config import ModelConfig
from .exact_attention import exact_attention
from .hofa_decode import fused_hofa_decode
from .modules import RotaryEmbedding, apply_rotary_pos_emb
from .prefill import prefill_fwd

_ATTN_WIDTHS = (16, 32, 64)
# RMSNorm epsilon of the inlier norm in prefill and decode alike: the one of
# nn.RMSNorm on float32 (src/HybridOutlierFactorizedAttention.py:64) and of the
# decode kernel (src/hofa_decode_triton.py:386).  The reference's prefill
# kernel hard-codes 1e-5 instead (src/chunk_gla_inlier.py:234), which makes
# its prefill and decode disagree for rows of small variance.
_NORM_EPS = float(torch.finfo(torch.float32).eps)


def _causal_attention(q, k, v, scale):
    """Full-width causal softmax attention (pure-MHA paths): the HIP kernel when
    its shapes are supported, else SDPA exactly as the reference calls it."""
    d = q.shape[-1]
    if q.is_cuda and d in (64, 128) and d in _ATTN_WIDTHS:
        return exact_attention(q, k, v, d, scale, None)
    return F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)


class HybridOutlierFactorizedAttention(nn.Module):
    def __init__(self, model_cfg: ModelConfig):
        super().__init__()
        self.d_model = model_cfg.d_model
        self.num_heads = model_cfg.num_heads
        self.d_head = model_cfg.d_head
        self.r = model_cfg.r
        self.j = self.d_head - self.r
        self.chunk_size = model_cfg.chunk_size
        if self.r > 0 and (self.r & (self.r - 1)) != 0:
            warnings.warn(f"HOFA: r={self.r} is not a power of 2; the kernels support r in {_ATTN_WIDTHS}.")

        # gate from the full (pre-routing) Q and K: W=0, b=-1 (:26-29)
        self.gate_proj = nn.Linear(2 * self.d_head, self.num_heads, bias=True)
        nn.init.constant_(self.gate_proj.bias, -1.0)
        nn.init.zeros_(self.gate_proj.weight)

        self.forced_mha_heads = getattr(model_cfg, "mha_heads_for_width_split", 0)
        self.fixed_blend_weight = getattr(model_cfg, "fixed_blend_weight", False)
        if not self.fixed_blend_weight and self.forced_mha_heads == 0:
            self.mix_proj = nn.Linear(2 * self.d_head, self.num_heads, bias=True)
            nn.init.zeros_(self.mix_proj.weight)
            nn.init.constant_(self.mix_proj.bias, model_cfg.mix_gate_bias_init)
        elif self.fixed_blend_weight and self.forced_mha_heads == 0:
            self.fixed_mix = nn.Parameter(torch.zeros(1, self.num_heads, 1, 1))

        self.learnable_alpha = getattr(model_cfg, "learnable_alpha", False)
        if self.learnable_alpha:
            n_decay = self.d_head if (self.forced_mha_heads > 0 or self.r == 0) else self.j
            self.log_alpha = nn.Parameter(torch.zeros(1, self.num_heads, 1, n_decay))
            self.log_alpha._is_alpha = True

        self.W_q = nn.Linear(self.d_model, self.d_model, bias=False)
        self.W_k = nn.Linear(self.d_model, self.d_model, bias=False)
        self.W_v = nn.Linear(self.d_model, self.d_model, bias=False)
        self.out_proj = nn.Linear(self.d_model, self.d_model, bias=False)

        if (self.r > 0 or self.forced_mha_heads > 0) and model_cfg.use_rope:
            self.rotary_emb = RotaryEmbedding(dim=self.r if self.r > 0 else self.d_head, base=model_cfg.rope_base)

        self.inlier_norm = nn.RMSNorm(self.d_head, elementwise_affine=False)
        self.gla_scale = nn.Parameter(torch.ones(1, self.num_heads, 1, self.d_head))

    # ------------------------------------------------------------------ helpers
    def _gate_terms(self, Q, K, weight, bias):
        wq, wk = weight[:, :self.d_head], weight[:, self.d_head:]
        return (torch.einsum("bhnf,hf->bhn", Q, wq) + torch.einsum("bhnf,hf->bhn", K, wk)
                + bias.view(1, -1, 1).to(Q.dtype))

    def _compute_gates_optimized(self, Q, K):
        """``(gate_logits [B,H,N,1], mix_g [B,H,N,1] or None)`` (:67-95)."""
        gate_logits = self._gate_terms(Q, K, self.gate_proj.weight, self.gate_proj.bias)
        if hasattr(self, "mix_proj"):
            mix_g = torch.sigmoid(self._gate_terms(Q, K, self.mix_proj.weight, self.mix_proj.bias)).to(Q.dtype)
            mix_g = mix_g.unsqueeze(-1)
        elif hasattr(self, "fixed_mix"):
            mix_g = torch.sigmoid(self.fixed_mix).to(Q.dtype).expand(Q.shape[0], -1, Q.shape[2], -1)
        else:
            mix_g = None
        return gate_logits.unsqueeze(-1), mix_g

    def _project(self, x):
        B, N, _ = x.shape
        s = self.d_head ** 0.25
        Q = (self.W_q(x) / s).view(B, N, self.num_heads, self.d_head).transpose(1, 2)
        K = (self.W_k(x) / s).view(B, N, self.num_heads, self.d_head).transpose(1, 2)
        V = self.W_v(x).view(B, N, self.num_heads, self.d_head).transpose(1, 2)
        return Q, K, V

    def _merge(self, Y, dtype_in):
        B, H, N, d = Y.shape
        return self.out_proj(Y.transpose(1, 2).reshape(B, N, H * d)).to(dtype_in)

    def _norm_scale(self, Y, gla_scale):
        return (self.inlier_norm(Y.float()) * gla_scale).to(Y.dtype)

    # ------------------------------------------------------------------ prefill
    def forward(self, x, return_state=False):
        B, N, D = x.shape
        dtype_in = x.dtype
        Q, K, V = self._project(x)

        if self.forced_mha_heads > 0:
            return self._forward_width_split(Q, K, V, dtype_in, return_state)
        if self.r == 0:
            gate_logits, _ = self._compute_gates_optimized(Q, K)
            log_gamma = F.logsigmoid(-gate_logits).squeeze(-1)
            Y_I, states_out = chunk_gla_inlier_fwd(Q, K, V, log_gamma, 0, self.chunk_size)
            Y_out = self._merge(self._norm_scale(Y_I, self.gla_scale), dtype_in)
            if return_state:
                state_I = states_out[:, :, :self.j, :self.d_head]
                return Y_out, None, (state_I, torch.empty_like(state_I))
            return Y_out
        if self.r == self.d_head:
            if hasattr(self, "rotary_emb"):
                cos, sin = self.rotary_emb(N)
                Q, K = apply_rotary_pos_emb(Q, K, cos, sin)
            Y_out = self._merge(_causal_attention(Q, K, V, 1.0), dtype_in)
            if return_state:
                return Y_out, (K.contiguous(), V.contiguous()), None
            return Y_out

        gate_logits, mix_g = self._compute_gates_optimized(Q, K)
        log_gamma = F.logsigmoid(-gate_logits).squeeze(-1)
        if hasattr(self, "rotary_emb"):
            cos, sin = self.rotary_emb(N)
            Q_O, K_O = apply_rotary_pos_emb(Q[..., :self.r], K[..., :self.r], cos, sin)
            Q[..., :self.r] = Q_O
            K[..., :self.r] = K_O
        if return_state:
            K_cache = K[..., :self.r].contiguous()
            V_cache = V.contiguous()
        log_alpha = self.log_alpha if self.learnable_alpha else None
        sm_scale = (self.d_head / self.r) ** 0.5
        Y, states_out = prefill_fwd(Q, K, V, log_gamma, self.r, sm_scale, mix_g.squeeze(-1), self.gla_scale,
                                    log_alpha=log_alpha, eps=_NORM_EPS)
        Y_out = self._merge(Y, dtype_in)
        if return_state:
            state_I = states_out[:, :, :self.j, :self.d_head].contiguous()
            return Y_out, (K_cache, V_cache), (state_I, torch.empty_like(state_I))
        return Y_out

    def _forward_width_split(self, Q, K, V, dtype_in, return_state):
        """Width-split ablation (:106-143): full-width MHA heads + pure-GLA heads."""
        B, H, N, d = Q.shape
        m = self.forced_mha_heads
        Q_mha, Q_gla = Q.split([m, H - m], dim=1)
        K_mha, K_gla = K.split([m, H - m], dim=1)
        V_mha, V_gla = V.split([m, H - m], dim=1)
        if hasattr(self, "rotary_emb"):
            cos, sin = self.rotary_emb(N)
            Q_mha, K_mha = apply_rotary_pos_emb(Q_mha, K_mha, cos, sin)
        Y_mha = _causal_attention(Q_mha, K_mha, V_mha, 1.0)
        wq, wk = self.gate_proj.weight[:, :d][m:], self.gate_proj.weight[:, d:][m:]
        gate_logits = (torch.einsum("bhnf,hf->bhn", Q_gla, wq) + torch.einsum("bhnf,hf->bhn", K_gla, wk)
                       + self.gate_proj.bias[m:].view(1, -1, 1).to(dtype_in))
        log_gamma = F.logsigmoid(-gate_logits)
        Y_gla, states_out = chunk_gla_inlier_fwd(Q_gla, K_gla, V_gla, log_gamma, 0, self.chunk_size)
        Y_gla = self._norm_scale(Y_gla, self.gla_scale[:, m:])
        Y_out = self._merge(torch.cat([Y_mha.to(Y_gla.dtype), Y_gla], dim=1), dtype_in)
        if return_state:
            state_I = states_out[:, :, :d, :d]
            return Y_out, (K_mha.contiguous(), V_mha.contiguous()), (state_I, torch.empty_like(state_I))
        return Y_out

    # ------------------------------------------------------------------ decode
    def forward_step(self, x, cache_O=None, state_I=None, cache_seq_len=None):
        """Single-step autoregressive decoding (:223-422)."""
        B, N, D = x.shape
        assert N == 1, "forward_step expects a single token (N=1)"
        dtype_in = x.dtype
        Q, K, V = self._project(x)

        if self.forced_mha_heads > 0:
            return self._step_width_split(Q, K, V, dtype_in, cache_O, state_I, cache_seq_len)
        if self.r == 0:
            return self._step_pure_gla(Q, K, V, dtype_in, state_I)
        if self.r == self.d_head:
            return self._step_pure_mha(Q, K, V, dtype_in, cache_O, cache_seq_len)

        gate_logits, mix_g = self._compute_gates_optimized(Q, K)
        log_gamma = F.logsigmoid(-gate_logits).squeeze(-1)
        if mix_g is not None:
            mix_g = mix_g.squeeze(-1)
        if hasattr(self, "rotary_emb"):
            pos = cache_seq_len if cache_seq_len is not None else (cache_O[0].shape[2] if cache_O is not None else 0)
            cos, sin = self.rotary_emb(pos + 1)
            Q_O, K_O = apply_rotary_pos_emb(Q[..., :self.r], K[..., :self.r], cos[-1:], sin[-1:])
            Q[..., :self.r] = Q_O
            K[..., :self.r] = K_O

        # append the token to the outlier cache (:377-392)
        if cache_O is None:
            cache_O_new = (K[..., :self.r], V)
            cache_seq_len = 0
        elif cache_seq_len is not None and cache_O[0].shape[2] > cache_seq_len:
            cache_O[0][:, :, cache_seq_len:cache_seq_len + 1, :] = K[..., :self.r]
            cache_O[1][:, :, cache_seq_len:cache_seq_len + 1, :] = V
            cache_O_new = cache_O
        else:
            cache_O_new = (torch.cat([cache_O[0], K[..., :self.r]], dim=2), torch.cat([cache_O[1], V], dim=2))
            cache_seq_len = cache_O_new[0].shape[2] - 1

        if state_I is None:
            z = torch.zeros(B, self.num_heads, self.j, self.d_head, device=x.device, dtype=torch.float32)
            state_I = (z, torch.empty_like(z))
        state_in, state_out = state_I
        assert state_in.dtype == torch.float32, f"Expected state_in to be float32, got {state_in.dtype}"
        assert state_in.is_contiguous(), "Expected state_in to be contiguous"

        Y = fused_hofa_decode(Q, K, V, cache_O_new[0], cache_O_new[1], state_in, state_out, log_gamma, mix_g,
                              self.gla_scale.view(self.num_heads, self.d_head), self.r, cache_seq_len + 1,
                              (self.d_head / self.r) ** 0.5,
                              log_alpha=self.log_alpha if self.learnable_alpha else None)
        return self._merge(Y, dtype_in), cache_O_new, (state_out, state_in)

    def _step_pure_gla(self, Q, K, V, dtype_in, state_I):
        """r == 0 (:298-331): decayed outer-product recurrence, update before read."""
        B, H, _, d = Q.shape
        gate_logits, _ = self._compute_gates_optimized(Q, K)
        log_gamma = F.logsigmoid(-gate_logits)
        if self.learnable_alpha:
            gamma = torch.exp(log_gamma * self.log_alpha.exp()).view(B, H, self.j, 1)
        else:
            gamma = torch.sigmoid(-gate_logits).view(B, H, 1, 1).expand(B, H, self.j, 1)
        if isinstance(state_I, tuple):
            state_I = state_I[0]
        if state_I is None:
            state_I = torch.zeros(B, H, self.j, d, device=Q.device, dtype=torch.float32)
        S = torch.baddbmm(state_I.reshape(B * H, self.j, d) * gamma.reshape(B * H, self.j, 1),
                          K.reshape(B * H, self.j, 1), V.reshape(B * H, 1, d))
        Y = torch.bmm(Q.reshape(B * H, 1, self.j), S).reshape(B, H, 1, d)
        S = S.reshape(B, H, self.j, d)
        return self._merge(self._norm_scale(Y, self.gla_scale), dtype_in), None, (S, torch.empty_like(S))

    def _append(self, cache_O, k_new, v_new, cache_seq_len):
        if cache_O is None:
            return (k_new, v_new), k_new, v_new
        if cache_seq_len is not None and cache_O[0].shape[2] > cache_seq_len:
            cache_O[0][:, :, cache_seq_len:cache_seq_len + 1, :] = k_new
            cache_O[1][:, :, cache_seq_len:cache_seq_len + 1, :] = v_new
            return cache_O, cache_O[0][:, :, :cache_seq_len + 1], cache_O[1][:, :, :cache_seq_len + 1]
        k_all, v_all = torch.cat([cache_O[0], k_new], dim=2), torch.cat([cache_O[1], v_new], dim=2)
        return (k_all, v_all), k_all, v_all

    def _step_pure_mha(self, Q, K, V, dtype_in, cache_O, cache_seq_len):
        """r == d_head (:333-356)."""
        if hasattr(self, "rotary_emb"):
            pos = cache_seq_len if cache_seq_len is not None else (cache_O[0].shape[2] if cache_O is not None else 0)
            cos, sin = self.rotary_emb(pos + 1)
            Q, K = apply_rotary_pos_emb(Q, K, cos[-1:], sin[-1:])
        cache_new, K_past, V_past = self._append(cache_O, K, V, cache_seq_len)
        Y = F.scaled_dot_product_attention(Q, K_past, V_past, is_causal=False, scale=1.0)
        return self._merge(Y, dtype_in), cache_new, None

    def _step_width_split(self, Q, K, V, dtype_in, cache_O, state_I, cache_seq_len):
        """Width-split ablation decode (:234-296)."""
        B, H, _, d = Q.shape
        m = self.forced_mha_heads
        Q_mha, Q_gla = Q.split([m, H - m], dim=1)
        K_mha, K_gla = K.split([m, H - m], dim=1)
        V_mha, V_gla = V.split([m, H - m], dim=1)
        if hasattr(self, "rotary_emb"):
            pos = cache_seq_len if cache_seq_len is not None else (cache_O[0].shape[2] if cache_O is not None else 0)
            cos, sin = self.rotary_emb(pos + 1)
            Q_mha, K_mha = apply_rotary_pos_emb(Q_mha, K_mha, cos[-1:], sin[-1:])
        cache_new, K_past, V_past = self._append(cache_O, K_mha, V_mha, cache_seq_len)
        Y_mha = F.scaled_dot_product_attention(Q_mha, K_past, V_past, is_causal=False, scale=1.0)
        wq, wk = self.gate_proj.weight[:, :d][m:], self.gate_proj.weight[:, d:][m:]
        gate_logits = (torch.einsum("bhnf,hf->bhn", Q_gla, wq) + torch.einsum("bhnf,hf->bhn", K_gla, wk)
                       + self.gate_proj.bias[m:].view(1, -1, 1).to(dtype_in))
        Hg = H - m
        gamma = torch.sigmoid(-gate_logits).reshape(B * Hg, 1, 1)
        S = state_I[0] if state_I is not None else torch.zeros(B, Hg, d, d, device=Q.device, dtype=torch.float32)
        S = torch.baddbmm(S.reshape(B * Hg, d, d) * gamma, K_gla.float().reshape(B * Hg, d, 1),
                          V_gla.float().reshape(B * Hg, 1, d))
        Y_gla = torch.bmm(Q_gla.float().reshape(B * Hg, 1, d), S).reshape(B, Hg, 1, d)
        Y_gla = (self.inlier_norm(Y_gla) * self.gla_scale[:, m:]).to(dtype_in)
        S = S.reshape(B, Hg, d, d)
        Y_out = self._merge(torch.cat([Y_mha.to(Y_gla.dtype), Y_gla], dim=1), dtype_in)
        return Y_out, cache_new, (S, torch.empty_like(S))


class TransformerBlock(nn.Module):
    """Pre-LN block: ``x + attn(LN(x))``, ``x + MLP(LN(x))`` with a 4x GELU MLP (:425-451)."""

    def __init__(self, model_cfg: ModelConfig):
        super().__init__()
        self.ln_1 = nn.LayerNorm(model_cfg.d_model)
        self.attn = HybridOutlierFactorizedAttention(model_cfg)
        self.ln_2 = nn.LayerNorm(model_cfg.d_model)
        self.mlp = nn.Sequential(nn.Linear(model_cfg.d_model, 4 * model_cfg.d_model), nn.GELU(),
                                 nn.Linear(4 * model_cfg.d_model, model_cfg.d_model))

    def forward(self, x, return_state=False):
        if return_state:
            a, cache_O, state_I = self.attn(self.ln_1(x), return_state=True)
            x = x + a
            return x + self.mlp(self.ln_2(x)), cache_O, state_I
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))

    def forward_step(self, x, cache_O=None, state_I=None, cache_seq_len=None):
        a, cache_O, state_I = self.attn.forward_step(self.ln_1(x), cache_O, state_I, cache_seq_len)
        x = x + a
        return x + self.mlp(self.ln_2(x)), cache_O, state_I


class SubwordLM(nn.Module):
    """Token embedding tied to the LM head, a stack of blocks with per-layer r (:454-513)."""

    def __init__(self, vocab_size: int, model_cfg: ModelConfig):
        super().__init__()
        self.token_emb = nn.Embedding(vocab_size, model_cfg.d_model)
        r_list = model_cfg.r if isinstance(model_cfg.r, (list, tuple)) else [model_cfg.r] * model_cfg.num_layers
        assert len(r_list) == model_cfg.num_layers, \
            f"Length of r ({len(r_list)}) must match num_layers ({model_cfg.num_layers})"
        self.layers = nn.ModuleList()
        for r in r_list:
            cfg = copy.copy(model_cfg)
            cfg.r = r
            self.layers.append(TransformerBlock(cfg))
        self.ln_f = nn.LayerNorm(model_cfg.d_model)
        self.lm_head = nn.Linear(model_cfg.d_model, vocab_size, bias=False)
        self.token_emb.weight = self.lm_head.weight

    def forward(self, x, targets=None, return_state=False):
        x = self.token_emb(x)
        if return_state:
            caches, states = [], []
            for layer in self.layers:
                x, c, s = layer(x, return_state=True)
                caches.append(c)
                states.append(s)
            return self.lm_head(self.ln_f(x)), caches, states
        for layer in self.layers:
            x = layer(x)
        logits = self.lm_head(self.ln_f(x))
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1))
        return logits, loss

    def forward_step(self, x, cache_O_list=None, state_I_list=None, cache_seq_len=None):
        x = self.token_emb(x)
        caches, states = [], []
        for i, layer in enumerate(self.layers):
            c = cache_O_list[i] if cache_O_list is not None else None
            s = state_I_list[i] if state_I_list is not None else None
            x, c, s = layer.forward_step(x, c, s, cache_seq_len)
            caches.append(c)
            states.append(s)
        return self.lm_head(self.ln_f(x)), caches, states
