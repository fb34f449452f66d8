"""Training HOFA module: drop-in for ``src/HybridOutlierFactorizedAttentionTrain.py``.

Same constructor (including the normal init of the projections), parameter
names, ``forward(x)`` / ``forward_step(x, cache_O, state_I)`` signatures and
return values as the reference class (src/HybridOutlierFactorizedAttentionTrain.py:13-438),
plus ``TransformerBlock`` and ``SubwordLM`` with per-layer activation
checkpointing (:441-501).

* ``forward`` (hybrid path): projections, gates and RoPE are PyTorch ops; the
  attention core (outlier softmax attention, inlier GLA, RMSNorm * gla_scale,
  the mix blend) is one autograd function over the gfx950 kernels
  (``autograd.hofa_core``), replacing SDPA + fla ``chunk_gla`` + ``lerp``
  (:233-296).
* ``forward_step`` (hybrid path): the split-K decode kernel on the growing
  caches and on the reference's zero-padded ``[d_head, d_head]`` state
  (:382-438).
"""
from __future__ import annotations

import copy
import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .autograd import hofa_core
from .config import ModelConfig
from .hofa_decode import fused_hofa_decode
from .modules import RotaryEmbedding, apply_rotary_pos_emb


class HybridOutlierFactorizedAttention(nn.Module):
    def __init__(self, model_cfg: ModelConfig):
        super().__init__()
        self.d_model = model_cfg.d_model
        self.num_heads = model_cfg.num_heads
        self.d_head = model_cfg.d_head
        self.r = model_cfg.r
        self.j = self.d_head - self.r
        self.chunk_size = model_cfg.chunk_size

        self.gate_proj = nn.Linear(2 * self.d_head, self.num_heads, bias=True)
        self.gate_proj._is_gate = True
        nn.init.constant_(self.gate_proj.bias, -1.0)
        nn.init.zeros_(self.gate_proj.weight)

        self.W_q = nn.Linear(self.d_model, self.d_model, bias=False)
        self.W_k = nn.Linear(self.d_model, self.d_model, bias=False)
        self.W_v = nn.Linear(self.d_model, self.d_model, bias=False)
        self.out_proj = nn.Linear(self.d_model, self.d_model, bias=False)

        self.pure_mha_low_rank_k = getattr(model_cfg, "pure_mha_low_rank_k", False)
        self.forced_mha_heads = getattr(model_cfg, "mha_heads_for_width_split", 0)
        self.fixed_blend_weight = model_cfg.fixed_blend_weight
        self.attention_scale = model_cfg.attention_scale

        if not self.fixed_blend_weight and self.forced_mha_heads == 0:
            self.mix_proj = nn.Linear(2 * self.d_head, self.num_heads, bias=True)
            self.mix_proj._is_gate = True
            nn.init.zeros_(self.mix_proj.weight)
            nn.init.constant_(self.mix_proj.bias, model_cfg.mix_gate_bias_init)
        elif self.fixed_blend_weight and self.forced_mha_heads == 0:
            self.fixed_mix = nn.Parameter(torch.zeros(1, self.num_heads, 1, 1))

        self.learnable_alpha = model_cfg.learnable_alpha
        if self.learnable_alpha:
            n_decay = self.d_head if (self.forced_mha_heads > 0 or self.r == 0) else self.j
            self.log_alpha = nn.Parameter(torch.zeros(1, self.num_heads, 1, n_decay))
            self.log_alpha._is_alpha = True

        if (self.r > 0 or self.forced_mha_heads > 0) and model_cfg.use_rope:
            self.rotary_emb = RotaryEmbedding(dim=self.r if self.r > 0 else self.d_head, base=model_cfg.rope_base)

        self.inlier_norm = nn.RMSNorm(self.d_head, elementwise_affine=False)
        self.gla_scale = nn.Parameter(torch.ones(1, self.num_heads, 1, self.d_head))

        std = model_cfg.initializer_range
        res_std = std / math.sqrt(2 * model_cfg.num_layers) if model_cfg.scale_residual_proj else std
        nn.init.normal_(self.W_q.weight, std=std)
        nn.init.normal_(self.W_k.weight, std=std)
        nn.init.normal_(self.W_v.weight, std=std)
        nn.init.normal_(self.out_proj.weight, std=res_std)

    # ------------------------------------------------------------------ helpers
    def _gate_terms(self, Q, K, weight, bias):
        wq, wk = weight[:, :self.d_head], weight[:, self.d_head:]
        return (torch.einsum("bhnf,hf->bhn", Q, wq) + torch.einsum("bhnf,hf->bhn", K, wk)
                + bias.view(1, -1, 1).to(Q.dtype))

    def _compute_gates_optimized(self, Q, K):
        """``(gate_logits [B,H,N,1], mix_g [B,H,N,1] or None)`` (:85-113)."""
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

    def _merge(self, Y):
        B, H, N, d = Y.shape
        return self.out_proj(Y.transpose(1, 2).reshape(B, N, H * d))

    # ------------------------------------------------------------------ prefill
    def forward(self, x):
        B, N, D = x.shape
        Q, K, V = self._project(x)
        if self.forced_mha_heads > 0:
            return self._forward_width_split(Q, K, V)
        if self.pure_mha_low_rank_k or self.r == self.d_head:
            return self._forward_attention_only(Q, K, V)
        gate_logits, mix_g = self._compute_gates_optimized(Q, K)
        if not torch.compiler.is_compiling():
            # gate telemetry (written, never read by the reference's training); a
            # module attribute set inside a checkpointed block would break the
            # compiled graph, so traced runs leave it unchanged
            self.last_mix_g = mix_g.detach() if mix_g is not None else None
        log_gamma = F.logsigmoid(-gate_logits).squeeze(-1)
        log_alpha = self.log_alpha if self.learnable_alpha else None
        if self.r == 0:
            Y = hofa_core(None, None, Q, K, V, log_gamma, log_alpha, None, self.gla_scale, 0, 1.0)
            return self._merge(Y)
        Q_O = K_O = None  # without RoPE the outlier channels are Q[..., :r], K[..., :r] in place
        if getattr(self, "rotary_emb", None) is not None:
            cos, sin = self.rotary_emb(N)
            Q_O, K_O = apply_rotary_pos_emb(Q[..., :self.r], K[..., :self.r], cos, sin)
            # the float32 tables promote 16-bit Q/K; the reference's SDPA runs
            # them in the autocast dtype (that of V), and so does the core
            Q_O, K_O = Q_O.to(V.dtype), K_O.to(V.dtype)
        sm_scale = ((self.d_head / self.r) ** 0.5) * self.attention_scale
        Y = hofa_core(Q_O, K_O, Q, K, V, log_gamma, log_alpha, mix_g.squeeze(-1), self.gla_scale, self.r, sm_scale)
        return self._merge(Y)

    def _forward_width_split(self, Q, K, V):
        """Width-split ablation (:139-175): the first ``mha_heads_for_width_split``
        heads run causal softmax attention over the full head (RoPE'd, scale
        ``attention_scale``, PyTorch SDPA as in the reference), the rest the
        normalized GLA over all ``d_head`` channels (the ``r = 0`` core on the
        HIP kernels) with their rows of ``gate_proj`` and ``gla_scale``.  With
        ``learnable_alpha`` the GLA heads take their own rows of ``log_alpha``
        (the reference multiplies the GLA heads' decay by all heads' alphas,
        which only broadcasts when no head is split off)."""
        B, H, N, d = Q.shape
        m = self.forced_mha_heads
        Q_mha, Q_gla = Q[:, :m], Q[:, m:]
        K_mha, K_gla = K[:, :m], K[:, m:]
        V_mha, V_gla = V[:, :m], V[:, m:]
        if getattr(self, "rotary_emb", None) is not None:
            cos, sin = self.rotary_emb(N)
            Q_mha, K_mha = apply_rotary_pos_emb(Q_mha, K_mha, cos, sin)
        Y_mha = F.scaled_dot_product_attention(Q_mha.to(V.dtype), K_mha.to(V.dtype), V_mha, is_causal=True,
                                               scale=self.attention_scale)
        W_g = self.gate_proj.weight
        gate_logits = self._gate_terms(Q_gla, K_gla, W_g[m:], self.gate_proj.bias[m:])
        log_gamma = F.logsigmoid(-gate_logits)
        log_alpha = self.log_alpha[:, m:] if self.learnable_alpha else None
        Y_gla = hofa_core(None, None, Q_gla, K_gla, V_gla, log_gamma, log_alpha, None, self.gla_scale[:, m:], 0, 1.0)
        return self._merge(torch.cat([Y_mha.to(Y_gla.dtype), Y_gla], dim=1))

    def _forward_attention_only(self, Q, K, V):
        """Ablations without the hybrid blend (:176-231): reduced-QK MHA and
        r == d_head.  PyTorch SDPA as in the reference."""
        B, H, N, d = Q.shape
        if self.pure_mha_low_rank_k:
            Q, K = Q[..., :self.r], K[..., :self.r]
            scale = ((self.d_head / self.r) ** 0.5) * self.attention_scale
        else:
            scale = self.attention_scale
        if getattr(self, "rotary_emb", None) is not None:
            cos, sin = self.rotary_emb(N)
            Q, K = apply_rotary_pos_emb(Q, K, cos, sin)
        Y = F.scaled_dot_product_attention(Q, K, V, is_causal=True, scale=scale)
        return self._merge(Y)

    # ------------------------------------------------------------------ decode
    def forward_step(self, x, cache_O=None, state_I=None):
        """Single-step decoding on growing caches and the zero-padded
        ``[B, H, d_head, d_head]`` float32 state (:298-438)."""
        B, N, D = x.shape
        assert N == 1, "forward_step expects a single token (N=1)"
        Q, K, V = self._project(x)
        if self.pure_mha_low_rank_k or self.r == 0 or self.r == self.d_head or self.forced_mha_heads > 0:
            return self._step_reference_ops(Q, K, V, cache_O, state_I)
        gate_logits, mix_g = self._compute_gates_optimized(Q, K)
        curr_len = 1 if cache_O is None else cache_O[0].shape[2] + 1
        Q_O, K_O = Q[..., :self.r], K[..., :self.r]
        if getattr(self, "rotary_emb", None) is not None:
            cos, sin = self.rotary_emb(curr_len)
            Q_O, K_O = apply_rotary_pos_emb(Q_O, K_O, cos[-1:], sin[-1:])
        if cache_O is None:
            cache_O = (K_O.contiguous(), V.contiguous())
        else:
            cache_O = (torch.cat([cache_O[0], K_O], dim=2), torch.cat([cache_O[1], V], dim=2))
        if state_I is None:
            state_I = torch.zeros(B, self.num_heads, self.d_head, self.d_head, device=x.device, dtype=torch.float32)
        state_new = torch.zeros_like(state_I)
        q = torch.cat([Q_O, Q[..., self.r:]], dim=-1)
        k = torch.cat([K_O, K[..., self.r:]], dim=-1)
        Y = fused_hofa_decode(q, k, V, cache_O[0], cache_O[1], state_I[:, :, :self.j, :], state_new[:, :, :self.j, :],
                              F.logsigmoid(-gate_logits).squeeze(-1), mix_g.squeeze(-1),
                              self.gla_scale.view(self.num_heads, self.d_head), self.r, cache_O[0].shape[2],
                              (self.d_head / self.r) ** 0.5,
                              log_alpha=self.log_alpha if self.learnable_alpha else None)
        return self._merge(Y), cache_O, state_new

    def _step_reference_ops(self, Q, K, V, cache_O, state_I):
        """The non-hybrid decode paths (:309-380) in PyTorch ops, as in the reference."""
        B, H, _, d = Q.shape
        if self.r == 0:
            gate_logits, _ = self._compute_gates_optimized(Q, K)
            log_gamma = F.logsigmoid(-gate_logits)
            if self.learnable_alpha:
                gamma = torch.exp(log_gamma * self.log_alpha.exp().transpose(-1, -2)).to(torch.float32)
            else:
                gamma = torch.exp(log_gamma).to(torch.float32)
            if state_I is None:
                state_I = torch.zeros(B, H, d, d, device=Q.device, dtype=torch.float32)
            S = gamma * state_I + K.squeeze(2).float().unsqueeze(-1) @ V.squeeze(2).float().unsqueeze(-2)
            Y = (Q.squeeze(2).float().unsqueeze(-2) @ S).squeeze(-2).unsqueeze(2)
            Y = (self.inlier_norm(Y.float()) * self.gla_scale).to(Q.dtype)
            return self._merge(Y), None, S
        if self.forced_mha_heads > 0:
            # the reference's forward_step has no width-split branch either
            raise NotImplementedError("forward_step does not support the width-split ablation")
        if self.pure_mha_low_rank_k:
            Qr, Kr = Q[..., :self.r], K[..., :self.r]
            scale = ((self.d_head / self.r) ** 0.5) * self.attention_scale
        else:
            Qr, Kr, scale = Q, K, 1.0
        curr_len = 1 if cache_O is None else cache_O[0].shape[2] + 1
        if getattr(self, "rotary_emb", None) is not None:
            cos, sin = self.rotary_emb(curr_len)
            Qr, Kr = apply_rotary_pos_emb(Qr, Kr, cos[-1:], sin[-1:])
        if cache_O is None:
            K_past, V_past = Kr, V
        else:
            K_past, V_past = torch.cat([cache_O[0], Kr], dim=2), torch.cat([cache_O[1], V], dim=2)
        Y = F.scaled_dot_product_attention(Qr, K_past, V_past, is_causal=False, scale=scale)
        return self._merge(Y), (K_past, V_past), None


class TransformerBlock(nn.Module):
    def __init__(self, model_cfg: ModelConfig):
        super().__init__()
        self.ln_1 = nn.LayerNorm(model_cfg.d_model)
        self.attn = HybridOutlierFactorizedAttention(model_cfg)
        self.ln_2 = nn.LayerNorm(model_cfg.d_model)
        self.mlp = nn.Sequential(nn.Linear(model_cfg.d_model, 4 * model_cfg.d_model), nn.GELU(),
                                 nn.Linear(4 * model_cfg.d_model, model_cfg.d_model))
        std = 0.02
        res_std = std / math.sqrt(2 * model_cfg.num_layers)
        nn.init.normal_(self.mlp[0].weight, std=std)
        nn.init.zeros_(self.mlp[0].bias)
        nn.init.normal_(self.mlp[2].weight, std=res_std)
        nn.init.zeros_(self.mlp[2].bias)

    def forward(self, x):
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))


class SubwordLM(nn.Module):
    def __init__(self, vocab_size: int, model_cfg: ModelConfig):
        super().__init__()
        self.config = model_cfg
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
        nn.init.normal_(self.lm_head.weight, std=0.02)
        self.token_emb.weight = self.lm_head.weight

    def forward(self, x, targets=None):
        x = self.token_emb(x)
        for layer in self.layers:
            x = torch.utils.checkpoint.checkpoint(layer, x, use_reentrant=False)
        logits = self.lm_head(self.ln_f(x))
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1))
        return logits, loss
