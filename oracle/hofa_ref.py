"""CPU restatement of the reference HOFA hybrid-attention path (the oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product package.

Everything here is plain PyTorch on the CPU and works in float32 or float64.
Each function cites the reference lines it restates (paths relative to the
reference repository root).  How each function is pinned (golden vectors
written by the reference itself, closed forms, invariants, library routines)
is listed in the test files that exercise it:

* ``rope_tables`` / ``rotate_half`` / ``apply_rope``  -> tests/test_oracle.py
  (golden vectors from the reference's Train ``forward_step``; rotation
  preserves norms and composes additively in position).
* ``compute_gates``  -> golden vectors.
* ``outlier_attention``  -> ``torch.nn.functional.scaled_dot_product_attention``
  (library routine) and golden vectors.
* ``gla_recurrent`` / ``gla_chunked`` / ``gla_quadratic``  -> three independent
  formulations checked against each other in float64, chunk-size independence,
  the scalar-decay special case, and golden vectors (decode recurrence).
* ``decode_step``  -> golden vectors; equality with the last row of a prefill.
* ``HOFARef``  -> golden vectors written by the reference's own Train module;
  its ``forward_variant`` (r = 0, r = d_h, width split) -> tests/test_oracle_variants.py
  (SDPA with RoPE on all channels, the GLA recurrence + ``nn.RMSNorm``, head
  independence); given RoPE tables (YaRN) enter as they are.
* ``layer_norm`` / ``gelu``  -> ``nn.LayerNorm`` / ``nn.GELU`` (library routines).
* ``SubwordLMRef``  -> golden logits written by the reference's own Train
  ``SubwordLM`` (tests/golden/make_golden_lm.py); decode == last prefill row.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F

FP32_EPS = float(torch.finfo(torch.float32).eps)


# ---------------------------------------------------------------------------
# RoPE (src/modules/modules.py:5-45)
# ---------------------------------------------------------------------------
def rope_tables(dim: int, n: int, base: float = 10000.0, device="cpu"):
    """cos/sin tables ``[n, dim]`` in float32.

    src/modules/modules.py:8-16: ``inv_freq = 1/base^(arange(0,dim,2)/dim)``,
    ``emb = cat(freqs, freqs)`` with ``freqs = outer(t, inv_freq)``.
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim))
    t = torch.arange(n, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """src/modules/modules.py:33-36: ``[x1, x2] -> [-x2, x1]`` (half split)."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """src/modules/modules.py:38-45 for one operand; ``cos/sin`` are ``[N, d]``."""
    return x * cos.to(x.dtype) + rotate_half(x) * sin.to(x.dtype)


# ---------------------------------------------------------------------------
# Gates (src/HybridOutlierFactorizedAttention.py:67-95, Train :85-113)
# ---------------------------------------------------------------------------
def compute_gates(Q, K, gate_w, gate_b, mix_w=None, mix_b=None, fixed_mix=None, rd=None):
    """Returns ``gate_logits [B,H,N]`` and ``mix [B,H,N]`` (or ``None``).

    The first ``d_h`` input features of each projection multiply Q and the
    last ``d_h`` multiply K (``W.chunk(2, dim=1)``, :70 / :81).  ``rd``
    (optional) rounds like a 16-bit module: each einsum, their sum, the sum
    with the bias and the sigmoid are rounded to the activation dtype.
    """
    rd = rd or (lambda t: t)
    d = Q.shape[-1]
    wq, wk = gate_w[:, :d], gate_w[:, d:]
    a = rd(torch.einsum("bhnf,hf->bhn", Q, wq.to(Q.dtype))) + rd(torch.einsum("bhnf,hf->bhn", K, wk.to(Q.dtype)))
    a = rd(rd(a) + gate_b.to(Q.dtype).view(1, -1, 1))
    mix = None
    if mix_w is not None:
        mq, mk = mix_w[:, :d], mix_w[:, d:]
        m = rd(torch.einsum("bhnf,hf->bhn", Q, mq.to(Q.dtype))) + rd(torch.einsum("bhnf,hf->bhn", K, mk.to(Q.dtype)))
        mix = rd(torch.sigmoid(rd(rd(m) + mix_b.to(Q.dtype).view(1, -1, 1))))
    elif fixed_mix is not None:
        mix = rd(torch.sigmoid(fixed_mix.to(Q.dtype))).view(1, -1, 1).expand(Q.shape[0], -1, Q.shape[2])
    return a, mix


def decay_from_gates(log_gamma: torch.Tensor, j: int, log_alpha: Optional[torch.Tensor] = None):
    """Per-channel log decay ``g [B,H,N,j]``.

    src/chunk_gla_inlier.py:47-52,90-107 and src/HybridOutlierFactorizedAttentionTrain.py:276:
    ``g_{t,c} = log_gamma_t * exp(log_alpha_c)``; without alpha every channel
    shares ``log_gamma_t`` (Train :283).
    """
    lg = log_gamma.unsqueeze(-1)
    if log_alpha is None:
        return lg.expand(*log_gamma.shape, j)
    la = log_alpha.reshape(1, log_gamma.shape[1], 1, j)
    return lg * la.exp().to(lg.dtype)


# ---------------------------------------------------------------------------
# Outlier pathway: causal softmax attention on the first r channels
# (src/exact_attention.py:46-161; Train SDPA :241-259)
# ---------------------------------------------------------------------------
def outlier_attention(q_o: torch.Tensor, k_o: torch.Tensor, v: torch.Tensor, sm_scale: float,
                      causal: bool = True, return_lse: bool = False, block_rows: int = 2048):
    """``softmax(q_o k_o^T * sm_scale + causal mask) v``; q_o,k_o ``[B,H,N,r]``, v ``[B,H,M,dv]``.

    With the module's pre-scaled Q/K (``d_h^{-1/4}`` each) and
    ``sm_scale = sqrt(d_h/r)`` the effective logit is ``q.k/sqrt(r)``
    (src/HybridOutlierFactorizedAttention.py:207).  ``lse`` is the natural-log
    log-sum-exp of the scaled logits per row.  Long inputs are processed per
    (batch, head) in blocks of ``block_rows`` query rows, which bounds the
    score matrix held at once; the arithmetic per row is unchanged.
    """
    B, H, n, _ = q_o.shape
    m = k_o.shape[2]
    if B * H * n * m <= (1 << 24):
        return _attention_rows(q_o, k_o, v, sm_scale, causal, return_lse, None)
    outs, lses = [], []
    for b in range(B):
        ob, lb = [], []
        for h in range(H):
            oh, lh = [], []
            for r0 in range(0, n, block_rows):
                r1 = min(n, r0 + block_rows)
                o, l = _attention_rows(q_o[b:b + 1, h:h + 1, r0:r1], k_o[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1],
                                       sm_scale, causal, True, r0 + (m - n))
                oh.append(o)
                lh.append(l)
            ob.append(torch.cat(oh, 2))
            lb.append(torch.cat(lh, 2))
        outs.append(torch.cat(ob, 1))
        lses.append(torch.cat(lb, 1))
    out, lse = torch.cat(outs, 0), torch.cat(lses, 0)
    return (out, lse) if return_lse else out


def _attention_rows(q_o, k_o, v, sm_scale, causal, return_lse, row0):
    """Query rows at key positions ``row0 .. row0 + n - 1`` of the causal
    softmax attention (``row0 = None``: the last query row sits at the last key)."""
    s = torch.matmul(q_o, k_o.transpose(-1, -2)) * sm_scale
    if causal:
        n, m = s.shape[-2], s.shape[-1]
        if row0 is None:
            mask = torch.ones(n, m, dtype=torch.bool).tril(diagonal=m - n)
        else:
            mask = torch.arange(m).view(1, m) <= (row0 + torch.arange(n)).view(n, 1)
        s = s.masked_fill(~mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse.unsqueeze(-1))
    out = torch.matmul(p, v)
    return (out, lse) if return_lse else out


# ---------------------------------------------------------------------------
# Inlier pathway: gated linear attention with per-channel log decay
# ---------------------------------------------------------------------------
def gla_recurrent(q, k, v, g, S0=None):
    """Sequential inclusive recurrence (one token at a time).

    src/HybridOutlierFactorizedAttentionTrain.py:425-433 and
    src/hofa_decode_triton.py:300-301: ``S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t``,
    then ``y_t = q_t S_t`` (state updated before it is read).
    q,k,g ``[B,H,T,J]``, v ``[B,H,T,D]``; returns ``y [B,H,T,D]``, ``S [B,H,J,D]``.
    """
    B, H, T, J = q.shape
    D = v.shape[-1]
    S = torch.zeros(B, H, J, D, dtype=q.dtype) if S0 is None else S0.clone()
    ys = []
    for t in range(T):
        S = S * torch.exp(g[:, :, t, :]).unsqueeze(-1) + k[:, :, t, :].unsqueeze(-1) * v[:, :, t, :].unsqueeze(-2)
        ys.append(torch.einsum("bhj,bhjd->bhd", q[:, :, t, :], S))
    return torch.stack(ys, dim=2), S


def gla_quadratic(q, k, v, g):
    """Parallel (quadratic) form of the same recurrence, no chunking:
    ``y_t = sum_{s<=t} sum_c q_tc k_sc exp(G_tc - G_sc) v_s`` with ``G = cumsum(g)``
    (preprint Eq. 4 unrolled).  Returns ``y`` only.  Used in float64 on tiny
    shapes as an independent check of the other two forms.
    """
    G = torch.cumsum(g, dim=2)
    diff = G.unsqueeze(3) - G.unsqueeze(2)            # [B,H,T(t),T(s),J]
    T = q.shape[2]
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    diff = diff.masked_fill(~causal.view(1, 1, T, T, 1), float("-inf"))
    A = torch.einsum("bhtc,bhsc,bhtsc->bhts", q, k, torch.exp(diff))
    return torch.matmul(A, v)


def gla_chunked(q, k, v, g, chunk: int = 64, S0=None):
    """Chunked form (src/chunk_gla_inlier.py:65-126).

    Per chunk with in-chunk inclusive cumsum ``G``:
      intra ``A_ij = sum_c q_ic k_jc exp(G_ic - G_jc)`` for ``j <= i``  (:109-118)
      ``y = A v + (q * exp(G)) S``                                     (:120)
      ``S <- exp(G_last) S + (k * exp(G_last - G))^T v``                (:122-126)
    Exponents are formed as differences so every factor is <= 1.
    """
    B, H, T, J = q.shape
    D = v.shape[-1]
    S = torch.zeros(B, H, J, D, dtype=q.dtype) if S0 is None else S0.clone()
    ys = []
    for c0 in range(0, T, chunk):
        c1 = min(c0 + chunk, T)
        qc, kc, vc, gc = q[:, :, c0:c1], k[:, :, c0:c1], v[:, :, c0:c1], g[:, :, c0:c1]
        G = torch.cumsum(gc, dim=2)
        n = c1 - c0
        diff = G.unsqueeze(3) - G.unsqueeze(2)
        causal = torch.ones(n, n, dtype=torch.bool).tril()
        diff = diff.masked_fill(~causal.view(1, 1, n, n, 1), float("-inf"))
        A = torch.einsum("bhtc,bhsc,bhtsc->bhts", qc, kc, torch.exp(diff))
        y = torch.matmul(A, vc) + torch.matmul(qc * torch.exp(G), S)
        Glast = G[:, :, -1:, :]
        S = S * torch.exp(Glast).transpose(-1, -2) + torch.matmul((kc * torch.exp(Glast - G)).transpose(-1, -2), vc)
        ys.append(y)
    return torch.cat(ys, dim=2), S


def rmsnorm(y: torch.Tensor, eps: float = FP32_EPS) -> torch.Tensor:
    """``nn.RMSNorm(d, elementwise_affine=False)``: ``y / sqrt(mean(y^2) + eps)``.

    eps: ``finfo(fp32).eps`` for the PyTorch path (Train :71, Infer :64) and the
    decode kernel (src/hofa_decode_triton.py:386); ``1e-5`` in the inference
    prefill kernel (src/chunk_gla_inlier.py:132-133,234).
    """
    return y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)


# ---------------------------------------------------------------------------
# Composed hot path
# ---------------------------------------------------------------------------
def hofa_core(q, k, v, g, mix, gla_scale, r: int, sm_scale: float, eps: float = FP32_EPS,
              chunk: int = 64, S0=None, return_parts: bool = False):
    """Attention core of one HOFA layer after projections, gates and RoPE.

    q,k ``[B,H,T,d_h]`` (RoPE already on ``[..., :r]``), v ``[B,H,T,d_h]``,
    g ``[B,H,T,j]`` per-channel log decay, mix ``[B,H,T]``, gla_scale
    broadcastable to ``[1,H,1,d_h]``.

    ``Y = (1-mix) * gla_scale * RMSNorm(GLA(q_I,k_I,v,g)) + mix * softmax_causal(q_O k_O^T sm_scale) v``
    (src/chunk_gla_inlier.py:130-141 + src/exact_attention.py:148-161;
    Train ``lerp`` :292-294).  Returns ``(Y, S_final)``.
    """
    y_i, S = gla_chunked(q[..., r:], k[..., r:], v, g, chunk=chunk, S0=S0)
    y_in = rmsnorm(y_i, eps) * gla_scale.reshape(1, -1, 1, q.shape[-1]).to(y_i.dtype)
    y_o = outlier_attention(q[..., :r], k[..., :r], v, sm_scale)
    m = mix.unsqueeze(-1).to(y_i.dtype)
    y = (1.0 - m) * y_in + m * y_o
    if return_parts:
        return y, S, y_i, y_in, y_o
    return y, S


def decode_step(q, k, v, cache_k, cache_v, seq_len: int, state_in, log_gamma, mix, norm_w,
                r: int, sm_scale: float, eps: float = FP32_EPS, log_alpha=None):
    """One decode token (src/hofa_decode_triton.py:242-340 semantics).

    q,k,v ``[B,H,d_h]`` (RoPE'd), caches ``[B,H,L,r]`` / ``[B,H,L,d_h]`` of which
    rows ``[0, seq_len)`` are used (the new token already written at row
    ``seq_len-1``), state_in ``[B,H,j,d_h]`` float32, log_gamma / mix ``[B,H]``,
    norm_w ``[H,d_h]``, log_alpha ``[H,j]`` or None.
    Returns ``(y [B,H,d_h], state_out)``.
    """
    d = q.shape[-1]
    s = torch.einsum("bhr,bhlr->bhl", q[..., :r], cache_k[:, :, :seq_len, :r]) * sm_scale
    p = torch.softmax(s, dim=-1)
    y_o = torch.einsum("bhl,bhld->bhd", p, cache_v[:, :, :seq_len, :])
    if log_alpha is None:
        gamma = torch.exp(log_gamma).unsqueeze(-1).unsqueeze(-1)                 # :278
    else:
        gamma = torch.exp(log_gamma.unsqueeze(-1) * log_alpha.reshape(1, -1, d - r).exp()).unsqueeze(-1)  # :296
    S = gamma * state_in + k[..., r:].unsqueeze(-1) * v.unsqueeze(-2)           # :300
    y_i = torch.einsum("bhj,bhjd->bhd", q[..., r:], S)                            # :301
    y_in = y_i * torch.rsqrt(y_i.pow(2).mean(-1, keepdim=True) + eps) * norm_w.unsqueeze(0)   # :332-336
    m = mix.unsqueeze(-1)
    return m * y_o + (1.0 - m) * y_in, S                                          # :339


# ---------------------------------------------------------------------------
# Module level (both reference classes), functional on a state dict
# ---------------------------------------------------------------------------
class HOFARef:
    """Functional restatement of ``HybridOutlierFactorizedAttention`` (inference,
    src/HybridOutlierFactorizedAttention.py:11-422) and its Train twin
    (src/HybridOutlierFactorizedAttentionTrain.py:13-438) on a state dict with
    the reference parameter names.  Computes in ``dtype`` (float32/float64).
    """

    def __init__(self, state: dict, d_model: int, num_heads: int, r: int, rope_base: float = 10000.0,
                 use_rope: bool = True, attention_scale: float = 1.0, chunk: int = 64,
                 dtype=torch.float64, act_dtype=None, rope_f32_tables: bool = False, rope_tables=None):
        self.act = act_dtype
        self.rope_f32 = rope_f32_tables
        # given (cos, sin) rows replace the computed tables (a context-extension
        # patch such as YaRN, src/yarn.py:74-82, stores its own, in 16 bits)
        self.rope_given = rope_tables
        self.p = {kk: vv.detach().to(dtype) for kk, vv in state.items()}
        if act_dtype is not None:  # weights enter the 16-bit ops rounded (a cast module or autocast)
            for kk in ("W_q.weight", "W_k.weight", "W_v.weight", "out_proj.weight", "gate_proj.weight",
                       "gate_proj.bias", "mix_proj.weight", "mix_proj.bias"):
                if kk in self.p:
                    self.p[kk] = self.p[kk].to(act_dtype).to(dtype)
        self.D, self.H = d_model, num_heads
        self.dh = d_model // num_heads
        self.r, self.j = r, self.dh - r
        self.rope_base, self.use_rope = rope_base, use_rope
        self.attention_scale = attention_scale
        self.chunk = chunk
        self.dtype = dtype

    # -- shared pieces ----------------------------------------------------
    def _rd(self, t):
        """Round to the activation dtype (identity without one)."""
        return t if self.act is None else t.to(self.act).to(self.dtype)

    def _qkv(self, x):
        """Projections (Infer :100-104, Train :132-137): Q,K scaled by d_h^{-1/4}."""
        B, N, _ = x.shape
        rd = self._rd
        x = rd(x.to(self.dtype))
        s = self.dh ** 0.25
        Q = rd(rd(x @ self.p["W_q.weight"].T) / s).view(B, N, self.H, self.dh).transpose(1, 2)
        K = rd(rd(x @ self.p["W_k.weight"].T) / s).view(B, N, self.H, self.dh).transpose(1, 2)
        V = rd(x @ self.p["W_v.weight"].T).view(B, N, self.H, self.dh).transpose(1, 2)
        return Q, K, V

    def _gates(self, Q, K):
        kw = {} if self.act is None else {"rd": self._rd}
        return compute_gates(Q, K, self.p["gate_proj.weight"], self.p["gate_proj.bias"],
                             self.p.get("mix_proj.weight"), self.p.get("mix_proj.bias"),
                             self.p.get("fixed_mix"), **kw)

    def _rope(self, n0, n1):
        if self.rope_given is not None:
            cos, sin = self.rope_given
            return cos[n0:n1].to(self.dtype), sin[n0:n1].to(self.dtype)
        cos, sin = rope_tables(self.r, n1, self.rope_base)
        cos, sin = cos[n0:n1].to(self.dtype), sin[n0:n1].to(self.dtype)
        if self.rope_f32:
            return cos, sin
        return self._rd(cos), self._rd(sin)

    def _apply_rope(self, x, cos, sin):
        if self.act is None:
            return apply_rope(x, cos, sin)
        if self.rope_f32:
            return self._rd(apply_rope(x, cos, sin))
        return self._rd(self._rd(x * cos) + self._rd(rotate_half(x) * sin))

    def _out(self, Y):
        B, H, N, d = Y.shape
        return self._rd(Y.transpose(1, 2).reshape(B, N, H * d) @ self.p["out_proj.weight"].T)

    def _log_alpha(self):
        return self.p.get("log_alpha")

    def _gla_scale(self):
        return self.p["gla_scale"]

    # -- prefill ----------------------------------------------------------
    def forward(self, x, eps: float = FP32_EPS, sm_extra: float = 1.0, return_state: bool = False):
        """Hybrid prefill (0 < r < d_h).  ``sm_extra`` is Train's ``attention_scale``
        (Train :248; the inference class omits it, Infer :207).  ``eps`` is the
        RMSNorm epsilon (Train ``finfo`` eps, inference prefill kernel 1e-5).
        Returns ``Y`` or ``(Y, (K_cache, V_cache), state_I)``.
        """
        Q, K, V = self._qkv(x)
        N = x.shape[1]
        a, mix = self._gates(Q, K)
        log_gamma = self._rd(F.logsigmoid(-a))                           # Infer :177
        if self.use_rope:
            cos, sin = self._rope(0, N)
            Q = torch.cat([self._apply_rope(Q[..., :self.r], cos, sin), Q[..., self.r:]], -1)
            K = torch.cat([self._apply_rope(K[..., :self.r], cos, sin), K[..., self.r:]], -1)
        g = decay_from_gates(log_gamma, self.j, self._log_alpha())
        sm = (self.dh / self.r) ** 0.5 * sm_extra
        Y, S = hofa_core(Q, K, V, g, mix, self._gla_scale(), self.r, sm, eps=eps, chunk=self.chunk)
        out = self._out(self._rd(Y))
        if return_state:
            return out, (K[..., :self.r].contiguous(), V.contiguous()), S
        return out

    # -- the non-hybrid variants ------------------------------------------
    def _rope_full(self, Q, K, n0, n1):
        """RoPE over all ``d_h`` channels (the rotary module's dim is ``d_h``
        when ``r`` is 0 or ``d_h``: Infer :57-61, Train :77-81)."""
        cos, sin = rope_tables(self.dh, n1, self.rope_base)
        cos, sin = cos[n0:n1].to(self.dtype), sin[n0:n1].to(self.dtype)
        return apply_rope(Q, cos, sin), apply_rope(K, cos, sin)

    def _pure_gla(self, Q, K, V, gate_w, gate_b, gla_scale, log_alpha=None, eps: float = FP32_EPS, S0=None):
        """``gla_scale * RMSNorm(GLA(Q, K, V, g))`` over all ``d_h`` channels with
        ``log_gamma = logsigmoid(-(Q w_q + K w_k + b))`` (Infer :146-159,
        Train :201-223; ``g`` carries ``exp(log_alpha)`` when given)."""
        a, _ = compute_gates(Q, K, gate_w, gate_b)
        g = decay_from_gates(F.logsigmoid(-a), self.dh, log_alpha)
        y, S = gla_chunked(Q, K, V, g, chunk=self.chunk, S0=S0)
        return rmsnorm(y, eps) * gla_scale.reshape(1, -1, 1, self.dh).to(y.dtype), S

    def forward_variant(self, x, mha_heads: int = 0, scale: float = 1.0, use_alpha: bool = False,
                        eps: float = FP32_EPS):
        """Prefill of the non-hybrid configurations, returning ``(out, S)``:

        * ``r == 0``: the pure normalized GLA on every head (``mha_heads`` = 0);
        * ``r == d_h``: causal softmax attention on every head with RoPE on all
          channels and logit scale ``scale`` (``mha_heads`` = H; Infer :161-171
          with 1.0, Train :225-231 with ``attention_scale``);
        * width split (Infer :106-143, Train :139-175): heads ``[0, mha_heads)``
          as above, the rest the pure GLA with their rows of ``gate_proj``,
          ``gla_scale`` (and ``log_alpha`` when ``use_alpha``).
        ``S`` is the GLA heads' final state ``[B, H - mha_heads, d_h, d_h]``.
        """
        Q, K, V = self._qkv(x)
        N, m = x.shape[1], mha_heads
        parts, S = [], None
        if m > 0:
            Qm, Km = Q[:, :m], K[:, :m]
            if self.use_rope:
                Qm, Km = self._rope_full(Qm, Km, 0, N)
            parts.append(outlier_attention(Qm, Km, V[:, :m], scale))
        if m < self.H:
            la = self._log_alpha()
            la = la.reshape(1, self.H, 1, self.dh)[:, m:] if (use_alpha and la is not None) else None
            y, S = self._pure_gla(Q[:, m:], K[:, m:], V[:, m:], self.p["gate_proj.weight"][m:],
                                  self.p["gate_proj.bias"][m:], self._gla_scale().reshape(1, self.H, 1, -1)[:, m:],
                                  la, eps)
            parts.append(y)
        return self._out(self._rd(torch.cat(parts, 1))), S

    # -- decode (Train forward_step semantics, :298-438) -----------------
    def forward_step(self, x, cache_O=None, state=None, eps: float = FP32_EPS):
        """One token.  ``cache_O`` is ``(K_cache [B,H,L,r], V_cache [B,H,L,d_h])``
        holding exactly the past rows; ``state`` ``[B,H,j,d_h]``.  RoPE position =
        current cache length (Train :388-393).  Returns ``(out, cache_O, state)``.
        """
        B = x.shape[0]
        Q, K, V = self._qkv(x)
        a, mix = self._gates(Q, K)
        pos = 0 if cache_O is None else cache_O[0].shape[2]
        if self.use_rope:
            cos, sin = self._rope(pos, pos + 1)
            Q = torch.cat([self._apply_rope(Q[..., :self.r], cos, sin), Q[..., self.r:]], -1)
            K = torch.cat([self._apply_rope(K[..., :self.r], cos, sin), K[..., self.r:]], -1)
        if cache_O is None:
            cache_O = (K[..., :self.r], V)
        else:
            cache_O = (torch.cat([cache_O[0], K[..., :self.r]], 2), torch.cat([cache_O[1], V], 2))
        if state is None:
            state = torch.zeros(B, self.H, self.j, self.dh, dtype=self.dtype)
        la = self._log_alpha()
        y, S = decode_step(Q[:, :, 0], K[:, :, 0], V[:, :, 0], cache_O[0], cache_O[1], cache_O[0].shape[2],
                           state, self._rd(F.logsigmoid(-a))[:, :, 0], mix[:, :, 0],
                           self._gla_scale().reshape(self.H, self.dh), self.r,
                           (self.dh / self.r) ** 0.5, eps=eps,
                           log_alpha=None if la is None else la.reshape(self.H, self.j))
        return self._out(self._rd(y).unsqueeze(2)), cache_O, S


# ---------------------------------------------------------------------------
# Language-model stack (src/HybridOutlierFactorizedAttention.py:425-513,
# Train src/HybridOutlierFactorizedAttentionTrain.py:441-502)
# ---------------------------------------------------------------------------
def layer_norm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``nn.LayerNorm(d)`` (biased variance, default eps 1e-5), as ``ln_1``/``ln_2``/``ln_f`` (:427,429,468)."""
    mu = x.mean(-1, keepdim=True)
    var = (x - mu).pow(2).mean(-1, keepdim=True)
    return (x - mu) * torch.rsqrt(var + eps) * w + b


def gelu(x: torch.Tensor) -> torch.Tensor:
    """``nn.GELU()`` (erf form, the default) of the block MLP (:432)."""
    return 0.5 * x * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0))))


class SubwordLMRef:
    """Functional restatement of ``SubwordLM`` / ``TransformerBlock`` on a state
    dict with the reference names: token embedding tied to ``lm_head``
    (:471), per layer ``x + attn(ln_1(x))`` then ``x + mlp(ln_2(x))`` with a
    4x GELU MLP (:436-451), ``ln_f`` and the LM head (:476-483).  Per-layer
    ``r`` comes from ``r_list`` (:459-467).  The attention of each layer is
    ``HOFARef`` (hybrid path, 0 < r < d_h).  ``attn_eps`` is the inlier
    RMSNorm epsilon used in prefill.
    """

    def __init__(self, state: dict, d_model: int, num_heads: int, r_list, rope_base: float = 10000.0,
                 attn_eps: float = FP32_EPS, dtype=torch.float64, act_dtype=None, rope_tables=None):
        self.dtype = dtype
        self.act = act_dtype
        self.attn_eps = attn_eps
        self.emb = state["lm_head.weight"].detach().to(dtype)
        self.lnf = (state["ln_f.weight"].detach().to(dtype), state["ln_f.bias"].detach().to(dtype))
        self.layers = []
        for i, r in enumerate(r_list):
            pre = f"layers.{i}."
            sub = {k[len(pre):]: v for k, v in state.items() if k.startswith(pre)}
            attn = HOFARef({k[len("attn."):]: v for k, v in sub.items() if k.startswith("attn.")}, d_model,
                           num_heads, r, rope_base=rope_base, dtype=dtype, act_dtype=act_dtype,
                           rope_tables=None if rope_tables is None else rope_tables[i])
            t = {k: v.detach().to(dtype) for k, v in sub.items() if not k.startswith("attn.")}
            self.layers.append((attn, t))

    def _rd(self, t):
        return t if self.act is None else t.to(self.act).to(self.dtype)

    def _ln(self, x, w, b):
        return self._rd(layer_norm(x, w, b))

    def _mlp(self, t, x):
        h = self._rd(gelu(self._rd(x @ t["mlp.0.weight"].T + t["mlp.0.bias"])))
        return self._rd(h @ t["mlp.2.weight"].T + t["mlp.2.bias"])

    def _head(self, x):
        return self._rd(self._ln(x, *self.lnf) @ self.emb.T)

    def forward(self, ids: torch.Tensor, return_state: bool = False, last_only: bool = False):
        """Logits ``[B, N, vocab]`` (``last_only``: ``[B, 1, vocab]``); with
        ``return_state`` also the per-layer caches and GLA states (:476-483)."""
        x = self.emb[ids]
        caches, states = [], []
        for attn, t in self.layers:
            a, cache, S = attn.forward(self._ln(x, t["ln_1.weight"], t["ln_1.bias"]), eps=self.attn_eps,
                                       return_state=True)
            caches.append(cache)
            states.append(S)
            x = self._rd(x + a)
            x = self._rd(x + self._mlp(t, self._ln(x, t["ln_2.weight"], t["ln_2.bias"])))
        logits = self._head(x[:, -1:] if last_only else x)
        return (logits, caches, states) if return_state else logits

    def forward_step(self, ids: torch.Tensor, caches, states):
        """One token ``ids [B, 1]`` per sequence on caches holding exactly the
        past rows (:446-451, :485-513); returns ``(logits [B,1,vocab], caches, states)``."""
        x = self.emb[ids]
        new_c, new_s = [], []
        for (attn, t), c, S in zip(self.layers, caches, states):
            a, c, S = attn.forward_step(self._ln(x, t["ln_1.weight"], t["ln_1.bias"]), c, S)
            new_c.append(c)
            new_s.append(S)
            x = self._rd(x + a)
            x = self._rd(x + self._mlp(t, self._ln(x, t["ln_2.weight"], t["ln_2.bias"])))
        return self._head(x), new_c, new_s
