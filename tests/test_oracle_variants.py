"""Pins the oracle's restatement of the non-hybrid configurations
(``HOFARef.forward_variant``: r = 0, r = d_h and the width split) against
independent forms on the CPU in float64:

* every head as attention == ``out_proj(SDPA(RoPE(Q), RoPE(K), V))`` with
  torch's ``scaled_dot_product_attention`` and RoPE on all channels;
* every head as GLA == ``gla_scale * nn.RMSNorm(GLA)`` with the GLA run as
  the sequential recurrence ``S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t``,
  ``y_t = q_t S_t`` written out here (not the oracle's chunked form);
* the width split == those two per head block (heads are independent), read
  through an identity ``out_proj``.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle import hofa_ref as ref

B, N, H, DH = 2, 37, 4, 16
D = H * DH


def _state(seed=0, alpha=True):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s, sd=1.0: torch.randn(*s, generator=g, dtype=torch.float64) * sd  # noqa: E731
    st = {"W_q.weight": rn(D, D, sd=D ** -0.5), "W_k.weight": rn(D, D, sd=D ** -0.5),
          "W_v.weight": rn(D, D, sd=D ** -0.5), "out_proj.weight": torch.eye(D, dtype=torch.float64),
          "gate_proj.weight": rn(H, 2 * DH, sd=0.3), "gate_proj.bias": rn(H, sd=0.5) - 1.0,
          "gla_scale": 1.0 + rn(1, H, 1, DH, sd=0.1)}
    if alpha:
        st["log_alpha"] = rn(1, H, 1, DH, sd=0.5)
    return st


def _x(seed=1):
    return torch.randn(B, N, D, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def _qkv(st, x):
    s = DH ** 0.25
    f = lambda w: (x @ st[w].T).view(B, N, H, DH).transpose(1, 2)  # noqa: E731
    return f("W_q.weight") / s, f("W_k.weight") / s, f("W_v.weight")


def _rope(x):
    # float32 tables, as the reference's rotary module builds them
    inv = 1.0 / (10000.0 ** (torch.arange(0, DH, 2, dtype=torch.float32) / DH))
    ang = torch.outer(torch.arange(N, dtype=torch.float32), inv)
    cos, sin = torch.cat([ang, ang], -1).cos().double(), torch.cat([ang, ang], -1).sin().double()
    x1, x2 = x[..., :DH // 2], x[..., DH // 2:]
    return x * cos + torch.cat([-x2, x1], -1) * sin


def _gla_recurrence(q, k, v, g):
    S = torch.zeros(q.shape[0], q.shape[1], q.shape[-1], v.shape[-1], dtype=q.dtype)
    ys = []
    for t in range(q.shape[2]):
        S = g[:, :, t].exp().unsqueeze(-1) * S + k[:, :, t].unsqueeze(-1) * v[:, :, t].unsqueeze(-2)
        ys.append((q[:, :, t].unsqueeze(-2) @ S).squeeze(-2))
    return torch.stack(ys, 2)


def _heads_gla(st, Q, K, V, h0, alpha):
    w, bias = st["gate_proj.weight"][h0:], st["gate_proj.bias"][h0:]
    a = torch.einsum("bhnf,hf->bhn", Q, w[:, :DH]) + torch.einsum("bhnf,hf->bhn", K, w[:, DH:]) + bias.view(1, -1, 1)
    lg = F.logsigmoid(-a).unsqueeze(-1)
    g = lg * st["log_alpha"][:, h0:].exp() if alpha else lg.expand(-1, -1, -1, DH)
    y = _gla_recurrence(Q, K, V, g)
    # the reference normalizes a float32 tensor: eps = finfo(float32).eps
    norm = torch.nn.RMSNorm(DH, eps=torch.finfo(torch.float32).eps, elementwise_affine=False, dtype=torch.float64)
    return norm(y) * st["gla_scale"][:, h0:]


def _heads_mha(Q, K, V, scale):
    return F.scaled_dot_product_attention(_rope(Q), _rope(K), V, is_causal=True, scale=scale)


def _oracle(st, r):
    return ref.HOFARef(st, D, H, r, dtype=torch.float64)


@pytest.mark.parametrize("scale", [1.0, 0.7])
def test_all_heads_attention_is_sdpa_with_full_rope(scale):
    st, x = _state(), _x()
    Q, K, V = _qkv(st, x)
    want = _heads_mha(Q, K, V, scale).transpose(1, 2).reshape(B, N, D)
    got, S = _oracle(st, DH).forward_variant(x, mha_heads=H, scale=scale)
    assert S is None
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("alpha", [False, True])
def test_all_heads_gla_is_normalized_recurrence(alpha):
    st, x = _state(alpha=alpha), _x()
    Q, K, V = _qkv(st, x)
    want = _heads_gla(st, Q, K, V, 0, alpha).transpose(1, 2).reshape(B, N, D)
    got, S = _oracle(st, 0).forward_variant(x, mha_heads=0, use_alpha=alpha)
    assert S.shape == (B, H, DH, DH)
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("m", [1, 3])
def test_width_split_is_the_two_per_head_blocks(m):
    st, x = _state(), _x()
    Q, K, V = _qkv(st, x)
    want = torch.cat([_heads_mha(Q[:, :m], K[:, :m], V[:, :m], 1.0),
                      _heads_gla(st, Q[:, m:], K[:, m:], V[:, m:], m, True)], 1).transpose(1, 2).reshape(B, N, D)
    got, S = _oracle(st, 0).forward_variant(x, mha_heads=m, use_alpha=True)
    assert S.shape == (B, H - m, DH, DH)
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)


def test_planted_mistake_in_variant_is_caught(monkeypatch):
    """Dropping the RoPE of the attention heads must fail the SDPA check."""
    st, x = _state(), _x()
    Q, K, V = _qkv(st, x)
    want = _heads_mha(Q, K, V, 1.0).transpose(1, 2).reshape(B, N, D)
    monkeypatch.setattr(ref.HOFARef, "_rope_full", lambda self, Q, K, n0, n1: (Q, K))
    got, _ = _oracle(st, DH).forward_variant(x, mha_heads=H)
    assert not torch.allclose(got, want, rtol=1e-6, atol=1e-6)
