"""Multi-step greedy decoding from captured HIP graphs (decode_loop.py).

Checks, on a small float32 SubwordLM:
* the graph-replayed loop (device-side position, RoPE row, cache slot and
  attended length) produces exactly the tokens of the module's own eager
  ``forward_step`` loop with Python ``cache_seq_len`` -- the reference's
  generation loop (src/inference.py:150-239);
* the logits of the last decoded token equal the last-row logits of one
  prefill over the whole sequence (the reference's decode-versus-prefill
  check, benchmarks/validate_kernels.py:312-337), to 2e-3 relative to the
  largest logit (the prefill's softmax probabilities enter the PV product in
  bf16);
* a second ``decode`` call continues from where the first stopped, and
  eager (``graphs=False``) and graph decoding agree token for token.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"
VOCAB = 384


def _model(seed=0, alpha=False, layers=2):
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    cfg = ModelConfig(d_model=256, num_heads=4, num_layers=layers, r=16, learnable_alpha=alpha, device=DEV)
    torch.manual_seed(seed)
    m = SubwordLM(VOCAB, cfg)
    with torch.no_grad():  # non-trivial gates, decay and scales (the defaults are zero / one)
        for layer in m.layers:
            a = layer.attn
            a.gate_proj.weight.normal_(0, 0.3)
            a.mix_proj.weight.normal_(0, 0.3)
            a.gla_scale.uniform_(0.5, 1.5)
            if alpha:
                a.log_alpha.normal_(0, 0.5)
    return m.to(DEV).eval()


def _eager_reference(m, ids, steps):
    """The module's own loop: prefill, pre-allocated caches, forward_step."""
    B, N = ids.shape
    cap = N + steps + 1
    with torch.no_grad():
        logits, caches, states = m(ids, return_state=True)
        big = []
        for k, v in caches:
            kk = torch.zeros(B, k.shape[1], cap, k.shape[3], device=DEV, dtype=k.dtype)
            vv = torch.zeros(B, v.shape[1], cap, v.shape[3], device=DEV, dtype=v.dtype)
            kk[:, :, :N] = k
            vv[:, :, :N] = v
            big.append((kk, vv))
        tok = logits[:, -1:].argmax(-1)
        first = tok.clone()
        out = []
        for i in range(steps):
            logits, big, states = m.forward_step(tok, big, states, cache_seq_len=N + i)
            tok = logits[:, -1:].argmax(-1)
            out.append(tok)
    return first, torch.cat(out, 1), logits


@pytest.mark.parametrize("alpha", [False, True])
def test_graph_decode_matches_eager_loop_and_prefill(alpha):
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    m = _model(seed=3, alpha=alpha)
    B, N, steps = 2, 37, 9
    gen = torch.Generator().manual_seed(11)
    ids = torch.randint(0, VOCAB, (B, N), generator=gen).to(DEV)
    first, ref_tokens, ref_logits = _eager_reference(m, ids, steps)

    dec = GreedyGraphDecoder(m, B, N + steps + 4)
    dec.prefill(ids)
    assert torch.equal(dec.tok, first)
    got = dec.decode(steps).clone()
    torch.cuda.synchronize()
    print(f"alpha={alpha} tokens graph {got.tolist()} eager {ref_tokens.tolist()}")
    assert torch.equal(got, ref_tokens)
    scale = ref_logits.abs().max().item()
    assert (dec.logits - ref_logits).abs().max().item() <= 1e-4 * scale

    # last decoded logits == last-row logits of a prefill over the whole sequence
    seq = torch.cat([ids, first, got[:, :-1]], 1)
    with torch.no_grad():
        full, _ = m(seq)
    err = (full[:, -1:] - dec.logits).abs().max().item()
    assert err <= 2e-3 * full[:, -1:].abs().max().item(), f"decode vs prefill: {err}"


def test_graph_decode_continues_and_matches_eager_steps():
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    m = _model(seed=5)
    B, N = 3, 50
    ids = torch.randint(0, VOCAB, (B, N), generator=torch.Generator().manual_seed(2)).to(DEV)
    g = GreedyGraphDecoder(m, B, N + 16)
    g.prefill(ids)
    a = g.decode(4).clone()
    b = g.decode(6).clone()   # continues from position N + 4 on the captured graphs
    e = GreedyGraphDecoder(m, B, N + 16)
    e.prefill(ids)
    c = e.decode(10, graphs=False).clone()
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([a, b], 1), c)
    assert (g.logits - e.logits).abs().max().item() <= 1e-5 * e.logits.abs().max().item()


def test_graph_decode_rejects_overflow_and_unsupported():
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    m = _model(seed=1, layers=1)
    dec = GreedyGraphDecoder(m, 1, 12)
    with pytest.raises(RuntimeError):
        dec.decode(1)
    dec.prefill(torch.zeros(1, 8, dtype=torch.int64, device=DEV))
    with pytest.raises(ValueError):
        dec.decode(5)
    cfg = ModelConfig(d_model=256, num_heads=4, num_layers=1, r=0, device=DEV)
    with pytest.raises(NotImplementedError):
        GreedyGraphDecoder(SubwordLM(VOCAB, cfg).to(DEV), 1, 8)
