"""HOFA hot-path benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 4] [--skip-cpu]
                    [--only decode|prefill|train|copy] [--eager]

A step is one pass of the hot path over one batch of synthetic input: one
decode token of the BASELINE cfg3 workload (H=16, d_h=64, r=16, 32768-row bf16
outlier cache, fp32 48x64 GLA state per head) for B sequences.  The headline
``value`` is decode tokens/s at B=4; B=1 is reported beside it.

Every step reads a different cache set from a rotation whose total size is at
least 1 GiB, so the timed steps stream from HBM instead of the 256 MB
last-level cache.  The K timed steps are replayed from captured HIP graphs and
bracketed by HIP events on the stream the kernels run on.

The CPU baseline times the build's own PyTorch restatement of the reference
path (``oracle/hofa_ref.py``; kind "port") on a bounded sample of the same
workload on this host.

Prints ONE JSON line (rank 0).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
MFMA_BF16_PEAK_TFS = 2500.0    # MI355X dense bf16 MFMA, vendor figure

H, D, R, L = 16, 64, 16, 32768
J = D - R


def decode_bytes(B: int) -> int:
    """Algorithmic HBM bytes of one decode step: both caches once, the fp32
    state read and written, plus q/k/v/y and the per-head scalars."""
    cache = B * H * L * (R + D) * 2
    state = B * H * J * D * 4 * 2
    small = B * H * (4 * D * 2 + 3 * 4) + H * D * 4
    return cache + state + small


def make_decode_set(B: int, gen: torch.Generator, dev="cuda"):
    f = dict(dtype=torch.float32)
    qkv = torch.randn(B, 1, H, 3 * D, generator=gen, **f).to(dev, torch.bfloat16)
    q, k, v = (qkv[..., i * D:(i + 1) * D].transpose(1, 2) for i in range(3))
    ck = torch.randn(B, H, L, R, generator=gen, **f).to(dev, torch.bfloat16)
    cv = torch.randn(B, H, L, D, generator=gen, **f).to(dev, torch.bfloat16)
    s_in = (0.1 * torch.randn(B, H, J, D, generator=gen, **f)).to(dev)
    s_out = torch.empty_like(s_in)
    lg = torch.clamp(F.logsigmoid(torch.randn(B, H, 1, generator=gen, **f)) / 16, -5, 0).to(dev)
    mix = torch.sigmoid(torch.randn(B, H, 1, generator=gen, **f)).to(dev)
    nw = torch.ones(H, D, device=dev)
    return dict(q=q, k=k, v=v, ck=ck, cv=cv, s_in=s_in, s_out=s_out, lg=lg, mix=mix, nw=nw)


def _decode_call(st):
    from outlierneuronattention_amd import fused_hofa_decode
    return fused_hofa_decode(st["q"], st["k"], st["v"], st["ck"], st["cv"], st["s_in"], st["s_out"], st["lg"],
                             st["mix"], st["nw"], R, L, math.sqrt(D / R))


def bench_decode(B: int, steps: int, warmup: int, rotate_bytes: int = 1 << 30, eager: bool = False):
    gen = torch.Generator().manual_seed(1234 + B)
    nbuf = max(1, math.ceil(rotate_bytes / decode_bytes(B)))
    sets = [make_decode_set(B, gen) for _ in range(nbuf)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(max(warmup, nbuf)):
            _decode_call(sets[i % nbuf])
        s.synchronize()
        if eager:  # plain launches (for counter collection, which follows eager dispatches)
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(s)
            for i in range(steps):
                _decode_call(sets[i % nbuf])
            t1.record(s)
            torch.cuda.synchronize()
            step_s = t0.elapsed_time(t1) / 1e3 / steps
            return dict(B=B, ms_per_step=step_s * 1e3, tok_per_s=B / step_s, bytes_per_step=decode_bytes(B),
                        gbs=decode_bytes(B) / step_s / 1e9, rotation_sets=nbuf, timing="eager launches")
        full = torch.cuda.CUDAGraph()
        with torch.cuda.graph(full, stream=s):
            for st in sets:
                _decode_call(st)
        rem = steps % nbuf
        part = None
        if rem:
            part = torch.cuda.CUDAGraph()
            with torch.cuda.graph(part, stream=s):
                for st in sets[:rem]:
                    _decode_call(st)
        full.replay()
        s.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(s)
        for _ in range(steps // nbuf):
            full.replay()
        if part is not None:
            part.replay()
        t1.record(s)
        torch.cuda.synchronize()
    ms = t0.elapsed_time(t1)
    step_s = ms / 1e3 / steps
    nbytes = decode_bytes(B)
    return dict(B=B, ms_per_step=ms / steps, tok_per_s=B / step_s, bytes_per_step=nbytes,
                gbs=nbytes / step_s / 1e9, rotation_sets=nbuf)


def bench_decode_hot(B: int, steps: int):
    """Same kernel on one cache set (last-level-cache resident when it fits)."""
    gen = torch.Generator().manual_seed(99)
    st = make_decode_set(B, gen)
    for _ in range(3):
        _decode_call(st)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _decode_call(st)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            for _ in range(10):
                _decode_call(st)
        g.replay()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(s)
        n = max(1, steps // 10)
        for _ in range(n):
            g.replay()
        t1.record(s)
        torch.cuda.synchronize()
    step_s = t0.elapsed_time(t1) / 1e3 / (n * 10)
    return dict(B=B, us_per_step=step_s * 1e6, gbs=decode_bytes(B) / step_s / 1e9)


# ---------------------------------------------------------------- prefill (cfg2)
P_B, P_T, P_H, P_D, P_R, P_C = 4, 4096, 16, 64, 16, 64
P_J = P_D - P_R


def prefill_flops(B=P_B, T=P_T, H=P_H, D=P_D, R=P_R) -> float:
    """Algorithmic FLOPs of the attention core (causal, preprint Eq. 7):
    B*H*T^2*(r + d_h) for the outlier softmax attention (QK^T and PV over the
    causal half) plus 6*B*H*T*j*d_h for the chunked GLA."""
    J = D - R
    return B * H * T * T * (R + D) + 6 * B * H * T * J * D


def make_prefill_inputs(gen, dev="cuda", B=P_B, T=P_T, H=P_H, D=P_D, R=P_R):
    """cfg2: q/k/v ~ N(0,1) as [B,H,T,d] views of [B,T,H,3d] memory; per-channel
    log decay clamp(logsigmoid(N(0,1))/16, -5, 0); mix = sigmoid(N(0,1)); gla_scale = 1."""
    J = D - R
    x = torch.randn(B, T, H, 3 * D, generator=gen).to(dev, torch.bfloat16)
    q, k, v = (x[..., i * D:(i + 1) * D].transpose(1, 2) for i in range(3))
    g = torch.clamp(F.logsigmoid(torch.randn(B, H, T, J, generator=gen)) / 16, -5, 0).to(dev)
    mix = torch.sigmoid(torch.randn(B, H, T, generator=gen)).to(dev, torch.bfloat16)
    gs = torch.ones(1, H, 1, D, device=dev)
    lg = torch.zeros(B, H, T, device=dev)
    return dict(q=q, k=k, v=v, g=g, mix=mix, gs=gs, lg=lg)


def _prefill_call(inp, y):
    """The inference module's prefill core: the GLA (general decay g, RMSNorm eps 1e-5 as the
    reference kernel) in float32, then the outlier attention adding mix * O with one rounding."""
    from outlierneuronattention_amd.prefill import prefill_fwd
    prefill_fwd(inp["q"], inp["k"], inp["v"], inp["lg"], P_R, math.sqrt(P_D / P_R), inp["mix"], inp["gs"],
                g=inp["g"], eps=1e-5, out=y)


def _warm_clocks(run, sync, seconds: float = 0.2):
    """Repeat `run` for at least `seconds` of wall time: the GPU's clocks ramp
    up over the first tens of milliseconds of sustained work (a cfg2 attention
    call measured 190 us at first, 165 us once settled), so the timed region
    starts at steady state."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(4):
            run()
        sync()


def bench_prefill(steps: int, warmup: int):
    gen = torch.Generator().manual_seed(4321)
    inp = make_prefill_inputs(gen)
    y = torch.empty(P_B, P_H, P_T, P_D, dtype=torch.bfloat16, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(max(2, warmup)):
            _prefill_call(inp, y)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            _prefill_call(inp, y)
        g.replay()
        s.synchronize()
        _warm_clocks(g.replay, s.synchronize)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(s)
        for _ in range(steps):
            g.replay()
        t1.record(s)
        torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    fl = prefill_flops()
    tfs = fl / (ms * 1e-3) / 1e12
    return dict(workload="cfg2: chunked prefill forward, B=4 T=4096 H=16 d_h=64 r=16 (j=48), GLA chunk 64, bf16",
                ms_per_call=round(ms, 4), gflop=round(fl / 1e9, 2), tflops=round(tfs, 1),
                mfma_frac=round(tfs / MFMA_BF16_PEAK_TFS, 4))


# ---------------------------------------------------------------- training (cfg4)
T_B, T_T, T_H, T_D, T_R = 8, 2048, 12, 64, 16


def train_flops(B=T_B, T=T_T, H=T_H, D=T_D, R=T_R):
    """Algorithmic FLOPs of the attention core, forward and backward (causal):
    forward B*H*T^2*(r + d_h) + 6*B*H*T*j*d_h; backward B*H*T^2*(3r + 2d_h)
    (QK^T recompute, dO V^T, dV, dK, dQ) + 12*B*H*T*j*d_h."""
    J = D - R
    fwd = B * H * T * T * (R + D) + 6 * B * H * T * J * D
    bwd = B * H * T * T * (3 * R + 2 * D) + 12 * B * H * T * J * D
    return fwd, bwd


def make_train_inputs(gen, dev="cuda"):
    """cfg4 at kernel level: bf16 q/k/v ~ N(0,1) ([B,H,T,d] views of [B,T,H,3d]),
    learnable per-(head, channel) decay: log_gamma = -1 and log_alpha =
    log(-logsigmoid(U(2,6))), so g[t, c] = logsigmoid(U(2,6))[c]; mix =
    sigmoid(N(0,1)); gla_scale = 1; dO ~ N(0,1).  Decay and gate parameters fp32."""
    B, T, H, D, R = T_B, T_T, T_H, T_D, T_R
    J = D - R
    x = torch.randn(B, T, H, 3 * D, generator=gen).to(dev, torch.bfloat16)
    # contiguous [B,H,T,d] leaves: the core's gradients are then stored as they are (no layout copies)
    q, k, v = (x[..., i * D:(i + 1) * D].transpose(1, 2).contiguous() for i in range(3))
    lg = torch.full((B, H, T), -1.0, device=dev)
    la = torch.log(-F.logsigmoid(2 + 4 * torch.rand(1, H, 1, J, generator=gen))).to(dev)
    mix = torch.sigmoid(torch.randn(B, H, T, generator=gen)).to(dev)
    gs = torch.ones(1, H, 1, D, device=dev)
    dy = torch.randn(B, H, T, D, generator=gen).to(dev, torch.bfloat16)
    leaves = dict(q=q.detach(), k=k.detach(), v=v.detach(), lg=lg, la=la, mix=mix, gs=gs)
    for t in leaves.values():
        t.requires_grad_()
    return leaves, dy


def _train_step(inp, dy, backward=True):
    from outlierneuronattention_amd.autograd import hofa_core
    q, k = inp["q"], inp["k"]
    y = hofa_core(None, None, q, k, inp["v"], inp["lg"], inp["la"], inp["mix"], inp["gs"], T_R,
                  math.sqrt(T_D / T_R))  # outlier channels = q[..., :r], k[..., :r] (RoPE is outside the core)
    if backward:
        for t in inp.values():
            t.grad = None
        y.backward(dy)
    return y


def bench_train(steps: int, warmup: int):
    gen = torch.Generator().manual_seed(777)
    inp, dy = make_train_inputs(gen)
    for _ in range(max(2, warmup)):
        _train_step(inp, dy)
    _warm_clocks(lambda: _train_step(inp, dy), torch.cuda.synchronize)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record(s)
    for _ in range(steps):
        _train_step(inp, dy)
    ev[1].record(s)
    with torch.no_grad():
        for _ in range(steps):
            _train_step(inp, dy, backward=False)
    ev[2].record(s)
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / steps
    ms_fwd = ev[1].elapsed_time(ev[2]) / steps
    # The same step (forward and backward, gradients into static tensors) captured
    # in one HIP graph and replayed: the launch gaps of the eager autograd step go.
    graph = torch.cuda.CUDAGraph()
    for t in inp.values():
        t.grad = None
    with torch.cuda.graph(graph):
        _train_step(inp, dy, backward=False).backward(dy)
    graph.replay()
    torch.cuda.synchronize()
    gs = torch.cuda.current_stream()
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record(gs)
    for _ in range(steps):
        graph.replay()
    g1.record(gs)
    torch.cuda.synchronize()
    ms_graph = g0.elapsed_time(g1) / steps
    del graph
    fwd, bwd = train_flops()
    tfs = (fwd + bwd) / (ms * 1e-3) / 1e12
    tfs_graph = (fwd + bwd) / (ms_graph * 1e-3) / 1e12
    return dict(workload="cfg4: attention core fwd+bwd, B=8 T=2048 H=12 d_h=64 r=16 (j=48), learnable "
                         "per-channel decay, bf16 operands, fp32 decay/gate grads (projections excluded)",
                ms_per_step=round(ms, 4), ms_fwd_only=round(ms_fwd, 4), gflop=round((fwd + bwd) / 1e9, 2),
                tflops=round(tfs, 1), mfma_frac=round(tfs / MFMA_BF16_PEAK_TFS, 4),
                timing="eager launches (autograd), HIP events on the current stream",
                ms_per_step_graph=round(ms_graph, 4), tflops_graph=round(tfs_graph, 1),
                mfma_frac_graph=round(tfs_graph / MFMA_BF16_PEAK_TFS, 4),
                timing_graph="the same forward+backward step captured in one HIP graph, replayed")


# ---------------------------------------------------------------- full model (cfg5)
M_LAYERS, M_D, M_H, M_R, M_VOCAB = 24, 1024, 16, 16, 50304


def model_decode_bytes(model, B: int, L: int) -> int:
    """Algorithmic HBM bytes of one greedy decode step at attended length L:
    every layer's outlier caches (B*H*L*(r + d_h) bf16) and fp32 GLA state
    (read and written), plus every parameter once (bf16)."""
    n = 0
    for layer in model.layers:
        a = layer.attn
        n += B * a.num_heads * L * (a.r + a.d_head) * 2 + B * a.num_heads * a.j * a.d_head * 4 * 2
    return n + sum(p.numel() * p.element_size() for p in model.parameters())


def model_prefill_flops(B: int, T: int) -> float:
    """Algorithmic FLOPs of the cfg5 prefill: per layer the Q/K/V/out
    projections and the 4x MLP (2*B*T*12*d^2), the causal outlier attention
    (B*H*T^2*(r + d_h)) and the chunked GLA (6*B*H*T*j*d_h); the LM head on
    the last row only (what generation needs)."""
    dh = M_D // M_H
    j = dh - M_R
    per_layer = 2 * B * T * 12 * M_D * M_D + B * M_H * T * T * (M_R + dh) + 6 * B * M_H * T * j * dh
    return M_LAYERS * per_layer + 2 * B * M_D * M_VOCAB


def bench_model(B: int, prompt: int = 65536, steps: int = 256, warm: int = 4, seed: int = 5):
    """cfg5: a 24-layer 350M-style SubwordLM (d_model 1024, H=16, d_h=64, r=16,
    vocab 50304, bf16, random init from seed) prefills ``prompt`` random ids,
    then decodes ``steps`` greedy tokens from captured HIP graphs
    (outlierneuronattention_amd.decode_loop)."""
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.decode_loop import GreedyGraphDecoder
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import SubwordLM
    torch.manual_seed(seed)
    cfg = ModelConfig(d_model=M_D, num_heads=M_H, num_layers=M_LAYERS, r=M_R, device="cuda")
    with torch.device("cuda"):
        model = SubwordLM(M_VOCAB, cfg)
    model = model.to(torch.bfloat16).eval()
    gen = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, M_VOCAB, (B, prompt), generator=gen).to("cuda")
    dec = GreedyGraphDecoder(model, B, prompt + warm + steps + 1)
    with torch.no_grad():
        dec.prefill(ids[:, :2048])  # warm-up (GEMM heuristics, workspaces)
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        ev[0].record()
        dec.prefill(ids)
        ev[1].record()
        dec.decode(warm)          # eager step + graph capture + replays
        torch.cuda.synchronize()
        ev[2].record()
        toks = dec.decode(steps)  # graph replays only
        ev[3].record()
        torch.cuda.synchronize()
    pre_ms = ev[0].elapsed_time(ev[1])
    dec_ms = ev[2].elapsed_time(ev[3]) / steps
    L_mid = prompt + warm + steps // 2
    nbytes = model_decode_bytes(model, B, L_mid)
    fl = model_prefill_flops(B, prompt)
    distinct = int(torch.unique(toks).numel())
    del dec, model
    torch.cuda.empty_cache()
    return dict(B=B, prompt=prompt, steps=steps, prefill_ms=round(pre_ms, 2),
                prefill_tok_per_s=round(B * prompt / pre_ms * 1e3, 1),
                prefill_tflops=round(fl / (pre_ms * 1e-3) / 1e12, 1),
                decode_ms_per_step=round(dec_ms, 4), decode_tok_per_s=round(B / dec_ms * 1e3, 1),
                decode_bytes_per_step=nbytes, decode_gbs=round(nbytes / (dec_ms * 1e-3) / 1e9, 1),
                decode_hbm_frac=round(nbytes / (dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                distinct_tokens=distinct)


def cpu_baseline_decode(B: int, budget_s: float = 10.0):
    """Oracle decode step (torch CPU fp32) on the cfg3 shape: time until the
    budget is spent (at least 2 steps after one warm-up)."""
    from oracle import hofa_ref as ref
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(B, H, D, generator=gen)
    k = torch.randn(B, H, D, generator=gen)
    v = torch.randn(B, H, D, generator=gen)
    ck = torch.randn(B, H, L, R, generator=gen)
    cv = torch.randn(B, H, L, D, generator=gen)
    st = 0.1 * torch.randn(B, H, J, D, generator=gen)
    lg = F.logsigmoid(torch.randn(B, H, generator=gen)) / 16
    mix = torch.sigmoid(torch.randn(B, H, generator=gen))
    nw = torch.ones(H, D)
    sm = math.sqrt(D / R)
    ref.decode_step(q, k, v, ck, cv, L, st, lg, mix, nw, R, sm)
    n, t0 = 0, time.perf_counter()
    while True:
        ref.decode_step(q, k, v, ck, cv, L, st, lg, mix, nw, R, sm)
        n += 1
        el = time.perf_counter() - t0
        if (el >= budget_s and n >= 2) or n >= 10000:
            break
    return dict(value=B * n / el, unit="tok/s", cores=torch.get_num_threads(), kind="port",
                cpu_count=os.cpu_count(), cpu_model=host_info()["cpu_model"],
                sample=f"{n} decode steps of cfg3 at B={B} (H=16, d_h=64, r=16, L=32768) in fp32, "
                       f"oracle/hofa_ref.decode_step, {el:.1f} s")


def host_info():
    """The host the CPU legs run on: core count, CPU model and torch's thread count."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(cpu_count=os.cpu_count(), cpu_model=model, torch_threads=torch.get_num_threads())


def _median_time(fn, warmup: int = 3, reps: int = 5, budget_s: float = 20.0):
    """Median wall time of ``fn`` over ``reps`` runs after ``warmup`` runs;
    both counts shrink (to 1 and 3) when the budget would be exceeded."""
    t0 = time.perf_counter()
    fn()
    one = time.perf_counter() - t0
    if one * (warmup + reps) > budget_s:
        warmup, reps = 1, 3
    for _ in range(warmup - 1):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], warmup, reps


def _rand_layer_state(d_model, H, r, gen, alpha=False):
    """Random parameters with the module's names (std 0.02 projections,
    non-trivial gates) for the oracle's functional layer."""
    dh = d_model // H
    rn = lambda *sh, sd=1.0: torch.randn(*sh, generator=gen) * sd  # noqa: E731
    st = {"W_q.weight": rn(d_model, d_model, sd=0.02), "W_k.weight": rn(d_model, d_model, sd=0.02),
          "W_v.weight": rn(d_model, d_model, sd=0.02), "out_proj.weight": rn(d_model, d_model, sd=0.02),
          "gate_proj.weight": rn(H, 2 * dh, sd=0.1), "gate_proj.bias": torch.full((H,), -1.0),
          "mix_proj.weight": rn(H, 2 * dh, sd=0.1), "mix_proj.bias": torch.zeros(H),
          "gla_scale": torch.ones(1, H, 1, dh)}
    if alpha:
        st["log_alpha"] = torch.zeros(1, H, 1, dh - r)
    return st


# cfg1: one fp32 layer, d_model 256, H=4, d_h=64, r=16, prefill 512 then 16 decode steps fed back
C1_D, C1_H, C1_R, C1_T, C1_STEPS = 256, 4, 16, 512, 16


def bench_cfg1(reps: int = 20):
    """cfg1 on the GPU through the inference module (fp32): prefill of 512
    tokens then 16 decode steps, each fed the layer's last output row."""
    from outlierneuronattention_amd.config import ModelConfig
    from outlierneuronattention_amd.HybridOutlierFactorizedAttention import HybridOutlierFactorizedAttention
    torch.manual_seed(0)
    m = HybridOutlierFactorizedAttention(ModelConfig(d_model=C1_D, num_heads=C1_H, num_layers=1, r=C1_R,
                                                     device="cuda")).cuda().eval()
    x = torch.randn(1, C1_T, C1_D, generator=torch.Generator().manual_seed(1)).cuda()

    def run():
        with torch.no_grad():
            y, cache, state = m(x, return_state=True)
            t = y[:, -1:]
            for _ in range(C1_STEPS):
                t, cache, state = m.forward_step(t, cache, state)
        return t

    for _ in range(3):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    return dict(workload="cfg1: one fp32 layer (d_model 256, H=4, d_h=64, r=16), prefill 512 + 16 decode steps "
                         "fed back", ms_per_run=round(ms, 3), timing="host wall clock per run, eager launches")


def cpu_cfg1():
    """cfg1 on the host: the oracle layer (fp32) doing the same prefill and 16 fed-back steps."""
    from oracle import hofa_ref as ref
    gen = torch.Generator().manual_seed(0)
    o = ref.HOFARef(_rand_layer_state(C1_D, C1_H, C1_R, gen), C1_D, C1_H, C1_R, dtype=torch.float32)
    x = torch.randn(1, C1_T, C1_D, generator=gen)

    def run():
        with torch.no_grad():
            y, cache, state = o.forward(x, return_state=True)
            t = y[:, -1:]
            for _ in range(C1_STEPS):
                t, cache, state = o.forward_step(t, cache, state)

    sec, w, n = _median_time(run)
    return dict(value=round(sec * 1e3, 2), unit="ms per run", kind="port", cores=torch.get_num_threads(),
                sample=f"the full cfg1 run (oracle HOFARef, fp32), {w} warm-up + median of {n}")


def cpu_prefill(heads: int = 4):
    """cfg2 attention core on the host (oracle hofa_core, fp32) over ``heads``
    of the 64 (b, h) heads at full T=4096: TFLOP/s of the same algorithmic count."""
    from oracle import hofa_ref as ref
    gen = torch.Generator().manual_seed(4321)
    q, k, v = (torch.randn(1, heads, P_T, P_D, generator=gen) for _ in range(3))
    g = torch.clamp(F.logsigmoid(torch.randn(1, heads, P_T, P_J, generator=gen)) / 16, -5, 0)
    mix = torch.sigmoid(torch.randn(1, heads, P_T, generator=gen))
    gs = torch.ones(1, heads, 1, P_D)
    with torch.no_grad():
        sec, w, n = _median_time(lambda: ref.hofa_core(q, k, v, g, mix, gs, P_R, math.sqrt(P_D / P_R), eps=1e-5))
    fl = prefill_flops(B=1, H=heads)
    return dict(value=round(fl / sec / 1e12, 4), unit="TFLOP/s", kind="port", cores=torch.get_num_threads(),
                sample=f"{heads} of the 64 heads of cfg2 at full T=4096 (fp32, oracle hofa_core), "
                       f"{sec * 1e3:.0f} ms per call, {w} warm-up + median of {n}")


def cpu_train(heads: int = 2):
    """cfg4 attention core forward + backward on the host (float32 autograd of
    the oracle) over ``heads`` of the 96 (b, h) heads at full T=2048."""
    from oracle import hofa_ref as ref
    gen = torch.Generator().manual_seed(777)
    q, k, v = (torch.randn(1, heads, T_T, T_D, generator=gen).requires_grad_() for _ in range(3))
    J = T_D - T_R
    lg = torch.full((1, heads, T_T), -1.0)
    la = torch.log(-F.logsigmoid(2 + 4 * torch.rand(1, heads, 1, J, generator=gen))).requires_grad_()
    mix = torch.sigmoid(torch.randn(1, heads, T_T, generator=gen)).requires_grad_()
    gs = torch.ones(1, heads, 1, T_D, requires_grad=True)
    dy = torch.randn(1, heads, T_T, T_D, generator=gen)

    def step():
        y, _ = ref.hofa_core(q, k, v, ref.decay_from_gates(lg, J, la), mix, gs, T_R, math.sqrt(T_D / T_R))
        y.backward(dy)

    sec, w, n = _median_time(step)
    fwd, bwd = train_flops(B=1, H=heads)
    return dict(value=round((fwd + bwd) / sec / 1e12, 4), unit="TFLOP/s", kind="port",
                cores=torch.get_num_threads(),
                sample=f"{heads} of the 96 heads of cfg4 at full T=2048 (fp32 autograd of oracle hofa_core), "
                       f"{sec * 1e3:.0f} ms per step, {w} warm-up + median of {n}")


def cpu_model(T: int = 1024, steps: int = 8):
    """cfg5 on the host at reduced length: the 24-layer oracle LM (fp32,
    random weights) prefills T ids, then decodes ``steps`` greedy tokens."""
    from oracle import hofa_ref as ref
    gen = torch.Generator().manual_seed(5)
    sd = {}
    for i in range(M_LAYERS):
        for kk, vv in _rand_layer_state(M_D, M_H, M_R, gen).items():
            sd[f"layers.{i}.attn.{kk}"] = vv
        for nm, shape in (("ln_1", (M_D,)), ("ln_2", (M_D,))):
            sd[f"layers.{i}.{nm}.weight"] = torch.ones(*shape)
            sd[f"layers.{i}.{nm}.bias"] = torch.zeros(*shape)
        sd[f"layers.{i}.mlp.0.weight"] = torch.randn(4 * M_D, M_D, generator=gen) * 0.02
        sd[f"layers.{i}.mlp.0.bias"] = torch.zeros(4 * M_D)
        sd[f"layers.{i}.mlp.2.weight"] = torch.randn(M_D, 4 * M_D, generator=gen) * 0.02
        sd[f"layers.{i}.mlp.2.bias"] = torch.zeros(M_D)
    sd["lm_head.weight"] = torch.randn(M_VOCAB, M_D, generator=gen) * 0.02
    sd["ln_f.weight"], sd["ln_f.bias"] = torch.ones(M_D), torch.zeros(M_D)
    o = ref.SubwordLMRef(sd, M_D, M_H, [M_R] * M_LAYERS, dtype=torch.float32)
    ids = torch.randint(0, M_VOCAB, (1, T), generator=gen)
    with torch.no_grad():
        t0 = time.perf_counter()
        logits, caches, states = o.forward(ids, return_state=True, last_only=True)
        pre = time.perf_counter() - t0
        tok = logits[:, -1].argmax(-1, keepdim=True)
        t0 = time.perf_counter()
        for _ in range(steps):
            logits, caches, states = o.forward_step(tok, caches, states)
            tok = logits[:, -1].argmax(-1, keepdim=True)
        dec = (time.perf_counter() - t0) / steps
    return dict(value=round(1.0 / dec, 3), unit="tok/s (decode)", kind="port", cores=torch.get_num_threads(),
                prefill_tok_per_s=round(T / pre, 1),
                sample=f"cfg5 reduced to a {T}-token prompt (from 65536), B=1, 24 layers, fp32 oracle LM "
                       f"(random weights): prefill once, then {steps} greedy steps")


def calibrate_copy(nbytes: int = 1 << 30, reps: int = 20):
    """Plain device streams of known size through torch: a copy (read and
    write 1 GiB: the reference point that scales the FETCH_SIZE / WRITE_SIZE
    counters to bytes), a sum (read only) and an add (two reads per write).
    Their rates are the practical HBM ceilings for a kernel's read/write mix."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    half = nbytes // 8  # add: two inputs and one output of half the size each

    def rate(fn, moved):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        s = t0.elapsed_time(t1) / 1e3 / reps
        return s, round(moved / s / 1e9, 1)

    s, copy_gbs = rate(lambda: dst.copy_(src), 2 * nbytes)
    acc = torch.empty((), dtype=torch.float32, device="cuda")
    _, read_gbs = rate(lambda: torch.sum(src, dim=0, out=acc), nbytes)
    a, b, c = src[:half], src[half:2 * half], dst[:half]
    _, add_gbs = rate(lambda: torch.add(a, b, out=c), 3 * half * 4)
    return dict(bytes_read=nbytes, bytes_written=nbytes, us=round(s * 1e6, 2), gbs=copy_gbs,
                read_only_gbs=read_gbs, two_reads_per_write_gbs=add_gbs)


def _traffic_from_profile(name: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary, if present."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1])
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--batch", type=int, default=4, help="batch of the headline decode line")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--only", choices=["all", "decode", "prefill", "train", "model", "copy", "cpu"], default="all",
                    help="run one leg and print its result (profiling runs); default: the full line")
    ap.add_argument("--eager", action="store_true", help="decode with plain launches instead of graph replay")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the multi-GPU "
              "layout is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)
    if args.only == "cpu":  # the host legs alone (no GPU needed)
        res = dict(host=host_info(), cfg1=cpu_cfg1(), cfg2=cpu_prefill(), cfg3=cpu_baseline_decode(args.batch, 2.0),
                   cfg4=cpu_train(), cfg5=cpu_model())
        print(json.dumps({"only": "cpu", "result": res}), flush=True)
        return
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.only != "all":
        if args.only == "decode":
            res = bench_decode(args.batch, args.steps, args.warmup, eager=args.eager)
        elif args.only == "prefill":
            res = bench_prefill(max(5, min(50, args.steps // 20)), 3)
        elif args.only == "train":
            res = bench_train(max(5, min(20, args.steps // 50)), 3)
        elif args.only == "model":
            res = bench_model(args.batch)
        else:
            res = calibrate_copy()
        print(json.dumps({"only": args.only, "result": res}), flush=True)
        return

    other = 1 if args.batch != 1 else 4
    head = bench_decode(args.batch, args.steps, args.warmup)
    side = bench_decode(other, args.steps, args.warmup)
    hot = bench_decode_hot(1, min(args.steps, 500))
    prefill = bench_prefill(max(5, min(50, args.steps // 20)), 3)
    train = bench_train(max(5, min(20, args.steps // 50)), 3)
    model = {}
    for mb in (1, 4):
        try:
            model[f"B{mb}"] = bench_model(mb)
        except Exception as e:  # the headline line must still print
            model[f"B{mb}"] = {"error": f"{type(e).__name__}: {e}"[:300]}
    cfg1 = bench_cfg1()
    cpu = None
    if not args.skip_cpu:
        cpu = cpu_baseline_decode(args.batch, args.cpu_budget)
        cfg1["cpu_baseline"] = cpu_cfg1()
        prefill["cpu_baseline"] = cpu_prefill()
        train["cpu_baseline"] = cpu_train()
        model["cpu_baseline"] = cpu_model()
    achieved = head["gbs"]
    line = {
        "metric": "decode tok/s (split-K HOFA decode, 32k ctx)",
        "value": round(head["tok_per_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) caches, N(0,0.1) fp32 state; random gates)",
        "config": {"workload": "cfg3: split-K decode of one token, H=16 d_h=64 r=16, L=32768 bf16 cache, "
                               "fp32 48x64 GLA state per head",
                   "global_batch": args.batch, "seq_len": L, "parallelism": "none (1 GPU)",
                   "rotation_sets": head["rotation_sets"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": _traffic_from_profile(f"decode_cfg3_B{args.batch}_pmc.txt")},
        "cpu_baseline": cpu,
        "decode": {f"B{head['B']}": {k: round(v, 4) if isinstance(v, float) else v for k, v in head.items()},
                   f"B{side['B']}": {k: round(v, 4) if isinstance(v, float) else v for k, v in side.items()},
                   "B1_llc_resident": {k: round(v, 3) if isinstance(v, float) else v for k, v in hot.items()}},
        "host": host_info(),
        "cfg1": cfg1,
        "prefill_fwd": prefill,
        "train_fwd_bwd": train,
        "model_cfg5": dict(workload="cfg5: 24-layer SubwordLM (d_model 1024, H=16, d_h=64, r=16, vocab 50304, bf16, "
                                    "random init), prefill 65536 random ids, then 256 greedy steps from captured "
                                    "HIP graphs", **model),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
