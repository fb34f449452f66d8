"""GPU parity of the split-K decode kernel against the CPU oracle.

Tolerances (stated by the build's parity bar):
* y (bf16/fp16 output) vs the float64 oracle on the same rounded inputs:
  max-abs <= 2e-2; float32 output: max-abs <= 1e-4.
* state_out (float32 arithmetic on both sides): relative L2 error <= 1e-5.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import hofa_ref as ref

pytestmark = pytest.mark.gpu

DEV = "cuda"


def make_case(B, H, L, seq_len, D, R, dtype, alpha=False, seed=0, fixed_mix=False, strided_q=False,
              alpha_layout=4):
    gen = torch.Generator().manual_seed(seed)
    J = D - R
    f32 = dict(dtype=torch.float32)
    qkv = torch.randn(B, 1, H, 3 * D, generator=gen, **f32).to(DEV, dtype)  # [B,N,H,d]-style memory
    q, k, v = (qkv[..., i * D:(i + 1) * D].transpose(1, 2) for i in range(3))
    cache_k = torch.randn(B, H, L, R, generator=gen, **f32)
    cache_v = torch.randn(B, H, L, D, generator=gen, **f32)
    cache_k[:, :, seq_len:] = float("nan")  # rows past seq_len must never be read
    cache_v[:, :, seq_len:] = float("nan")
    state = 0.1 * torch.randn(B, H, J, D, generator=gen, **f32)
    lg = torch.clamp(F.logsigmoid(torch.randn(B, H, 1, generator=gen, **f32)) / 16, -5, 0)
    if fixed_mix:
        mix = torch.sigmoid(torch.randn(1, H, 1, 1, generator=gen, **f32)).expand(B, H, 1, 1)[..., 0]
    else:
        mix = torch.sigmoid(torch.randn(B, H, 1, generator=gen, **f32))
    norm_w = 1 + 0.2 * torch.randn(H, D, generator=gen, **f32)
    la = 0.5 * torch.randn(1, H, 1, J, generator=gen, **f32) if alpha else None
    sm = math.sqrt(D / R)

    g = dict(q=q, k=k, v=v,
             cache_k=cache_k.to(DEV, dtype), cache_v=cache_v.to(DEV, dtype),
             state_in=state.to(DEV), log_gamma=lg.to(DEV), mix=mix.to(DEV), norm_w=norm_w.to(DEV),
             log_alpha=None)
    if alpha:
        g["log_alpha"] = {4: la, 2: la.reshape(H, J), 1: la.reshape(H * J)}[alpha_layout].to(DEV)
    if strided_q:
        assert not g["q"].is_contiguous()
    # oracle inputs: the exact values the GPU sees, in float64
    c = {kk: (vv.detach().cpu().double() if vv is not None else None) for kk, vv in g.items()}
    y_ref, s_ref = ref.decode_step(c["q"][:, :, 0], c["k"][:, :, 0], c["v"][:, :, 0], c["cache_k"], c["cache_v"],
                                   seq_len, c["state_in"], c["log_gamma"][..., 0], c["mix"][..., 0], c["norm_w"],
                                   R, sm, eps=float(torch.finfo(torch.float32).eps),
                                   log_alpha=None if la is None else la.double().reshape(H, J))
    return g, sm, y_ref, s_ref


def run(g, R, seq_len, sm, split_k=None, seq_len_dev=None):
    from outlierneuronattention_amd import fused_hofa_decode
    out = torch.empty_like(g["state_in"])
    y = fused_hofa_decode(g["q"], g["k"], g["v"], g["cache_k"], g["cache_v"], g["state_in"], out,
                          g["log_gamma"], g["mix"], g["norm_w"], R, seq_len, sm, split_k=split_k,
                          log_alpha=g["log_alpha"], seq_len_dev=seq_len_dev)
    torch.cuda.synchronize()
    return y, out


def check(y, s, y_ref, s_ref, dtype):
    assert torch.isfinite(y).all()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    err = (y[:, :, 0].double().cpu() - y_ref).abs().max().item()
    assert err <= tol, f"y max-abs err {err}"
    rel = ((s.double().cpu() - s_ref).norm() / s_ref.norm()).item()
    assert rel <= 1e-5, f"state rel err {rel}"


CASES = [
    # B, H, L, seq_len, D, R, dtype, alpha, split_k
    (2, 3, 1000, 777, 64, 16, torch.bfloat16, False, None),
    (1, 16, 4096, 4096, 64, 16, torch.bfloat16, True, None),
    (1, 4, 300, 1, 64, 16, torch.bfloat16, False, None),
    (2, 2, 5000, 4999, 64, 16, torch.bfloat16, True, 1),
    (2, 2, 5000, 4999, 64, 16, torch.bfloat16, True, 7),
    (1, 2, 70000, 65537, 64, 16, torch.bfloat16, False, 64),
    (2, 4, 2048, 1500, 64, 32, torch.bfloat16, True, None),
    (2, 4, 2048, 2048, 128, 16, torch.bfloat16, True, None),
    (1, 4, 3000, 2222, 128, 32, torch.float16, False, None),
    (1, 4, 3000, 2999, 128, 64, torch.bfloat16, True, None),
    (2, 3, 1024, 1000, 64, 16, torch.float32, True, None),
    (1, 2, 2048, 2047, 128, 16, torch.float32, False, 3),
]


@pytest.mark.parametrize("B,H,L,seq_len,D,R,dtype,alpha,split_k", CASES)
def test_decode_matches_oracle(B, H, L, seq_len, D, R, dtype, alpha, split_k):
    print(f"decode case B={B} H={H} L={L} seq={seq_len} D={D} R={R} {dtype} alpha={alpha} split={split_k}",
          flush=True)
    g, sm, y_ref, s_ref = make_case(B, H, L, seq_len, D, R, dtype, alpha, strided_q=True)
    y, s = run(g, R, seq_len, sm, split_k)
    check(y, s, y_ref, s_ref, dtype)


@pytest.mark.parametrize("B", [1, 4])
def test_decode_cfg3_full_size(B):
    """BASELINE cfg3: H=16, d_h=64, r=16, 32768-row bf16 cache."""
    print(f"decode cfg3 B={B}", flush=True)
    g, sm, y_ref, s_ref = make_case(B, 16, 32768, 32768, 64, 16, torch.bfloat16, seed=B)
    y, s = run(g, 16, 32768, sm)
    check(y, s, y_ref, s_ref, torch.bfloat16)


def test_decode_variants_fixed_mix_and_alpha_layouts():
    for layout in (4, 2, 1):
        g, sm, y_ref, s_ref = make_case(2, 3, 512, 300, 64, 16, torch.bfloat16, alpha=True, fixed_mix=True,
                                        alpha_layout=layout, seed=layout)
        y, s = run(g, 16, 300, sm)
        check(y, s, y_ref, s_ref, torch.bfloat16)


def test_decode_device_seq_len_and_repeat():
    """seq_len read on the device; repeated calls reuse the workspace and are bitwise stable."""
    g, sm, y_ref, s_ref = make_case(1, 4, 8192, 5000, 64, 16, torch.bfloat16, alpha=True, seed=11)
    sl = torch.tensor([5000], dtype=torch.int32, device=DEV)
    y1, s1 = run(g, 16, 0, sm, seq_len_dev=sl)
    check(y1, s1, y_ref, s_ref, torch.bfloat16)
    for _ in range(3):
        y2, s2 = run(g, 16, 0, sm, seq_len_dev=sl)
        assert torch.equal(y1, y2) and torch.equal(s1, s2)
    # a shorter length through the same device scalar
    g2, _, y_ref2, s_ref2 = make_case(1, 4, 8192, 1234, 64, 16, torch.bfloat16, alpha=True, seed=11)
    sl.fill_(1234)
    y3, s3 = run(g2, 16, 0, sm, seq_len_dev=sl)
    check(y3, s3, y_ref2, s_ref2, torch.bfloat16)


def test_decode_graph_replay_advancing_length():
    """A captured decode replays correctly while the device-side length advances."""
    g, sm, _, _ = make_case(1, 4, 4096, 4096, 64, 16, torch.bfloat16, seed=5)
    from outlierneuronattention_amd import fused_hofa_decode
    sl = torch.tensor([100], dtype=torch.int32, device=DEV)
    out = torch.empty_like(g["state_in"])
    args = (g["q"], g["k"], g["v"], g["cache_k"], g["cache_v"], g["state_in"], out, g["log_gamma"], g["mix"],
            g["norm_w"], 16, 0, sm)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fused_hofa_decode(*args, seq_len_dev=sl)  # warm-up allocates the workspace
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            y_g = fused_hofa_decode(*args, seq_len_dev=sl)
    torch.cuda.synchronize()
    for n in (100, 2000, 4096, 1):
        sl.fill_(n)
        graph.replay()
        torch.cuda.synchronize()
        y_e = fused_hofa_decode(*args[:11], n, sm)
        torch.cuda.synchronize()
        assert torch.equal(y_g, y_e), n


def test_workspace_outlives_graph_capture():
    """A graph captured with a small decode workspace still owns it after an
    eager call on the same stream needs a larger one: replays must not write
    into memory the allocator has handed to other tensors."""
    from outlierneuronattention_amd import _lib, fused_hofa_decode
    L, short = 40000, 512
    g, sm, _, _ = make_case(1, 16, L, L, 64, 16, torch.bfloat16, seed=21)
    out = torch.empty_like(g["state_in"])
    base = (g["q"], g["k"], g["v"], g["cache_k"], g["cache_v"], g["state_in"], out, g["log_gamma"], g["mix"],
            g["norm_w"], 16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    print("workspace vs graph: capture at a short length", flush=True)
    with torch.cuda.stream(s):
        fused_hofa_decode(*base, short, sm)  # sizes this stream's workspace for the short plan
        s.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            y_g = fused_hofa_decode(*base, short, sm)
        s.synchronize()
        retired0 = _lib.WORKSPACES.retired_bytes()
        fused_hofa_decode(*base, L, sm)  # needs a larger workspace on the same stream
        s.synchronize()
        assert _lib.WORKSPACES.retired_bytes() > retired0
        # tensors that would reuse a freed workspace block
        bystanders = [torch.full((16384,), 0x5A, dtype=torch.uint8, device=DEV) for _ in range(64)]
        s.synchronize()
        graph.replay()
        s.synchronize()
        y_e = fused_hofa_decode(*base, short, sm)
        s.synchronize()
    assert torch.equal(y_g, y_e)
    for t in bystanders:
        assert bool((t == 0x5A).all())
