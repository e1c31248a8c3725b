"""Chains of decode-shaped LoRA linears in one persistent launch (wsl_lora_linear_chain_fwd):
every stage's output equals the stage run alone (wsl_lora_linear_fused_fwd or the grouped
launch) bit for bit, for the weight-shared Qwen3 decode layer's dependent chain (o with the
residual, gate|up with RMSNorm and SwiGLU, down with the residual, the next layer's q|k|v
with RMSNorm) and for independent grouped projections; graph replays repeat the eager
result; a stage wait forced to give up from the host is reported by the status word and the
launch still drains."""
import sys

import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _r(g, *shape, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


def _layer(dev, M, seed, dim=1024, q=2048, kv=1024, hidden=3072, r=32):
    """Operands of one weight-shared Qwen3-0.6B decode layer's chain stages (config 4 dims)."""
    g = torch.Generator().manual_seed(seed)
    t = {
        "attn": _r(g, M, q), "h": _r(g, M, dim),
        "wo": _r(g, dim, q, scale=0.02), "ao": _r(g, r, q, scale=0.02), "bo": _r(g, dim, r, scale=0.02),
        "ffn_norm": (1.0 + 0.1 * torch.randn(dim, generator=g)).bfloat16(),
        "wgu": _r(g, 2 * hidden, dim, scale=0.02), "agu": _r(g, 2 * r, dim, scale=0.02),
        "bgu": _r(g, 2 * hidden, 2 * r, scale=0.02),
        "w2": _r(g, dim, hidden, scale=0.02), "a2": _r(g, r, hidden, scale=0.02), "b2": _r(g, dim, r, scale=0.02),
        "attn_norm": (1.0 + 0.1 * torch.randn(dim, generator=g)).bfloat16(),
        "wqkv": _r(g, q + 2 * kv, dim, scale=0.02), "aqkv": _r(g, 3 * r, dim, scale=0.02),
        "bqkv": _r(g, q + 2 * kv, 3 * r, scale=0.02),
    }
    return {k: v.to(dev) for k, v in t.items()}


def _separate(t, eps=1e-6):
    from weightshared_torchtitan_amd import ops
    fl = ops.lora_linear_fused_op
    h1 = fl(t["attn"], None, 0.0, t["wo"], t["ao"], t["bo"], 2.0, t["h"], 4)
    act = fl(h1, t["ffn_norm"], eps, t["wgu"], t["agu"], t["bgu"], 2.0, None, 3)
    h2 = fl(act, None, 0.0, t["w2"], t["a2"], t["b2"], 2.0, h1, 4)
    qkv = fl(h2, t["attn_norm"], eps, t["wqkv"], t["aqkv"], t["bqkv"], 2.0, None, 1)
    return h1, act, h2, qkv


def _chain_stages(t, outs, eps=1e-6):
    from weightshared_torchtitan_amd import ops
    from weightshared_torchtitan_amd._native import WSL_FUSE_RESIDUAL as RES, WSL_FUSE_RMSNORM as NORM, \
        WSL_FUSE_SWIGLU as ACT
    h1, act, h2, qkv = outs
    S = ops.ChainStage
    return [S(t["attn"], t["wo"], t["ao"], t["bo"], 2.0, h1, fuse=RES, residual=t["h"]),
            S(h1, t["wgu"], t["agu"], t["bgu"], 2.0, act, fuse=NORM | ACT, norm_w=t["ffn_norm"], eps=eps,
              after_previous=True),
            S(act, t["w2"], t["a2"], t["b2"], 2.0, h2, fuse=RES, residual=h1, after_previous=True),
            S(h2, t["wqkv"], t["aqkv"], t["bqkv"], 2.0, qkv, fuse=NORM, norm_w=t["attn_norm"], eps=eps,
              after_previous=True)]


def _empty_outs(t, M, dev):
    e = lambda n: torch.empty(M, n, dtype=torch.bfloat16, device=dev)  # noqa: E731
    return e(1024), e(3072), e(1024), e(4096)


@pytest.mark.parametrize("M", [8, 1, 16])
def test_decode_layer_chain_equals_separate_launches(gpu, M):
    from weightshared_torchtitan_amd import ops
    _say(f"[chain] decode layer o -> gate|up -> down -> q|k|v, M={M}")
    t = _layer(gpu, M, seed=100 + M)
    want = _separate(t)
    outs = _empty_outs(t, M, gpu)
    stages = _chain_stages(t, outs)
    assert ops.chain_supported(stages, M)
    ops.lora_linear_chain(stages, M)
    torch.cuda.synchronize()
    assert not ops.chain_status(gpu)
    for name, got, w in zip(("h1", "act", "h2", "qkv"), outs, want):
        assert torch.equal(got, w), name
    # and against the float64 oracle for the first stage (the residual epilogue)
    f = lambda x: x.float().cpu().numpy()  # noqa: E731
    o = O.lora_linear(f(t["attn"]), f(t["wo"]), f(t["ao"]), f(t["bo"]), 2.0)
    ref = f(t["h"]).astype(np.float64) + O.bf16_round(o)
    assert O.max_rel_err(f(outs[0]), ref) <= BF16_TOL


@pytest.mark.parametrize("M", [1, 8])
def test_independent_grouped_chain_equals_grouped_launches(gpu, M):
    """Qwen3-1.7B's four grouped projections of a layer (q|k|v, o, gate|up, down; rank 64) as
    independent stages of one chain against each grouped or single launch alone."""
    from weightshared_torchtitan_amd import ops
    _say(f"[chain] independent 1.7B projections, M={M}")
    g = torch.Generator().manual_seed(7 + M)
    r = 64
    specs = [((2048, 1024, 1024), 2048), ((2048,), 2048), ((6144, 6144), 2048), ((2048,), 6144)]
    stages, want = [], []
    for ns, K in specs:
        N = sum(ns)
        x = _r(g, M, K).to(gpu)
        w = _r(g, N, K, scale=0.02).to(gpu)
        a = _r(g, len(ns) * r, K, scale=0.02).to(gpu)
        b = _r(g, N, r, scale=0.02).to(gpu)
        y = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        stages.append(ops.ChainStage(x, w, a, b, 2.0, y, group_n=ns))
        want.append(ops.lora_linear_grouped_op(x, w, None, a, b, 2.0, list(ns)) if len(ns) > 1
                    else ops.lora_linear_op(x, w, None, a, b, 2.0))
    assert ops.chain_supported(stages, M)
    ops.lora_linear_chain(stages, M)
    torch.cuda.synchronize()
    assert not ops.chain_status(gpu)
    for i, (st, w) in enumerate(zip(stages, want)):
        assert torch.equal(st.y, w), i


def test_chain_graph_replays(gpu):
    """A captured chain replayed three times, with eager work between the replays: every
    replay's outputs equal the eager chain's."""
    from weightshared_torchtitan_amd import ops
    M = 8
    _say("[chain] graph replays")
    t = _layer(gpu, M, seed=31)
    outs = _empty_outs(t, M, gpu)
    stages = _chain_stages(t, outs)
    ops.lora_linear_chain(stages, M)
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.lora_linear_chain(stages, M)  # the stream's workspace, before the capture
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        ops.lora_linear_chain(stages, M)
    for _ in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            assert torch.equal(o, w)
        _separate(t)  # eager work between the replays
    with torch.cuda.stream(s):
        assert not ops.chain_status(gpu)


def test_chain_wait_given_up_is_reported(gpu, wsl_opts):
    """With the decode poll bound forced to no polling from the host, the gate|up stage's
    workgroups that had no o work reach their wait before o can be done and give up: the
    launch drains, the status word reports it once, and the next chain with the default
    bound is correct and reports nothing."""
    from weightshared_torchtitan_amd import ops
    M = 8
    _say("[chain] forced wait failure")
    t = _layer(gpu, M, seed=37)
    want = _separate(t)
    outs = _empty_outs(t, M, gpu)
    stages = _chain_stages(t, outs)
    wsl_opts(decode_spin_limit=-1)
    ops.lora_linear_chain(stages, M)
    torch.cuda.synchronize()
    assert ops.chain_status(gpu)
    assert not ops.chain_status(gpu)  # cleared by the read
    wsl_opts(decode_spin_limit=0)
    ops.lora_linear_chain(stages, M)
    torch.cuda.synchronize()
    assert not ops.chain_status(gpu)
    for got, w in zip(outs, want):
        assert torch.equal(got, w)


def test_chain_refuses_unsupported_stages(gpu):
    """M above one token block, or a stage whose x needs a K split, is refused on the host."""
    from weightshared_torchtitan_amd import ops
    t = _layer(gpu, 32, seed=3)
    outs = _empty_outs(t, 32, gpu)
    assert not ops.chain_supported(_chain_stages(t, outs), 32)
    with pytest.raises(ValueError):
        ops.lora_linear_chain(_chain_stages(t, outs), 32)
