"""Shared T on the prefill path (the SKT form of prefill_kernel): a launch of one wave of
tiles with one in-loop rank block lets the column tiles of each row block (and group) share
T = s x . A^T. The group's first four tiles each compute one class of T's k steps (k step c
of every K tile), publish the fp32 partial and arrive at the row block's counter; every
tile sums the four classes in class order.

- The plan reports it where it applies (K >= 4096: the 1.7B down, a ragged M, grouped
  one-wave launches whose groups have four or more tiles) and not for shorter K, for
  persistent strips or for two rank blocks.
- Bit for bit against its no-wait path (WSL_OPT_PREFILL_SHARED_T = 1: every tile computes
  the four classes from x and A in global memory), on two calls in a row (the counters
  return to zero) and across graph replays.
- Within the bf16 bar of T computed in every tile (option -1; T's sums run in another order)
  and of the float64 oracle on rows sampled from every 128-row block."""
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


def _inputs(M, group_n, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    Ws = [(torch.randn(n, K, generator=g) * 0.02).bfloat16() for n in group_n]
    As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16() for _ in group_n]
    Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16() for n in group_n]
    return x, Ws, As, Bs


def _run(gpu, x, Ws, As, Bs, s):
    from weightshared_torchtitan_amd import ops
    d = lambda t: t.to(gpu)  # noqa: E731
    if len(Ws) == 1:
        return ops.lora_linear_op(d(x), d(Ws[0]), None, d(As[0]), d(Bs[0]), s)
    return ops.lora_linear_grouped_op(d(x), d(torch.cat(Ws)), None, d(torch.cat(As)), d(torch.cat(Bs)), s,
                                      [w.shape[0] for w in Ws])


def _with_option(value, fn):
    from weightshared_torchtitan_amd import _native
    _native.set_option("prefill_shared_t", value)
    try:
        out = fn()
        torch.cuda.synchronize()
        return out
    finally:
        _native.set_option("prefill_shared_t", 0)


CASES = [
    # name, M, group sizes, K, r, tile (m, n)
    ("1.7b down", 8192, (2048,), 6144, 32, (256, 256)),
    ("8192 x 4096 -> 1024", 8192, (1024,), 4096, 32, (128, 256)),
    ("ragged M, rank 24", 8000, (1024,), 4096, 24, (128, 256)),
    ("two groups", 4096, (1024, 1024), 4096, 32, (128, 256)),
    ("q|k|v-like groups", 2048, (2048, 1024, 1024), 4096, 16, (128, 256)),
    ("four groups, rank 8", 2048, (1024, 1024, 1024, 1024), 4096, 8, (128, 256)),
]


@pytest.mark.parametrize("name,M,group_n,K,r,tile", CASES, ids=[c[0] for c in CASES])
def test_shared_t_matches_its_fallback_and_the_oracle(gpu, name, M, group_n, K, r, tile):
    from weightshared_torchtitan_amd import ops
    _say(f"[shared T] {name}: M={M} groups={group_n} K={K} r={r}")
    p = ops.plan(M, K, r, list(group_n))
    assert p["path"] == "prefill" and (p["tile_m"], p["tile_n"]) == tile and p["launches"] == 1
    assert p["shared_t"] == 1 and p["strip_tiles"] == 1 and p["rank_blocks"] == 1
    x, Ws, As, Bs = _inputs(M, group_n, K, r, seed=M + sum(group_n) + K + r)
    y = _with_option(0, lambda: _run(gpu, x, Ws, As, Bs, 2.0))
    y2 = _with_option(0, lambda: _run(gpu, x, Ws, As, Bs, 2.0))
    assert torch.equal(y, y2), "two calls in a row differ (counters left set?)"
    y_fb = _with_option(1, lambda: _run(gpu, x, Ws, As, Bs, 2.0))
    assert torch.equal(y, y_fb), "the no-wait path differs from the shared classes"
    y_every = _with_option(-1, lambda: _run(gpu, x, Ws, As, Bs, 2.0))
    e_every = O.max_rel_err(y.cpu().float().numpy(), y_every.cpu().float().numpy())
    assert e_every <= BF16_TOL, e_every
    rows = sorted({min(b + o, M - 1) for b in range(0, M, 128) for o in (0, 61, 127)})
    yc = y.cpu()
    n0 = 0
    f = lambda t: t.float().numpy()  # noqa: E731
    for g, n in enumerate(group_n):
        ref = O.lora_linear(f(x[rows]), f(Ws[g]), f(As[g]), f(Bs[g]), 2.0)
        err = O.max_rel_err(f(yc[rows, n0:n0 + n]), ref)
        _say(f"   group {g}: max_rel_err {err:.2e} (against T in every tile {e_every:.2e})")
        assert np.isfinite(err) and err <= BF16_TOL
        n0 += n


def test_shared_t_not_taken_where_it_does_not_pay(gpu):
    """K below 4096 (config 2's o and down: the exchange costs what the rank MFMAs it saves
    do), multi-wave launches (persistent strips: T once per strip), ranks 33-64 (two rank
    blocks) and the pre-pass ranks keep T in every tile; so does option -1."""
    from weightshared_torchtitan_amd import _native, ops
    assert ops.plan(8192, 2048, 32, [1024])["shared_t"] == 0
    assert ops.plan(8192, 3072, 32, [1024])["shared_t"] == 0
    p = ops.plan(8192, 4096, 32, [2048, 1024, 1024])  # strips of two tiles
    assert p["strip_tiles"] == 2 and p["shared_t"] == 0
    assert ops.plan(8192, 4096, 64, [1024])["shared_t"] == 0
    assert ops.plan(8192, 4096, 128, [1024])["shared_t"] == 0
    _native.set_option("prefill_shared_t", -1)
    try:
        assert ops.plan(8192, 4096, 32, [1024])["shared_t"] == 0
    finally:
        _native.set_option("prefill_shared_t", 0)
    assert ops.plan(8192, 4096, 32, [1024])["shared_t"] == 1


def test_shared_t_graph_replays(gpu):
    """Captured in a HIP graph: every replay (with eager launches of other shapes between
    them, which use the same counters) equals the eager result."""
    from weightshared_torchtitan_amd import ops
    M, N, K, r = 8192, 1024, 4096, 32
    x, Ws, As, Bs = _inputs(M, (N,), K, r, seed=5)
    d = lambda t: t.to(gpu)  # noqa: E731
    xd, wd, ad, bd = d(x), d(Ws[0]), d(As[0]), d(Bs[0])
    want = ops.lora_linear_op(xd, wd, None, ad, bd, 2.0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.lora_linear_op(xd, wd, None, ad, bd, 2.0)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = ops.lora_linear_op(xd, wd, None, ad, bd, 2.0)
    x2, W2, A2, B2 = _inputs(4096, (1024, 1024), 4096, 32, seed=6)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
        _run(gpu, x2, W2, A2, B2, 2.0)  # another shared-T launch between replays
        torch.cuda.synchronize()


def test_shared_t_at_any_k_for_timing(gpu):
    """WSL_OPT_PREFILL_SHARED_T = 2 takes the shared form below 4096 too (the side-by-side
    timings of config 2's o): the plan reports it, and the output is within the bar of T in
    every tile and of the oracle."""
    from weightshared_torchtitan_amd import _native, ops
    M, N, K, r = 8192, 1024, 2048, 32
    assert ops.plan(M, K, r, [N])["shared_t"] == 0
    _native.set_option("prefill_shared_t", 2)
    try:
        assert ops.plan(M, K, r, [N])["shared_t"] == 1
    finally:
        _native.set_option("prefill_shared_t", 0)
    x, Ws, As, Bs = _inputs(M, (N,), K, r, seed=17)
    y = _with_option(2, lambda: _run(gpu, x, Ws, As, Bs, 2.0))
    y_every = _with_option(-1, lambda: _run(gpu, x, Ws, As, Bs, 2.0))
    assert O.max_rel_err(y.cpu().float().numpy(), y_every.cpu().float().numpy()) <= BF16_TOL
    rows = sorted({min(b + o, M - 1) for b in range(0, M, 128) for o in (0, 127)})
    f = lambda t: t.float().numpy()  # noqa: E731
    ref = O.lora_linear(f(x[rows]), f(Ws[0]), f(As[0]), f(Bs[0]), 2.0)
    assert O.max_rel_err(f(y.cpu()[rows]), ref) <= BF16_TOL
