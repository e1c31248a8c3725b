"""The prefill path's in-launch split-K form: shapes whose 128 x 128 tiles would leave most
CUs idle (a few rows of tokens, or narrow N) cut K over a second grid dimension; every split
runs the fused K loop (T included) over its part and leaves fp32 partial records, and the
split that arrives last at the tile's counter sums them in split order and finishes the
tile. Checked against the float64 oracle (bar max|y - y_ref| / max|y_ref| <= 1e-2), bitwise
repeatable (the sum does not depend on which split arrives last), at forced split counts
(the prefill_split override) against the unsplit tiles (prefill_split at -1; another summation
order, so within the bar), in graph replays, with shapes of different tile counts sharing
one workspace, and with every arrival counter back at zero after the launches."""
import ctypes
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


def _inputs(M, N, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16() if r else None
    return x, W, A, B


def _np(t):
    return None if t is None else t.float().numpy()


def _mode(wsl_opts, mode):
    if mode is None:
        wsl_opts(prefill_split=0)
    else:
        wsl_opts(prefill_split=-1 if mode == "off" else int(mode))


CASES = [
    # M, N, K, r
    (256, 2048, 2048, 64),   # o at 1.7B: 32 tiles, four splits
    (256, 2048, 6144, 64),   # down at 1.7B
    (192, 4096, 2048, 32),   # q|k|v width, one rank block
    (129, 1024, 1024, 16),   # one token past the decode path
    (200, 1000, 2048, 24),   # M and N off the tile grid, partial rank block
    (384, 1024, 3072, 0),    # plain linear
    (512, 2048, 1024, 64),
]


@pytest.mark.parametrize("M,N,K,r", CASES)
def test_split_form_matches_oracle(gpu, M, N, K, r, wsl_opts):
    import weightshared_torchtitan_amd as wsl
    _mode(wsl_opts, None)
    _say(f"[prefill split] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=7 * M + N + K + r)
    d = lambda t: None if t is None else t.to(gpu)
    y1 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    y2 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    err = O.max_rel_err(y1.float().cpu().numpy(), ref)
    _say(f"   max_rel_err {err:.2e}")
    assert np.isfinite(err) and err <= BF16_TOL
    # the unsplit tiles on the same inputs: the same bar, another order of the K sum
    _mode(wsl_opts, "off")
    y3 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    torch.cuda.synchronize()
    assert O.max_rel_err(y3.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("splits", [2, 4, 8, 16])
def test_forced_split_counts(gpu, splits, wsl_opts):
    """Every split count the form takes, on one shape (32 K tiles), against the oracle;
    the counts sum K in different orders, so they agree with each other to the bar."""
    import weightshared_torchtitan_amd as wsl
    M, N, K, r = 160, 640, 2048, 64
    _say(f"[prefill split forced] S={splits} M={M} N={N} K={K} r={r}")
    x, W, A, B = (t.to(gpu) for t in _inputs(M, N, K, r, seed=splits))
    _mode(wsl_opts, splits)
    y = wsl.lora_linear(x, W, A, B, 2.0)
    y2 = wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref = O.lora_linear(_np(x.cpu()), _np(W.cpu()), _np(A.cpu()), _np(B.cpu()), 2.0)
    assert O.max_rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL


@pytest.mark.parametrize("M,K,r,group_n", [
    (256, 2048, 64, (2048, 1024, 1024)),  # q|k|v at 1.7B
    (150, 2048, 32, (3072, 3072)),        # gate|up: the grouped launch splits in two, each group alone in four
    (300, 1024, 8, (1024, 512, 512)),
])
def test_split_form_grouped(gpu, M, K, r, group_n, wsl_opts):
    """A grouped launch runs whole; its split count follows its own tiles, so each group
    agrees with its single call within the bar, and with the oracle."""
    import weightshared_torchtitan_amd as wsl
    from weightshared_torchtitan_amd import ops
    _mode(wsl_opts, None)
    _say(f"[prefill split grouped] M={M} K={K} r={r} groups={group_n}")
    g = torch.Generator().manual_seed(M + K + r)
    x = torch.randn(M, K, generator=g).bfloat16().to(gpu)
    Ws = [(torch.randn(n, K, generator=g) * 0.02).bfloat16().to(gpu) for n in group_n]
    As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16().to(gpu) for _ in group_n]
    Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16().to(gpu) for n in group_n]
    y = ops.lora_linear_grouped_op(x, torch.cat(Ws), None, torch.cat(As), torch.cat(Bs), 2.0, list(group_n))
    xn = x.float().cpu().numpy()
    n0 = 0
    for i, n in enumerate(group_n):
        yi = wsl.lora_linear(x, Ws[i], As[i], Bs[i], 2.0).float()
        yg = y[:, n0:n0 + n].float()
        assert ((yg - yi).abs().max() / yi.abs().max()).item() <= BF16_TOL, i
        ref = O.lora_linear(xn, Ws[i].float().cpu().numpy(), As[i].float().cpu().numpy(),
                            Bs[i].float().cpu().numpy(), 2.0)
        err = O.max_rel_err(yg.cpu().numpy(), ref)
        _say(f"   group {i} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, i
        n0 += n


def test_split_form_graph_replays(gpu, wsl_opts):
    """Captured once and replayed with eager work between the replays: every replay equals
    the eager launch (the counters the replays leave behind start the next one at zero)."""
    import weightshared_torchtitan_amd as wsl
    _mode(wsl_opts, None)
    M, N, K, r = 256, 2048, 2048, 64
    _say(f"[prefill split graph] M={M} N={N} K={K} r={r}")
    x, W, A, B = (t.to(gpu) for t in _inputs(M, N, K, r, seed=11))
    eager = wsl.lora_linear(x, W, A, B, 2.0)
    s = torch.cuda.Stream(gpu)
    s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s):
        wsl.lora_linear(x, W, A, B, 2.0)  # the capture stream's workspace exists before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.current_stream(gpu).wait_stream(s)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        other = wsl.lora_linear(x[:200], W, A, B, 2.0)  # eager work in between
        torch.cuda.synchronize()
        assert other.shape == (200, N)


def test_split_counters_return_to_zero(gpu, wsl_opts):
    """Launches of two tile counts and split counts through one workspace, through the C ABI:
    the arrival counters in the workspace prefix are all zero afterwards, and each output
    equals its launch on a fresh workspace."""
    from weightshared_torchtitan_amd import _native as N_
    _mode(wsl_opts, None)
    shapes = [(256, 2048, 2048, 64), (160, 1024, 6144, 32), (256, 2048, 2048, 64)]
    nb = max(N_.workspace_bytes(M, N, K, r, N_.WSL_DTYPE_BF16) for M, N, K, r in shapes)
    ws = torch.zeros(nb // 8, dtype=torch.int64, device=gpu)
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    outs = []
    for i, (M, N, K, r) in enumerate(shapes):
        _say(f"[prefill split counters] M={M} N={N} K={K} r={r}")
        x, W, A, B = (t.to(gpu) for t in _inputs(M, N, K, r, seed=100 + M + K))
        y = torch.empty(M, N, dtype=torch.bfloat16, device=gpu)
        N_.check(N_.lib().wsl_lora_linear_fwd(p(x), K, p(W), K, N_.WSL_DTYPE_BF16, None, p(A), K, p(B), r, 2.0,
                                              p(y), N, M, N, K, r, p(ws), nb, stream), "wsl_lora_linear_fwd")
        fresh = torch.zeros_like(ws)
        y0 = torch.empty_like(y)
        N_.check(N_.lib().wsl_lora_linear_fwd(p(x), K, p(W), K, N_.WSL_DTYPE_BF16, None, p(A), K, p(B), r, 2.0,
                                              p(y0), N, M, N, K, r, p(fresh), nb, stream), "wsl_lora_linear_fwd")
        torch.cuda.synchronize()
        assert torch.equal(y, y0), i
        outs.append(y)
    assert torch.equal(outs[0], outs[2])
    prefix = ws[4096 // 8:65536 // 8].cpu()
    assert int((prefix != 0).sum()) == 0


@pytest.mark.parametrize("M,N,K,r", [
    (200, 16, 512, 0), (200, 100, 64, 0), (200, 1000, 128, 0), (130, 640, 192, 0), (256, 256, 256, 8),
    (300, 384, 320, 16), (129, 2048, 2048, 64), (512, 512, 4096, 40), (24 * 8, 16, 1024, 0),
])
def test_deep_ring_unsplit(gpu, M, N, K, r, wsl_opts):
    """The 128 x 128 tile's four-buffer ring (no more tiles than CUs) without the K split,
    every K tile count from one up: against the oracle."""
    import weightshared_torchtitan_amd as wsl
    _mode(wsl_opts, "off")
    _say(f"[deep ring] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=M * 3 + N + K + r)
    d = lambda t: None if t is None else t.to(gpu)
    y = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    torch.cuda.synchronize()
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    err = O.max_rel_err(y.float().cpu().numpy(), ref)
    _say(f"   max_rel_err {err:.2e}")
    assert err <= BF16_TOL
