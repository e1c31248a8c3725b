"""The prefill path's persistent strips: where a launch's tiles are a whole number k >= 2 of
waves over the 256 CUs, 256 workgroups each run k consecutive column tiles of one row block
(one group), and T = bf16(s x A^T), which depends only on the row block and the group, is
computed in the strip's first K loop and reused by the rest. The arithmetic is that of one
tile per workgroup, so the outputs are compared bit for bit with the prefill_strips override at -1, and
against the float64 oracle on rows sampled from every row block (rows are independent; bar
max|y - y_ref| / max|y_ref| <= 1e-2)."""
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


CASES = [
    # M, group widths, K, r; tiles -> workgroups x tiles per strip
    (8192, (2048, 1024, 1024), 1024, 32),  # q|k|v at config 2: 512 tiles of 256 x 256 -> 256 x 2
    (8192, (3072, 3072), 1024, 32),        # gate|up at config 2: 768 tiles -> 256 x 3
    (8192, (3072,), 1024, 32),             # one gate projection: 512 tiles of 256 x 192 -> 256 x 2
    (8000, (2048, 1024, 1024), 1024, 16),  # a partial last row block, one rank block of 16
    (4096, (4096,), 1024, 64),             # ranks 33-64: 512 tiles of 128 x 256 -> 256 x 2
    (4096, (2048, 2048), 2048, 48),        # grouped, two rank blocks, partial second block
]


def _inputs(M, ns, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    N = sum(ns)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(len(ns) * r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16()
    return x, W, A, B


def _run(gpu, x, W, A, B, ns):
    from weightshared_torchtitan_amd import ops
    d = lambda t: t.to(gpu)
    if len(ns) == 1:
        y = ops.lora_linear_op(d(x), d(W), None, d(A), d(B), 2.0)
    else:
        y = ops.lora_linear_grouped_op(d(x), d(W), None, d(A), d(B), 2.0, list(ns))
    torch.cuda.synchronize()
    return y.cpu()


@pytest.mark.parametrize("M,ns,K,r", CASES)
def test_strips_match_single_tiles_and_oracle(gpu, M, ns, K, r, wsl_opts):
    _say(f"[prefill strips] M={M} groups={ns} K={K} r={r}")
    x, W, A, B = _inputs(M, ns, K, r, seed=M + sum(ns) + K + r)
    wsl_opts(prefill_strips=0)
    y = _run(gpu, x, W, A, B, ns)
    wsl_opts(prefill_strips=-1)
    y_off = _run(gpu, x, W, A, B, ns)
    assert torch.equal(y, y_off), "strips differ from one tile per workgroup"
    # oracle on 3 rows of every 128-row block (first, middle, last row present)
    rows = sorted({min(b + o, M - 1) for b in range(0, M, 128) for o in (0, 61, 127)})
    xs = x[rows].float().numpy()
    yf = y[rows].float().numpy()
    c0 = 0
    for g, n in enumerate(ns):
        ref = O.lora_linear(xs, W[c0:c0 + n].float().numpy(), A[g * r:(g + 1) * r].float().numpy(),
                            B[c0:c0 + n].float().numpy(), 2.0)
        err = O.max_rel_err(yf[:, c0:c0 + n], ref)
        _say(f"   group {g}: max_rel_err {err:.2e} over {len(rows)} rows")
        assert np.isfinite(err) and err <= BF16_TOL
        c0 += n


def test_strips_on_the_shared_base_form(gpu, wsl_opts):
    """The shared-base launch (wsl::lora_linear_bcast, the reference's head sharing: one base
    W [1024, 1024] read through the broadcast_add row map by two LoRA pairs of width 2048,
    g = 8) at M = 8192: 512 tiles, strips of 2. Bit for bit against one tile per workgroup,
    and against the float64 oracle of broadcast_add on sampled rows."""
    from weightshared_torchtitan_amd import ops
    M, N, K, r, base_n, g, G = 8192, 2048, 1024, 32, 1024, 8, 2
    _say(f"[prefill strips, shared base] M={M} N={N} K={K} r={r} base_n={base_n} g={g} groups={G}")
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(M, K, generator=gen).bfloat16()
    W = (torch.randn(base_n, K, generator=gen) * 0.02).bfloat16()
    A = (torch.randn(G * r, K, generator=gen) * 0.02).bfloat16()
    B = (torch.randn(G * N, r, generator=gen) * 0.02).bfloat16()

    def run():
        y = ops.lora_linear_bcast_op(x.to(gpu), W.to(gpu), None, A.to(gpu), B.to(gpu), 2.0, g, G)
        torch.cuda.synchronize()
        return y.cpu()

    wsl_opts(prefill_strips=0)
    y = run()
    wsl_opts(prefill_strips=-1)
    assert torch.equal(y, run()), "strips differ from one tile per workgroup"
    rows = sorted({min(b + o, M - 1) for b in range(0, M, 256) for o in (0, 255)})
    xs = x[rows].float().numpy().astype("float64")
    base = xs @ W.float().numpy().T
    yf = y[rows].float().numpy()
    for j in range(G):
        delta = O.lora_delta(x[rows].float().numpy(), A[j * r:(j + 1) * r].float().numpy(),
                             B[j * N:(j + 1) * N].float().numpy(), 2.0)
        ref = O.broadcast_add(base, delta, dim=-1, g=g)
        err = O.max_rel_err(yf[:, j * N:(j + 1) * N], ref)
        _say(f"   group {j}: max_rel_err {err:.2e}")
        assert np.isfinite(err) and err <= BF16_TOL
