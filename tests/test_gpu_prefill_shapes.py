"""Forward parity of the prefill launches the benchmarks time, at their full shapes, with the
tile form each takes asserted through wsl_lora_linear_plan:

- config 2's o (8192 x 2048 -> 1024) and down (8192 x 3072 -> 1024): 128 x 256 tiles with one
  in-loop rank block, one tile per workgroup (two T blocks spread over four waves along n);
- Qwen3-1.7B o (8192 x 2048 -> 2048) and down (8192 x 6144 -> 2048): 256 x 256 tiles, one
  rank block, one tile per workgroup.

All four are one wave of tiles; over K >= 4096 (the 1.7B down) their column tiles share T
(tests/test_gpu_shared_t.py).

Rows are independent, so the float64 oracle runs on rows sampled from every 128-row block
(first, middle, last) of the GPU output (bar max|y - y_ref| / max|y_ref| <= 1e-2). Also the
grouped in-launch split-K case whose group ends fall on 192 but not 128 columns, which must
run group by group and match the oracle, and the shared-base backward above the kernels'
rank limit (three LoRA pairs of rank 128 on one base)."""
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


SHAPES = [
    # name, M, N, K, r, tile (m, n)
    ("c2 o", 8192, 1024, 2048, 32, (128, 256)),
    ("c2 down", 8192, 1024, 3072, 32, (128, 256)),
    ("1.7b o", 8192, 2048, 2048, 32, (256, 256)),
    ("1.7b down", 8192, 2048, 6144, 32, (256, 256)),
]


@pytest.mark.parametrize("name,M,N,K,r,tile", SHAPES, ids=[s[0] for s in SHAPES])
def test_one_wave_launches_match_oracle(gpu, name, M, N, K, r, tile):
    from weightshared_torchtitan_amd import ops
    _say(f"[prefill shape] {name}: M={M} N={N} K={K} r={r}")
    p = ops.plan(M, K, r, [N])
    assert p["path"] == "prefill" and (p["tile_m"], p["tile_n"]) == tile
    assert p["rank_blocks"] == 1 and p["strip_tiles"] == 1 and p["k_splits"] == 1 and p["launches"] == 1
    assert p["shared_t"] == (1 if K >= 4096 else 0)  # T shared by the column tiles over a long K
    g = torch.Generator().manual_seed(M + N + K + r)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16()
    y = ops.lora_linear_op(x.to(gpu), W.to(gpu), None, A.to(gpu), B.to(gpu), 2.0)
    y2 = ops.lora_linear_op(x.to(gpu), W.to(gpu), None, A.to(gpu), B.to(gpu), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rows = sorted({min(b + o, M - 1) for b in range(0, M, 128) for o in (0, 61, 127)})
    f = lambda t: t.float().numpy()
    ref = O.lora_linear(f(x[rows]), f(W), f(A), f(B), 2.0)
    err = O.max_rel_err(y.cpu()[rows].float().numpy(), ref)
    # the LoRA term alone, against its oracle (a wrong T block would show here first)
    delta = ops.lora_linear_op(x.to(gpu), None, None, A.to(gpu), B.to(gpu), 2.0).cpu()
    err_d = O.max_rel_err(delta[rows].float().numpy(), O.lora_delta(f(x[rows]), f(A), f(B), 2.0))
    _say(f"   max_rel_err {err:.2e} (delta alone {err_d:.2e}) over {len(rows)} rows")
    assert np.isfinite(err) and err <= BF16_TOL
    assert np.isfinite(err_d) and err_d <= BF16_TOL


@pytest.mark.parametrize("group_n", [(192, 192, 192), (256, 128, 128)])
def test_split_form_grouped_off_its_tiles(gpu, group_n):
    """M = 256, K = 4096, r = 16: the in-launch split-K form (128 x 128 tiles, each computing
    one group's T). Group ends at 192 and 384 are off its tiles, so the groups run one by one;
    ends at 256 and 384 keep one launch. Every group against the oracle."""
    from weightshared_torchtitan_amd import ops
    M, K, r = 256, 4096, 16
    p = ops.plan(M, K, r, list(group_n))
    _say(f"[split-K grouped] groups={group_n}: {p}")
    assert p["path"] == "prefill_splitk"
    assert p["launches"] == (3 if group_n[0] == 192 else 1)
    g = torch.Generator().manual_seed(sum(group_n) + 7)
    N = sum(group_n)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(len(group_n) * r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16()
    y = ops.lora_linear_grouped_op(x.to(gpu), W.to(gpu), None, A.to(gpu), B.to(gpu), 2.0, list(group_n))
    y = y.float().cpu().numpy()
    f = lambda t: t.float().numpy()
    c0 = 0
    for j, n in enumerate(group_n):
        ref = O.lora_linear(f(x), f(W[c0:c0 + n]), f(A[j * r:(j + 1) * r]), f(B[c0:c0 + n]), 2.0)
        err = O.max_rel_err(y[:, c0:c0 + n], ref)
        _say(f"   group {j}: max_rel_err {err:.2e}")
        assert np.isfinite(err) and err <= BF16_TOL
        c0 += n


def test_bcast_backward_above_rank_limit(gpu):
    """One base W [512, 512] shared by three LoRA pairs of rank 128 (the reference's
    qkv_sharing; 3 * 128 = 384 stacked ranks, above WSL_MAX_RANK): forward and every gradient
    against torch fp32 autograd of the composition on the CPU."""
    from weightshared_torchtitan_amd import ops
    M, K, N, r, G = 384, 512, 512, 128, 3
    _say(f"[bcast backward] M={M} K={K} N={N} r={r} groups={G}")
    g = torch.Generator().manual_seed(23)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(G * r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(G * N, r, generator=g) * 0.02).bfloat16()
    gy = torch.randn(M, G * N, generator=g).bfloat16()
    leaves = [t.float().requires_grad_(True) for t in (x, W, A, B)]
    xr, Wr, Ar, Br = leaves
    base = xr @ Wr.t()
    ref = torch.cat([base + 2.0 * (xr @ Ar[j * r:(j + 1) * r].t()) @ Br[j * N:(j + 1) * N].t() for j in range(G)], -1)
    ref.backward(gy.float())
    dl = [t.to(gpu).requires_grad_(True) for t in (x, W, A, B)]
    y = ops.lora_linear_bcast_op(dl[0], dl[1], None, dl[2], dl[3], 2.0, 1, G)
    y.backward(gy.to(gpu))
    torch.cuda.synchronize()
    assert O.max_rel_err(y.detach().float().cpu().numpy(), ref.detach().numpy()) <= BF16_TOL
    for name, got, want in zip(("dx", "dW", "dA", "dB"), dl, leaves):
        err = O.max_rel_err(got.grad.float().cpu().numpy(), want.grad.numpy())
        _say(f"   {name}: max_rel_err {err:.2e}")
        assert np.isfinite(err) and err <= BF16_TOL, name


@pytest.mark.parametrize("M,K,r,group_n", [
    (8192, 2048, 64, (6144, 6144)),        # 1.7B gate|up, 256 x 256 tiles
    (1024, 2048, 64, (6144, 6144)),        # 256 x 192 tiles
    (2000, 1024, 40, (2048, 1024, 1024)),  # ragged M, rank 40
])
def test_rank_33_to_64_from_the_prepass(gpu, M, K, r, group_n):
    """Ranks 33-64 on tiles wider than 128 x 128: T from the rank pre-pass over all groups,
    the K loop without rank work. Each group against the oracle on rows of every 128-row
    block, and the grouped launch against the single-group calls within the bar."""
    from weightshared_torchtitan_amd import ops
    _say(f"[rank 33-64 pre-pass] M={M} K={K} r={r} groups={group_n}")
    p = ops.plan(M, K, r, list(group_n))
    assert p["path"] == "prefill" and p["rank_prepass"] == 1 and p["rank_blocks"] == 0 and p["launches"] == 1
    g = torch.Generator().manual_seed(M + K + r)
    x = torch.randn(M, K, generator=g).bfloat16()
    Ws = [(torch.randn(n, K, generator=g) * 0.02).bfloat16() for n in group_n]
    As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16() for _ in group_n]
    Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16() for n in group_n]
    d = lambda t: t.to(gpu)  # noqa: E731
    y = ops.lora_linear_grouped_op(d(x), d(torch.cat(Ws)), None, d(torch.cat(As)), d(torch.cat(Bs)), 2.0,
                                   list(group_n))
    y2 = ops.lora_linear_grouped_op(d(x), d(torch.cat(Ws)), None, d(torch.cat(As)), d(torch.cat(Bs)), 2.0,
                                    list(group_n))
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    rows = sorted({min(b + o, M - 1) for b in range(0, M, 128) for o in (0, 61, 127)})
    f = lambda t: t.float().numpy()  # noqa: E731
    yc = y.cpu()
    n0 = 0
    for i, n in enumerate(group_n):
        ref = O.lora_linear(f(x[rows]), f(Ws[i]), f(As[i]), f(Bs[i]), 2.0)
        err = O.max_rel_err(f(yc[rows, n0:n0 + n]), ref)
        ys = ops.lora_linear_op(d(x), d(Ws[i]), None, d(As[i]), d(Bs[i]), 2.0).cpu()
        e_single = O.max_rel_err(f(yc[:, n0:n0 + n]), f(ys).astype("float64"))
        _say(f"   group {i}: max_rel_err {err:.2e}, against the single call {e_single:.2e}")
        assert np.isfinite(err) and err <= BF16_TOL
        assert e_single <= BF16_TOL
        n0 += n
