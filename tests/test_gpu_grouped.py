"""GPU parity of the grouped LoRA linear (wsl_lora_linear_grouped_fwd): projections that
read the same x, stacked in N. Each group's output block must equal the single-projection
op on that group bit for bit (same kernels, same accumulation order; the grouped prefill
launch only selects each tile's rank block), and the float64 oracle within the forward's
bar (1e-2 bf16, 3e-2 fp8 base). Covers the one-launch prefill path (rank in-kernel and
through the pre-pass; 256-, 192- and 128-wide tiles), the per-group fallback (decode M,
group ends off the tile grid, unaligned K) and the backward against per-projection
autograd summed over the fan-out of x.
"""
import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP8_TOL = 3e-2


def _say(msg):
    print(msg, flush=True)


def _inputs(M, K, r, group_n, seed, fp8=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    Ws = [(torch.randn(n, K, generator=g) * 0.02) for n in group_n]
    As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16() for _ in group_n] if r else None
    Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16() for n in group_n] if r else None
    return x, Ws, As, Bs


CASES = [
    # M, K, r, group_n, s: the case it covers
    (1000, 256, 32, (2048, 1024, 1024), 2.0),   # q|k|v of Qwen3-0.6B, rank in-kernel (one block)
    (700, 512, 64, (1024, 512, 512), 2.0),      # two rank blocks: 128 x 256 tiles only
    (600, 256, 128, (512, 256, 256), 1.0),      # rank pre-pass over all groups (N = 3r)
    (8192, 128, 32, (3072, 3072), 2.0),         # gate|up: 256 x 192 or 256 x 256 tiles
    (4096, 256, 16, (384, 640), 2.0),           # boundary at 384: 128-wide tiles only
    (300, 192, 24, (128, 128, 256, 128), 2.0),  # four groups, odd rank
    (8, 512, 32, (1024, 512, 512), 2.0),        # decode-shaped M: one launch, T over 3 rank blocks
    (1, 2048, 64, (2048, 1024, 1024), 2.0),     # config-3 q|k|v at M = 1
    (32, 1024, 64, (1024, 512, 512), 2.0),      # M = 32: two token blocks
    (64, 512, 32, (1536, 1536), 2.0),           # M = 64, gate|up
    (3, 256, 16, (96, 160), 2.0),               # decode, boundary off the row groups: per group
    (500, 256, 16, (200, 120), 2.0),            # boundary off every tile grid: per group
    (260, 200, 16, (256, 128), 2.0),            # K % 64 != 0: generic path per group
    (512, 256, 0, (512, 256), 2.0),             # no LoRA: plain stacked linear
]


@pytest.mark.parametrize("M,K,r,group_n,s", CASES)
def test_grouped_matches_single_and_oracle(gpu, M, K, r, group_n, s):
    import weightshared_torchtitan_amd as wsl
    from weightshared_torchtitan_amd import ops
    _say(f"[grouped] M={M} K={K} r={r} groups={group_n} s={s}")
    x, Ws, As, Bs = _inputs(M, K, r, group_n, seed=M + K + r + len(group_n))
    Ws = [w.bfloat16() for w in Ws]
    w = torch.cat(Ws, 0)
    a = torch.cat(As, 0) if r else None
    b = torch.cat(Bs, 0) if r else None
    d = lambda t: None if t is None else t.to(gpu)
    y = ops.lora_linear_grouped_op(d(x), d(w), None, d(a), d(b), s, list(group_n)).cpu()
    n0 = 0
    for g, n in enumerate(group_n):
        yg = wsl.lora_linear(d(x), d(Ws[g]), d(As[g]) if r else None, d(Bs[g]) if r else None, s).cpu()
        assert torch.equal(y[:, n0:n0 + n], yg), f"group {g} differs from the single-projection op"
        ref = O.lora_linear(x.float().numpy(), Ws[g].float().numpy(), As[g].float().numpy() if r else None,
                            Bs[g].float().numpy() if r else None, s)
        err = O.max_rel_err(y[:, n0:n0 + n].float().numpy(), ref)
        _say(f"   group {g} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (g, err)
        n0 += n


def test_grouped_fp8_base(gpu):
    from weightshared_torchtitan_amd import lora, ops
    M, K, r, group_n = 512, 512, 128, (1024, 256, 256)
    _say(f"[grouped fp8] M={M} K={K} r={r} groups={group_n}")
    x, Ws, As, Bs = _inputs(M, K, r, group_n, seed=5)
    wq, sc = lora.quantize_fp8_per_channel(torch.cat(Ws, 0))
    y = ops.lora_linear_grouped_op(x.to(gpu), wq.to(gpu), sc.to(gpu), torch.cat(As).to(gpu),
                                   torch.cat(Bs).to(gpu), 1.0, list(group_n)).cpu()
    n0 = 0
    for g, n in enumerate(group_n):
        ref = O.lora_linear(x.float().numpy(), Ws[g].float().numpy(), As[g].float().numpy(),
                            Bs[g].float().numpy(), 1.0)
        err = O.max_rel_err(y[:, n0:n0 + n].float().numpy(), ref)
        _say(f"   group {g} max_rel_err {err:.2e} (against the fp32 W)")
        assert err <= FP8_TOL, (g, err)
        n0 += n


def test_grouped_in_graph_replays_match_eager(gpu):
    from weightshared_torchtitan_amd import ops
    M, K, r, group_n = 2048, 512, 128, (1024, 512, 512)
    _say(f"[grouped graph] M={M} K={K} r={r} groups={group_n}")
    x, Ws, As, Bs = _inputs(M, K, r, group_n, seed=9)
    args = [t.to(gpu) for t in (x, torch.cat(Ws).bfloat16(), torch.cat(As), torch.cat(Bs))]
    eager = ops.lora_linear_grouped_op(args[0], args[1], None, args[2], args[3], 2.0, list(group_n))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.lora_linear_grouped_op(args[0], args[1], None, args[2], args[3], 2.0, list(group_n))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = ops.lora_linear_grouped_op(args[0], args[1], None, args[2], args[3], 2.0, list(group_n))
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("M,K,r,group_n", [
    (1000, 256, 32, (512, 256, 256)),   # one launch, in-kernel rank
    (600, 256, 96, (256, 256)),         # one launch, pre-pass rank; dx at rank 192
    (8, 256, 16, (256, 128, 128)),      # decode-shaped: one grouped launch
    (300, 128, 128, (128, 128, 128)),   # G*r = 384 > WSL_MAX_RANK: dx per group, summed
])
def test_grouped_backward(gpu, M, K, r, group_n):
    """Gradients of the grouped op against the float64 oracle of the per-projection
    backward, with x's gradient summed over the groups (x fans out to every group)."""
    from weightshared_torchtitan_amd import ops
    _say(f"[grouped backward] M={M} K={K} r={r} groups={group_n}")
    x, Ws, As, Bs = _inputs(M, K, r, group_n, seed=M + r)
    Ws = [w.bfloat16() for w in Ws]
    g = torch.Generator().manual_seed(3)
    gy = torch.randn(M, sum(group_n), generator=g).bfloat16()
    leaf = lambda t: t.to(gpu).requires_grad_(True)
    tx, tw, ta, tb = leaf(x), leaf(torch.cat(Ws)), leaf(torch.cat(As)), leaf(torch.cat(Bs))
    y = ops.lora_linear_grouped_op(tx, tw, None, ta, tb, 2.0, list(group_n))
    y.backward(gy.to(gpu))
    torch.cuda.synchronize()
    dx_ref = 0
    n0 = 0
    checks = []
    for gi, n in enumerate(group_n):
        dx, dW, dA, dB = O.lora_linear_backward(x.float().numpy(), Ws[gi].float().numpy(), As[gi].float().numpy(),
                                                Bs[gi].float().numpy(), 2.0, gy[:, n0:n0 + n].float().numpy())
        dx_ref = dx_ref + dx
        checks += [(f"dW{gi}", tw.grad[n0:n0 + n], dW), (f"dA{gi}", ta.grad[gi * r:(gi + 1) * r], dA),
                   (f"dB{gi}", tb.grad[n0:n0 + n], dB)]
        n0 += n
    checks.append(("dx", tx.grad, dx_ref))
    for name, got, ref in checks:
        err = O.max_rel_err(got.float().cpu().numpy(), ref)
        _say(f"   {name} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (name, err)


def test_grouped_decode_t_wait_fallback(gpu, wsl_opts):
    """With the T poll bound at zero every W workgroup computes its group's T columns
    itself from x and the stacked A (the fallback reads rows g*r.. of a): same bits as
    the published path."""
    from weightshared_torchtitan_amd import ops
    M, K, r, group_n = 8, 1024, 32, (1024, 512, 512)
    _say(f"[grouped decode fallback] M={M} K={K} r={r} groups={group_n}")
    x, Ws, As, Bs = _inputs(M, K, r, group_n, seed=13)
    args = [t.to(gpu) for t in (x, torch.cat(Ws).bfloat16(), torch.cat(As), torch.cat(Bs))]
    y0 = ops.lora_linear_grouped_op(args[0], args[1], None, args[2], args[3], 2.0, list(group_n))
    torch.cuda.synchronize()
    wsl_opts(decode_spin_limit=-1)
    y1 = ops.lora_linear_grouped_op(args[0], args[1], None, args[2], args[3], 2.0, list(group_n))
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


def test_grouped_decode_fp8_base(gpu):
    from weightshared_torchtitan_amd import lora, ops
    M, K, r, group_n = 16, 1024, 128, (1024, 256, 256)
    _say(f"[grouped decode fp8] M={M} K={K} r={r} groups={group_n}")
    x, Ws, As, Bs = _inputs(M, K, r, group_n, seed=17)
    wq, sc = lora.quantize_fp8_per_channel(torch.cat(Ws, 0))
    d = lambda t: t.to(gpu)
    y = ops.lora_linear_grouped_op(d(x), d(wq), d(sc), d(torch.cat(As)), d(torch.cat(Bs)), 1.0, list(group_n)).cpu()
    import weightshared_torchtitan_amd as wsl
    n0 = 0
    for g, n in enumerate(group_n):
        yg = wsl.lora_linear(d(x), d(wq[n0:n0 + n].contiguous()), d(As[g]), d(Bs[g]), 1.0,
                             w_scale=d(sc[n0:n0 + n].contiguous())).cpu()
        assert torch.equal(y[:, n0:n0 + n], yg), g
        ref = O.lora_linear(x.float().numpy(), Ws[g].float().numpy(), As[g].float().numpy(), Bs[g].float().numpy(), 1.0)
        err = O.max_rel_err(y[:, n0:n0 + n].float().numpy(), ref)
        _say(f"   group {g} max_rel_err {err:.2e}")
        assert err <= FP8_TOL, (g, err)
        n0 += n
