"""The decode path's wide form from 65 to 72 tokens (plain bf16 launches, taken with the
decode_wide override at 1; by default these shapes run on the prefill path's split-K form):
five token blocks, four waves along K, x walked in pass slices of 512 or 1024 columns, the
slices spread over the K splits that keep one wave of workgroups. Against the float64 oracle
(1e-2), bitwise repeatable, with the T wait forced to its local fallback, beside the prefill
path (the default) on the same inputs, and as grouped launches. The K split count
fills one wave of workgroups, so it depends on N: a grouped launch may sum a group's rows in
another order than the group's single launch, and the two agree within the bar (below 65
tokens they agree bit for bit)."""
import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


def _np(t):
    return None if t is None else t.float().numpy()


def _inputs(M, N, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16() if r else None
    return x, W, A, B


CASES = [
    # M, N, K, r
    (65, 2048, 2048, 64),    # 1024-column passes (x of 65 rows fits), o at 1.7B
    (72, 6144, 2048, 64),    # 512-column passes, 64 rows per workgroup
    (72, 2048, 6144, 64),    # twelve slices over K splits and passes (down at 1.7B)
    (70, 1000, 2048, 24),    # N tail, partial rank group
    (68, 4096, 1024, 16),
    (72, 12288, 2048, 64),   # gate|up at 1.7B, one wave of workgroups
    (66, 3072, 1024, 0),     # plain linear
    (71, 640, 4096, 8),
]


@pytest.mark.parametrize("M,N,K,r", CASES)
def test_wide_decode_matches_oracle(gpu, M, N, K, r, wsl_opts):
    import weightshared_torchtitan_amd as wsl
    wsl_opts(decode_wide=1)
    _say(f"[decode wide] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=5 * M + N + K + r)
    d = lambda t: None if t is None else t.to(gpu)
    y1 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    y2 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    err = O.max_rel_err(y1.float().cpu().numpy(), ref)
    _say(f"  max_rel_err={err:.3e}")
    assert np.isfinite(err) and err <= BF16_TOL
    # the prefill path's split-K form (the default) on the same inputs: same bar, a different kernel
    wsl_opts(decode_wide=0)
    y3 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    torch.cuda.synchronize()
    assert O.max_rel_err(y3.float().cpu().numpy(), ref) <= BF16_TOL


def test_wide_decode_t_fallback(gpu, wsl_opts):
    """T wait bound forced to zero from the host: the W workgroups compute T themselves."""
    import weightshared_torchtitan_amd as wsl
    wsl_opts(decode_wide=1)
    M, N, K, r = 72, 2048, 6144, 64
    _say(f"[decode wide T fallback] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=53)
    d = lambda t: t.to(gpu)
    wsl_opts(decode_spin_limit=-1)
    y = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0).float().cpu().numpy()
    torch.cuda.synchronize()
    wsl_opts(decode_spin_limit=0)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    assert O.max_rel_err(y, ref) <= BF16_TOL


@pytest.mark.parametrize("M,K,group_n", [
    (72, 2048, (6144, 6144)),        # gate|up
    (70, 2048, (2048, 1024, 1024)),  # q|k|v
    (72, 6144, (2048, 2048)),
    (65, 1024, (3072, 3072, 1024)),
])
def test_wide_decode_grouped_matches_single(gpu, M, K, group_n, wsl_opts):
    import weightshared_torchtitan_amd as wsl
    from weightshared_torchtitan_amd import ops
    wsl_opts(decode_wide=1)
    r = 64
    _say(f"[decode wide grouped] M={M} K={K} r={r} groups={group_n}")
    g = torch.Generator().manual_seed(M + K + len(group_n))
    x = torch.randn(M, K, generator=g).bfloat16().to(gpu)
    Ws = [(torch.randn(n, K, generator=g) * 0.02).bfloat16().to(gpu) for n in group_n]
    As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16().to(gpu) for _ in group_n]
    Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16().to(gpu) for n in group_n]
    y = ops.lora_linear_grouped_op(x, torch.cat(Ws), None, torch.cat(As), torch.cat(Bs), 2.0, list(group_n))
    n0 = 0
    xn = x.float().cpu().numpy()
    for i, n in enumerate(group_n):
        yi = wsl.lora_linear(x, Ws[i], As[i], Bs[i], 2.0).float()
        yg = y[:, n0:n0 + n].float()
        assert ((yg - yi).abs().max() / yi.abs().max()).item() <= BF16_TOL, i
        ref = O.lora_linear(xn, Ws[i].float().cpu().numpy(), As[i].float().cpu().numpy(),
                            Bs[i].float().cpu().numpy(), 2.0)
        assert O.max_rel_err(yg.cpu().numpy(), ref) <= BF16_TOL, i
        n0 += n
