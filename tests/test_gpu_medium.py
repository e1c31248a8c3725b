"""Medium M: from 65 tokens the prefill path's in-launch split-K form (ranks up to 64)
or, above rank 64 up to 160 tokens over long K, its medium split form (split-K base
product, rank pre-pass, combine kernel); each against the float64 oracle, bar
max|y - y_ref| / max|y_ref| <= 1e-2. Grouped launches against the single calls within the
bar (the K split counts of both forms above 64 tokens depend on N). The shared-base form,
and agreement across the M = 64 / 65 cut-over."""
import sys

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


CASES = [
    # M, N, K, r
    (65, 6144, 2048, 64),    # one token past the decode path, 1.7B gate shape
    (100, 2048, 2048, 32),
    (128, 1024, 1024, 16),
    (150, 3072, 1024, 32),
    (160, 1024, 2048, 128),  # r > 64: unsplit tiles, T by the rank pre-pass
    (130, 2048, 6144, 128),  # r > 64 over 96 K tiles: the medium split form
    (65, 200, 512, 8),       # N off every tile grid
    (96, 512, 4096, 0),      # plain linear
]


@pytest.mark.parametrize("M,N,K,r", CASES)
def test_medium_m_matches_oracle(gpu, M, N, K, r):
    from weightshared_torchtitan_amd import lora_linear
    _say(f"[medium] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, M + N + K + r)
    d = lambda t: None if t is None else t.to(gpu)
    y = lora_linear(d(x), d(W), d(A), d(B), 2.0).float().cpu().numpy()
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    err = O.max_rel_err(y, ref)
    _say(f"   max_rel_err {err:.2e}")
    assert err <= BF16_TOL


@pytest.mark.parametrize("M,K,r,group_n", [
    (100, 1024, 32, (2048, 1024, 1024)),   # q|k|v on the decode path
    (150, 1024, 32, (3072, 3072)),         # gate|up: in-launch split-K
    (150, 2048, 64, (1024, 512, 512)),
])
def test_medium_m_grouped_matches_single(gpu, M, K, r, group_n):
    import weightshared_torchtitan_amd as wsl
    from weightshared_torchtitan_amd import ops
    _say(f"[medium grouped] M={M} K={K} r={r} groups={group_n}")
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).bfloat16().to(gpu)
    Ws = [(torch.randn(n, K, generator=g) * 0.02).bfloat16().to(gpu) for n in group_n]
    As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16().to(gpu) for _ in group_n]
    Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16().to(gpu) for n in group_n]
    y = ops.lora_linear_grouped_op(x, torch.cat(Ws), None, torch.cat(As), torch.cat(Bs), 2.0, list(group_n))
    n0 = 0
    for i, n in enumerate(group_n):
        yi = wsl.lora_linear(x, Ws[i], As[i], Bs[i], 2.0)
        assert ((y[:, n0:n0 + n].float() - yi.float()).abs().max() / yi.float().abs().max()).item() <= BF16_TOL, i
        n0 += n
    ref = O.lora_linear(x.float().cpu().numpy(), Ws[0].float().cpu().numpy(), As[0].float().cpu().numpy(),
                        Bs[0].float().cpu().numpy(), 2.0)
    assert O.max_rel_err(y[:, :group_n[0]].float().cpu().numpy(), ref) <= BF16_TOL


def test_medium_m_shared_base(gpu):
    """Head sharing (g = 2) and q|k|v sharing one base at M = 120: the base product reads
    the base rows through the column map in the split form too."""
    from weightshared_torchtitan_amd import ops
    for (N, base_n, g, G) in ((512, 128, 2, 1), (1024, 1024, 1, 3)):
        M, K, r = 120, 1024, 16
        _say(f"[medium bcast] M={M} N={N} base_n={base_n} g={g} groups={G}")
        gen = torch.Generator().manual_seed(N + G)
        x = torch.randn(M, K, generator=gen).bfloat16()
        W = (torch.randn(base_n, K, generator=gen) * 0.02).bfloat16()
        A = (torch.randn(G * r, K, generator=gen) * 0.02).bfloat16()
        B = (torch.randn(G * N, r, generator=gen) * 0.02).bfloat16()
        y = ops.lora_linear_bcast_op(x.to(gpu), W.to(gpu), None, A.to(gpu), B.to(gpu), 2.0, g, G)
        y = y.float().cpu().numpy()
        xn, Wn, An, Bn = x.float().numpy(), W.float().numpy(), A.float().numpy(), B.float().numpy()
        base = xn.astype("float64") @ Wn.T.astype("float64")
        for j in range(G):
            delta = O.lora_delta(xn, An[j * r:(j + 1) * r], Bn[j * N:(j + 1) * N], 2.0)
            ref = O.broadcast_add(base, delta, dim=-1, g=g)
            assert O.max_rel_err(y[:, j * N:(j + 1) * N], ref) <= BF16_TOL, j


def test_medium_m_continues_the_decode_path(gpu):
    """Rows of an M = 65 call (split form) agree with the same rows at M = 64 (decode path)
    to the bar, and every row is independent of the others in the split form."""
    from weightshared_torchtitan_amd import lora_linear
    M, N, K, r = 65, 2048, 2048, 64
    _say(f"[medium cut-over] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, 77)
    d = lambda t: t.to(gpu)
    y65 = lora_linear(d(x), d(W), d(A), d(B), 2.0).float().cpu()
    y64 = lora_linear(d(x[:64]), d(W), d(A), d(B), 2.0).float().cpu()
    assert O.max_rel_err(y65[:64].numpy(), y64.numpy().astype("float64")) <= BF16_TOL
    perm = torch.randperm(M, generator=torch.Generator().manual_seed(1))
    yp = lora_linear(d(x[perm]), d(W), d(A), d(B), 2.0).float().cpu()
    assert torch.equal(yp, y65[perm])
