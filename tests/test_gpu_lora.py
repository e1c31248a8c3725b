"""GPU parity of the fused LoRA linear (prefill, decode and generic paths) against the
CPU oracle, plus size-independent properties at the benchmark shapes.

Bar: max|y - y_ref| / max|y_ref| <= 1e-2 for the bf16 path and
<= 3e-2 for the fp8-base path, y_ref = float64 oracle on the same bf16-rounded inputs.
"""
import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP8_TOL = 3e-2


def _inputs(M, N, K, r, seed=0, has_w=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16() if has_w else None
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16() if r else None
    return x, W, A, B


def _np(t):
    return None if t is None else t.float().numpy()


def _gpu(t, dev):
    return None if t is None else t.to(dev)


def _run(dev, x, W, A, B, s, w_scale=None):
    import weightshared_torchtitan_amd as wsl
    y = wsl.lora_linear(_gpu(x, dev), _gpu(W, dev), _gpu(A, dev), _gpu(B, dev), s,
                        w_scale=_gpu(w_scale, dev))
    torch.cuda.synchronize()
    return y.cpu()


def _say(msg):
    print(msg, flush=True)


PREFILL_CASES = [
    # M, N, K, r, s, has_w
    (2048, 1024, 1024, 16, 2.0, True),   # BASELINE config 1 shape
    (512, 2048, 1024, 32, 2.0, True),
    (300, 520, 192, 24, 2.0, True),      # M, N tails, odd rank
    (256, 256, 64, 8, 2.0, True),        # reference default rank 8, one K tile
    (1000, 768, 512, 64, 2.0, True),     # largest in-kernel rank
    (640, 512, 256, 128, 1.0, True),     # pre-pass rank, scale 1
    (320, 384, 256, 256, 2.0, True),     # WSL_MAX_RANK
    (384, 1024, 512, 0, 2.0, True),      # plain linear
    (400, 640, 320, 32, 2.0, False),     # delta only (LoRAModule.forward)
    (65, 1024, 1024, 32, 2.0, True),     # just above the decode cut-over
    (8192, 3072, 64, 32, 2.0, True),     # 256 x 192 tiles (two full waves for N = 3072)
    (8000, 2900, 128, 16, 2.0, True),    # 256 x 192 tiles with M and N tails
    (8192, 3072, 64, 0, 2.0, True),      # 256 x 192, plain linear
    (8192, 3072, 64, 128, 1.0, True),    # 256 x 192 consuming the pre-pass T
    (1000, 1024, 2048, 128, 2.0, True),  # pre-pass split 8 ways over K, M tail
    (700, 512, 1024, 256, 1.0, True),    # pre-pass split 4 ways, two rank tiles
    (64 + 1, 640, 4096, 128, 2.0, False),  # delta only, pre-pass split 16 ways
    (4096, 1024, 512, 0, 2.0, True),     # 128 x 128 tiles (256 of them), plain linear
    (4096, 1000, 256, 128, 1.0, True),   # 128 x 128 tiles, pre-pass T, N tail
    (2000, 1024, 512, 32, 2.0, False),   # 128 x 128 tiles, delta only, M tail
]


@pytest.mark.parametrize("M,N,K,r,s,has_w", PREFILL_CASES)
def test_prefill_parity(gpu, M, N, K, r, s, has_w):
    _say(f"[prefill] M={M} N={N} K={K} r={r} s={s} has_w={has_w}")
    x, W, A, B = _inputs(M, N, K, r, seed=M + N + K + r, has_w=has_w)
    y = _run(gpu, x, W, A, B, s)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), s)
    err = O.max_rel_err(y.float().numpy(), ref)
    _say(f"  max_rel_err={err:.3e}")
    assert np.isfinite(err) and err <= BF16_TOL


DECODE_CASES = [
    (1, 2048, 2048, 64, 2.0, True),
    (8, 2048, 2048, 64, 2.0, True),
    (32, 1024, 2048, 64, 2.0, True),
    (64, 6144, 2048, 64, 2.0, True),
    (64, 2048, 6144, 64, 2.0, True),
    (3, 1000, 1024, 16, 2.0, True),      # N not a multiple of the row group
    (17, 512, 512, 8, 2.0, True),
    (49, 768, 1024, 40, 2.0, True),
    (8, 4096, 256, 0, 2.0, True),        # r = 0, direct-write path
    (5, 640, 1024, 32, 2.0, False),      # delta only
    (16, 1024, 1024, 256, 2.0, True),    # max rank
    (33, 1000, 2048, 24, 2.0, True),     # 32-row groups with an N tail, partial rank group
    (64, 1000, 6144, 24, 2.0, True),     # six-way K split with tails
    (1, 2048, 6144, 128, 1.0, True),     # one token, long K, rank 128
    (8, 151936, 256, 0, 2.0, True),      # tied output head: short K, 2 waves per row block
    (3, 5000, 256, 16, 2.0, True),       # short K with rank rows
    (20, 2000, 512, 24, 2.0, True),      # 4 waves per row block
    (64, 1000, 256, 64, 2.0, True),      # short K at the largest M
    # rows per workgroup chosen by the plan's cost model (16, 32 or 64)
    (64, 1024, 2048, 64, 2.0, True),     # 16 rows, four token blocks
    (48, 1024, 2048, 64, 2.0, True),     # 16 rows, three token blocks
    (40, 6144, 2048, 32, 2.0, True),     # 64 rows, three token blocks
    (32, 12288, 1024, 16, 2.0, True),    # 64 rows, two token blocks
    (20, 4096, 1024, 16, 2.0, True),     # 32 rows, two token blocks
]


@pytest.mark.parametrize("M,N,K,r,s,has_w", DECODE_CASES)
def test_decode_parity(gpu, M, N, K, r, s, has_w):
    _say(f"[decode] M={M} N={N} K={K} r={r} s={s} has_w={has_w}")
    x, W, A, B = _inputs(M, N, K, r, seed=7 * M + N + K + r, has_w=has_w)
    y = _run(gpu, x, W, A, B, s)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), s)
    err = O.max_rel_err(y.float().numpy(), ref)
    _say(f"  max_rel_err={err:.3e}")
    assert np.isfinite(err) and err <= BF16_TOL


GENERIC_CASES = [
    (70, 100, 100, 5, 2.0),    # K % 64 != 0, odd rank -> generic path
    (3, 33, 40, 3, 2.0),       # tiny decode-size, odd everything
    (129, 64, 72, 12, 2.0),
]


@pytest.mark.parametrize("M,N,K,r,s", GENERIC_CASES)
def test_generic_parity(gpu, M, N, K, r, s):
    _say(f"[generic] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=11 + M)
    y = _run(gpu, x, W, A, B, s)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), s)
    err = O.max_rel_err(y.float().numpy(), ref)
    _say(f"  max_rel_err={err:.3e}")
    assert err <= BF16_TOL


def test_strided_inputs(gpu):
    """Leading dimensions larger than K (views into wider buffers)."""
    import weightshared_torchtitan_amd as wsl
    _say("[strided] M=300 N=256 K=256 r=16, ldx=ldw=320")
    g = torch.Generator().manual_seed(5)
    xb = torch.randn(300, 320, generator=g).bfloat16()
    wb = (torch.randn(256, 320, generator=g) * 0.02).bfloat16()
    A = (torch.randn(16, 256, generator=g) * 0.02).bfloat16()
    B = (torch.randn(256, 16, generator=g) * 0.02).bfloat16()
    x, W = xb[:, :256], wb[:, :256]
    y = wsl.lora_linear(xb.to(gpu)[:, :256], wb.to(gpu)[:, :256], A.to(gpu), B.to(gpu), 2.0)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    assert O.max_rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL


def test_golden_vectors_on_gpu(gpu):
    """The brute-force fixtures, run through the HIP kernels (generic/decode paths)."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "lora_small.npz"), allow_pickle=False)
    for name in g["names"]:
        x = torch.from_numpy(g[f"{name}_x"]).bfloat16()
        W = torch.from_numpy(g[f"{name}_W"]).bfloat16() if g[f"{name}_W"].shape[0] else None
        A = torch.from_numpy(g[f"{name}_A"]).bfloat16() if g[f"{name}_A"].shape[0] else None
        B = torch.from_numpy(g[f"{name}_B"]).bfloat16() if A is not None else None
        _say(f"[golden] {name} x{tuple(x.shape)}")
        y = _run(gpu, x, W, A, B, float(g[f"{name}_s"]))
        assert O.max_rel_err(y.float().numpy(), g[f"{name}_y"]) <= BF16_TOL, str(name)


# ------------------------------------------------------------------ fp8 base
@pytest.mark.parametrize("M,N,K", [(16, 1024, 4096), (512, 1024, 1024), (4, 512, 2048), (4096, 1024, 4096)])
def test_fp8_base_parity(gpu, M, N, K):
    from weightshared_torchtitan_amd import quantize_fp8_per_channel
    _say(f"[fp8] M={M} N={N} K={K} r=128 s=1")
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    Wf = torch.randn(N, K, generator=g) * 0.02
    A = (torch.randn(128, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, 128, generator=g) * 0.02).bfloat16()
    q, sc = quantize_fp8_per_channel(Wf)
    y = _run(gpu, x, q, A, B, 1.0, w_scale=sc).float().numpy()
    ref = O.lora_linear(_np(x), Wf.numpy(), _np(A), _np(B), 1.0)
    err = O.max_rel_err(y, ref)
    wdq = O.dequantize_fp8(q.view(torch.uint8).numpy(), sc.numpy())
    err_dq = O.max_rel_err(y, O.lora_linear(_np(x), wdq, _np(A), _np(B), 1.0))
    _say(f"  vs fp32 W: {err:.3e}   vs dequantised W: {err_dq:.3e}")
    assert err <= FP8_TOL
    assert err_dq <= BF16_TOL


@pytest.mark.parametrize("M", [16, 4096])
@pytest.mark.parametrize("N,K", [(4096, 4096), (12288, 4096), (4096, 12288)])  # q/o, gate/up, down at 8B
def test_fp8_base_parity_c5_shapes(gpu, M, N, K):
    """Config 5's fp8 projections at their full size (rank 128, scale 1). The kernel runs on
    all M rows; the float64 oracle checks every row at M = 16 and every 16th row at
    M = 4096 (rows are independent, so the sample is exact for the rows it covers)."""
    from weightshared_torchtitan_amd import quantize_fp8_per_channel
    _say(f"[fp8 c5] M={M} N={N} K={K} r=128 s=1")
    g = torch.Generator().manual_seed(N + K + M)
    x = torch.randn(M, K, generator=g).bfloat16()
    Wf = torch.randn(N, K, generator=g) * 0.02
    A = (torch.randn(128, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, 128, generator=g) * 0.02).bfloat16()
    q, sc = quantize_fp8_per_channel(Wf)
    y = _run(gpu, x, q, A, B, 1.0, w_scale=sc).float().numpy()
    rows = np.arange(0, M, 1 if M <= 64 else 16)
    ref = O.lora_linear(_np(x)[rows], Wf.numpy(), _np(A), _np(B), 1.0)
    err = O.max_rel_err(y[rows], ref)
    wdq = O.dequantize_fp8(q.view(torch.uint8).numpy(), sc.numpy())
    err_dq = O.max_rel_err(y[rows], O.lora_linear(_np(x)[rows], wdq, _np(A), _np(B), 1.0))
    _say(f"  vs fp32 W: {err:.3e}   vs dequantised W: {err_dq:.3e}")
    assert err <= FP8_TOL
    assert err_dq <= BF16_TOL


@pytest.mark.parametrize("path", [1, 2], ids=["decoded_w", "fp8_matrix_cores"])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1024, 4096), (4096, 12288)])  # q/o, k/v, down at 8B
def test_fp8_base_parity_c5_forced_paths(gpu, N, K, path, wsl_opts):
    """Config 5's one-wave fp8 launches (M = 4096) on each path, forced (by default the
    launch width picks W decoded onto the bf16 matrix cores for these; wider launches take
    the fp8 matrix cores, test_fp8_base_parity_c5_shapes), so both stay pinned at these
    shapes. Every 16th row against the float64 oracle: within the
    bf16 bar of the exact product on the dequantised W, and against the fp32 W no more than
    2e-3 above the per-channel e4m3 quantiser's own error on these inputs (2.5-3.1e-2 for
    N(0, 0.02^2) weights at these shapes, whatever the kernel)."""
    from weightshared_torchtitan_amd import _native, quantize_fp8_per_channel
    M = 4096
    wsl_opts(fp8_prefill=path)
    p = _native.plan(M, K, 128, (N,), _native.WSL_DTYPE_FP8_E4M3)
    assert p["path"] == ("prefill_fp8" if path == 2 else "prefill")
    _say(f"[fp8 c5 forced] path={p['path']} M={M} N={N} K={K} r=128 s=1")
    g = torch.Generator().manual_seed(N + K + M)
    x = torch.randn(M, K, generator=g).bfloat16()
    Wf = torch.randn(N, K, generator=g) * 0.02
    A = (torch.randn(128, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, 128, generator=g) * 0.02).bfloat16()
    q, sc = quantize_fp8_per_channel(Wf)
    y = _run(gpu, x, q, A, B, 1.0, w_scale=sc).float().numpy()
    rows = np.arange(0, M, 16)
    ref = O.lora_linear(_np(x)[rows], Wf.numpy(), _np(A), _np(B), 1.0)
    err = O.max_rel_err(y[rows], ref)
    wdq = O.dequantize_fp8(q.view(torch.uint8).numpy(), sc.numpy())
    exact_dq = O.lora_linear(_np(x)[rows], wdq, _np(A), _np(B), 1.0)
    err_dq = O.max_rel_err(y[rows], exact_dq)
    q_err = O.max_rel_err(exact_dq, ref)  # the quantiser's share
    _say(f"  vs fp32 W: {err:.3e} (quantiser alone {q_err:.3e})   vs dequantised W: {err_dq:.3e}")
    assert err_dq <= BF16_TOL
    assert err <= q_err + 2e-3


@pytest.mark.parametrize("terms", [2, 1])
def test_fp8_activation_split_pinned_by_identity_weight(gpu, terms, monkeypatch, wsl_opts):
    """The fp8 matrix-core path with W = I (code 1.0 on the diagonal, scale 1): y is the
    activations the kernel multiplied, 2^e (hi + lo/16) (or 2^e hi), rounded to bf16. It must
    equal the oracle's split (oracle.fp8_split_activations) bit for bit: exponent choice, the
    two nearest-even roundings and the residual scale are all pinned. Rows span magnitudes
    from 1e-6 to 1e6 and include maxima on both sides of the 1.75 * 2^k boundary."""
    from weightshared_torchtitan_amd import ops
    monkeypatch.setattr(ops, "FP8_ACTIVATIONS", terms == 1)
    wsl_opts(fp8_prefill=2)  # one 256 x 256 tile: the fp8 matrix cores only when forced
    _say(f"[fp8 split] terms={terms}")
    M, K = 256, 256
    g = torch.Generator().manual_seed(17)
    mags = 10.0 ** torch.randint(-6, 7, (M, 1), generator=g).float()
    x = (torch.randn(M, K, generator=g) * mags).bfloat16()
    x[0, :] = 0.0
    x[1, 5] = 448.0
    x[2, 7] = 1.75
    x[3, 9] = -1.7578125
    x[4, 11] = 3.5
    q = torch.eye(K).to(torch.float8_e4m3fn)
    sc = torch.ones(K)
    y = _run(gpu, x, q, None, None, 0.0, w_scale=sc).float().numpy()
    codes, e = O.fp8_split_activations(_np(x), terms=terms)
    want = O.bf16_round(O.fp8_activations_value(codes, e).astype(np.float32))
    np.testing.assert_array_equal(y, want)
    if terms == 2:
        assert np.mean(y == _np(x)) > 0.95  # two terms carry almost every bf16 value exactly


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (512, 12288, 4096), (320, 4096, 12288)])
def test_fp8_one_term_activations(gpu, M, N, K, monkeypatch):
    """The opt-in one-term path (WSL_DTYPE_FP8_E4M3_ACT8) against the oracle of the same
    arithmetic (e4m3 activations under a per-token power-of-two scale, dequantised W, bf16 T):
    kernel error within the bf16 bar. Its error against the fp32-W reference is reported;
    the north star's 3e-2 bar is the default path's (the CPU test pins the difference)."""
    from weightshared_torchtitan_amd import ops, quantize_fp8_per_channel
    monkeypatch.setattr(ops, "FP8_ACTIVATIONS", True)
    _say(f"[fp8 act8] M={M} N={N} K={K} r=128 s=1")
    g = torch.Generator().manual_seed(M + N + 3 * K)
    x = torch.randn(M, K, generator=g).bfloat16()
    Wf = torch.randn(N, K, generator=g) * 0.02
    A = (torch.randn(128, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, 128, generator=g) * 0.02).bfloat16()
    q, sc = quantize_fp8_per_channel(Wf)
    y = _run(gpu, x, q, A, B, 1.0, w_scale=sc).float().numpy()
    rows = np.arange(0, M, max(1, M // 256))
    codes, e = O.fp8_split_activations(_np(x)[rows], terms=1)
    xv = O.fp8_activations_value(codes, e)
    wdq = O.dequantize_fp8(q.view(torch.uint8).numpy(), sc.numpy())
    same = xv @ wdq.T + O.lora_delta(_np(x)[rows], _np(A), _np(B), 1.0)
    err_k = O.max_rel_err(y[rows], same)
    err_fp32 = O.max_rel_err(y[rows], O.lora_linear(_np(x)[rows], Wf.numpy(), _np(A), _np(B), 1.0))
    _say(f"  vs its own arithmetic: {err_k:.3e}   vs fp32 W: {err_fp32:.3e}")
    assert err_k <= BF16_TOL
    assert err_fp32 <= 6e-2


def test_fp8_decode_table_on_gpu(gpu):
    """Every finite e4m3fn code through the kernel's decoder: x = e_k one-hot rows."""
    _say("[fp8 table] K=256 one-hot")
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=torch.uint8)
    n = codes.numel()
    K = 256
    q = torch.zeros(n, K, dtype=torch.uint8)
    q[:, 0] = codes
    x = torch.zeros(1, K, dtype=torch.bfloat16)
    x[0, 0] = 1.0
    y = _run(gpu, x, q.view(torch.float8_e4m3fn), None, None, 0.0, w_scale=torch.ones(n))
    expect = O.fp8_e4m3_decode(codes.numpy())
    np.testing.assert_array_equal(y.float().numpy()[0], expect.astype(np.float32))


# ------------------------------------------------------------------ properties at benchmark size
def test_properties_at_benchmark_shape(gpu):
    """Config-2 gate/up projection (M=8192, N=3072, K=1024, r=32): determinism, row
    independence, B = 0 reducing to the plain linear, linearity in the scale."""
    import weightshared_torchtitan_amd as wsl
    _say("[props] M=8192 N=3072 K=1024 r=32")
    M, N, K, r = 8192, 3072, 1024, 32
    x, W, A, B = (t.to(gpu) for t in _inputs(M, N, K, r, seed=99))
    y1 = wsl.lora_linear(x, W, A, B, 2.0)
    y2 = wsl.lora_linear(x, W, A, B, 2.0)
    assert torch.equal(y1, y2), "not deterministic"
    # A slice large enough to take the same tile configuration (configurations differ in
    # how they split the rank down-projection's K sum, so only equal ones are bit-equal).
    ys = wsl.lora_linear(x[1024:5120], W, A, B, 2.0)
    assert torch.equal(ys, y1[1024:5120]), "rows not independent"
    y0 = wsl.lora_linear(x, W, A, torch.zeros_like(B), 2.0)
    yp = wsl.lora_linear(x, W, None, None, 0.0)
    assert torch.equal(y0, yp), "B = 0 must equal the plain linear"
    ya = wsl.lora_linear(x, W, A, B, 1.0).float()
    yb = wsl.lora_linear(x, W, A, B, 3.0).float()
    d1 = ya - yp.float()
    d3 = yb - yp.float()
    rel = ((d3 - 3 * d1).abs().max() / (3 * d1).abs().max()).item()
    _say(f"  linearity residual {rel:.3e}")
    assert rel < 5e-2
    # spot-check 64 rows against the oracle at full K
    rows = torch.arange(0, M, M // 64)
    ref = O.lora_linear(_np(x[rows].cpu()), _np(W.cpu()), _np(A.cpu()), _np(B.cpu()), 2.0)
    assert O.max_rel_err(y1[rows].float().cpu().numpy(), ref) <= BF16_TOL


def test_decode_matches_prefill_path(gpu):
    """The same rows through the decode (M <= 64) and prefill (M > 64) kernels agree."""
    import weightshared_torchtitan_amd as wsl
    _say("[decode vs prefill] N=2048 K=2048 r=64")
    x, W, A, B = (t.to(gpu) for t in _inputs(128, 2048, 2048, 64, seed=3))
    big = wsl.lora_linear(x, W, A, B, 2.0).float()
    small = wsl.lora_linear(x[:8], W, A, B, 2.0).float()
    rel = ((big[:8] - small).abs().max() / big[:8].abs().max()).item()
    assert rel < 1e-2


# ------------------------------------------------------------------ factorized embedding
def test_factorized_embedding_golden(gpu):
    import os
    import weightshared_torchtitan_amd as wsl
    _say("[embedding golden]")
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "embedding_small.npz"), allow_pickle=False)
    E = torch.from_numpy(g["E"]).bfloat16().to(gpu)
    P = torch.from_numpy(g["P"]).bfloat16().to(gpu)
    out = wsl.factorized_embedding(torch.from_numpy(g["ids"]).to(gpu), E, P).float().cpu().numpy()
    assert O.max_rel_err(out, g["out"]) <= BF16_TOL
    assert np.all(out[3] == 0) and np.all(out[5] == 0)  # out-of-range ids


@pytest.mark.parametrize("n_tok", [8, 4096])
def test_factorized_embedding_benchmark_shape(gpu, n_tok):
    import weightshared_torchtitan_amd as wsl
    _say(f"[embedding] V=151936 k=256 H=1024 tokens={n_tok}")
    g = torch.Generator().manual_seed(n_tok)
    V, k, H = 151936, 256, 1024
    E = (torch.randn(V, k, generator=g) * 0.02).bfloat16()
    P = (torch.randn(H, k, generator=g) * 0.02).bfloat16()
    ids = torch.randint(0, V, (n_tok,), generator=g)
    out = wsl.factorized_embedding(ids.to(gpu), E.to(gpu), P.to(gpu)).float().cpu().numpy()
    ref = O.factorized_embedding(ids.numpy(), _np(E), _np(P))
    assert O.max_rel_err(out, ref) <= BF16_TOL


# ------------------------------------------------------------------ decode workspace contract
def _check_counters(gpu, calls_before, calls_after):
    """The workspace prefix holds only the launch counter, spread over 8 words 128 bytes
    apart (every other byte of the 64 KB prefix is zero); their sum advanced by exactly
    2^20 per decode launch."""
    from weightshared_torchtitan_amd import ops
    ws = ops.workspace(gpu, torch.cuda.current_stream(gpu).cuda_stream, 0)
    prefix = ws[:65536].cpu().numpy()
    words = prefix.view(np.uint64)
    counters = words[::16][:8]
    rest = np.delete(words, np.arange(0, 8 * 16, 16))
    assert int(np.count_nonzero(rest)) == 0, "prefix bytes outside the launch counter words"
    launch = int(counters.sum())
    if calls_before is not None:
        assert launch - calls_before == (calls_after << 20)
    return launch


def test_decode_counters_return_to_zero_and_deterministic(gpu):
    """The split-K decode path leaves its arrival counters zero, advances the launch
    counter by one unit per launch and sums slices in a fixed order: repeated calls are
    bitwise identical."""
    import weightshared_torchtitan_amd as wsl
    _say("[decode counters] M=8 N=2048 K=6144 r=64")
    x, W, A, B = (t.to(gpu) for t in _inputs(8, 2048, 6144, 64, seed=17))
    wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.synchronize()
    before = _check_counters(gpu, None, 0)
    ys = [wsl.lora_linear(x, W, A, B, 2.0) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(torch.equal(ys[0], v) for v in ys[1:])
    _check_counters(gpu, before, 3)
    x2, W2, A2, B2 = (t.to(gpu) for t in _inputs(64, 1000, 6144, 24, seed=18))
    wsl.lora_linear(x2, W2, A2, B2, 2.0)
    torch.cuda.synchronize()
    _check_counters(gpu, before, 4)


@pytest.mark.parametrize("M,N,K,r", [(4, 1024, 2048, 32), (64, 2048, 6144, 64), (64, 6144, 2048, 64),
                                     (72, 2048, 6144, 64)])
def test_decode_in_graph_replays_match_eager(gpu, M, N, K, r, wsl_opts):
    """Captured decode calls replay correctly several times (counters reset per replay);
    72 tokens on the decode path's wide form (the decode_wide override at 1)."""
    import weightshared_torchtitan_amd as wsl
    if M > 64:
        wsl_opts(decode_wide=1)
    _say(f"[decode graph] M={M} N={N} K={K} r={r}, 3 replays")
    x, W, A, B = (t.to(gpu) for t in _inputs(M, N, K, r, seed=23))
    eager = wsl.lora_linear(x, W, A, B, 2.0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = wsl.lora_linear(x, W, A, B, 2.0)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        wsl.lora_linear(x, W, A, B, 2.0)  # eager work on the default stream between replays


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_workspace_growth_refused_during_capture(gpu):
    """A workspace that would have to grow inside a graph capture raises instead of being
    allocated (and zero-filled) by the graph; after an eager call on the capture stream the
    same capture succeeds."""
    import weightshared_torchtitan_amd as wsl
    x, W, A, B = (t.to(gpu) for t in _inputs(4, 512, 1024, 16, seed=41))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="during graph capture"):
        with torch.cuda.graph(g, stream=s):
            wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        eager = wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.current_stream().wait_stream(s)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        out = wsl.lora_linear(x, W, A, B, 2.0)
    g2.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)


@pytest.mark.parametrize("M,N,K,r", [(1, 2048, 2048, 64), (40, 1000, 6144, 24)])
def test_decode_t_wait_fallback(gpu, M, N, K, r, wsl_opts):
    """With the T wait bound forced to zero from the host, every W workgroup computes T
    itself: the result stays within tolerance and the counters still return to zero."""
    import weightshared_torchtitan_amd as wsl
    _say(f"[decode T fallback] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=29)
    xg, Wg, Ag, Bg = (t.to(gpu) for t in (x, W, A, B))
    normal = wsl.lora_linear(xg, Wg, Ag, Bg, 2.0).float()
    wsl_opts(decode_spin_limit=-1)
    forced = wsl.lora_linear(xg, Wg, Ag, Bg, 2.0).float()
    torch.cuda.synchronize()
    wsl_opts(decode_spin_limit=0)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    assert O.max_rel_err(forced.cpu().numpy(), ref) <= BF16_TOL
    assert ((forced - normal).abs().max() / normal.abs().max()).item() < 1e-2
    _check_counters(gpu, None, 0)
    again = wsl.lora_linear(xg, Wg, Ag, Bg, 2.0).float()  # the normal path still works after it
    assert torch.equal(again, normal)
