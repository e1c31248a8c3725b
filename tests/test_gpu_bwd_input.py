"""The input gradient with W read where it lies (wsl_lora_linear_bwd_input): dx = gy . W +
s (gy . B) . A against the float64 oracle's backward (oracle.lora_oracle.lora_linear_backward)
on every tile form the entry point picks (256 x 256, 128 x 256, 128 x 128; in-loop rank
blocks 1 and 2; T from the rank pre-pass above rank 64), config 2's projection shapes,
decode-sized and ragged token counts, strided views, and the fallback for layouts it does
not take. Bar: max|dx - dx_ref| / max|dx_ref| <= 1e-2."""
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


def _np(t):
    return t.detach().float().cpu().numpy()


def _inputs(M, N, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    gy = torch.randn(M, N, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16() if r else None
    return gy, W, A, B


def _ref_dx(gy, W, A, B, s):
    K = W.shape[1]
    x = np.zeros((gy.shape[0], K), dtype=np.float32)  # dx does not depend on x
    if A is None:
        return _np(gy).astype(np.float64) @ _np(W).astype(np.float64)
    return O.lora_linear_backward(x, _np(W), _np(A), _np(B), s, _np(gy))[0]


CASES = [
    # M, N (the reduction), K (dx columns), r
    (8192, 4096, 1024, 96),   # config 2 grouped q|k|v (W [4096, 1024], block-diagonal B of rank 3 x 32)
    (8192, 2048, 1024, 32),   # config 2 q: W [2048, 1024], dx [8192, 1024]
    (8192, 1024, 2048, 32),   # config 2 o
    (8192, 3072, 1024, 32),   # config 2 gate
    (8192, 1024, 3072, 32),   # config 2 down
    (4096, 2048, 2048, 64),   # rank 33-64 on 128 x 256 tiles: T from the rank pre-pass
    (1024, 2048, 2048, 64),   # rank 33-64 on 128 x 128 tiles: two in-loop rank blocks
    (8192, 6144, 2048, 48),   # rank 33-64 on 256 x 256 tiles (1.7B gate's dx): the pre-pass
    (2048, 1024, 1024, 128),  # T from the rank pre-pass
    (512, 1024, 1024, 0),     # no LoRA term
    (384, 512, 512, 16),      # 128 x 128 tiles
    (8, 1024, 2048, 32),      # decode-sized token count
    (1000, 512, 776, 24),     # ragged M and K (K % 8 == 0), rank off 32
]


@pytest.mark.parametrize("M,N,K,r", CASES, ids=[f"M{c[0]}_N{c[1]}_K{c[2]}_r{c[3]}" for c in CASES])
def test_bwd_input_matches_oracle(gpu, M, N, K, r):
    from weightshared_torchtitan_amd import ops
    _say(f"[bwd input] M={M} N={N} K={K} r={r}")
    gy, W, A, B = _inputs(M, N, K, r, seed=M + N + K + r)
    dev = lambda t: t.to(gpu) if t is not None else None  # noqa: E731
    dx = ops.lora_linear_bwd_input_op(dev(gy), dev(W), None, dev(A), dev(B), 2.0)
    dx2 = ops.lora_linear_bwd_input_op(dev(gy), dev(W), None, dev(A), dev(B), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(dx, dx2)
    rows = np.arange(M) if M <= 1024 else np.unique(np.concatenate([np.arange(0, M, 64), np.arange(63, M, 64)]))
    ref = _ref_dx(gy[rows], W, A, B, 2.0)
    err = O.max_rel_err(_np(dx)[rows], ref)
    _say(f"   max_rel_err {err:.2e} over {len(rows)} rows")
    assert np.isfinite(err) and err <= BF16_TOL


def test_bwd_input_through_the_c_abi_and_views(gpu):
    """Direct C-ABI call on strided views (gy a column slice of a wider buffer, dx written
    into a wider buffer): equal to the op on contiguous copies, bit for bit, and the
    columns past dx untouched."""
    from weightshared_torchtitan_amd import _native, ops
    M, N, K, r = 512, 1024, 768, 32
    gy, W, A, B = _inputs(M, N, K, r, seed=7)
    big = torch.randn(M, N + 64).bfloat16().to(gpu)
    big[:, 32:32 + N] = gy.to(gpu)
    gyv = big[:, 32:32 + N]
    out = torch.full((M, K + 40), 7.0, dtype=torch.bfloat16, device=gpu)
    L = _native.lib()
    Wd, Ad, Bd = W.to(gpu), A.to(gpu), B.to(gpu)
    bf = _native.WSL_DTYPE_BF16
    assert L.wsl_lora_linear_bwd_input_supported(gyv.data_ptr(), gyv.stride(0), Wd.data_ptr(), K, bf, None,
                                                 Ad.data_ptr(), K, Bd.data_ptr(), r, out.data_ptr(), out.stride(0),
                                                 M, N, K, r) == 1
    ws = torch.zeros(_native.bwd_input_workspace_bytes(M, N, K, r), dtype=torch.uint8, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    rc = L.wsl_lora_linear_bwd_input(gyv.data_ptr(), gyv.stride(0), Wd.data_ptr(), K, bf, None, Ad.data_ptr(), K,
                                     Bd.data_ptr(), r, 2.0, out.data_ptr(), out.stride(0), M, N, K, r,
                                     ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, _native.last_error()
    want = ops.lora_linear_bwd_input_op(gy.to(gpu), Wd, None, Ad, Bd, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(out[:, :K], want)
    assert torch.all(out[:, K:] == 7.0)


def test_bwd_input_unsupported_layout_falls_back(gpu):
    """N off the 64 grid: the entry point refuses with WSL_E_SHAPE, and the op multiplies by
    a transposed copy of W on the forward kernel instead, to the same bar."""
    from weightshared_torchtitan_amd import _native, ops
    M, N, K, r = 256, 200, 512, 16
    gy, W, A, B = _inputs(M, N, K, r, seed=11)
    L = _native.lib()
    Wd = W.to(gpu)
    gyd = gy.to(gpu)
    dx = torch.empty(M, K, dtype=torch.bfloat16, device=gpu)
    bf = _native.WSL_DTYPE_BF16
    assert L.wsl_lora_linear_bwd_input_supported(gyd.data_ptr(), N, Wd.data_ptr(), K, bf, None, None, 0, None, 0,
                                                 dx.data_ptr(), K, M, N, K, 0) == 0
    ws = torch.zeros(_native.bwd_input_workspace_bytes(M, N, K, 0), dtype=torch.uint8, device=gpu)
    rc = L.wsl_lora_linear_bwd_input(gyd.data_ptr(), N, Wd.data_ptr(), K, bf, None, None, 0, None, 0, 1.0,
                                     dx.data_ptr(), K, M, N, K, 0, ws.data_ptr(), ws.numel(),
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == _native.WSL_E_SHAPE
    got = ops.lora_linear_bwd_input_op(gyd, Wd, None, A.to(gpu), B.to(gpu), 2.0)
    err = O.max_rel_err(_np(got), _ref_dx(gy, W, A, B, 2.0))
    assert err <= BF16_TOL


FP8_CASES = [(4096, 4096, 4096, 128), (2048, 1024, 4096, 32), (512, 12288, 4096, 0), (300, 512, 784, 16)]


@pytest.mark.parametrize("M,N,K,r", FP8_CASES, ids=[f"M{c[0]}_N{c[1]}_K{c[2]}_r{c[3]}" for c in FP8_CASES])
def test_bwd_input_fp8_base(gpu, M, N, K, r):
    """An fp8 W (e4m3 codes, per-row scales, config 5's shapes among them): decoded to
    bf16(code * scale) as its tiles are staged. Against the float64 oracle on that
    dequantised W (the bf16 bar), and bit for bit against the bf16 entry point given the
    same dequantised W."""
    from weightshared_torchtitan_amd import ops, quantize_fp8_per_channel
    _say(f"[bwd input fp8] M={M} N={N} K={K} r={r}")
    g = torch.Generator().manual_seed(M + N + K + r + 1)
    gy = torch.randn(M, N, generator=g).bfloat16()
    q, sc = quantize_fp8_per_channel(torch.randn(N, K, generator=g) * 0.02)
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16() if r else None
    wdq = (q.float() * sc[:, None]).bfloat16()  # the dequantised W, rounded as the kernel rounds it
    dev = lambda t: t.to(gpu) if t is not None else None  # noqa: E731
    dx = ops.lora_linear_bwd_input_op(dev(gy), dev(q), dev(sc), dev(A), dev(B), 1.0)
    want = ops.lora_linear_bwd_input_op(dev(gy), dev(wdq), None, dev(A), dev(B), 1.0)
    torch.cuda.synchronize()
    assert torch.equal(dx, want)
    rows = np.arange(0, M, max(1, M // 256))
    err = O.max_rel_err(_np(dx)[rows], _ref_dx(gy[rows], wdq, A, B, 1.0))
    _say(f"   max_rel_err {err:.2e}")
    assert np.isfinite(err) and err <= BF16_TOL


def test_backward_calls_no_transpose_of_w(gpu):
    """A training step's backward through wsl::lora_linear: dx runs on
    wsl::lora_linear_bwd_input, and no W-sized transposed copy is made (no aten copy of
    W^T's shape in the trace)."""
    import weightshared_torchtitan_amd as wsl
    M, N, K, r = 1024, 2048, 1024, 32
    g = torch.Generator().manual_seed(3)
    x = torch.randn(M, K, generator=g).bfloat16().to(gpu).requires_grad_(True)
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16().to(gpu).requires_grad_(True)
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16().to(gpu).requires_grad_(True)
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16().to(gpu).requires_grad_(True)
    y = wsl.lora_linear(x, W, A, B, 2.0)
    gy = torch.randn_like(y)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU], record_shapes=True) as prof:
        y.backward(gy)
        torch.cuda.synchronize()
    names = [e.name for e in prof.events()]
    assert "wsl::lora_linear_bwd_input" in names
    wt_copies = [e for e in prof.events() if e.name in ("aten::contiguous", "aten::clone", "aten::copy_")
                 and e.input_shapes and list(e.input_shapes[0]) in ([K, N], [N, K])]
    assert not wt_copies, [(e.name, e.input_shapes) for e in wt_copies]
    dx = O.lora_linear_backward(_np(x), _np(W), _np(A), _np(B), 2.0, _np(gy))[0]
    assert O.max_rel_err(_np(x.grad), dx) <= BF16_TOL
