"""Weight gradients on the HIP path (wsl_lora_linear_bwd_weights, called through the C ABI):
dW = gy^T x, dA = s (gy B)^T x, dB = s gy^T (x A^T), by both routes (dA and dB from dW when
dW is asked for, over the tokens without it), against the float64 oracle
(oracle.lora_oracle.lora_linear_backward) on the same bf16 inputs, bar max|g - g_ref| /
max|g_ref| <= 1e-2 per gradient. The full config-2 shape is checked against torch fp32 on
the device (the oracle's float64 products there take minutes). Split reductions are summed
in a fixed order, so repeated calls, and calls asking for a subset of the gradients, agree
bit for bit."""
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


def _bwd(x, gy, a, b, s, want=(True, True, True), outs=None):
    """One C-ABI call; returns (dw, da, db) (None where not asked for). `outs` may give
    destination views (any leading dimension)."""
    from weightshared_torchtitan_amd import _native
    M, K = x.shape
    N = gy.shape[1]
    r = a.shape[0] if a is not None else 0
    dev = x.device
    if outs is None:
        outs = (torch.empty(N, K, dtype=torch.bfloat16, device=dev) if want[0] else None,
                torch.empty(r, K, dtype=torch.bfloat16, device=dev) if want[1] else None,
                torch.empty(N, r, dtype=torch.bfloat16, device=dev) if want[2] else None)
    dw, da, db = outs
    nbytes = _native.bwd_weights_workspace_bytes(M, N, K, r)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    L = _native.lib()
    p = lambda t: None if t is None else t.data_ptr()
    ld = lambda t: 0 if t is None else t.stride(0)
    with torch.cuda.device(dev):
        rc = L.wsl_lora_linear_bwd_weights(
            p(x), ld(x), p(gy), ld(gy), p(a), ld(a), p(b), ld(b), float(s), M, N, K, r,
            p(dw), ld(dw), p(da), ld(da), p(db), ld(db), ws.data_ptr(), ws.numel(),
            torch.cuda.current_stream(dev).cuda_stream)
    _native.check(rc, "wsl_lora_linear_bwd_weights")
    torch.cuda.synchronize()
    return dw, da, db


def _inputs(M, N, K, r, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    gy = torch.randn(M, N, generator=g).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.05).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.05).bfloat16() if r else None
    to = lambda t: None if t is None else t.to(dev)
    return x, gy, A, B, to(x), to(gy), to(A), to(B)


CASES = [
    # M, N, K, r: which split counts the plan takes
    (2048, 1024, 1024, 16),   # config-1 shape
    (8192, 1024, 1024, 32),   # config-2 k/v shape: dW split 4, dA/dB split 32
    (8192, 3072, 1024, 32),   # gate/up
    (8192, 1024, 3072, 32),   # down
    (1, 512, 256, 8),         # one token: 63 padded zero tokens
    (65, 256, 512, 64),       # ragged token count
    (1000, 640, 320, 128),    # r = 128
    (384, 512, 384, 0),       # plain linear: dW only
]


@pytest.mark.parametrize("M,N,K,r", CASES)
def test_weight_grads_match_oracle(gpu, M, N, K, r):
    _say(f"[weight grads] M={M} N={N} K={K} r={r}")
    s = 2.0
    x, gy, A, B, tx, tgy, tA, tB = _inputs(M, N, K, r, M + N + K + r, gpu)
    dw, da, db = _bwd(tx, tgy, tA, tB, s, want=(True, r > 0, r > 0))             # dW route
    got = [("dW", dw), ("dA", da), ("dB", db)]
    if r > 0:                                                                       # token route
        _, ta, tb = _bwd(tx, tgy, tA, tB, s, want=(False, True, True))
        got += [("dA token route", ta), ("dB token route", tb)]
    _, dW, dA, dB = O.lora_linear_backward(_np(x), np.zeros((N, K), np.float32), None if A is None else _np(A),
                                           None if B is None else _np(B), s, _np(gy))
    refs = {"dW": dW, "dA": dA, "dB": dB}
    for name, t in got:
        if t is None:
            continue
        err = O.max_rel_err(_np(t), refs[name[:2]])
        _say(f"   {name} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (name, err)


def test_weight_grads_config2_full_shape(gpu):
    """Config 2's projection at its full shape (M = 8192, N = K = 4096, r = 32: dW unsplit
    on 256 x 256 tiles) against torch fp32 on the device."""
    M, N, K, r, s = 8192, 4096, 4096, 32, 2.0
    _say(f"[weight grads] full config-2 M={M} N={N} K={K} r={r}")
    g = torch.Generator(device=gpu).manual_seed(9)
    x = torch.randn(M, K, device=gpu, generator=g).bfloat16()
    gy = torch.randn(M, N, device=gpu, generator=g).bfloat16()
    A = (torch.randn(r, K, device=gpu, generator=g) * 0.05).bfloat16()
    B = (torch.randn(N, r, device=gpu, generator=g) * 0.05).bfloat16()
    dw, da, db = _bwd(x, gy, A, B, s)
    xf, gf = x.float(), gy.float()
    for name, got, ref in (("dW", dw, gf.t() @ xf),
                           ("dA", da, s * (gf @ B.float()).t() @ xf),
                           ("dB", db, s * gf.t() @ (xf @ A.float().t()))):
        err = ((got.float() - ref).abs().max() / ref.abs().max()).item()
        _say(f"   {name} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (name, err)


def test_weight_grads_deterministic_and_subsets(gpu):
    """Repeated calls agree bit for bit. With dW asked for, dA and dB come from dW (the dW
    route), so any subset that includes dW gives the full call's bits; without dW they take
    the token route (T, U over the tokens), whose da and db do not depend on each other and
    meet the oracle bar."""
    M, N, K, r = 4096, 1024, 2048, 32
    _say(f"[weight grads] determinism M={M} N={N} K={K} r={r}")
    x, gy, A, B, tx, tgy, tA, tB = _inputs(M, N, K, r, 21, gpu)
    full = _bwd(tx, tgy, tA, tB, 0.5)
    again = _bwd(tx, tgy, tA, tB, 0.5)
    for a_, b_ in zip(full, again):
        assert torch.equal(a_, b_)
    for want in ((True, False, False), (True, True, False), (True, False, True)):
        sub = _bwd(tx, tgy, tA, tB, 0.5, want=want)
        for j in range(3):
            assert (sub[j] is None) == (not want[j])
            if want[j]:
                assert torch.equal(sub[j], full[j]), (want, j)
    tok = _bwd(tx, tgy, tA, tB, 0.5, want=(False, True, True))
    tok_a = _bwd(tx, tgy, tA, tB, 0.5, want=(False, True, False))
    tok_b = _bwd(tx, tgy, tA, tB, 0.5, want=(False, False, True))
    assert tok[0] is None and torch.equal(tok_a[1], tok[1]) and torch.equal(tok_b[2], tok[2])
    _, _, dA, dB = O.lora_linear_backward(_np(x), None, _np(A), _np(B), 0.5, _np(gy))
    for name, got, ref in (("dA dW route", full[1], dA), ("dB dW route", full[2], dB),
                           ("dA token route", tok[1], dA), ("dB token route", tok[2], dB)):
        err = O.max_rel_err(_np(got), ref)
        _say(f"   {name} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (name, err)


@pytest.mark.parametrize("M,N,K,r,exact", [
    (1536, 512, 768, 16, True),     # dW split over the tokens in both calls
    (512, 4096, 4096, 16, False),   # dW unsplit: straight from the tile kernel when aligned,
])                                  # through the reduce kernel into the unaligned view
def test_weight_grads_strided_operands_and_destinations(gpu, M, N, K, r, exact):
    """Row strides wider than the rows (x and gy as column slices of wider tensors) and
    destinations that are strided views off the 8-byte grid (the reduce kernels' scalar
    stores) give the contiguous call's values: bit for bit when both take the same route,
    else within one bf16 rounding."""
    _say(f"[weight grads] strided M={M} N={N} K={K} r={r}")
    _, _, _, _, tx, tgy, tA, tB = _inputs(M, N, K, r, 33, gpu)
    ref = _bwd(tx, tgy, tA, tB, 2.0)
    xw = torch.zeros(M, K + 64, dtype=torch.bfloat16, device=gpu)
    xw[:, 8:8 + K] = tx
    gw = torch.zeros(M, N + 128, dtype=torch.bfloat16, device=gpu)
    gw[:, 64:64 + N] = tgy
    dwb = torch.full((N, K + 3), 7.0, dtype=torch.bfloat16, device=gpu)
    dab = torch.full((r, K + 3), 7.0, dtype=torch.bfloat16, device=gpu)
    dbb = torch.full((N, r + 3), 7.0, dtype=torch.bfloat16, device=gpu)
    outs = (dwb[:, 1:1 + K], dab[:, 1:1 + K], dbb[:, 1:1 + r])
    got = _bwd(xw[:, 8:8 + K], gw[:, 64:64 + N], tA, tB, 2.0, outs=outs)
    for a_, b_ in zip(got, ref):
        if exact:
            assert torch.equal(a_, b_)
        else:
            assert O.max_rel_err(_np(a_), _np(b_).astype(np.float64)) <= 4e-3
    for buf, w in ((dwb, K), (dab, K), (dbb, r)):  # nothing written outside the views
        assert bool((buf[:, 0] == 7.0).all()) and bool((buf[:, 1 + w:] == 7.0).all())


def test_weight_grads_op_and_autograd(gpu):
    """wsl::lora_linear_weight_grads (the op the backward calls) and loss.backward() through
    wsl.lora_linear give the C-ABI call's gradients, bit for bit."""
    import weightshared_torchtitan_amd as wsl
    from weightshared_torchtitan_amd import ops
    M, N, K, r = 2048, 1024, 512, 32
    _say(f"[weight grads] op + autograd M={M} N={N} K={K} r={r}")
    _, _, _, _, tx, tgy, tA, tB = _inputs(M, N, K, r, 44, gpu)
    W = (torch.randn(N, K, device=gpu) * 0.02).bfloat16()
    ref = _bwd(tx, tgy, tA, tB, 2.0)
    got = ops.lora_linear_weight_grads_op(tx, tgy, tA, tB, 2.0, True, True, True)
    for a_, b_ in zip(got, ref):
        assert torch.equal(a_, b_)
    lx, lW, lA, lB = (t.clone().requires_grad_(True) for t in (tx, W, tA, tB))
    wsl.lora_linear(lx, lW, lA, lB, 2.0).backward(tgy)
    torch.cuda.synchronize()
    for t, want in ((lW, ref[0]), (lA, ref[1]), (lB, ref[2])):
        assert torch.equal(t.grad, want)


GENERIC_CASES = [
    # M, N, K, r, x column offset: layouts the tile kernels do not take
    (200, 256, 136, 8, 0),    # K off the 64 grid
    (100, 72, 136, 8, 0),     # N and K off the grid
    (300, 192, 256, 12, 0),   # rank not a multiple of 8
    (130, 128, 128, 16, 1),   # x rows not 16-byte aligned (a view one column in)
    (1, 96, 40, 4, 0),        # one token
]


@pytest.mark.parametrize("M,N,K,r,xoff", GENERIC_CASES)
def test_weight_grads_generic_layouts(gpu, M, N, K, r, xoff):
    """Layouts off the tile kernels' grid run on the library's scalar kernels (the token
    route: dW = gy^T x, dB = gy^T T, dA = U^T x with T, U rounded to bf16 once): the query
    says so, every gradient meets the oracle bar, and repeated calls agree bit for bit."""
    from weightshared_torchtitan_amd import _native
    _say(f"[weight grads, generic] M={M} N={N} K={K} r={r} x offset {xoff}")
    x, gy, A, B, tx, tgy, tA, tB = _inputs(M, N, K, r, 55 + M, gpu)
    if xoff:
        big = torch.zeros(M, K + 8, dtype=torch.bfloat16, device=gpu)
        big[:, xoff:xoff + K] = tx
        tx = big[:, xoff:xoff + K]
    assert _native.lib().wsl_lora_linear_bwd_weights_supported(
        tx.data_ptr(), tx.stride(0), tgy.data_ptr(), N, tA.data_ptr(), K, tB.data_ptr(), r, M, N, K, r) == 0
    got = _bwd(tx, tgy, tA, tB, 2.0)
    again = _bwd(tx, tgy, tA, tB, 2.0)
    _, dW, dA, dB = O.lora_linear_backward(_np(x), np.zeros((N, K), np.float32), _np(A), _np(B), 2.0, _np(gy))
    for name, g, g2, ref in zip(("dW", "dA", "dB"), got, again, (dW, dA, dB)):
        err = O.max_rel_err(_np(g), ref)
        _say(f"   {name}: max_rel_err {err:.2e}")
        assert err <= BF16_TOL, name
        assert torch.equal(g, g2), name
    dw_only = _bwd(tx, tgy, tA, tB, 2.0, want=(True, False, False))[0]
    assert torch.equal(dw_only, got[0])
