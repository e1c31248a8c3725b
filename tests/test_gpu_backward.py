"""GPU parity of the LoRA linear's backward against the CPU oracle's gradients.

dx runs on the fused kernel (the forward of the same op on gy, W^T, B^T, A^T); dW, dA, dB
on plain GEMMs. Bar, as for the forward: max|g - g_ref| / max|g_ref| <= 1e-2 for each
gradient, g_ref = float64 oracle (oracle.lora_oracle.lora_linear_backward) on the same
bf16-rounded inputs; 3e-2 for dx with an fp8 base.
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


def _leaf(t, dev):
    return None if t is None else t.to(dev).requires_grad_(True)


def _np(t):
    return None if t is None else t.detach().float().cpu().numpy()


CASES = [
    # M, N, K, r, s, has_w: which kernel runs dx (its K is the forward's N)
    (2048, 1024, 1024, 16, 2.0, True),   # config-1 shape: prefill kernel
    (512, 2048, 768, 32, 2.0, True),     # prefill, N != K
    (640, 512, 256, 128, 1.0, True),     # r > 64: dx through the rank pre-pass
    (4, 2048, 1024, 64, 2.0, True),      # decode-shaped M: dx on the decode kernel
    (100, 72, 136, 8, 2.0, True),        # N = 72 is not a multiple of 64: generic kernel
    (384, 640, 320, 32, 2.0, False),     # delta only (LoRAModule.forward)
    (256, 512, 384, 0, 2.0, True),       # plain linear
]


@pytest.mark.parametrize("M,N,K,r,s,has_w", CASES)
def test_backward_parity(gpu, M, N, K, r, s, has_w):
    import weightshared_torchtitan_amd as wsl
    _say(f"[backward] M={M} N={N} K={K} r={r} has_w={has_w}")
    g = torch.Generator().manual_seed(M + N + K + r)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16() if has_w else None
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16() if r else None
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16() if r else None
    gy = torch.randn(M, N, generator=g).bfloat16()
    tx, tW, tA, tB = (_leaf(t, gpu) for t in (x, W, A, B))
    y = wsl.lora_linear(tx, tW, tA, tB, s)
    y.backward(gy.to(gpu))
    torch.cuda.synchronize()
    ref = O.lora_linear_backward(_np(x), _np(W), _np(A), _np(B), s, _np(gy))
    for name, t, g_ref in zip(("dx", "dW", "dA", "dB"), (tx, tW, tA, tB), ref):
        if t is None:
            continue
        assert t.grad is not None, name
        assert t.grad.dtype == torch.bfloat16 and t.grad.shape == t.shape, name
        err = O.max_rel_err(_np(t.grad), g_ref)
        _say(f"   {name} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (name, err)


def test_backward_fp8_base_dx(gpu):
    import weightshared_torchtitan_amd as wsl
    M, N, K, r = 256, 1024, 512, 32
    _say(f"[backward fp8] M={M} N={N} K={K} r={r}")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = torch.randn(N, K, generator=g) * 0.02
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16()
    gy = torch.randn(M, N, generator=g).bfloat16()
    q, ws = wsl.quantize_fp8_per_channel(W)
    tx, tA, tB = (_leaf(t, gpu) for t in (x, A, B))
    y = wsl.lora_linear(tx, q.to(gpu), tA, tB, 1.0, w_scale=ws.to(gpu))
    y.backward(gy.to(gpu))
    torch.cuda.synchronize()
    # against the fp32 W (quantisation error included) and against the dequantised W
    for W_ref, tol in ((W.numpy(), FP8_TOL), (O.dequantize_fp8(q.view(torch.uint8).numpy(), ws.numpy()), BF16_TOL)):
        dx, _, dA, dB = O.lora_linear_backward(_np(x), W_ref, _np(A), _np(B), 1.0, _np(gy))
        assert O.max_rel_err(_np(tx.grad), dx) <= tol
        assert O.max_rel_err(_np(tA.grad), dA) <= BF16_TOL
        assert O.max_rel_err(_np(tB.grad), dB) <= BF16_TOL


def test_lora_linear_module_trains(gpu):
    # the module path: shared base weight, per-instance LoRA; gradients reach every
    # parameter and one SGD step lowers the loss
    import weightshared_torchtitan_amd as wsl
    torch.manual_seed(0)
    base = torch.nn.Linear(512, 512, bias=False).to(gpu).bfloat16()
    with torch.no_grad():
        base.weight.normal_(0, 0.02)
    mods = [wsl.LoRALinear(base, wsl.LoRAModule(512, 512, rank=16)).to(gpu).bfloat16() for _ in range(2)]
    for m in mods:
        with torch.no_grad():
            m.lora.w_a.weight.normal_(0, 0.02)
            m.lora.w_b.weight.normal_(0, 0.02)
    x = torch.randn(256, 512, device=gpu).bfloat16()
    target = torch.randn(256, 512, device=gpu).bfloat16()

    def loss_fn():
        h = mods[1](mods[0](x).float().tanh().bfloat16())
        return ((h.float() - target.float()) ** 2).mean()

    loss = loss_fn()
    loss.backward()
    params = [base.weight] + [p for m in mods for p in (m.lora.w_a.weight, m.lora.w_b.weight)]
    for p in params:
        assert p.grad is not None and torch.isfinite(p.grad.float()).all()
    with torch.no_grad():
        for p in params:  # a descent step of 2 % of each parameter's norm (bf16 resolves it)
            p -= 0.02 * p.float().norm() * p.grad / p.grad.float().norm()
    assert loss_fn().item() < loss.item()


def test_shared_weight_updates_seen_by_next_backward(gpu):
    # dx of two layers sharing one W reads W where it lies; an in-place update of W between
    # steps must be seen by the next backward
    import weightshared_torchtitan_amd as wsl
    M, N, K, r = 256, 512, 384, 16
    g = torch.Generator().manual_seed(21)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16()
    gy = torch.randn(M, N, generator=g).bfloat16()
    tW = W.to(gpu).requires_grad_(True)
    for step in range(3):
        _say(f"[shared W] step {step}")
        tx = x.to(gpu).requires_grad_(True)
        ys = [wsl.lora_linear(tx, tW, A.to(gpu), B.to(gpu), 2.0) for _ in range(2)]  # two layers
        torch.autograd.backward(ys, [gy.to(gpu)] * 2)
        torch.cuda.synchronize()
        Wn = _np(tW)
        dx = 2 * O.lora_linear_backward(_np(x), Wn, _np(A), _np(B), 2.0, _np(gy))[0]
        assert O.max_rel_err(_np(tx.grad), dx) <= BF16_TOL
        with torch.no_grad():
            tW.mul_(-1.5).add_(0.01)  # an optimizer-like in-place update
        tW.grad = None


@pytest.mark.parametrize("M,N,K,r,need_w", [(24, 1024, 512, 16, False), (40, 512, 1024, 8, True),
                                            (100, 256, 768, 32, True)])
def test_weight_grads_partial_token_tile_repeats(gpu, M, N, K, r, need_w):
    """Token counts off the 64-token tile: the rows past the tokens are zeroed in the last
    token tile after every wave's fill has landed. Twenty launches in a row give the same
    bits, and the oracle's gradients to the bar."""
    from weightshared_torchtitan_amd import ops
    _say(f"[weight grads repeats] M={M} N={N} K={K} r={r} dW={need_w}")
    g = torch.Generator().manual_seed(M * 5 + N + K)
    x = torch.randn(M, K, generator=g).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.05).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.05).bfloat16()
    gy = torch.randn(M, N, generator=g).bfloat16()
    d = lambda t: t.to(gpu)
    first = None
    for i in range(20):
        dw, da, db = ops.lora_linear_weight_grads_op(d(x), d(gy), d(A), d(B), 2.0, need_w, True, True)
        got = ([dw.cpu()] if need_w else []) + [da.cpu(), db.cpu()]
        if first is None:
            first = got
        else:
            for a_, b_ in zip(first, got):
                assert torch.equal(a_, b_), i
    W = torch.zeros(N, K).bfloat16()
    ref = O.lora_linear_backward(_np(x), _np(W), _np(A), _np(B), 2.0, _np(gy))
    names = (["dW"] if need_w else []) + ["dA", "dB"]
    refs = ([ref[1]] if need_w else []) + [ref[2], ref[3]]
    for name, t, g_ref in zip(names, first, refs):
        err = O.max_rel_err(t.float().numpy(), g_ref)
        _say(f"   {name} max_rel_err {err:.2e}")
        assert err <= BF16_TOL, (name, err)


def test_off_grid_backward_runs_no_vendor_gemm(gpu):
    """The backward at a layout off the tile grid (N = 72, K = 136) runs dx on the library's
    generic forward and dW, dA, dB on its generic weight-gradient kernels: no hipBLASLt or
    rocBLAS GEMM kernel appears in a trace of the backward."""
    from torch.profiler import ProfilerActivity, profile
    import weightshared_torchtitan_amd as wsl
    M, N, K, r = 100, 72, 136, 8
    _say(f"[backward, no vendor GEMM] M={M} N={N} K={K} r={r}")
    g = torch.Generator().manual_seed(3)
    x, W, A, B = (_leaf(t, gpu) for t in (torch.randn(M, K, generator=g).bfloat16(),
                                          (torch.randn(N, K, generator=g) * 0.02).bfloat16(),
                                          (torch.randn(r, K, generator=g) * 0.02).bfloat16(),
                                          (torch.randn(N, r, generator=g) * 0.02).bfloat16()))
    gy = torch.randn(M, N, generator=g).bfloat16().to(gpu)
    wsl.lora_linear(x, W, A, B, 2.0).backward(gy)  # warm-up: workspaces
    torch.cuda.synchronize()
    for t in (x, W, A, B):
        t.grad = None
    y = wsl.lora_linear(x, W, A, B, 2.0)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        y.backward(gy)
        torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    if not kernels:
        pytest.skip("the profiler recorded no device activity on this build")
    vendor = [k for k in kernels if any(s in k for s in ("Cijk", "gemm", "Gemm", "GEMM", "rocblas", "hipblaslt"))]
    assert vendor == [], vendor
    assert all(t.grad is not None for t in (x, W, A, B))
