"""The decode path's two ways to cover a K whose x rows do not fit the LDS at once: K split
over several workgroups (partials handed to the last split) and the pass form (one workgroup
walks its K range in passes, refilling x between them), and the plan's own mix of the two
(two passes per split for an even slice count). Each form, forced with the decode_passes override (-1 splits, 1 passes)
/ on or left to the plan (auto), against the float64 oracle (1e-2 bf16, 3e-2 fp8 base against
fp32 W and 1e-2 against the dequantised W), bitwise repeatable, and with the T wait forced
to its local fallback. The forms sum K in different orders, so they agree with each other
only to the bar."""
import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP8_TOL = 3e-2


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
    # M, N, K, r: x is M x K bf16, more than one slice of the LDS at these sizes
    (64, 6144, 2048, 64),    # two slices (gate at 1.7B)
    (64, 2048, 6144, 64),    # six slices (down at 1.7B; auto: three splits of two passes)
    (48, 1024, 2048, 64),    # three token blocks
    (48, 1000, 6144, 40),    # six slices at three token blocks, N tail
    (33, 1000, 6144, 24),    # N tail, partial rank group
    (64, 1000, 6144, 24),
    (17, 640, 12288, 8),     # two token blocks, three slices
    (16, 2048, 6144, 64),    # one token block, two slices
    (40, 2048, 4096, 0),     # plain linear (no T workgroups)
]


PASS_MODES = {"off": -1, "on": 1, "auto": 0}


def _mode(wsl_opts, mode):
    wsl_opts(decode_passes=PASS_MODES[mode])


@pytest.mark.parametrize("mode", ["off", "on", "auto"])
@pytest.mark.parametrize("M,N,K,r", CASES)
def test_decode_forms_match_oracle(gpu, M, N, K, r, mode, wsl_opts):
    import weightshared_torchtitan_amd as wsl
    _mode(wsl_opts, mode)
    _say(f"[decode {mode}] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=3 * M + N + K + r)
    d = lambda t: None if t is None else t.to(gpu)
    y1 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    y2 = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    err = O.max_rel_err(y1.float().cpu().numpy(), ref)
    _say(f"  max_rel_err={err:.3e}")
    assert np.isfinite(err) and err <= BF16_TOL


def test_override_reaches_the_plan(gpu, wsl_opts):
    """The two forms sum K in different orders, so at a six-slice shape their outputs differ
    in some elements (both within the bar above): the override switched the kernel's form."""
    import weightshared_torchtitan_amd as wsl
    M, N, K, r = 64, 2048, 6144, 64
    x, W, A, B = (t.to(gpu) for t in _inputs(M, N, K, r, seed=43))
    ys = {}
    for mode in ("off", "on"):
        wsl_opts(decode_passes=PASS_MODES[mode])
        ys[mode] = wsl.lora_linear(x, W, A, B, 2.0)
    torch.cuda.synchronize()
    assert not torch.equal(ys["off"], ys["on"])
    assert ((ys["off"].float() - ys["on"].float()).abs().max() / ys["off"].float().abs().max()).item() < BF16_TOL


@pytest.mark.parametrize("mode", ["off", "on", "auto"])
def test_decode_forms_grouped(gpu, mode, wsl_opts):
    """gate|up and q|k|v of Qwen3-1.7B at M = 64 as grouped launches; every group's block
    against the oracle."""
    from weightshared_torchtitan_amd import ops
    _mode(wsl_opts, mode)
    M, K, r = 64, 2048, 64
    for group_n in ((6144, 6144), (2048, 1024, 1024)):
        _say(f"[decode grouped {mode}] M={M} K={K} r={r} groups={group_n}")
        g = torch.Generator().manual_seed(sum(group_n))
        x = torch.randn(M, K, generator=g).bfloat16()
        Ws = [(torch.randn(n, K, generator=g) * 0.02).bfloat16() for n in group_n]
        As = [(torch.randn(r, K, generator=g) * 0.02).bfloat16() for _ in group_n]
        Bs = [(torch.randn(n, r, generator=g) * 0.02).bfloat16() for n in group_n]
        y = ops.lora_linear_grouped_op(x.to(gpu), torch.cat(Ws).to(gpu), None, torch.cat(As).to(gpu),
                                       torch.cat(Bs).to(gpu), 2.0, list(group_n)).float().cpu().numpy()
        n0 = 0
        for i, n in enumerate(group_n):
            ref = O.lora_linear(_np(x), _np(Ws[i]), _np(As[i]), _np(Bs[i]), 2.0)
            err = O.max_rel_err(y[:, n0:n0 + n], ref)
            _say(f"  group {i}: max_rel_err={err:.3e}")
            assert err <= BF16_TOL
            n0 += n


@pytest.mark.parametrize("mode", ["on", "auto"])
def test_pass_form_t_fallback(gpu, mode, wsl_opts):
    """The pass forms with the T wait bound forced to zero from the host: the W workgroups
    compute T themselves, within the bar."""
    import weightshared_torchtitan_amd as wsl
    _mode(wsl_opts, mode)
    M, N, K, r = 64, 2048, 6144, 64
    _say(f"[decode pass T fallback] M={M} N={N} K={K} r={r}")
    x, W, A, B = _inputs(M, N, K, r, seed=41)
    d = lambda t: t.to(gpu)
    wsl_opts(decode_spin_limit=-1)
    y = wsl.lora_linear(d(x), d(W), d(A), d(B), 2.0).float().cpu().numpy()
    torch.cuda.synchronize()
    wsl_opts(decode_spin_limit=0)
    ref = O.lora_linear(_np(x), _np(W), _np(A), _np(B), 2.0)
    assert O.max_rel_err(y, ref) <= BF16_TOL


@pytest.mark.parametrize("mode", ["off", "on"])
def test_decode_forms_fp8(gpu, mode, wsl_opts):
    """Config 5's down projection at M = 16 (fp8 base, K = 12288: three x slices)."""
    import weightshared_torchtitan_amd as wsl
    from weightshared_torchtitan_amd import quantize_fp8_per_channel
    wsl_opts(decode_passes=PASS_MODES[mode])
    M, N, K, r = 16, 4096, 12288, 128
    _say(f"[decode fp8 {mode}] M={M} N={N} K={K} r={r}")
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M, K, generator=g).bfloat16()
    Wf = torch.randn(N, K, generator=g) * 0.02
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N, r, generator=g) * 0.02).bfloat16()
    q, sc = quantize_fp8_per_channel(Wf)
    y = wsl.lora_linear(x.to(gpu), q.to(gpu), A.to(gpu), B.to(gpu), 1.0, w_scale=sc.to(gpu)).float().cpu().numpy()
    err = O.max_rel_err(y, O.lora_linear(_np(x), Wf.numpy(), _np(A), _np(B), 1.0))
    wdq = O.dequantize_fp8(q.view(torch.uint8).numpy(), sc.numpy())
    err_dq = O.max_rel_err(y, O.lora_linear(_np(x), wdq, _np(A), _np(B), 1.0))
    _say(f"  vs fp32 W: {err:.3e}   vs dequantised W: {err_dq:.3e}")
    assert err <= FP8_TOL
    assert err_dq <= BF16_TOL


def test_split_partials_are_consumed(gpu, wsl_opts):
    """After split-form launches (T and W split six ways) the workspace past the counter
    prefix holds no partial-sum word (bit 63 clear, tag bits set): the last split takes
    each word, so none can meet a launch whose 31-bit tag repeats its own. T words (bit 63
    set) stay, as their readers are many."""
    import ctypes
    from weightshared_torchtitan_amd import _native as N
    wsl_opts(decode_passes=-1)
    M, N_, K, r = 64, 2048, 6144, 64
    _say(f"[decode split partials consumed] M={M} N={N_} K={K} r={r}")
    x, W, A, B = (t.to(gpu) for t in _inputs(M, N_, K, r, seed=47))
    y = torch.empty(M, N_, dtype=torch.bfloat16, device=gpu)
    nb = N.workspace_bytes(M, N_, K, r, N.WSL_DTYPE_BF16)
    ws = torch.zeros(nb // 8, dtype=torch.int64, device=gpu)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    for _ in range(3):
        N.check(N.lib().wsl_lora_linear_fwd(p(x), K, p(W), K, N.WSL_DTYPE_BF16, None, p(A), K, p(B), r, 2.0,
                                            p(y), N_, M, N_, K, r, p(ws), nb, stream), "wsl_lora_linear_fwd")
    torch.cuda.synchronize()
    words = ws[65536 // 8:].cpu()
    partial = (words >= 0) & ((words >> 32) != 0)  # bit 63 clear, upper half non-zero
    assert int(partial.sum()) == 0
    assert int((words < 0).sum()) > 0  # the T words of the launch are there
    ref = O.lora_linear(_np(x.cpu()), _np(W.cpu()), _np(A.cpu()), _np(B.cpu()), 2.0)
    assert O.max_rel_err(y.float().cpu().numpy(), ref) <= BF16_TOL
