"""wsl_lora_linear_fwd_noalloc (scratch in a static device array, nothing allocated) against
wsl_lora_linear_fwd (caller's workspace) on the same inputs, through the C ABI.

Each case runs two calls in a row on the no-allocation entry point, the second with a
smaller input, and compares each with the workspace entry point's output: the same kernels
run, so the outputs must be equal bit for bit, and both within the bf16 bar (1e-2) of the
float64 oracle. The cases reach every use of the scratch: the decode path's tagged hand-off
words (K split, so split partials too), the prefill rank pre-pass (T and split partials),
and the generic path's T buffer."""
import ctypes
import sys

import pytest
import torch

from oracle import lora_oracle as O
from weightshared_torchtitan_amd import _native as N

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _inputs(M, N_, K, r, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).bfloat16()
    W = (torch.randn(N_, K, generator=g) * 0.02).bfloat16()
    A = (torch.randn(r, K, generator=g) * 0.02).bfloat16()
    B = (torch.randn(N_, r, generator=g) * 0.02).bfloat16()
    return x, W, A, B


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _with_workspace(dev, x, W, A, B, s):
    M, K = x.shape
    N_, r = B.shape
    y = torch.empty(M, N_, dtype=torch.bfloat16, device=dev)
    nb = N.workspace_bytes(M, N_, K, r, N.WSL_DTYPE_BF16)
    ws = torch.zeros(nb, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = N.lib().wsl_lora_linear_fwd(_ptr(x), x.stride(0), _ptr(W), W.stride(0), N.WSL_DTYPE_BF16, None,
                                     _ptr(A), A.stride(0), _ptr(B), B.stride(0), s, _ptr(y), y.stride(0),
                                     M, N_, K, r, _ptr(ws), ws.numel(), ctypes.c_void_p(stream))
    N.check(rc, "wsl_lora_linear_fwd")
    torch.cuda.synchronize()
    return y


def _noalloc(dev, x, W, A, B, s):
    M, K = x.shape
    N_, r = B.shape
    y = torch.empty(M, N_, dtype=torch.bfloat16, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = N.lib().wsl_lora_linear_fwd_noalloc(_ptr(x), x.stride(0), _ptr(W), W.stride(0), N.WSL_DTYPE_BF16, None,
                                             _ptr(A), A.stride(0), _ptr(B), B.stride(0), s, _ptr(y), y.stride(0),
                                             M, N_, K, r, ctypes.c_void_p(stream))
    N.check(rc, "wsl_lora_linear_fwd_noalloc")
    torch.cuda.synchronize()
    return y


CASES = [
    # (first shape, second smaller shape): M, N, K, r
    ((64, 1024, 4096, 64), (8, 1024, 4096, 64)),      # decode path, K split (partials + T words)
    ((72, 2048, 6144, 64), (64, 6144, 2048, 64)),     # prefill split-K at 72 tokens, then two decode passes
    ((256, 2048, 2048, 64), (160, 1024, 6144, 32)),   # prefill in-launch split-K (arrival counters in the scratch)
    ((4, 2048, 2048, 32), (1, 2048, 2048, 32)),       # decode path, one slice
    ((1024, 768, 1024, 128), (512, 768, 1024, 128)),  # prefill rank pre-pass with split partials
    ((300, 520, 192, 24), (100, 520, 192, 24)),       # prefill, in-kernel rank
    ((100, 200, 72, 8), (50, 200, 72, 8)),            # generic path (K % 64 != 0): T in scratch
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_workspace_entry(gpu, first, second):
    for i, (M, N_, K, r) in enumerate((first, second)):
        _say(f"[noalloc] call {i}: M={M} N={N_} K={K} r={r}")
        x, W, A, B = _inputs(M, N_, K, r, seed=M + N_ + K + r)
        xd, Wd, Ad, Bd = (t.to(gpu) for t in (x, W, A, B))
        want = _with_workspace(gpu, xd, Wd, Ad, Bd, 2.0)
        got = _noalloc(gpu, xd, Wd, Ad, Bd, 2.0)
        assert torch.equal(got, want)
        ref = O.lora_linear(x.float().numpy(), W.float().numpy(), A.float().numpy(), B.float().numpy(), 2.0)
        assert O.max_rel_err(got.float().cpu().numpy(), ref) <= 1e-2


def test_noalloc_repeated_decode_calls_stay_equal(gpu):
    """The launch counter and hand-off words persist in the static array between calls:
    many decode calls in a row (alternating shapes) keep matching the workspace entry."""
    shapes = [(16, 1024, 2048, 64), (2, 1024, 2048, 64), (64, 2048, 4096, 32)]
    data = []
    for M, N_, K, r in shapes:
        x, W, A, B = _inputs(M, N_, K, r, seed=7 * M + r)
        dev_t = tuple(t.to(gpu) for t in (x, W, A, B))
        data.append((dev_t, _with_workspace(gpu, *dev_t, 2.0)))
    _say("[noalloc] 30 alternating decode calls")
    for it in range(30):
        dev_t, want = data[it % len(data)]
        assert torch.equal(_noalloc(gpu, *dev_t, 2.0), want), f"call {it}"


def test_noalloc_wide_decode_form(gpu, wsl_opts):
    """The decode path's wide form (72 tokens, taken with the decode_wide override at 1:
    splits of passes, their partials and T words in the scratch), then a smaller call."""
    wsl_opts(decode_wide=1)
    for i, (M, N_, K, r) in enumerate(((72, 2048, 6144, 64), (66, 3072, 1024, 16))):
        _say(f"[noalloc wide] call {i}: M={M} N={N_} K={K} r={r}")
        x, W, A, B = _inputs(M, N_, K, r, seed=3 * M + K)
        xd, Wd, Ad, Bd = (t.to(gpu) for t in (x, W, A, B))
        want = _with_workspace(gpu, xd, Wd, Ad, Bd, 2.0)
        assert torch.equal(_noalloc(gpu, xd, Wd, Ad, Bd, 2.0), want)
