"""torch custom ops over libwsl: ``wsl::lora_linear``, ``wsl::lora_linear_grouped`` (the
projections that read one activation in one call), ``wsl::factorized_embedding`` and the
decode-step ops of the weight-shared Qwen3 harness.

Every op has a HIP (device type "cuda" on ROCm) implementation only. Called with CPU
tensors they raise; there is no CPU or eager-PyTorch fallback. Each op has a fake
(meta) implementation so models can be built on the meta device and traced by
torch.compile, matching how the reference builds its model
(torchtitan/train.py:156-157) and compiles blocks
(torchtitan/models/llama3/infra/parallelize.py:348-357).
"""
from __future__ import annotations

from typing import Optional

import contextlib
import ctypes
import os

import torch

from . import _native

_FP8 = torch.float8_e4m3fn

# fp8 base weights: on prefill shapes the product runs on the fp8 matrix cores with bf16-quality
# activations (two e4m3 terms per element). When set (or with WSL_FP8_ACTIVATIONS=1), one
# e4m3 term per activation instead (WSL_DTYPE_FP8_E4M3_ACT8): half the matrix-core work, and
# an error of about 3.7e-2 against the fp32-weight reference at config-5 shapes, above the
# 3e-2 bar the default keeps (2.4-2.6e-2).
FP8_ACTIVATIONS = os.environ.get("WSL_FP8_ACTIVATIONS", "") not in ("", "0")


@contextlib.contextmanager
def path_options(**opts: int):
    """Forces kernel forms for the duration of the block through libwsl's path overrides
    (``_native.OPTIONS``: e.g. ``prefill_strips=-1``, ``prefill_split=4``,
    ``decode_passes=1``), restoring the previous values on exit. The overrides are
    process-wide; use them for side-by-side timing and tests, not in concurrent code."""
    saved = {k: _native.get_option(k) for k in opts}
    try:
        for k, v in opts.items():
            _native.set_option(k, v)
        yield
    finally:
        for k, v in saved.items():
            _native.set_option(k, v)


def plan(M: int, K: int, r: int, group_n, fp8: bool = False) -> dict:
    """The kernel plan libwsl takes for a (grouped) LoRA linear of these sizes on dense,
    aligned operands: path, launches, tile, in-loop rank blocks, pre-pass, strips, K splits,
    workgroups, and whether the column tiles share T (shared_t)."""
    return _native.plan(M, K, r, list(group_n), _fp8_code() if fp8 else _native.WSL_DTYPE_BF16)


def _fp8_code() -> int:
    return _native.WSL_DTYPE_FP8_E4M3_ACT8 if FP8_ACTIVATIONS else _native.WSL_DTYPE_FP8_E4M3


def _dev_ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _row_major(t: torch.Tensor, name: str) -> torch.Tensor:
    """2-D view with a contiguous inner dimension (copies only if it is strided)."""
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        t = t.contiguous()
    return t


def _check_device(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "wsl ops run on the GPU only (HIP kernels for gfx950); got a tensor on "
                f"{t.device}. There is no CPU implementation.")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"all tensors must be on one device ({dev} vs {t.device})")
    assert dev is not None
    return dev


_WS_MIN_BYTES = 16 << 20
_workspaces: dict = {}
# Workspaces that were replaced (grown, or dropped after a failed launch). A HIP graph
# captured while one of them was current keeps its raw address and writes to it on every
# replay, so none of them is ever returned to the caching allocator: they stay referenced
# here until the process ends.
_retired: list = []


def _retire(key) -> None:
    """Replaces the workspace of `key` after a failed kernel launch (WSL_E_LAUNCH), which may
    leave its counters mid-update. Argument, shape and workspace errors return before any
    launch and keep the buffer."""
    buf = _workspaces.pop(key, None)
    if buf is not None:
        _retired.append(buf)


def workspace(dev: torch.device, stream: int, nbytes: int, kind: str = "lora") -> torch.Tensor:
    """The persistent scratch buffer of (device, stream, kind).

    libwsl requires its workspaces to be zero-filled before first use (the leading
    counters of the decode kernels) and keeps those counters valid across calls, so one
    zero-filled buffer per stream and kind is reused by every call on that stream; it only
    grows (a grown buffer starts zeroed again). A replaced buffer is kept alive for the
    life of the process (graphs captured earlier still address it).
    """
    key = (dev.index, stream, kind)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if dev.type == "cuda" and torch.cuda.is_current_stream_capturing():
            # allocated inside a capture, the buffer would come from the graph's private
            # pool and its zero-fill would replay with the graph
            raise RuntimeError(
                f"libwsl: the {kind!r} workspace would have to grow to {nbytes} bytes during graph "
                "capture; run the op once eagerly with the same shapes before capturing")
        _retire(key)
        buf = torch.zeros(max(2 * nbytes, _WS_MIN_BYTES), dtype=torch.uint8, device=dev)
        _workspaces[key] = buf
    return buf


def _out_features(w: Optional[torch.Tensor], b: Optional[torch.Tensor]) -> int:
    if w is not None:
        return w.shape[0]
    if b is not None:
        return b.shape[0]
    raise ValueError("lora_linear needs w or (a, b)")


@torch.library.custom_op("wsl::lora_linear", mutates_args=(), device_types="cuda")
def lora_linear_op(x: torch.Tensor, w: Optional[torch.Tensor], w_scale: Optional[torch.Tensor],
                   a: Optional[torch.Tensor], b: Optional[torch.Tensor],
                   scale: float) -> torch.Tensor:
    """y = (x . w^T) * w_scale + scale * (x . a^T) . b^T  (bf16 in/out, fp32 accumulate)."""
    dev = _check_device(x, w, w_scale, a, b)
    K = x.shape[-1]
    N = _out_features(w, b)
    lead = x.shape[:-1]
    x2 = _row_major(x.reshape(-1, K), "x")
    M = x2.shape[0]
    if x2.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x2.dtype}")
    w_dtype = _native.WSL_DTYPE_BF16
    if w is not None:
        w = _row_major(w, "w")
        if w.shape[1] != K:
            raise ValueError(f"w is {tuple(w.shape)} but x has K={K}")
        if w.dtype == _FP8:
            w_dtype = _fp8_code()
            if w_scale is None:
                raise ValueError("an fp8 w needs w_scale [N] fp32")
            if w_scale.dtype != torch.float32 or w_scale.shape != (N,):
                raise ValueError(f"w_scale must be fp32 [{N}], got {w_scale.dtype} {tuple(w_scale.shape)}")
            w_scale = w_scale.contiguous()
        elif w.dtype != torch.bfloat16:
            raise TypeError(f"w must be bfloat16 or float8_e4m3fn, got {w.dtype}")
        elif w_scale is not None:
            raise ValueError("w_scale is only valid with an fp8 w")
    r = 0
    if a is not None or b is not None:
        if a is None or b is None:
            raise ValueError("a and b must be given together")
        a = _row_major(a, "a")
        b = _row_major(b, "b")
        r = a.shape[0]
        if a.shape[1] != K or b.shape != (N, r):
            raise ValueError(f"LoRA shapes a {tuple(a.shape)}, b {tuple(b.shape)} do not match K={K}, N={N}")
        if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise TypeError("a and b must be bfloat16")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if M > 0:
        ws_bytes = _native.workspace_bytes(M, N, K, r, w_dtype)
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = workspace(dev, stream, ws_bytes)
        with torch.cuda.device(dev):
            rc = _native.lib().wsl_lora_linear_fwd(
                x2.data_ptr(), x2.stride(0),
                _dev_ptr(w), w.stride(0) if w is not None else 0, w_dtype, _dev_ptr(w_scale),
                _dev_ptr(a), a.stride(0) if a is not None else 0,
                _dev_ptr(b), b.stride(0) if b is not None else 0,
                float(scale),
                y.data_ptr(), y.stride(0),
                M, N, K, r,
                ws.data_ptr(), ws.numel(), stream)
        if rc == _native.WSL_E_LAUNCH:
            _retire((dev.index, stream, "lora"))  # a failed launch may leave counters mid-update
        _native.check(rc, "wsl_lora_linear_fwd")
    return y.reshape(*lead, N)


@lora_linear_op.register_fake
def _lora_linear_fake(x, w, w_scale, a, b, scale):
    N = _out_features(w, b)
    return x.new_empty((*x.shape[:-1], N), dtype=torch.bfloat16)


@torch.library.custom_op("wsl::lora_linear_bwd_input", mutates_args=(), device_types="cuda")
def lora_linear_bwd_input_op(gy: torch.Tensor, w: torch.Tensor, w_scale: Optional[torch.Tensor],
                             a: Optional[torch.Tensor], b: Optional[torch.Tensor], scale: float) -> torch.Tensor:
    """dx [M, K] = gy . W + scale * (gy . b) . a for bf16 gy [M, N], w [N, K] (bf16, or
    float8_e4m3fn with w_scale [N] fp32: W = bf16(w * w_scale[:, None]) row by row),
    a [r, K] and b [N, r] as the forward takes them (a and b None: r = 0):
    wsl_lora_linear_bwd_input, the fused kernel reading w where it lies as the reduction rows
    of its tiles. Layouts that entry point does not take (N off the 64 grid, K or r off 8,
    unaligned rows) run the forward op on a transposed copy of W."""
    dev = _check_device(gy, w, w_scale, a, b)
    gy2 = _row_major(gy.reshape(-1, gy.shape[-1]), "grad_y")
    w = _row_major(w, "w")
    M, N = gy2.shape
    if w.dim() != 2 or w.shape[0] != N:
        raise ValueError(f"w {tuple(w.shape)} does not match grad_y's {N} columns")
    K = w.shape[1]
    fp8 = w.dtype == _FP8
    if gy2.dtype != torch.bfloat16 or (w.dtype != torch.bfloat16 and not fp8):
        raise TypeError("grad_y must be bfloat16 and w bfloat16 or float8_e4m3fn")
    if fp8 and (w_scale is None or w_scale.dtype != torch.float32 or w_scale.shape != (N,)):
        raise ValueError("an fp8 w needs w_scale [N] float32")
    if fp8:
        w_scale = w_scale.contiguous()
    r = 0
    if a is not None or b is not None:
        if a is None or b is None:
            raise ValueError("a and b go together")
        a = _row_major(a, "a")
        b = _row_major(b, "b")
        r = a.shape[0]
        if a.shape[1] != K or b.shape != (N, r):
            raise ValueError(f"LoRA shapes a {tuple(a.shape)}, b {tuple(b.shape)} do not match K={K}, N={N}")
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    if M == 0:
        return dx
    L = _native.lib()
    wdt = _native.WSL_DTYPE_FP8_E4M3 if fp8 else _native.WSL_DTYPE_BF16
    ws_ptr = w_scale.data_ptr() if fp8 else None
    if not L.wsl_lora_linear_bwd_input_supported(gy2.data_ptr(), gy2.stride(0), w.data_ptr(), w.stride(0), wdt,
                                                 ws_ptr, _dev_ptr(a), a.stride(0) if r else 0, _dev_ptr(b),
                                                 b.stride(0) if r else 0, dx.data_ptr(), K, M, N, K, r):
        wt = ((w.float() * w_scale[:, None]).to(torch.bfloat16) if fp8 else w).t().contiguous()
        return lora_linear_op(gy2, wt, None, b.t().contiguous() if r else None, a.t().contiguous() if r else None,
                              float(scale))
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = workspace(dev, stream, _native.bwd_input_workspace_bytes(M, N, K, r))
    with torch.cuda.device(dev):
        rc = L.wsl_lora_linear_bwd_input(gy2.data_ptr(), gy2.stride(0), w.data_ptr(), w.stride(0), wdt, ws_ptr,
                                         _dev_ptr(a), a.stride(0) if r else 0, _dev_ptr(b), b.stride(0) if r else 0,
                                         float(scale), dx.data_ptr(), K, M, N, K, r, ws.data_ptr(), ws.numel(),
                                         stream)
    _native.check(rc, "wsl_lora_linear_bwd_input")
    return dx


@lora_linear_bwd_input_op.register_fake
def _lora_linear_bwd_input_fake(gy, w, w_scale, a, b, scale):
    return gy.new_empty((gy.numel() // gy.shape[-1], w.shape[1]), dtype=torch.bfloat16)


def _input_grad(gy2, w, w_scale, a, b, s):
    """dx = gy . W + s (gy . b) . a with W read where it lies (an fp8 W decoded with its
    per-row scale as it is staged; a and b None: the base term alone)."""
    return lora_linear_bwd_input_op(gy2, w, w_scale if w.dtype == _FP8 else None, a, b, float(s))


@torch.library.custom_op("wsl::lora_linear_weight_grads", mutates_args=(), device_types="cuda")
def lora_linear_weight_grads_op(x: torch.Tensor, gy: torch.Tensor, a: Optional[torch.Tensor],
                                b: Optional[torch.Tensor], scale: float, need_w: bool, need_a: bool,
                                need_b: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """dw = gy^T . x [N, K], da = scale (gy . b)^T . x [r, K], db = scale gy^T . (x . a^T)
    [N, r], each only when asked for (else an empty tensor), bf16 from bf16 x [M, K],
    gy [M, N], a [r, K], b [N, r] (wsl_lora_linear_bwd_weights: dW over the tokens on the
    fused kernel's tile loop, reading x and gy as they lie, da and db from dW; layouts off
    the tile grid on the library's scalar kernels)."""
    dev = _check_device(x, gy, a, b)
    x2 = _row_major(x.reshape(-1, x.shape[-1]), "x")
    gy2 = _row_major(gy.reshape(-1, gy.shape[-1]), "grad_y")
    M, K = x2.shape
    N = gy2.shape[1]
    if gy2.shape[0] != M:
        raise ValueError(f"x has {M} rows but grad_y has {gy2.shape[0]}")
    if x2.dtype != torch.bfloat16 or gy2.dtype != torch.bfloat16:
        raise TypeError("x and grad_y must be bfloat16")
    r = 0
    if need_a or need_b:
        if a is None or b is None:
            raise ValueError("da and db need a and b")
        a = _row_major(a, "a")
        b = _row_major(b, "b")
        r = a.shape[0]
        if a.shape[1] != K or b.shape != (N, r):
            raise ValueError(f"LoRA shapes a {tuple(a.shape)}, b {tuple(b.shape)} do not match K={K}, N={N}")
        if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise TypeError("a and b must be bfloat16")
    empty = lambda: x2.new_empty(0)  # a fresh one per unused output: returns may not alias
    if M == 0:
        return (x2.new_zeros(N, K) if need_w else empty(), x2.new_zeros(r, K) if need_a else empty(),
                x2.new_zeros(N, r) if need_b else empty())
    L = _native.lib()
    dw = torch.empty((N, K), dtype=torch.bfloat16, device=dev) if need_w else None
    da = torch.empty((r, K), dtype=torch.bfloat16, device=dev) if need_a else None
    db = torch.empty((N, r), dtype=torch.bfloat16, device=dev) if need_b else None
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = workspace(dev, stream, _native.bwd_weights_workspace_bytes(M, N, K, r))
    with torch.cuda.device(dev):
        rc = L.wsl_lora_linear_bwd_weights(
            x2.data_ptr(), x2.stride(0), gy2.data_ptr(), gy2.stride(0),
            _dev_ptr(a), a.stride(0) if r else 0, _dev_ptr(b), b.stride(0) if r else 0,
            float(scale), M, N, K, r,
            _dev_ptr(dw), K, _dev_ptr(da), K, _dev_ptr(db), r,
            ws.data_ptr(), ws.numel(), stream)
    _native.check(rc, "wsl_lora_linear_bwd_weights")
    return dw if need_w else empty(), da if need_a else empty(), db if need_b else empty()


@lora_linear_weight_grads_op.register_fake
def _lora_linear_weight_grads_fake(x, gy, a, b, scale, need_w, need_a, need_b):
    K, N = x.shape[-1], gy.shape[-1]
    r = a.shape[0] if a is not None else 0
    empty = lambda: x.new_empty(0, dtype=torch.bfloat16)
    return (x.new_empty((N, K), dtype=torch.bfloat16) if need_w else empty(),
            x.new_empty((r, K), dtype=torch.bfloat16) if need_a else empty(),
            x.new_empty((N, r), dtype=torch.bfloat16) if need_b else empty())


def weight_grads(x2, gy2, a, b, s, need_w, need_a, need_b):
    """(dw, da, db) with None for the ones not asked for (see lora_linear_weight_grads_op)."""
    if not (need_w or need_a or need_b):
        return None, None, None
    dw, da, db = lora_linear_weight_grads_op(x2, gy2, a, b, float(s), bool(need_w), bool(need_a), bool(need_b))
    return dw if need_w else None, da if need_a else None, db if need_b else None


def _lora_linear_setup(ctx, inputs, output):
    x, w, w_scale, a, b, scale = inputs
    ctx.save_for_backward(x, w, w_scale, a, b)
    ctx.scale = scale


def _lora_linear_backward(ctx, gy):
    """Backward of ``wsl::lora_linear``. With T = x . a^T and U = gy . b:

        dx = gy . W + scale * U . a     one wsl::lora_linear_bwd_input launch: the fused
                                        kernel on (gy, b^T, a^T) with W's rows as the
                                        reduction of its tiles, read where they lie
        dW = gy^T . x                   one wsl::lora_linear_weight_grads call: dW over the
        da = scale * U^T . x            tokens on the fused kernel's tile loop (operands
        db = scale * gy^T . T           read as they lie), da and db from dW

    The reference has no backward of its own: torch autograd differentiates
    LoRAModule.forward (torchtitan/models/llama3/model/model.py:189-192) and the base
    nn.Linear (:257-273) composed by broadcast_add with g = 1 (:392-398); the trainer runs
    it at torchtitan/train.py:456. An fp8 ``w`` gets no gradient (it is not a trainable
    dtype); its dx uses the dequantised weight. ``w_scale`` gets no gradient.
    """
    x, w, w_scale, a, b = ctx.saved_tensors
    s = float(ctx.scale)
    need_x, need_w, _, need_a, need_b, _ = ctx.needs_input_grad
    K = x.shape[-1]
    gy2 = _row_major(gy.reshape(-1, gy.shape[-1]).to(torch.bfloat16), "grad_y")
    x2 = x.reshape(-1, K)
    has_lora = a is not None and a.shape[0] > 0
    dx = dw = da = db = None
    if need_x:
        if w is not None:
            dx = _input_grad(gy2, w, w_scale, a if has_lora else None, b if has_lora else None, s)
        elif has_lora:  # the delta alone: s (gy . b) . a on the fused kernel's delta form
            dx = lora_linear_op(gy2, None, None, b.t().contiguous(), a.t().contiguous(), s)
        else:
            dx = torch.zeros_like(x2)
        dx = dx.reshape(x.shape)
    dw, da, db = weight_grads(x2, gy2, a, b, s, need_w and w is not None and w.dtype == torch.bfloat16,
                              has_lora and need_a, has_lora and need_b)
    return dx, dw, None, da, db, None


lora_linear_op.register_autograd(_lora_linear_backward, setup_context=_lora_linear_setup)


@torch.library.custom_op("wsl::lora_linear_grouped", mutates_args=(), device_types="cuda")
def lora_linear_grouped_op(x: torch.Tensor, w: torch.Tensor, w_scale: Optional[torch.Tensor],
                           a: Optional[torch.Tensor], b: Optional[torch.Tensor], scale: float,
                           group_n: list[int]) -> torch.Tensor:
    """Projections that read the same x, side by side in N (wsl_lora_linear_grouped_fwd).

    w [N, K] and b [N, r] stack the groups' rows (N = sum(group_n)); a [G*r, K] stacks
    their A factors (group g uses rows g*r..g*r+r-1). Output column block g is
    ``x . w_g^T (* w_scale_g) + scale * (x . a_g^T) . b_g^T``, the result of
    ``lora_linear_op`` on that group alone.
    """
    dev = _check_device(x, w, w_scale, a, b)
    K = x.shape[-1]
    G = len(group_n)
    if not 1 <= G <= _native.WSL_MAX_GROUPS or any(int(n) < 1 for n in group_n):
        raise ValueError(f"group_n must hold 1..{_native.WSL_MAX_GROUPS} positive widths, got {group_n}")
    N = sum(int(n) for n in group_n)
    lead = x.shape[:-1]
    x2 = _row_major(x.reshape(-1, K), "x")
    M = x2.shape[0]
    if x2.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x2.dtype}")
    w = _row_major(w, "w")
    if w.shape != (N, K):
        raise ValueError(f"w is {tuple(w.shape)}, expected ({N}, {K}) for groups {group_n}")
    w_dtype = _native.WSL_DTYPE_BF16
    if w.dtype == _FP8:
        w_dtype = _fp8_code()
        if w_scale is None or w_scale.dtype != torch.float32 or w_scale.shape != (N,):
            raise ValueError(f"an fp8 w needs w_scale fp32 [{N}]")
        w_scale = w_scale.contiguous()
    elif w.dtype != torch.bfloat16:
        raise TypeError(f"w must be bfloat16 or float8_e4m3fn, got {w.dtype}")
    elif w_scale is not None:
        raise ValueError("w_scale is only valid with an fp8 w")
    r = 0
    if a is not None or b is not None:
        if a is None or b is None:
            raise ValueError("a and b must be given together")
        a = _row_major(a, "a")
        b = _row_major(b, "b")
        r = b.shape[1]
        if a.shape != (G * r, K) or b.shape[0] != N:
            raise ValueError(f"LoRA shapes a {tuple(a.shape)}, b {tuple(b.shape)} do not match "
                             f"{G} groups of rank {r}, K={K}, N={N}")
        if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise TypeError("a and b must be bfloat16")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    if M > 0:
        gn = _native.group_array(group_n)
        ws_bytes = _native.grouped_workspace_bytes(M, K, r, group_n, w_dtype)
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = workspace(dev, stream, ws_bytes)
        with torch.cuda.device(dev):
            rc = _native.lib().wsl_lora_linear_grouped_fwd(
                x2.data_ptr(), x2.stride(0),
                w.data_ptr(), w.stride(0), w_dtype, _dev_ptr(w_scale),
                _dev_ptr(a), a.stride(0) if a is not None else 0,
                _dev_ptr(b), b.stride(0) if b is not None else 0,
                float(scale),
                y.data_ptr(), y.stride(0),
                M, K, r, G, gn,
                ws.data_ptr(), ws.numel(), stream)
        if rc == _native.WSL_E_LAUNCH:
            _retire((dev.index, stream, "lora"))
        _native.check(rc, "wsl_lora_linear_grouped_fwd")
    return y.reshape(*lead, N)


@lora_linear_grouped_op.register_fake
def _lora_linear_grouped_fake(x, w, w_scale, a, b, scale, group_n):
    return x.new_empty((*x.shape[:-1], sum(int(n) for n in group_n)), dtype=torch.bfloat16)


@torch.library.custom_op("wsl::lora_linear_bcast", mutates_args=(), device_types="cuda")
def lora_linear_bcast_op(x: torch.Tensor, w: torch.Tensor, w_scale: Optional[torch.Tensor],
                         a: Optional[torch.Tensor], b: Optional[torch.Tensor], scale: float, g: int,
                         n_groups: int) -> torch.Tensor:
    """Shared-base LoRA linears in one launch (wsl_lora_linear_bcast_fwd): w [base_n, K] serves
    n_groups projections of width N = b.shape[0] / n_groups (N = w.shape[0] without LoRA), and
    output block j is the reference's broadcast_add(x . w^T, scale * (x . a_j^T) . b_j^T, g),
    a = [a_0; a_1; ...] [n_groups * r, K], b = [b_0; b_1; ...] [n_groups * N, r]."""
    dev = _check_device(x, w, w_scale, a, b)
    K = x.shape[-1]
    G = int(n_groups)
    if not 1 <= G <= _native.WSL_MAX_GROUPS:
        raise ValueError(f"n_groups must be in [1, {_native.WSL_MAX_GROUPS}], got {G}")
    lead = x.shape[:-1]
    x2 = _row_major(x.reshape(-1, K), "x")
    M = x2.shape[0]
    if x2.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x2.dtype}")
    w = _row_major(w, "w")
    base_n = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"w is {tuple(w.shape)} but x has K={K}")
    w_dtype = _native.WSL_DTYPE_BF16
    if w.dtype == _FP8:
        w_dtype = _fp8_code()
        if w_scale is None or w_scale.dtype != torch.float32 or w_scale.shape != (base_n,):
            raise ValueError(f"an fp8 w needs w_scale fp32 [{base_n}]")
        w_scale = w_scale.contiguous()
    elif w.dtype != torch.bfloat16:
        raise TypeError(f"w must be bfloat16 or float8_e4m3fn, got {w.dtype}")
    elif w_scale is not None:
        raise ValueError("w_scale is only valid with an fp8 w")
    r = 0
    N = base_n
    if a is not None or b is not None:
        if a is None or b is None:
            raise ValueError("a and b must be given together")
        a = _row_major(a, "a")
        b = _row_major(b, "b")
        r = b.shape[1]
        if b.shape[0] % G != 0 or a.shape != (G * r, K):
            raise ValueError(f"LoRA shapes a {tuple(a.shape)}, b {tuple(b.shape)} do not match {G} groups, K={K}")
        N = b.shape[0] // G
        if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
            raise TypeError("a and b must be bfloat16")
    if N % base_n != 0 or base_n % int(g) != 0:
        raise ValueError(f"broadcast needs N % base_n == 0 and base_n % g == 0 (N {N}, base_n {base_n}, g {g})")
    y = torch.empty((M, G * N), dtype=torch.bfloat16, device=dev)
    if M > 0:
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = workspace(dev, stream, _native.bcast_workspace_bytes(M, N, K, r, G, w_dtype))
        with torch.cuda.device(dev):
            rc = _native.lib().wsl_lora_linear_bcast_fwd(
                x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), w_dtype, _dev_ptr(w_scale),
                _dev_ptr(a), a.stride(0) if a is not None else 0, _dev_ptr(b), b.stride(0) if b is not None else 0,
                float(scale), y.data_ptr(), y.stride(0), M, N, K, r, base_n, int(g), G,
                ws.data_ptr(), ws.numel(), stream)
        if rc == _native.WSL_E_LAUNCH:
            _retire((dev.index, stream, "lora"))
        _native.check(rc, "wsl_lora_linear_bcast_fwd")
    return y.reshape(*lead, G * N)


@lora_linear_bcast_op.register_fake
def _lora_linear_bcast_fake(x, w, w_scale, a, b, scale, g, n_groups):
    N = b.shape[0] // int(n_groups) if b is not None else w.shape[0]
    return x.new_empty((*x.shape[:-1], int(n_groups) * N), dtype=torch.bfloat16)


def _lora_linear_bcast_setup(ctx, inputs, output):
    x, w, w_scale, a, b, scale, g, n_groups = inputs
    ctx.save_for_backward(x, w, w_scale, a, b)
    ctx.scale = scale
    ctx.g = int(g)
    ctx.G = int(n_groups)


def _lora_linear_bcast_backward(ctx, gy):
    """Backward of ``wsl::lora_linear_bcast``. Every output column c of group j reads base row
    base(c) = (c / (hpg D)) D + c % D, so W's gradient gathers them: with gy_b [M, base_n]
    the sum of gy over the groups and the heads of each template,

        dx = gy_b . W + scale * (gy . Bd) . a       two launches of the fused kernel
        dW = gy_b^T . x
        da = scale * (gy . Bd)^T . x,   db_j = scale * gy_j^T . (x . a_j^T)

    (Bd: b block-diagonal over the groups). The reference differentiates broadcast_add's
    expand and the separate projections (torchtitan/models/llama3/model/model.py:111-145,
    381-398); these are the same sums."""
    x, w, w_scale, a, b, scale = *ctx.saved_tensors, ctx.scale
    s = float(scale)
    G, g = ctx.G, ctx.g
    need_x, need_w, _, need_a, need_b, _, _, _ = ctx.needs_input_grad
    K = x.shape[-1]
    base_n = w.shape[0]
    gy2 = _row_major(gy.reshape(-1, gy.shape[-1]).to(torch.bfloat16), "grad_y")
    M = gy2.shape[0]
    N = gy2.shape[1] // G
    D = base_n // g
    hpg = N // base_n
    x2 = x.reshape(-1, K)
    gyb = gy2.float().view(M, G, g, hpg, D).sum(dim=(1, 3)).reshape(M, base_n).to(torch.bfloat16)
    has_lora = a is not None and b is not None and b.shape[1] > 0
    r = b.shape[1] if has_lora else 0
    bd = _block_diag_rows(b, [N] * G, r) if has_lora else None
    dx = dw = da = db = None
    if need_x:
        dx = _input_grad(gyb, w, w_scale, None, None, 0.0)
        if has_lora and G * r <= _native.WSL_MAX_RANK:
            dx = dx + lora_linear_op(gy2, None, None, bd.t().contiguous(), a.t().contiguous(), s)
        elif has_lora:  # G*r above the kernels' rank limit: one delta launch per group, summed
            for j in range(G):
                dx = dx + lora_linear_op(gy2[:, j * N:(j + 1) * N], None, None, b[j * N:(j + 1) * N].t().contiguous(),
                                         a[j * r:(j + 1) * r].t().contiguous(), s)
        dx = dx.reshape(x.shape)
    dw, _, _ = weight_grads(x2, gyb, None, None, s, need_w and w.dtype == torch.bfloat16, False, False)
    if has_lora and (need_a or need_b):
        if G * r <= _native.WSL_MAX_RANK:
            _, da, full = weight_grads(x2, gy2, a, bd, s, False, need_a, need_b)
            if full is not None:
                db = torch.empty_like(b)
                for j in range(G):
                    db[j * N:(j + 1) * N] = full[j * N:(j + 1) * N, j * r:(j + 1) * r]
        else:  # G*r above the rank limit: per group
            da = torch.empty_like(a) if need_a else None
            db = torch.empty_like(b) if need_b else None
            for j in range(G):
                _, daj, dbj = weight_grads(x2, gy2[:, j * N:(j + 1) * N], a[j * r:(j + 1) * r],
                                           b[j * N:(j + 1) * N], s, False, need_a, need_b)
                if need_a:
                    da[j * r:(j + 1) * r] = daj
                if need_b:
                    db[j * N:(j + 1) * N] = dbj
    return dx, dw, None, da, db, None, None, None


lora_linear_bcast_op.register_autograd(_lora_linear_bcast_backward, setup_context=_lora_linear_bcast_setup)


def _block_diag_rows(b: torch.Tensor, group_n, r: int) -> torch.Tensor:
    """[N, G*r] with group g's rows of b in column block g and zeros elsewhere."""
    out = b.new_zeros(b.shape[0], len(group_n) * r)
    n0 = 0
    for g, n in enumerate(group_n):
        out[n0:n0 + n, g * r:(g + 1) * r] = b[n0:n0 + n]
        n0 += n
    return out


def _lora_linear_grouped_setup(ctx, inputs, output):
    x, w, w_scale, a, b, scale, group_n = inputs
    ctx.save_for_backward(x, w, w_scale, a, b)
    ctx.scale = scale
    ctx.group_n = [int(n) for n in group_n]


def _lora_linear_grouped_backward(ctx, gy):
    """Backward of ``wsl::lora_linear_grouped``: the per-group backward of
    ``wsl::lora_linear`` summed over the groups for dx. With Bd the block-diagonal
    [N, G*r] form of b (group g's rows in column block g):

        dx = gy . W + scale * (gy . Bd) . a      one launch of the fused kernel, rank G*r
        dW = gy^T . x                            one GEMM over all groups
        da = scale * (gy . Bd)^T . x             one GEMM over all groups
        db_g = scale * gy_g^T . (x . a_g^T)      the diagonal blocks of one [N, G*r] GEMM

    The reference differentiates each projection separately (torch autograd over
    torchtitan/models/llama3/model/model.py:189-192,392-398) and sums the three dx of
    q, k and v where x fans out; this is the same sum.
    """
    x, w, w_scale, a, b = ctx.saved_tensors
    s = float(ctx.scale)
    gn = ctx.group_n
    need_x, need_w, _, need_a, need_b, _, _ = ctx.needs_input_grad
    K = x.shape[-1]
    gy2 = _row_major(gy.reshape(-1, gy.shape[-1]).to(torch.bfloat16), "grad_y")
    x2 = x.reshape(-1, K)
    has_lora = a is not None and b is not None and b.shape[1] > 0
    r = b.shape[1] if has_lora else 0
    bd = _block_diag_rows(b, gn, r) if has_lora else None
    dx = dw = da = db = None
    if need_x:
        if has_lora and len(gn) * r <= _native.WSL_MAX_RANK:
            dx = _input_grad(gy2, w, w_scale, a, bd, s)
        elif has_lora:  # G*r above the kernels' rank limit: the base term, then one delta per group
            dx = _input_grad(gy2, w, w_scale, None, None, s)
            n0 = 0
            for g, n in enumerate(gn):
                dx = dx + lora_linear_op(gy2[:, n0:n0 + n], None, None, b[n0:n0 + n].t().contiguous(),
                                         a[g * r:(g + 1) * r].t().contiguous(), s)
                n0 += n
        else:
            dx = _input_grad(gy2, w, w_scale, None, None, s)
        dx = dx.reshape(x.shape)
    # one weight-gradient call over all groups (x and gy read once): da from Bd, db as the
    # diagonal blocks of the [N, G*r] product (the off-diagonal blocks are a few GFLOP,
    # cheaper than G strided skinny products)
    lora_ab = has_lora and len(gn) * r <= _native.WSL_MAX_RANK
    dw, da, full = weight_grads(x2, gy2, a, bd, s, need_w and w.dtype == torch.bfloat16,
                                lora_ab and need_a, lora_ab and need_b)
    if has_lora and not lora_ab and (need_a or need_b):  # G*r above the rank limit: per group
        da = torch.empty_like(a) if need_a else None
        db = torch.empty_like(b) if need_b else None
        n0 = 0
        for g, n in enumerate(gn):
            _, dag, dbg = weight_grads(x2, gy2[:, n0:n0 + n], a[g * r:(g + 1) * r], b[n0:n0 + n], s, False,
                                       need_a, need_b)
            if need_a:
                da[g * r:(g + 1) * r] = dag
            if need_b:
                db[n0:n0 + n] = dbg
            n0 += n
    elif full is not None:
        db = torch.empty_like(b)
        n0 = 0
        for g, n in enumerate(gn):
            db[n0:n0 + n] = full[n0:n0 + n, g * r:(g + 1) * r]
            n0 += n
    return dx, dw, None, da, db, None, None


lora_linear_grouped_op.register_autograd(_lora_linear_grouped_backward, setup_context=_lora_linear_grouped_setup)


def lora_linear_grouped(x: torch.Tensor, ws, as_=None, bs=None, scale: float = 2.0) -> list:
    """Several LoRA linears over the same x in one call: ``ws`` lists the base weights
    [N_g, K], ``as_`` / ``bs`` the LoRA factors [r, K] / [N_g, r] (all of rank r), one scale.
    Returns the per-group outputs as views of one [..., sum N_g] tensor. The operands are
    stacked with torch.cat (differentiable), so callers that reuse them should stack once
    and call ``lora_linear_grouped_op`` directly."""
    group_n = [int(w_.shape[0]) for w_ in ws]
    w = torch.cat(list(ws), 0) if len(ws) > 1 else ws[0]
    a = b = None
    if as_ is not None:
        a = torch.cat(list(as_), 0)
        b = torch.cat(list(bs), 0)
    y = lora_linear_grouped_op(x, w, None, a, b, float(scale), group_n)
    return list(torch.split(y, group_n, dim=-1))


@torch.library.custom_op("wsl::factorized_embedding", mutates_args=(), device_types="cuda")
def factorized_embedding_op(ids: torch.Tensor, emb: torch.Tensor, proj: torch.Tensor) -> torch.Tensor:
    """out[..., :] = emb[ids[...], :] . proj^T   (emb [V,k], proj [H,k], bf16)."""
    dev = _check_device(ids, emb, proj)
    if ids.dtype != torch.int64:
        raise TypeError(f"ids must be int64, got {ids.dtype}")
    if emb.dtype != torch.bfloat16 or proj.dtype != torch.bfloat16:
        raise TypeError("emb and proj must be bfloat16")
    emb = _row_major(emb, "emb")
    proj = _row_major(proj, "proj")
    V, k = emb.shape
    H = proj.shape[0]
    if proj.shape[1] != k:
        raise ValueError(f"proj {tuple(proj.shape)} does not match emb rank {k}")
    flat = ids.reshape(-1).contiguous()
    out = torch.empty((flat.numel(), H), dtype=torch.bfloat16, device=dev)
    if flat.numel() > 0:
        stream = torch.cuda.current_stream(dev).cuda_stream
        with torch.cuda.device(dev):
            rc = _native.lib().wsl_factorized_embedding_fwd(
                flat.data_ptr(), flat.numel(), emb.data_ptr(), emb.stride(0), V, k,
                proj.data_ptr(), proj.stride(0), H, out.data_ptr(), out.stride(0), stream)
        _native.check(rc, "wsl_factorized_embedding_fwd")
    return out.reshape(*ids.shape, H)


@factorized_embedding_op.register_fake
def _factorized_embedding_fake(ids, emb, proj):
    return emb.new_empty((*ids.shape, proj.shape[0]), dtype=torch.bfloat16)


# ------------------------------------------------------------------------------------------
# Autocast rules. The reference trains under torch.autocast(device, dtype=bf16) on the
# single-device / DDP path (torchtitan/distributed/utils.py:219-239), where nn.Linear casts
# its floating inputs to the autocast dtype. The wsl ops compute in bf16 only, so inside an
# autocast region their activation and weight operands are cast to bf16, whatever the region's
# dtype; an fp8 base weight keeps its storage type and its fp32 per-channel scale stays fp32.
# The rules sit on the ops themselves (dispatch key AutocastCUDA, which ROCm's autocast uses),
# so torch.ops.wsl.* called directly, a compiled graph or the Python wrappers all get them.
# ------------------------------------------------------------------------------------------
def autocast_operand(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """bf16 for a floating operand of another type; fp8, bf16 and non-floating tensors and
    None pass unchanged."""
    if t is None or not t.is_floating_point() or t.dtype in (torch.bfloat16, _FP8):
        return t
    return t.to(torch.bfloat16)


_AUTOCAST_KEYS = (torch._C.DispatchKeySet(torch._C.DispatchKey.AutocastCUDA)
                  | torch._C.DispatchKeySet(torch._C.DispatchKey.AutocastCPU))
_autocast_lib = torch.library.Library("wsl", "IMPL")


def _autocast_lora_linear(_ks, x, w, w_scale, a, b, scale):
    with torch._C._ExcludeDispatchKeyGuard(_AUTOCAST_KEYS):
        return lora_linear_op(autocast_operand(x), autocast_operand(w), w_scale, autocast_operand(a),
                              autocast_operand(b), scale)


def _autocast_lora_linear_grouped(_ks, x, w, w_scale, a, b, scale, group_n):
    with torch._C._ExcludeDispatchKeyGuard(_AUTOCAST_KEYS):
        return lora_linear_grouped_op(autocast_operand(x), autocast_operand(w), w_scale, autocast_operand(a),
                                      autocast_operand(b), scale, group_n)


def _autocast_factorized_embedding(_ks, ids, emb, proj):
    with torch._C._ExcludeDispatchKeyGuard(_AUTOCAST_KEYS):
        return factorized_embedding_op(ids, autocast_operand(emb), autocast_operand(proj))


def _autocast_lora_linear_bcast(_ks, x, w, w_scale, a, b, scale, g, n_groups):
    with torch._C._ExcludeDispatchKeyGuard(_AUTOCAST_KEYS):
        return lora_linear_bcast_op(autocast_operand(x), autocast_operand(w), w_scale, autocast_operand(a),
                                    autocast_operand(b), scale, g, n_groups)


_autocast_lib.impl("lora_linear", _autocast_lora_linear, "AutocastCUDA", with_keyset=True)
_autocast_lib.impl("lora_linear_bcast", _autocast_lora_linear_bcast, "AutocastCUDA", with_keyset=True)
_autocast_lib.impl("lora_linear_grouped", _autocast_lora_linear_grouped, "AutocastCUDA", with_keyset=True)
_autocast_lib.impl("factorized_embedding", _autocast_factorized_embedding, "AutocastCUDA", with_keyset=True)


def lora_linear(x: torch.Tensor, w: Optional[torch.Tensor], a: Optional[torch.Tensor] = None,
                b: Optional[torch.Tensor] = None, scale: float = 2.0,
                w_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused LoRA linear ``x . w^T + scale * (x . a^T) . b^T`` (``torch.ops.wsl.lora_linear``;
    under autocast its operands are cast by the op's autocast rule above)."""
    return lora_linear_op(x, w, w_scale, a, b, float(scale))


# When set (or with WSL_CHECK_EMBEDDING_IDS=1 in the environment), factorized_embedding raises
# IndexError for an id outside [0, vocab), as the reference's nn.Embedding does. Off by default:
# the check reads the ids' range back to the host (a synchronisation, and impossible inside a
# graph capture). Unchecked, the kernel turns an out-of-range id into a zero row and never
# reads outside the table.
CHECK_EMBEDDING_IDS = os.environ.get("WSL_CHECK_EMBEDDING_IDS", "") not in ("", "0")


def check_embedding_ids(ids: torch.Tensor, vocab: int) -> None:
    """Raises IndexError unless every id is in [0, vocab) (one host read of the ids' range)."""
    if ids.numel() == 0:
        return
    lo, hi = int(ids.min()), int(ids.max())
    if lo < 0 or hi >= vocab:
        raise IndexError(f"token id out of range: ids span [{lo}, {hi}] but the vocabulary has {vocab} rows")


def factorized_embedding(ids: torch.Tensor, emb: torch.Tensor, proj: torch.Tensor) -> torch.Tensor:
    if CHECK_EMBEDDING_IDS and not torch.cuda.is_current_stream_capturing():
        check_embedding_ids(ids, emb.shape[0])
    return factorized_embedding_op(ids, emb, proj)


# ------------------------------------------------------------------------------------------
# Decode-step ops of the weight-shared Qwen3 harness (include/wsl_decode.h). GPU only.
# ------------------------------------------------------------------------------------------
def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _bf16_2d(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    t = t.reshape(-1, t.shape[-1])
    if t.stride(-1) != 1 or t.stride(0) % 8 != 0 or t.data_ptr() % 16 != 0:
        t = t.contiguous()
    return t


def _check_rope(rope: torch.Tensor, cache_len: int, head_dim: int) -> None:
    """The RoPE table must cover every cache position: [>= cache_len, 2 * head_dim] (cos
    then sin). The kernels index row `pos` of it for any pos < cache_len; a position at or
    past cache_len gives NaN outputs and writes nothing."""
    if rope.dim() != 2 or rope.shape[1] != 2 * head_dim or rope.shape[0] < cache_len:
        raise ValueError(f"rope must be [>= {cache_len}, {2 * head_dim}] (cos | sin) to cover the cache; "
                         f"got {tuple(rope.shape)}")


def _rmsnorm_launch(x, weight, eps, residual):
    dev = _check_device(x, weight, residual)
    dim = x.shape[-1]
    x2 = _bf16_2d(x, "x")
    r2 = _bf16_2d(residual, "residual") if residual is not None else None
    w = weight.to(torch.bfloat16).contiguous()
    out = torch.empty((x2.shape[0], dim), dtype=torch.bfloat16, device=dev)
    h = torch.empty_like(out) if residual is not None else None
    with torch.cuda.device(dev):
        rc = _native.lib().wsl_rmsnorm_fwd(
            x2.data_ptr(), x2.stride(0), _dev_ptr(r2), r2.stride(0) if r2 is not None else 0,
            w.data_ptr(), float(eps), out.data_ptr(), out.stride(0),
            _dev_ptr(h), h.stride(0) if h is not None else 0, x2.shape[0], dim, _stream(dev))
    _native.check(rc, "wsl_rmsnorm_fwd", decode=True)
    return out.view(x.shape), (h.view(x.shape) if h is not None else None)


@torch.library.custom_op("wsl::rmsnorm", mutates_args=(), device_types="cuda")
def rmsnorm_op(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm(x) * weight over the last dimension (bf16 in/out, fp32 arithmetic)."""
    return _rmsnorm_launch(x, weight, eps, None)[0]


@rmsnorm_op.register_fake
def _rmsnorm_fake(x, weight, eps):
    return x.new_empty(x.shape, dtype=torch.bfloat16)


@torch.library.custom_op("wsl::add_rmsnorm", mutates_args=(), device_types="cuda")
def add_rmsnorm_op(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                   eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(RMSNorm(h) * weight, h) with h = bf16(x + residual): the residual add of a block and
    the next norm in one launch."""
    return _rmsnorm_launch(x, weight, eps, residual)


@add_rmsnorm_op.register_fake
def _add_rmsnorm_fake(x, residual, weight, eps):
    return x.new_empty(x.shape, dtype=torch.bfloat16), x.new_empty(x.shape, dtype=torch.bfloat16)


@torch.library.custom_op("wsl::qk_norm_rope", mutates_args=("k_cache", "v_cache"), device_types="cuda")
def qk_norm_rope_op(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, eps: float,
                    rope: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    n_heads: int, n_kv_heads: int) -> torch.Tensor:
    """q [b, n_heads, hd] after q-norm + RoPE; k (normed, rotated) and v written into the
    caches [b, n_kv_heads, L, hd] at position `pos`."""
    dev = _check_device(qkv, q_norm_w, k_norm_w, rope, pos, k_cache, v_cache)
    b, _, L, hd = k_cache.shape
    q2 = _bf16_2d(qkv, "qkv")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache and v_cache must be contiguous [b, n_kv_heads, L, head_dim]")
    _check_rope(rope, L, hd)
    qw = q_norm_w.to(torch.bfloat16).contiguous()
    kw = k_norm_w.to(torch.bfloat16).contiguous()
    rope = rope.float().contiguous()
    pos = pos.to(torch.int64).contiguous()
    q = torch.empty((b, n_heads, hd), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        rc = _native.lib().wsl_qk_norm_rope_fwd(
            q2.data_ptr(), q2.stride(0), b, n_heads, n_kv_heads, hd, qw.data_ptr(), kw.data_ptr(), float(eps),
            rope.data_ptr(), pos.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), L, _stream(dev))
    _native.check(rc, "wsl_qk_norm_rope_fwd", decode=True)
    return q


@qk_norm_rope_op.register_fake
def _qk_norm_rope_fake(qkv, q_norm_w, k_norm_w, eps, rope, pos, k_cache, v_cache, n_heads, n_kv_heads):
    return qkv.new_empty((k_cache.shape[0], n_heads, k_cache.shape[3]), dtype=torch.bfloat16)


@torch.library.custom_op("wsl::decode_attention", mutates_args=(), device_types="cuda")
def decode_attention_op(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                        scale: float) -> torch.Tensor:
    """softmax(q . K^T * scale) . V over cache positions 0..pos; q [b, n_heads, hd],
    caches [b, n_kv_heads, L, hd] -> [b, n_heads * hd]."""
    dev = _check_device(q, k_cache, v_cache, pos)
    b, nh, hd = q.shape
    nkv, L = k_cache.shape[1], k_cache.shape[2]
    q = q.contiguous()
    pos = pos.to(torch.int64).contiguous()
    out = torch.empty((b, nh * hd), dtype=torch.bfloat16, device=dev)
    nbytes = _native.lib().wsl_decode_attention_workspace_bytes(b, nh, nkv, hd, L)
    part = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)  # partial softmax records
    with torch.cuda.device(dev):
        rc = _native.lib().wsl_decode_attention_fwd(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), b, nh, nkv, hd, L, pos.data_ptr(),
            float(scale), out.data_ptr(), part.data_ptr(), part.numel(), _stream(dev))
    _native.check(rc, "wsl_decode_attention_fwd", decode=True)
    return out


@decode_attention_op.register_fake
def _decode_attention_fake(q, k_cache, v_cache, pos, scale):
    return q.new_empty((q.shape[0], q.shape[1] * q.shape[2]), dtype=torch.bfloat16)


@torch.library.custom_op("wsl::swiglu", mutates_args=(), device_types="cuda")
def swiglu_op(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(g) * u for gate_up = [g | u] along the last dimension."""
    dev = _check_device(gate_up)
    ffn = gate_up.shape[-1] // 2
    g2 = _bf16_2d(gate_up, "gate_up")
    out = torch.empty((g2.shape[0], ffn), dtype=torch.bfloat16, device=dev)
    with torch.cuda.device(dev):
        rc = _native.lib().wsl_swiglu_fwd(g2.data_ptr(), g2.stride(0), g2.shape[0], ffn, out.data_ptr(),
                                          out.stride(0), _stream(dev))
    _native.check(rc, "wsl_swiglu_fwd", decode=True)
    return out.view(*gate_up.shape[:-1], ffn)


@swiglu_op.register_fake
def _swiglu_fake(gate_up):
    return gate_up.new_empty((*gate_up.shape[:-1], gate_up.shape[-1] // 2), dtype=torch.bfloat16)


@torch.library.custom_op("wsl::argmax_rows", mutates_args=(), device_types="cuda")
def argmax_rows_op(x: torch.Tensor) -> torch.Tensor:
    """int64 index of the largest element of each row (first on ties, NaN largest)."""
    dev = _check_device(x)
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16, got {x.dtype}")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    out = torch.empty(x2.shape[0], dtype=torch.int64, device=dev)
    lib = _native.lib()
    stream = _stream(dev)
    ws = workspace(dev, stream, lib.wsl_argmax_rows_workspace_bytes(x2.shape[0], x2.shape[1]), kind="argmax")
    with torch.cuda.device(dev):
        rc = lib.wsl_argmax_rows_fwd(x2.data_ptr(), x2.stride(0), x2.shape[0], x2.shape[1], out.data_ptr(),
                                     ws.data_ptr(), ws.numel(), stream)
    if rc == _native.WSL_E_LAUNCH:
        _retire((dev.index, stream, "argmax"))  # a failed launch may leave keys set
    _native.check(rc, "wsl_argmax_rows_fwd", decode=True)
    return out.view(x.shape[:-1])


@argmax_rows_op.register_fake
def _argmax_rows_fake(x):
    return x.new_empty(x.shape[:-1], dtype=torch.int64)


@torch.library.custom_op("wsl::decode_attention_step", mutates_args=("k_cache", "v_cache"), device_types="cuda")
def decode_attention_step_op(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, eps: float,
                             rope: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                             n_heads: int, n_kv_heads: int, scale: float) -> torch.Tensor:
    """q/k norm + RoPE + cache write + attention of one decode step in one launch:
    qkv [b, (n_heads + 2 n_kv_heads) hd] -> [b, n_heads * hd]; k, v written into the
    caches [b, n_kv_heads, L, hd] at `pos`."""
    dev = _check_device(qkv, q_norm_w, k_norm_w, rope, pos, k_cache, v_cache)
    b, _, L, hd = k_cache.shape
    q2 = _bf16_2d(qkv, "qkv")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache and v_cache must be contiguous [b, n_kv_heads, L, head_dim]")
    _check_rope(rope, L, hd)
    qw = q_norm_w.to(torch.bfloat16).contiguous()
    kw = k_norm_w.to(torch.bfloat16).contiguous()
    rope = rope.float().contiguous()
    pos = pos.to(torch.int64).contiguous()
    out = torch.empty((b, n_heads * hd), dtype=torch.bfloat16, device=dev)
    lib = _native.lib()
    stream = _stream(dev)
    ws = workspace(dev, stream, lib.wsl_decode_attention_step_workspace_bytes(b, n_heads, n_kv_heads, hd, L),
                   kind="attention")
    with torch.cuda.device(dev):
        rc = lib.wsl_decode_attention_step_fwd(
            q2.data_ptr(), q2.stride(0), b, n_heads, n_kv_heads, hd, qw.data_ptr(), kw.data_ptr(), float(eps),
            rope.data_ptr(), pos.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), L, float(scale),
            out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    if rc == _native.WSL_E_LAUNCH:
        _retire((dev.index, stream, "attention"))
    _native.check(rc, "wsl_decode_attention_step_fwd", decode=True)
    return out


@decode_attention_step_op.register_fake
def _decode_attention_step_fake(qkv, q_norm_w, k_norm_w, eps, rope, pos, k_cache, v_cache, n_heads, n_kv_heads,
                                scale):
    return qkv.new_empty((k_cache.shape[0], n_heads * k_cache.shape[3]), dtype=torch.bfloat16)


def tied_head_argmax_supported(M: int, N: int, K: int) -> bool:
    """Whether wsl::tied_head_argmax covers these sizes (16-byte aligned operands)."""
    return bool(_native.lib().wsl_tied_head_argmax_supported(M, N, K))


@torch.library.custom_op("wsl::tied_head_argmax", mutates_args=(), device_types="cuda")
def tied_head_argmax_op(z: torch.Tensor, emb: torch.Tensor) -> torch.Tensor:
    """Greedy token of the tied head: argmax over n of bf16(z[m] . emb[n]) for every row of z
    [M, k] (M <= 64), without writing the [M, vocab] logits (include/wsl_decode.h)."""
    dev = _check_device(z, emb)
    z2 = _bf16_2d(z, "z")
    if emb.dtype != torch.bfloat16:
        raise TypeError(f"emb must be bfloat16, got {emb.dtype}")
    emb = _row_major(emb, "emb")
    M, K = z2.shape
    V = emb.shape[0]
    if emb.shape[1] != K:
        raise ValueError(f"emb {tuple(emb.shape)} does not match z's width {K}")
    out = torch.empty(M, dtype=torch.int64, device=dev)
    lib = _native.lib()
    stream = _stream(dev)
    ws = workspace(dev, stream, lib.wsl_tied_head_argmax_workspace_bytes(M), kind="head_argmax")
    with torch.cuda.device(dev):
        rc = lib.wsl_tied_head_argmax_fwd(z2.data_ptr(), z2.stride(0), emb.data_ptr(), emb.stride(0), V, K, M,
                                          out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    if rc == _native.WSL_E_LAUNCH:
        _retire((dev.index, stream, "head_argmax"))  # a failed launch may leave keys set
    _native.check(rc, "wsl_tied_head_argmax_fwd")
    return out


@tied_head_argmax_op.register_fake
def _tied_head_argmax_fake(z, emb):
    return z.new_empty((z.reshape(-1, z.shape[-1]).shape[0],), dtype=torch.int64)


def lora_linear_fused_supported(M: int, N: int, K: int, r: int, fuse: int) -> bool:
    """Whether wsl::lora_linear_fused covers these sizes (16-byte aligned operands)."""
    return bool(_native.lib().wsl_lora_linear_fused_supported(M, N, K, r, fuse))


@torch.library.custom_op("wsl::lora_linear_fused", mutates_args=(), device_types="cuda")
def lora_linear_fused_op(x: torch.Tensor, norm_w: Optional[torch.Tensor], eps: float, w: torch.Tensor,
                         a: Optional[torch.Tensor], b: Optional[torch.Tensor], scale: float,
                         residual: Optional[torch.Tensor], fuse: int) -> torch.Tensor:
    """The decode-step fused LoRA linear (include/wsl_decode.h): bf16 W, 1 <= M <= 64, with
    an RMSNorm prologue on x (norm_w), a SwiGLU epilogue over interleaved gate/up rows
    (y [M, N/2]) and/or a residual-add epilogue (y = bf16(residual + bf16(y)))."""
    dev = _check_device(x, norm_w, w, a, b, residual)
    x2 = _bf16_2d(x, "x")
    M, K = x2.shape
    N = w.shape[0]
    nw = norm_w.to(torch.bfloat16).contiguous() if norm_w is not None else None
    res = _bf16_2d(residual, "residual") if residual is not None else None
    w = _row_major(w, "w")
    r = 0
    if a is not None:
        a, b = _row_major(a, "a"), _row_major(b, "b")
        r = a.shape[0]
    ny = N // 2 if fuse & _native.WSL_FUSE_SWIGLU else N
    y = torch.empty((M, ny), dtype=torch.bfloat16, device=dev)
    stream = _stream(dev)
    ws = workspace(dev, stream, _native.workspace_bytes(M, N, K, r, _native.WSL_DTYPE_BF16))
    with torch.cuda.device(dev):
        rc = _native.lib().wsl_lora_linear_fused_fwd(
            x2.data_ptr(), x2.stride(0), _dev_ptr(nw), float(eps), w.data_ptr(), w.stride(0),
            _dev_ptr(a), a.stride(0) if a is not None else 0, _dev_ptr(b), b.stride(0) if b is not None else 0,
            float(scale), _dev_ptr(res), res.stride(0) if res is not None else 0, y.data_ptr(), y.stride(0),
            M, N, K, r, int(fuse), ws.data_ptr(), ws.numel(), stream)
    if rc == _native.WSL_E_LAUNCH:
        _retire((dev.index, stream, "lora"))
    _native.check(rc, "wsl_lora_linear_fused_fwd")
    return y


@lora_linear_fused_op.register_fake
def _lora_linear_fused_fake(x, norm_w, eps, w, a, b, scale, residual, fuse):
    M = x.reshape(-1, x.shape[-1]).shape[0]
    ny = w.shape[0] // 2 if fuse & 2 else w.shape[0]
    return x.new_empty((M, ny), dtype=torch.bfloat16)



# ------------------------------------------------------------------------------------------
# Chains: several decode-shaped LoRA linears in one persistent launch
# (wsl_lora_linear_chain_fwd, include/wsl_decode.h). Inference only (no autograd): the decode
# step of the weight-shared Qwen3 harness runs o, gate|up, down and the next layer's q|k|v as
# one chain between two attention steps.
# ------------------------------------------------------------------------------------------
class ChainStage:
    """One stage of a chain: ``y = fused(x; w, a, b, scale)`` as wsl::lora_linear_fused with
    ``fuse`` (WSL_FUSE_* flags; 0 = the plain or grouped LoRA linear over ``group_n``).
    ``y`` is written in place (allocate it before the call); ``after_previous`` marks a stage
    whose x or residual is an earlier stage's y."""

    def __init__(self, x, w, a, b, scale, y, fuse=0, norm_w=None, eps=0.0, residual=None, group_n=None,
                 after_previous=False):
        self.x, self.w, self.a, self.b, self.scale, self.y = x, w, a, b, float(scale), y
        self.fuse, self.norm_w, self.eps, self.residual = int(fuse), norm_w, float(eps), residual
        self.group_n = list(group_n) if group_n else [w.shape[0]]
        self.after_previous = bool(after_previous)

    def _c(self, M: int) -> "_native.ChainStage":
        c = _native.ChainStage()
        x2 = self.x.reshape(M, -1)
        c.x, c.ldx = x2.data_ptr(), x2.stride(0)
        c.norm_w = _dev_ptr(self.norm_w)
        c.eps = self.eps
        c.w, c.ldw = self.w.data_ptr(), self.w.stride(0)
        r = 0
        if self.a is not None:
            r = self.b.shape[1]
            c.a, c.lda, c.b, c.ldb = self.a.data_ptr(), self.a.stride(0), self.b.data_ptr(), self.b.stride(0)
        c.scale = self.scale
        if self.residual is not None:
            res2 = self.residual.reshape(M, -1)
            c.residual, c.ldr = res2.data_ptr(), res2.stride(0)
        y2 = self.y.reshape(M, -1)
        c.y, c.ldy = y2.data_ptr(), y2.stride(0)
        c.N, c.K, c.r = self.w.shape[0], self.w.shape[1], r
        c.fuse = self.fuse
        c.n_groups = len(self.group_n)
        for i, n in enumerate(self.group_n):
            c.group_n[i] = int(n)
        c.after_previous = 1 if self.after_previous else 0
        return c


def _chain_array(stages, M):
    arr = (_native.ChainStage * len(stages))(*[st._c(M) for st in stages])
    return arr


def chain_supported(stages, M: int) -> bool:
    """Whether one chain launch takes these stages at M tokens (wsl_lora_linear_chain_supported)."""
    if not 1 <= len(stages) <= _native.WSL_CHAIN_MAX_STAGES:
        return False
    return bool(_native.lib().wsl_lora_linear_chain_supported(M, len(stages), _chain_array(stages, M)))


def lora_linear_chain(stages, M: int) -> None:
    """Runs the stages as one persistent launch on the current stream (each stage's y is
    written; results equal the per-stage fused or grouped calls bit for bit). Raises if the
    chain is not supported (chain_supported)."""
    dev = _check_device(*[st.x for st in stages], *[st.y for st in stages])
    arr = _chain_array(stages, M)
    L = _native.lib()
    need = ctypes.c_size_t(0)
    _native.check(L.wsl_lora_linear_chain_workspace_bytes(M, len(stages), arr, ctypes.byref(need)),
                  "wsl_lora_linear_chain_workspace_bytes")
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = workspace(dev, stream, int(need.value), kind="chain")
    with torch.cuda.device(dev):
        rc = L.wsl_lora_linear_chain_fwd(M, len(stages), arr, ws.data_ptr(), ws.numel(), stream)
    if rc == _native.WSL_E_LAUNCH:
        _retire((dev.index, stream, "chain"))
    _native.check(rc, "wsl_lora_linear_chain_fwd")


def chain_status(dev: Optional[torch.device] = None) -> bool:
    """True when a chain launch on the current stream's workspace gave up a stage wait since
    the last call (the sticky failure word, then cleared); synchronizes the stream."""
    dev = dev or torch.device("cuda", torch.cuda.current_device())
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = _workspaces.get((dev.index, stream, "chain"))
    if ws is None:
        return False
    failed = ctypes.c_int32(0)
    with torch.cuda.device(dev):
        _native.check(_native.lib().wsl_lora_linear_chain_status(ws.data_ptr(), stream, ctypes.byref(failed)),
                      "wsl_lora_linear_chain_status")
    return bool(failed.value)
