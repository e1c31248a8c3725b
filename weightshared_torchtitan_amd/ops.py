"""torch custom ops over libwsl: ``wsl::lora_linear`` and ``wsl::factorized_embedding``.

Both ops have a HIP (device type "cuda" on ROCm) implementation only. Called with CPU
tensors they raise; there is no CPU or eager-PyTorch fallback. Each op has a fake
(meta) implementation so models can be built on the meta device and traced by
torch.compile, matching how the reference builds its model
(torchtitan/train.py:156-157) and compiles blocks
(torchtitan/models/llama3/infra/parallelize.py:348-357).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _native

_FP8 = torch.float8_e4m3fn


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


def workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """The persistent scratch buffer of (device, stream).

    libwsl requires its workspace to be zero-filled before first use (the leading
    counters of the decode kernels) and keeps those counters valid across calls, so one
    zero-filled buffer per stream is reused by every call on that stream; it only grows
    (a grown buffer starts zeroed again).
    """
    key = (dev.index, stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
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
            w_dtype = _native.WSL_DTYPE_FP8_E4M3
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
        if rc != _native.WSL_OK:
            _workspaces.pop((dev.index, stream), None)  # a failed launch may leave counters mid-update
        _native.check(rc, "wsl_lora_linear_fwd")
    return y.reshape(*lead, N)


@lora_linear_op.register_fake
def _lora_linear_fake(x, w, w_scale, a, b, scale):
    N = _out_features(w, b)
    return x.new_empty((*x.shape[:-1], N), dtype=torch.bfloat16)


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


def lora_linear(x: torch.Tensor, w: Optional[torch.Tensor], a: Optional[torch.Tensor] = None,
                b: Optional[torch.Tensor] = None, scale: float = 2.0,
                w_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Fused LoRA linear ``x . w^T + scale * (x . a^T) . b^T``.

    Under ``torch.autocast("cuda", dtype=torch.bfloat16)`` floating inputs are cast to
    bf16 (an fp8 ``w`` and its fp32 ``w_scale`` are left as they are), mirroring the
    reference's AMP path (torchtitan/distributed/utils.py:219-239).
    """
    if torch.is_autocast_enabled("cuda"):
        def cast(t):
            return t.to(torch.bfloat16) if (t is not None and t.is_floating_point()
                                             and t.dtype not in (torch.bfloat16, _FP8)) else t
        x, a, b = cast(x), cast(a), cast(b)
        if w is not None and w.dtype != _FP8:
            w = cast(w)
    return lora_linear_op(x, w, w_scale, a, b, float(scale))


def factorized_embedding(ids: torch.Tensor, emb: torch.Tensor, proj: torch.Tensor) -> torch.Tensor:
    return factorized_embedding_op(ids, emb, proj)
