"""Module interface of the fused LoRA linear (drop-in for the reference's LoRA path).

* ``LoRAModule`` keeps the reference's constructor, attributes and state-dict names
  (``w_a.weight [r, in]``, ``w_b.weight [out, r]``, ``alpha = 2 * rank``) and its
  forward still returns the delta alone, so the reference's composition
  ``broadcast_add(base(x), lora(x), g=...)`` keeps working
  (torchtitan/models/llama3/model/model.py:148-192, 376-398).
* ``LoRALinear`` is the fused form of that composition for the ``g = 1`` case: one
  kernel computes ``base(x) + lora(x)``.
* ``broadcast_add`` restates the reference helper (model.py:111-145) for the
  head-sharing compositions.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
from torch import nn

from . import ops

FP8_MAX = 448.0  # largest finite float8_e4m3fn


def broadcast_add(base: torch.Tensor, delta: torch.Tensor, *, dim: int = -1, g: int = 1) -> torch.Tensor:
    """``broadcast(base) + delta`` along ``dim``: base holds g templates of width D that
    are shared by the H/g heads of each group of ``delta`` (H*D wide).

    Same contract as torchtitan/models/llama3/model/model.py:111-145, including the
    assertion that the delta width is a multiple of the base width.
    """
    if dim < 0:
        dim += base.dim()
    big = delta.shape[dim]
    small = base.shape[dim]
    assert big % small == 0, "delta and base feature dims incompatible"
    per_group = big // small
    d = small // g
    split = list(base.shape[:dim]) + [g, 1, d] + list(base.shape[dim + 1:])
    tiled = list(base.shape[:dim]) + [g, per_group, d] + list(base.shape[dim + 1:])
    expanded = base.reshape(split).expand(tiled).reshape(delta.shape)
    return expanded + delta


class LoRAModule(nn.Module):
    """Rank-``rank`` adapter: ``forward(x) = w_b(w_a(x)) * (alpha / rank)``.

    Constructor and attributes as torchtitan/models/llama3/model/model.py:148-182.
    ``scale`` overrides ``alpha / rank`` when given (the reference fixes
    ``alpha = 2 * rank``, i.e. scale 2).
    """

    def __init__(self, in_dim: int, out_dim: int, rank: int = 8, bias: bool = False,
                 w_a_override: Optional[nn.Linear] = None,
                 w_b_override: Optional[nn.Linear] = None,
                 scale: Optional[float] = None, device=None, dtype=None):
        super().__init__()
        self.in_dim = in_dim
        self.out_dim = out_dim
        self.rank = rank
        self.alpha = rank * 2
        self.bias = bias
        self._scale = scale
        fk = {"device": device, "dtype": dtype}
        self.w_a = w_a_override if w_a_override is not None else nn.Linear(in_dim, rank, bias=False, **fk)
        self.w_b = w_b_override if w_b_override is not None else nn.Linear(rank, out_dim, bias=False, **fk)

    @property
    def scale(self) -> float:
        return float(self._scale) if self._scale is not None else self.alpha / self.rank

    def reset_parameters(self) -> None:
        """A ~ kaiming_uniform(a=sqrt(5)), B = 0 (model.py:184-186): the delta starts at 0."""
        nn.init.kaiming_uniform_(self.w_a.weight, a=math.sqrt(5))
        nn.init.zeros_(self.w_b.weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return ops.lora_linear(x, None, self.w_a.weight, self.w_b.weight, self.scale)


class LoRALinear(nn.Module):
    """Fused ``base(x) + lora(x)``: ``x . W^T (* w_scale) + s * (x . A^T) . B^T``.

    ``base`` is an ``nn.Linear`` without bias whose weight may be shared by many
    ``LoRALinear`` instances (the weight-shared model reuses one base per block).
    For an fp8 base, pass ``weight_fp8`` / ``w_scale`` from
    :func:`quantize_fp8_per_channel` instead of ``base``.
    """

    def __init__(self, base: Optional[nn.Linear], lora: Optional[LoRAModule],
                 weight_fp8: Optional[torch.Tensor] = None, w_scale: Optional[torch.Tensor] = None):
        super().__init__()
        if base is not None and base.bias is not None:
            raise ValueError("LoRALinear fuses bias-free projections only (the reference uses bias=False)")
        if base is None and weight_fp8 is None and lora is None:
            raise ValueError("LoRALinear needs a base weight, an fp8 weight or a LoRA adapter")
        self.base = base
        self.lora = lora
        if weight_fp8 is not None:
            if w_scale is None:
                raise ValueError("weight_fp8 needs w_scale")
            self.register_buffer("weight_fp8", weight_fp8)
            self.register_buffer("w_scale", w_scale)
        else:
            self.weight_fp8 = None
            self.w_scale = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.weight_fp8 is not None:
            w, ws = self.weight_fp8, self.w_scale
        else:
            w, ws = (self.base.weight if self.base is not None else None), None
        if self.lora is not None:
            return ops.lora_linear(x, w, self.lora.w_a.weight, self.lora.w_b.weight, self.lora.scale, w_scale=ws)
        return ops.lora_linear(x, w, None, None, 0.0, w_scale=ws)


def quantize_fp8_per_channel(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel e4m3fn quantisation: s_n = max|W_n| / 448, Q = fp8(W / s_n).

    Returns (Q [N,K] float8_e4m3fn, s [N] fp32); W ~= Q * s[:, None]. All-zero rows get
    s_n = 1.
    """
    wf = w.float()
    amax = wf.abs().amax(dim=1)
    s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (wf / s[:, None]).clamp_(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, s.contiguous()
