"""Model converter that moves a torchtitan-style model's LoRA linears onto libwsl.

Follows the reference's converter protocol (torchtitan/protocols/model_converter.py:15-33):
constructed with ``(job_config, parallel_dims)``, ``convert(model)`` rewrites the model in
place, ``post_optimizer_hook(model)`` runs after each optimizer step; converters are
registered by name (:36-50) and applied by the trainer (torchtitan/train.py:160-161).

The reference's attention holds each LoRA projection as a pair (model.py:246-273,
302-324) and adds the two outputs in its forward (:392-398):

    xq = broadcast_add(self.wq_base(x), self.wq_offset(x), g)

``WslLoRAConverter.convert`` rewrites every such pair whose widths match (g = 1, where
broadcast_add is a plain add) so the parent's forward runs one fused launch:

- ``<p>_base`` becomes a ``FusedBase`` whose forward is the fused
  ``x . W^T + s (x . A^T) . B^T``;
- ``<p>_offset`` becomes a wsl ``LoRAModule`` in folded mode, whose forward returns a
  broadcast zero (no memory of its own), so the parent's add is the identity on the fused
  output.

Any other LoRA module (an unpaired one, or one whose base is expanded over head groups)
becomes a wsl ``LoRAModule``: the delta in one launch instead of two GEMMs and a multiply.
Every Parameter object is kept, so the optimizer's state and the state-dict keys
(``<p>_base.weight``, ``<p>_offset.w_a.weight``, ``<p>_offset.w_b.weight``) do not change.
"""
from __future__ import annotations

from typing import Dict, List, Union

import torch
import torch.nn as nn

from . import ops
from .lora import LoRAModule


class FusedBase(nn.Module):
    """The base half of a fused pair: ``weight`` is the original base Parameter; the LoRA
    factors are read from the paired offset module (held outside the module tree so its
    parameters keep their one state-dict key)."""

    def __init__(self, base: nn.Linear, lora: LoRAModule):
        super().__init__()
        self.weight = base.weight
        self.in_features = base.in_features
        self.out_features = base.out_features
        object.__setattr__(self, "_lora", lora)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lora = self._lora
        return ops.lora_linear(x, self.weight, lora.w_a.weight, lora.w_b.weight, lora.scale)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, fused LoRA rank={self._lora.rank}"


class _FoldedLoRA(LoRAModule):
    """A wsl LoRAModule whose delta is already inside its paired ``FusedBase`` output."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x.new_zeros((), dtype=torch.bfloat16).expand(*x.shape[:-1], self.out_dim)


def _is_lora(m: nn.Module) -> bool:
    """The reference's LoRAModule shape (model.py:148-192): bias-free w_a, w_b, rank, alpha."""
    return (isinstance(getattr(m, "w_a", None), nn.Linear) and isinstance(getattr(m, "w_b", None), nn.Linear)
            and m.w_a.bias is None and m.w_b.bias is None and hasattr(m, "rank") and hasattr(m, "alpha"))


def _as_wsl(m: nn.Module, cls=LoRAModule) -> LoRAModule:
    scale = m.scale if isinstance(m, LoRAModule) else m.alpha / m.rank
    return cls(m.w_a.in_features, m.w_b.out_features, rank=m.rank, w_a_override=m.w_a,
               w_b_override=m.w_b, scale=scale)


class WslLoRAConverter:
    """``model.converters = ["wsl_lora"]``: fused LoRA linears (see the module docstring)."""

    def __init__(self, job_config=None, parallel_dims=None):
        self.fused: List[str] = []
        self.converted: List[str] = []

    def convert(self, model: nn.Module) -> None:
        for pname, parent in list(model.named_modules()):
            for name, child in list(parent.named_children()):
                path = f"{pname}.{name}" if pname else name
                if not name.endswith("_offset") or not _is_lora(child) or isinstance(child, _FoldedLoRA):
                    continue
                base = getattr(parent, name[: -len("_offset")] + "_base", None)
                if (isinstance(base, nn.Linear) and base.bias is None
                        and base.out_features == child.w_b.out_features
                        and base.in_features == child.w_a.in_features):
                    lora = _as_wsl(child, _FoldedLoRA)
                    setattr(parent, name, lora)
                    setattr(parent, name[: -len("_offset")] + "_base", FusedBase(base, lora))
                    self.fused.append(path)
            for name, child in list(parent.named_children()):
                if _is_lora(child) and type(child) not in (LoRAModule, _FoldedLoRA):
                    setattr(parent, name, _as_wsl(child))
                    self.converted.append(f"{pname}.{name}" if pname else name)

    def post_optimizer_hook(self, model: Union[nn.Module, List[nn.Module]]) -> None:
        return None


_registry: Dict[str, type] = {}


def register_model_converter(converter_cls: type, name: str) -> None:
    """As torchtitan/protocols/model_converter.py:41-50: one class per name."""
    if name in _registry:
        raise ValueError(f"A model converter {name!r} is already registered.")
    _registry[name] = converter_cls


def build_model_converters(names: List[str], job_config=None, parallel_dims=None) -> list:
    return [_registry[n](job_config, parallel_dims) for n in names]


register_model_converter(WslLoRAConverter, "wsl_lora")
