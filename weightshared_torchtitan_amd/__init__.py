"""MI355X (gfx950) fused LoRA linear for weight-shared Qwen3 models.

Public surface:
  ops.lora_linear / torch.ops.wsl.lora_linear           fused y = x.W^T + s (x.A^T).B^T
  ops.factorized_embedding / torch.ops.wsl.factorized_embedding
  lora.LoRAModule, lora.LoRALinear, lora.broadcast_add, lora.quantize_fp8_per_channel
  converter.WslLoRAConverter                           the "wsl_lora" model converter
"""
from . import ops  # noqa: F401  (registers torch.ops.wsl.*)
from .lora import LoRALinear, LoRAModule, broadcast_add, quantize_fp8_per_channel  # noqa: F401
from .ops import factorized_embedding, lora_linear  # noqa: F401

__all__ = [
    "LoRALinear",
    "LoRAModule",
    "broadcast_add",
    "factorized_embedding",
    "lora_linear",
    "quantize_fp8_per_channel",
]
