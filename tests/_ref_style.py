"""Reference-style modules for the converter tests: the attribute layout of
torchtitan/models/llama3/model/model.py:148-192 (LoRAModule) and :246-273, 376-398 (an
attention that adds <p>_base and <p>_offset with broadcast_add), in plain torch."""
import torch
import torch.nn as nn

from weightshared_torchtitan_amd.lora import broadcast_add


class RefLoRA(nn.Module):
    def __init__(self, in_dim, out_dim, rank=8):
        super().__init__()
        self.in_dim, self.out_dim, self.rank, self.alpha = in_dim, out_dim, rank, 2 * rank
        self.w_a = nn.Linear(in_dim, rank, bias=False)
        self.w_b = nn.Linear(rank, out_dim, bias=False)

    def forward(self, x):
        return self.w_b(self.w_a(x)) * (self.alpha / self.rank)


class RefAttentionProjections(nn.Module):
    """q and k as base + offset pairs; k's base is narrower than its offset (grouped
    heads, g = 2), so only q can be fused; o is a plain linear."""

    def __init__(self, dim=512, q_out=512, k_group=128, k_out=256, rank=16):
        super().__init__()
        self.wq_base = nn.Linear(dim, q_out, bias=False)
        self.wq_offset = RefLoRA(dim, q_out, rank)
        self.wk_base = nn.Linear(dim, k_group, bias=False)
        self.wk_offset = RefLoRA(dim, k_out, rank)
        self.wo = nn.Linear(q_out, dim, bias=False)
        self.g = k_out // k_group

    def forward(self, x):
        q = broadcast_add(self.wq_base(x), self.wq_offset(x), g=1)
        k = broadcast_add(self.wk_base(x), self.wk_offset(x), g=self.g)
        return self.wo(q), k
