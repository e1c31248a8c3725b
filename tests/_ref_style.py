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


class RefSharedAttention(nn.Module):
    """The projection part of the reference's Attention with its sharing switches: base widths
    as its constructor sets them (torchtitan/models/llama3/model/model.py:218-273: one base per
    qkv_sharing group named str(group), GQA off under qkv_sharing; g = grouping templates under
    head_sharing; k/v bases g / n_rep templates wide), the two_step offsets (:275-300: one
    head_offset as wide as q, and per-projection w{q,k,v}_only_offset one head wide) and the
    composition of its forward (:366-398: under two_step each offset is
    broadcast_add(w<p>_only_offset(x), head_offset(x)).contiguous(); every projection is
    broadcast_add(base, offset, g=self.grouping)). Returns (xq, xk, xv)."""

    def __init__(self, dim=512, n_heads=16, n_kv_heads=8, rank=8, head_sharing=False, grouping=1,
                 qkv_sharing=None, two_step=False):
        super().__init__()
        self.n_heads, self.n_kv_heads = n_heads, n_kv_heads
        self.qkv_sharing, self.head_sharing = qkv_sharing, head_sharing
        self.grouping = grouping if grouping else 1
        self.two_step = two_step
        self.head_dim = dim // n_heads
        self.n_rep = n_heads // n_kv_heads
        if qkv_sharing:
            self.n_kv_heads, self.n_rep = n_heads, 1
            base_dim = self.head_dim * self.grouping if head_sharing else self.head_dim * n_heads
            for grp in qkv_sharing:
                setattr(self, str(grp), nn.Linear(dim, base_dim, bias=False))
        else:
            dim_mult = self.grouping if head_sharing else n_heads
            kv_dim_mult = dim_mult // self.n_rep
            self.wq_base = nn.Linear(dim, self.head_dim * dim_mult, bias=False)
            self.wk_base = nn.Linear(dim, self.head_dim * kv_dim_mult, bias=False)
            self.wv_base = nn.Linear(dim, self.head_dim * kv_dim_mult, bias=False)
        if two_step:
            self.head_offset = RefLoRA(dim, n_heads * self.head_dim, rank)
            self.wq_only_offset = RefLoRA(dim, self.head_dim, rank)
            self.wk_only_offset = RefLoRA(dim, self.head_dim, rank)
            self.wv_only_offset = RefLoRA(dim, self.head_dim, rank)
        else:
            self.wq_offset = RefLoRA(dim, n_heads * self.head_dim, rank)
            self.wk_offset = RefLoRA(dim, self.n_kv_heads * self.head_dim, rank)
            self.wv_offset = RefLoRA(dim, self.n_kv_heads * self.head_dim, rank)

    def forward(self, x):
        if self.two_step:
            head_offset = self.head_offset(x)
            wq_only_offset = self.wq_only_offset(x)
            wk_only_offset = self.wk_only_offset(x)
            wv_only_offset = self.wv_only_offset(x)
            wq_offset = broadcast_add(wq_only_offset, head_offset).contiguous()
            wk_offset = broadcast_add(wk_only_offset, head_offset).contiguous()
            wv_offset = broadcast_add(wv_only_offset, head_offset).contiguous()
        else:
            wq_offset, wk_offset, wv_offset = self.wq_offset(x), self.wk_offset(x), self.wv_offset(x)
        if self.qkv_sharing:
            for grp in self.qkv_sharing:
                val = getattr(self, str(grp))(x)
                for wgt in grp:
                    if wgt == "q":
                        q_base = val
                    elif wgt == "k":
                        k_base = val
                    elif wgt == "v":
                        v_base = val
        else:
            q_base, k_base, v_base = self.wq_base(x), self.wk_base(x), self.wv_base(x)
        xq = broadcast_add(q_base, wq_offset, g=self.grouping)
        xk = broadcast_add(k_base, wk_offset, g=self.grouping)
        xv = broadcast_add(v_base, wv_offset, g=self.grouping)
        return xq, xk, xv
