"""Weight-shared Qwen3 decoder whose every projection is the fused LoRA linear.

Layer l runs base block b(l) (one of ``n_unique_blocks`` sets of q/k/v/o/gate/up/down
weights and norms, shared by n_layers / n_unique_blocks layers) plus its own rank-r
LoRA adapters on all seven projections. Tokens enter through a factorized embedding
E [vocab, k] . P^T and leave through the tied head (h . P) . E^T.

Block semantics follow the reference's Qwen3 block:
  attention with q/k RMSNorm, HF-style RoPE and GQA   torchtitan/experiments/qwen3/model/model.py:167-218
  SwiGLU feed-forward                                  :250-251
  pre-norm residual block                              :296-314
Cross-layer sharing, the factorized embedding and LoRA on all projections are the
configuration this path serves; the reference applies LoRA to q/k/v only
(torchtitan/models/llama3/model/model.py:302-324).

Decoding keeps a KV cache (the reference re-runs the full prefix each step,
scripts/generate/_generation.py:43) and can replay one decode step as a HIP graph.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn.functional as F
from torch import nn

from . import ops
from .lora import LoRAModule

PROJS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


@dataclass
class SharedQwen3Args:
    dim: int = 1024
    n_layers: int = 28
    n_unique_blocks: int = 4
    n_heads: int = 16
    n_kv_heads: int = 8
    head_dim: int = 128
    hidden_dim: int = 3072
    vocab_size: int = 151936
    embed_rank: int = 256
    lora_rank: int = 32
    lora_scale: Optional[float] = None  # None: alpha / rank with alpha = 2 * rank
    norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_seq_len: int = 1024
    block_map: str = "cyclic"  # "cyclic": b(l) = l % n_unique; "contiguous": l // (n_layers / n_unique)

    def block_of(self, layer: int) -> int:
        if self.block_map == "cyclic":
            return layer % self.n_unique_blocks
        if self.block_map == "contiguous":
            return layer // (self.n_layers // self.n_unique_blocks)
        raise ValueError(f"unknown block_map {self.block_map!r}")

    def proj_shapes(self) -> dict:
        """(out, in) of each projection."""
        q = self.n_heads * self.head_dim
        kv = self.n_kv_heads * self.head_dim
        return {"wq": (q, self.dim), "wk": (kv, self.dim), "wv": (kv, self.dim), "wo": (self.dim, q),
                "w1": (self.hidden_dim, self.dim), "w3": (self.hidden_dim, self.dim),
                "w2": (self.dim, self.hidden_dim)}


def qwen3_0p6b_shared() -> SharedQwen3Args:
    """The benchmark configuration: Qwen3-0.6B dims, 28 layers from 4 unique blocks."""
    return SharedQwen3Args()


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return (y * self.weight.float()).to(x.dtype)


class _Attention(nn.Module):
    def __init__(self, a: SharedQwen3Args):
        super().__init__()
        sh = a.proj_shapes()
        for name in ("wq", "wk", "wv", "wo"):
            out, inp = sh[name]
            setattr(self, name, nn.Linear(inp, out, bias=False))
        self.q_norm = RMSNorm(a.head_dim, a.norm_eps)
        self.k_norm = RMSNorm(a.head_dim, a.norm_eps)


class _FeedForward(nn.Module):
    def __init__(self, a: SharedQwen3Args):
        super().__init__()
        sh = a.proj_shapes()
        for name in ("w1", "w2", "w3"):
            out, inp = sh[name]
            setattr(self, name, nn.Linear(inp, out, bias=False))


class SharedBlockBase(nn.Module):
    """The shared (base) weights of one unique block."""

    def __init__(self, a: SharedQwen3Args):
        super().__init__()
        self.attention = _Attention(a)
        self.feed_forward = _FeedForward(a)
        self.attention_norm = RMSNorm(a.dim, a.norm_eps)
        self.ffn_norm = RMSNorm(a.dim, a.norm_eps)

    def base(self, name: str) -> nn.Linear:
        return getattr(self.attention if name in ("wq", "wk", "wv", "wo") else self.feed_forward, name)


class LayerLoRA(nn.Module):
    """Per-layer adapters: one LoRAModule per projection."""

    def __init__(self, a: SharedQwen3Args):
        super().__init__()
        for name, (out, inp) in a.proj_shapes().items():
            setattr(self, name, LoRAModule(inp, out, rank=a.lora_rank, scale=a.lora_scale))


class FactorizedEmbedding(nn.Module):
    """E [vocab, k] and P = proj.weight [dim, k]: embed(ids) = E[ids] . P^T."""

    def __init__(self, vocab: int, rank: int, dim: int):
        super().__init__()
        self.emb = nn.Parameter(torch.empty(vocab, rank))
        self.proj = nn.Linear(rank, dim, bias=False)
        self._pt = None
        self._pt_key = None

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return ops.factorized_embedding(ids, self.emb, self.proj.weight)

    def proj_t(self) -> torch.Tensor:
        """P^T [k, dim] contiguous, cached while P is unchanged."""
        w = self.proj.weight
        key = (w.data_ptr(), w._version)
        if self._pt is None or self._pt_key != key:
            self._pt = w.detach().t().contiguous()
            self._pt_key = key
        return self._pt

    def tied_logits(self, h: torch.Tensor) -> torch.Tensor:
        """(h . P) . E^T as two fused-linear calls (r = 0): [.., dim] -> [.., k] -> [.., vocab]."""
        z = ops.lora_linear(h, self.proj_t(), None, None, 0.0)
        return ops.lora_linear(z, self.emb, None, None, 0.0)


class KVCache:
    """Per-layer K and V, each [n_layers, b, kv_heads, max_len, head_dim] (one position's
    head_dim vector contiguous, as the decode attention kernel streams them)."""

    def __init__(self, a: SharedQwen3Args, batch: int, max_len: int, device, dtype=torch.bfloat16):
        self.k = torch.zeros(a.n_layers, batch, a.n_kv_heads, max_len, a.head_dim, device=device, dtype=dtype)
        self.v = torch.zeros(a.n_layers, batch, a.n_kv_heads, max_len, a.head_dim, device=device, dtype=dtype)
        self.max_len = max_len


def _rope_cache(head_dim: int, max_seq_len: int, theta: float) -> torch.Tensor:
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2)[: head_dim // 2].float() / head_dim))
    t = torch.arange(max_seq_len, dtype=freqs.dtype)
    idx = torch.outer(t, freqs).float()
    f = torch.cat([idx, idx], dim=-1)
    return torch.cat([f.cos(), f.sin()], dim=-1)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


class SharedQwen3(nn.Module):
    def __init__(self, a: SharedQwen3Args):
        super().__init__()
        if a.n_layers % a.n_unique_blocks != 0:
            raise ValueError("n_layers must be a multiple of n_unique_blocks")
        self.args = a
        self.tok_embeddings = FactorizedEmbedding(a.vocab_size, a.embed_rank, a.dim)
        self.base_blocks = nn.ModuleList([SharedBlockBase(a) for _ in range(a.n_unique_blocks)])
        self.layer_loras = nn.ModuleList([LayerLoRA(a) for _ in range(a.n_layers)])
        self.norm = RMSNorm(a.dim, a.norm_eps)
        self.register_buffer("rope", _rope_cache(a.head_dim, a.max_seq_len, a.rope_theta), persistent=False)

    # ------------------------------------------------------------------ init
    @torch.no_grad()
    def init_random(self, seed: int = 0, std: float = 0.02) -> None:
        """Every weight matrix ~ N(0, std^2) (LoRA B non-zero), norms = 1, drawn on the CPU
        from one seeded generator in parameter order, then copied to the module's device."""
        g = torch.Generator().manual_seed(seed)
        for name, p in self.named_parameters():
            if name.endswith("norm.weight"):
                p.fill_(1.0)
            else:
                p.copy_((torch.randn(p.shape, generator=g) * std).to(p.dtype))

    # ------------------------------------------------------------------ helpers
    def _proj(self, layer: int, name: str, x: torch.Tensor) -> torch.Tensor:
        base = self.base_blocks[self.args.block_of(layer)].base(name)
        lora = getattr(self.layer_loras[layer], name)
        return ops.lora_linear(x, base.weight, lora.w_a.weight, lora.w_b.weight, lora.scale)

    def _rope(self, x: torch.Tensor, rc: torch.Tensor) -> torch.Tensor:
        hd = x.shape[-1]
        cos = rc[..., :hd].to(x.dtype)
        sin = rc[..., hd:].to(x.dtype)
        return x * cos + _rotate_half(x) * sin

    def _ffn(self, layer: int, h: torch.Tensor, pk: Optional[dict] = None) -> torch.Tensor:
        blk = self.base_blocks[self.args.block_of(layer)]
        x = blk.ffn_norm(h)
        gu = self._grouped(layer, "gu", x, pk)
        if gu is not None:
            g, u = gu
        else:
            g = self._proj(layer, "w1", x)
            u = self._proj(layer, "w3", x)
        return h + self._proj(layer, "w2", F.silu(g) * u)

    # With prefill_grouped, inference prefill runs q|k|v and gate|up as grouped launches (one
    # each, on the stacked operands cached with the decode pack); with autograd on, always
    # one launch per projection so the gradients reach the module parameters. Off by
    # default: at the config-4 prompt (M = 4096) the per-projection launches fill the CUs
    # with better-suited tiles (128 x 256 and 128 x 128 against one wave of 256 x 256), and
    # the forward measured 21.9 ms against 22.2 ms grouped on MI355X.
    prefill_grouped = False

    def _grouped(self, layer: int, group: str, x: torch.Tensor, pk: Optional[dict]):
        """The group's projections of x in one grouped launch, as a list of views, or None
        when this call takes the per-projection path."""
        if pk is None or pk["g_" + group][layer] is None:
            return None
        A, B, sc, widths = pk["g_" + group][layer]
        y = ops.lora_linear_grouped_op(x, pk["w_" + group][self.args.block_of(layer)], None, A, B, sc, widths)
        return list(y.split(widths, -1))

    # ------------------------------------------------------------------ prefill
    def forward(self, tokens: torch.Tensor, cache: Optional[KVCache] = None) -> torch.Tensor:
        """Full-sequence causal forward from position 0 -> logits [b, s, vocab].
        Fills `cache` (positions 0..s-1) when given."""
        a = self.args
        b, s = tokens.shape
        if s > a.max_seq_len:
            raise IndexError(f"sequence of {s} tokens exceeds max_seq_len {a.max_seq_len} (the RoPE table)")
        pk = self._decode_pack() if (self.prefill_grouped and not torch.is_grad_enabled()) else None
        h = self.tok_embeddings(tokens)
        rc = self.rope[:s].view(1, s, 1, 2 * a.head_dim)
        rep = a.n_heads // a.n_kv_heads
        from torch.nn.attention import SDPBackend, sdpa_kernel
        for l in range(a.n_layers):
            blk = self.base_blocks[a.block_of(l)]
            x = blk.attention_norm(h)
            qkv = self._grouped(l, "qkv", x, pk)
            if qkv is None:
                qkv = [self._proj(l, n, x) for n in ("wq", "wk", "wv")]
            xq = qkv[0].view(b, s, a.n_heads, a.head_dim)
            xk = qkv[1].view(b, s, a.n_kv_heads, a.head_dim)
            xv = qkv[2].view(b, s, a.n_kv_heads, a.head_dim)
            xq = self._rope(blk.attention.q_norm(xq), rc)
            xk = self._rope(blk.attention.k_norm(xk), rc)
            if cache is not None:
                cache.k[l, :, :, :s] = xk.transpose(1, 2)
                cache.v[l, :, :, :s] = xv.transpose(1, 2)
            kk = xk.repeat_interleave(rep, dim=2).transpose(1, 2).contiguous()
            vv = xv.repeat_interleave(rep, dim=2).transpose(1, 2).contiguous()
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
                o = F.scaled_dot_product_attention(xq.transpose(1, 2).contiguous(), kk, vv, is_causal=True)
            o = o.transpose(1, 2).reshape(b, s, a.n_heads * a.head_dim)
            h = h + self._proj(l, "wo", o)
            h = self._ffn(l, h, pk)
        h = self.norm(h)
        return self.tok_embeddings.tied_logits(h)

    # ------------------------------------------------------------------ decode
    def _decode_pack(self) -> dict:
        """Concatenated operands for the decode step's fused q|k|v and gate|up projections.

        [W_q; W_k; W_v] (per unique block) with per-layer [A_q; A_k; A_v] and the
        block-diagonal [B_q, 0, 0; 0, B_k, 0; 0, 0, B_v] give exactly the three LoRA linears
        (each output row meets only its own rank block; the zero blocks add exact zeros), in
        one launch that streams all three weights; likewise [W_1; W_3] for gate|up. Rebuilt
        when any parameter changes."""
        key = tuple((p.data_ptr(), p._version) for p in self.parameters())
        pk = getattr(self, "_pack_cache", None)
        if pk is not None and pk["key"] == key:
            return pk
        a = self.args

        def cat_w(blk, names):
            return torch.cat([blk.base(n).weight for n in names], 0).contiguous()

        def cat_lora(layer, names):
            mods = [getattr(self.layer_loras[layer], n) for n in names]
            scales = {m.scale for m in mods}
            if len(scales) != 1:
                return None
            A = torch.cat([m.w_a.weight for m in mods], 0).contiguous()
            rows = sum(m.w_b.weight.shape[0] for m in mods)
            ranks = sum(m.w_b.weight.shape[1] for m in mods)
            B = mods[0].w_b.weight.new_zeros(rows, ranks)
            r0 = c0 = 0
            for m in mods:
                n, r = m.w_b.weight.shape
                B[r0:r0 + n, c0:c0 + r] = m.w_b.weight
                r0, c0 = r0 + n, c0 + r
            return A, B, scales.pop()

        def stack_lora(layer, names):
            # [A_1; A_2; ...] and [B_1; B_2; ...] for wsl::lora_linear_grouped (one rank, one scale)
            mods = [getattr(self.layer_loras[layer], n) for n in names]
            if len({m.scale for m in mods}) != 1 or len({m.w_a.weight.shape[0] for m in mods}) != 1:
                return None
            A = torch.cat([m.w_a.weight for m in mods], 0).contiguous()
            B = torch.cat([m.w_b.weight for m in mods], 0).contiguous()
            return A, B, mods[0].scale, [m.w_b.weight.shape[0] for m in mods]

        def interleave8(g, u):
            # rows 16j..16j+7 <- g rows 8j..8j+7, rows 16j+8..16j+15 <- u rows 8j..8j+7
            n = g.shape[0]
            return torch.stack((g.reshape(n // 8, 8, -1), u.reshape(n // 8, 8, -1)), 1).reshape(2 * n, -1)

        def gu_interleaved(layer, blk):
            w1, w3 = blk.base("w1").weight, blk.base("w3").weight
            if w1.shape[0] % 8 != 0:
                return None
            lo = self.layer_loras[layer]
            if lo.w1.scale != lo.w3.scale:
                return None
            b1, b3 = lo.w1.w_b.weight, lo.w3.w_b.weight
            A = torch.cat([lo.w1.w_a.weight, lo.w3.w_a.weight], 0).contiguous()
            B = interleave8(torch.cat([b1, torch.zeros_like(b3)], 1), torch.cat([torch.zeros_like(b1), b3], 1))
            return A, B.contiguous(), lo.w1.scale

        with torch.no_grad():
            pk = {"key": key,
                  "w_qkv": [cat_w(blk, ("wq", "wk", "wv")) for blk in self.base_blocks],
                  "w_gu": [cat_w(blk, ("w1", "w3")) for blk in self.base_blocks],
                  "l_qkv": [cat_lora(l, ("wq", "wk", "wv")) for l in range(a.n_layers)],
                  "l_gu": [cat_lora(l, ("w1", "w3")) for l in range(a.n_layers)],
                  "g_qkv": [stack_lora(l, ("wq", "wk", "wv")) for l in range(a.n_layers)],
                  "g_gu": [stack_lora(l, ("w1", "w3")) for l in range(a.n_layers)]}
            if a.hidden_dim % 8 == 0:
                pk["w_gu_il"] = [interleave8(blk.base("w1").weight, blk.base("w3").weight).contiguous()
                                 for blk in self.base_blocks]
                pk["l_gu_il"] = [gu_interleaved(l, self.base_blocks[a.block_of(l)]) for l in range(a.n_layers)]
        self._pack_cache = pk
        return pk

    def _fusion_plan(self, b: int, pk: dict) -> dict:
        """Which decode-step launches take the fused forms (include/wsl_decode.h) at batch b:
        q|k|v with the RMSNorm prologue, o and down projections with the residual epilogue,
        gate|up with RMSNorm + SwiGLU, the head's first factor with RMSNorm. A group whose
        adapters differ in scale, or whose shape the fused kernel does not cover, keeps the
        separate kernels."""
        a = self.args
        r = a.lora_rank
        sup = ops.lora_linear_fused_supported
        qkv_n = (a.n_heads + 2 * a.n_kv_heads) * a.head_dim
        plan = {
            "qkv": all(x is not None for x in pk["l_qkv"]) and sup(b, qkv_n, a.dim, 3 * r, 1),
            "wo": sup(b, a.dim, a.n_heads * a.head_dim, r, 4),
            "gu": "l_gu_il" in pk and all(x is not None for x in pk["l_gu_il"])
                  and sup(b, 2 * a.hidden_dim, a.dim, 2 * r, 3),
            "w2": sup(b, a.dim, a.hidden_dim, r, 4),
            "head": sup(b, a.embed_rank, a.dim, 0, 1),
        }
        plan["on"] = self.decode_fusion and all(plan.values())
        return plan

    def _rope32(self) -> torch.Tensor:
        """The RoPE table in fp32 (the `rope` buffer follows the module's dtype, and cos/sin
        in bf16 would lose precision), cached per device."""
        dev = self.rope.device
        t = getattr(self, "_rope32_cache", None)
        if t is None or t.device != dev:
            t = _rope_cache(self.args.head_dim, self.args.max_seq_len, self.args.rope_theta).to(dev)
            self._rope32_cache = t
        return t

    def _proj_group(self, layer: int, group: str, names, x: torch.Tensor, pk: dict) -> torch.Tensor:
        lo = pk["l_" + group][layer]
        if lo is None:  # adapters with different scales: one call per projection
            return torch.cat([self._proj(layer, n, x) for n in names], -1)
        w = pk["w_" + group][self.args.block_of(layer)]
        A, B, sc = lo
        return ops.lora_linear(x, w, A, B, sc)

    decode_fusion = True  # use the fused decode-step launches where _fusion_plan allows

    # Run each layer's o, gate|up and down projections and the next layer's q|k|v (the head's
    # first factor after the last layer) as one chain launch between two attention steps,
    # where the library takes the chain (wsl_lora_linear_chain_fwd; same results bit for bit):
    # 58 launches per step instead of 142. Off by default: at config 4 it measured at parity
    # with the separate launches (5409 against 5440 tok/s, one box), the stage waits inside
    # the launch costing about what the launch boundaries did.
    decode_chain = False

    def _chain_layer_stages(self, l, o, h, nxt, pk, outs):
        """The chain of layer l: o (+ residual h) -> gate|up (RMSNorm, SwiGLU) -> down
        (+ residual) -> `nxt` = (x-consuming weights of the next launch: the next layer's
        q|k|v with its RMSNorm, or the head's first factor with the final RMSNorm)."""
        from ._native import WSL_FUSE_RESIDUAL as RES, WSL_FUSE_RMSNORM as NORM, WSL_FUSE_SWIGLU as ACT
        a = self.args
        blk = self.base_blocks[a.block_of(l)]
        lo = self.layer_loras[l]
        h1, act, h2, y4 = outs
        Ag, Bg, sg = pk["l_gu_il"][l]
        S = ops.ChainStage
        nw, w, A, B, sc = nxt
        return [S(o, blk.base("wo").weight, lo.wo.w_a.weight, lo.wo.w_b.weight, lo.wo.scale, h1, fuse=RES,
                  residual=h),
                S(h1, pk["w_gu_il"][a.block_of(l)], Ag, Bg, sg, act, fuse=NORM | ACT, norm_w=blk.ffn_norm.weight,
                  eps=a.norm_eps, after_previous=True),
                S(act, blk.base("w2").weight, lo.w2.w_a.weight, lo.w2.w_b.weight, lo.w2.scale, h2, fuse=RES,
                  residual=h1, after_previous=True),
                S(h2, w, A, B, sc, y4, fuse=NORM, norm_w=nw, eps=a.norm_eps, after_previous=True)]

    def _decode_step_chain(self, h, pos, cache, pk, rope):
        """The fused decode step with chain launches: q|k|v of layer 0, then per layer the
        attention step and one chain (o, gate|up, down, and the next layer's q|k|v or the
        head's first factor). Returns None where the library does not take the chain."""
        a = self.args
        b = h.shape[0]
        sm_scale = a.head_dim ** -0.5
        fl = ops.lora_linear_fused_op
        dev = h.device
        qkv_n = (a.n_heads + 2 * a.n_kv_heads) * a.head_dim

        def nxt_of(l):
            if l + 1 < a.n_layers:
                A, B, sc = pk["l_qkv"][l + 1]
                nb = self.base_blocks[a.block_of(l + 1)]
                return nb.attention_norm.weight, pk["w_qkv"][a.block_of(l + 1)], A, B, sc
            return self.norm.weight, self.tok_embeddings.proj_t(), None, None, 0.0

        def outs_of(l):
            e = lambda n: torch.empty(b, n, dtype=torch.bfloat16, device=dev)  # noqa: E731
            return e(a.dim), e(a.hidden_dim), e(a.dim), e(qkv_n if l + 1 < a.n_layers else a.embed_rank)

        o_probe = torch.empty(b, a.n_heads * a.head_dim, dtype=torch.bfloat16, device=dev)
        for l in (0, a.n_layers - 1):  # every layer's chain has one of these two shapes
            if not ops.chain_supported(self._chain_layer_stages(l, o_probe, h, nxt_of(l), pk, outs_of(l)), b):
                return None
        blk = self.base_blocks[a.block_of(0)]
        A, B, sc = pk["l_qkv"][0]
        qkv = fl(h, blk.attention_norm.weight, a.norm_eps, pk["w_qkv"][a.block_of(0)], A, B, sc, None, 1)
        for l in range(a.n_layers):
            blk = self.base_blocks[a.block_of(l)]
            o = ops.decode_attention_step_op(qkv, blk.attention.q_norm.weight, blk.attention.k_norm.weight,
                                             a.norm_eps, rope, pos, cache.k[l], cache.v[l], a.n_heads,
                                             a.n_kv_heads, sm_scale)
            outs = outs_of(l)
            ops.lora_linear_chain(self._chain_layer_stages(l, o, h, nxt_of(l), pk, outs), b)
            h, qkv = outs[2], outs[3]
        return qkv  # after the last layer: z = rmsnorm(h) . P

    def _decode_step_fused(self, h, pos, cache, pk, rope) -> torch.Tensor:
        """The decode step in fused launches up to the head input z = rmsnorm(h) . P [b, k]:
        q|k|v (RMSNorm prologue), the fused attention step, o projection (+ residual),
        gate|up (RMSNorm prologue, SwiGLU epilogue), down projection (+ residual); then the
        head's first factor with the final RMSNorm. With decode_chain, the projections
        between two attention steps run as one chain launch."""
        if self.decode_chain:
            z = self._decode_step_chain(h, pos, cache, pk, rope)
            if z is not None:
                return z
        a = self.args
        b = h.shape[0]
        sm_scale = a.head_dim ** -0.5
        fl = ops.lora_linear_fused_op
        for l in range(a.n_layers):
            blk = self.base_blocks[a.block_of(l)]
            lo = self.layer_loras[l]
            A, B, sc = pk["l_qkv"][l]
            qkv = fl(h, blk.attention_norm.weight, a.norm_eps, pk["w_qkv"][a.block_of(l)], A, B, sc, None, 1)
            o = ops.decode_attention_step_op(qkv, blk.attention.q_norm.weight, blk.attention.k_norm.weight,
                                             a.norm_eps, rope, pos, cache.k[l], cache.v[l], a.n_heads,
                                             a.n_kv_heads, sm_scale)
            wo, Ao, Bo, so = blk.base("wo").weight, lo.wo.w_a.weight, lo.wo.w_b.weight, lo.wo.scale
            Ag, Bg, sg = pk["l_gu_il"][l]
            h = fl(o, None, 0.0, wo, Ao, Bo, so, h, 4)
            act = fl(h, blk.ffn_norm.weight, a.norm_eps, pk["w_gu_il"][a.block_of(l)], Ag, Bg, sg, None, 3)
            w2, A2, B2, s2 = blk.base("w2").weight, lo.w2.w_a.weight, lo.w2.w_b.weight, lo.w2.scale
            h = fl(act, None, 0.0, w2, A2, B2, s2, h, 4)
        return fl(h, self.norm.weight, a.norm_eps, self.tok_embeddings.proj_t(), None, None, 0.0, None, 1)

    def _decode_z(self, token: torch.Tensor, pos: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """One decode step at position `pos` (0-d int64 device tensor) up to the head input
        z = rmsnorm(h) . P [b, k]. Shape-static and host-sync-free, so it can be captured in
        a HIP graph. Per layer: residual add + RMSNorm, fused q|k|v projection, q/k norm +
        RoPE + cache write, decode attention, o projection, residual add + RMSNorm, fused
        gate|up projection, SwiGLU, down projection (its residual add joins the next layer's
        norm)."""
        a = self.args
        b = token.shape[0]
        pk = self._decode_pack()
        rope = self._rope32()
        h = self.tok_embeddings(token.view(b)).view(b, a.dim)
        fused_attn = a.n_heads // a.n_kv_heads in (1, 2, 4) and a.head_dim in (64, 128)
        if fused_attn:
            plan = self._fusion_plan(b, pk)
            if plan["on"]:
                return self._decode_step_fused(h, pos, cache, pk, rope)
        sm_scale = a.head_dim ** -0.5
        pending = None
        for l in range(a.n_layers):
            blk = self.base_blocks[a.block_of(l)]
            if pending is None:
                x = ops.rmsnorm_op(h, blk.attention_norm.weight, a.norm_eps)
            else:
                x, h = ops.add_rmsnorm_op(pending, h, blk.attention_norm.weight, a.norm_eps)
            qkv = self._proj_group(l, "qkv", ("wq", "wk", "wv"), x, pk)
            if fused_attn:
                o = ops.decode_attention_step_op(qkv, blk.attention.q_norm.weight, blk.attention.k_norm.weight,
                                                 a.norm_eps, rope, pos, cache.k[l], cache.v[l], a.n_heads,
                                                 a.n_kv_heads, sm_scale)
            else:
                q = ops.qk_norm_rope_op(qkv, blk.attention.q_norm.weight, blk.attention.k_norm.weight, a.norm_eps,
                                        rope, pos, cache.k[l], cache.v[l], a.n_heads, a.n_kv_heads)
                o = ops.decode_attention_op(q, cache.k[l], cache.v[l], pos, sm_scale)
            o = self._proj(l, "wo", o)
            x, h = ops.add_rmsnorm_op(o, h, blk.ffn_norm.weight, a.norm_eps)
            gu = self._proj_group(l, "gu", ("w1", "w3"), x, pk)
            pending = self._proj(l, "w2", ops.swiglu_op(gu))
        x, _ = ops.add_rmsnorm_op(pending, h, self.norm.weight, a.norm_eps)
        return ops.lora_linear(x, self.tok_embeddings.proj_t(), None, None, 0.0)

    def decode_step(self, token: torch.Tensor, pos: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """One step at position `pos` -> logits [b, vocab] (the tied head (h . P) . E^T)."""
        z = self._decode_z(token, pos, cache)
        return ops.lora_linear(z, self.tok_embeddings.emb, None, None, 0.0).view(token.shape[0], -1)

    # Greedy steps take the head fused with the argmax (wsl_tied_head_argmax_fwd: E streamed
    # once, no logits written) where it covers the shape; off, the logits are written and a
    # separate argmax reads them.
    head_argmax_fusion = True

    def decode_next(self, token: torch.Tensor, pos: torch.Tensor, cache: KVCache) -> torch.Tensor:
        """One greedy step at position `pos` -> the next tokens [b] (int64): the argmax of
        the step's bf16 logits (first index on ties, NaN largest, as torch.argmax; the
        reference's top_k = 1 sampling, scripts/generate/_generation.py:19-32)."""
        z = self._decode_z(token, pos, cache)
        emb = self.tok_embeddings.emb
        if self.head_argmax_fusion and ops.tied_head_argmax_supported(z.shape[0], emb.shape[0], emb.shape[1]):
            return ops.tied_head_argmax_op(z, emb)
        return ops.argmax_rows_op(ops.lora_linear(z, emb, None, None, 0.0))

    @torch.no_grad()
    def generate(self, prompt: torch.Tensor, n_new: int, use_graph: bool = True, return_logits: bool = False):
        """Greedy decoding with a KV cache. Returns (new tokens [b, n_new], timings dict); with
        `return_logits` the dict also holds "logits" [b, n_new, vocab], the logits each new
        token was chosen from (copied out of the step's buffer after every step).

        Positions 0..s + n_new - 2 are embedded (the last new token is not fed back), so
        s + n_new - 1 may not exceed max_seq_len, the length of the RoPE table; the
        reference's rope cache lookup raises an IndexError in that case too."""
        b, s = prompt.shape
        if n_new < 1:
            raise ValueError("n_new must be >= 1")
        if s + n_new - 1 > self.args.max_seq_len:
            raise IndexError(f"prompt {s} + {n_new} new tokens needs {s + n_new - 1} positions; "
                             f"max_seq_len is {self.args.max_seq_len}")
        dev = prompt.device
        cache = KVCache(self.args, b, s + n_new - 1, dev)  # positions 0 .. s + n_new - 2
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t2 = torch.cuda.Event(enable_timing=True)
        t0.record()
        logits = self.forward(prompt, cache)[:, -1]
        tok = logits.argmax(-1).view(b, 1)
        t1.record()
        out = torch.empty(b, n_new, dtype=torch.int64, device=dev)
        out[:, 0] = tok[:, 0]
        logits_out = None
        if return_logits:
            logits_out = torch.empty(b, n_new, logits.shape[-1], dtype=logits.dtype, device=dev)
            logits_out[:, 0] = logits
        pos = torch.full((), s, dtype=torch.int64, device=dev)
        tok_buf = tok.clone()
        if use_graph and n_new > 1:
            # warm up outside the graph (kernel selection, allocator), then capture one step
            def step():
                if logits_out is None:
                    return None, self.decode_next(tok_buf, pos, cache).view(b, 1)
                lg = self.decode_step(tok_buf, pos, cache)
                return lg, ops.argmax_rows_op(lg).view(b, 1)

            stream = torch.cuda.Stream()
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                step()
            torch.cuda.current_stream().wait_stream(stream)
            graph = torch.cuda.CUDAGraph()
            # captured on the warm-up stream: the ops' per-stream workspaces already exist
            with torch.cuda.graph(graph, stream=stream):
                g_logits, g_next = step()
            # the warm-up wrote position s; the first replay rewrites it identically
            for i in range(1, n_new):
                graph.replay()
                out[:, i] = g_next[:, 0]
                if logits_out is not None:
                    logits_out[:, i] = g_logits
                tok_buf.copy_(g_next)
                pos.add_(1)
        else:
            for i in range(1, n_new):
                if logits_out is None:
                    nxt = self.decode_next(tok_buf, pos, cache).view(b, 1)
                else:
                    logits = self.decode_step(tok_buf, pos, cache)
                    nxt = ops.argmax_rows_op(logits).view(b, 1)
                    logits_out[:, i] = logits
                out[:, i] = nxt[:, 0]
                tok_buf.copy_(nxt)
                pos.add_(1)
        t2.record()
        t2.synchronize()
        res = {"prefill_ms": t0.elapsed_time(t1), "decode_ms": t1.elapsed_time(t2)}
        if logits_out is not None:
            res["logits"] = logits_out
        return out, res
