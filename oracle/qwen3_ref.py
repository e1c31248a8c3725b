"""torch-CPU float32 restatement of the reference arithmetic around the LoRA path
(test infrastructure only; never imported by the product package).

* reference_lora_linear: the reference's CPU path for one LoRA'd projection, op for op
  (nn.Linear base, LoRAModule delta, add).
* reference_forward / reference_generate: a weight-shared Qwen3 forward with no KV
  cache and the greedy generation loop that re-runs the whole prefix every step, as the
  reference's generator does. Parameters are read from the same state-dict keys the
  product model (weightshared_torchtitan_amd.qwen3_shared) uses.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

PROJS = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


def reference_lora_linear(x, W, A, B, scale):
    """F.linear(x, W) + F.linear(F.linear(x, A), B) * scale.

    torchtitan/models/llama3/model/model.py:392 (base nn.Linear), :189-192
    (LoRAModule.forward: w_b(w_a(x)) * (alpha / rank)), :396-398 (broadcast_add, g = 1).
    Pinned by: tests/test_oracle.py::test_oracle_matches_reference_style_torch_cpu_path
    (agrees with the float64 numpy oracle, itself pinned by brute-force golden vectors).
    """
    base = F.linear(x, W) if W is not None else 0.0
    if A is None:
        return base
    return base + F.linear(F.linear(x, A), B) * scale


def rope_cache(head_dim: int, max_seq_len: int, theta: float) -> torch.Tensor:
    """[max_seq_len, 2*head_dim] = cat(cos, sin) of cat(idx_theta, idx_theta).

    torchtitan/experiments/qwen3/model/model.py:20-36.
    Pinned by: position 0 gives cos = 1, sin = 0 (identity rotation) and the rotation
    preserves the per-pair norm (tests/test_model_cpu.py).
    """
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2)[: head_dim // 2].float() / head_dim))
    t = torch.arange(max_seq_len, dtype=freqs.dtype)
    idx = torch.outer(t, freqs).float()
    f = torch.cat([idx, idx], dim=-1)
    return torch.cat([f.cos(), f.sin()], dim=-1)


def _rotate_half(x):
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def _rope(x, rc):
    """x [b, s, heads, hd]; rc [s, 2*hd]. qwen3/model/model.py:73-90."""
    hd = x.shape[-1]
    rc = rc.view(1, rc.shape[0], 1, 2 * hd)
    cos, sin = rc[..., :hd], rc[..., hd:]
    return x * cos + _rotate_half(x) * sin


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def block_of(layer: int, n_layers: int, n_unique: int, block_map: str) -> int:
    """Base block used by `layer`: cyclic (l % n_unique) or contiguous (l // (n_layers/n_unique))."""
    if block_map == "cyclic":
        return layer % n_unique
    return layer // (n_layers // n_unique)


def reference_forward(p: dict, args, tokens: torch.Tensor) -> torch.Tensor:
    """Full-sequence forward (no cache) -> logits [b, s, vocab] in float32.

    Block semantics of torchtitan/experiments/qwen3/model/model.py:167-218 (attention
    with q/k RMSNorm, RoPE, GQA via repeat_kv, causal SDPA), :250-251 (SwiGLU),
    :296-314 (pre-norm residual block); every projection is base (shared block
    b(l)) + per-layer LoRA delta; token embedding factorised E . P^T, output tied
    (h . P) . E^T.
    Pinned by: tests/test_model_cpu.py (a single-token forward equals the explicit
    per-op computation; the generation loop's first token equals the argmax of this
    forward) — parity with the reference model itself is unpinned (the reference has no
    weight-shared Qwen3).
    """
    b, s = tokens.shape
    E = p["tok_embeddings.emb"].float()
    P = p["tok_embeddings.proj.weight"].float()
    h = F.linear(E[tokens], P)
    rc = rope_cache(args.head_dim, max(s, 1), args.rope_theta)[:s]
    scale = args.lora_scale if args.lora_scale is not None else 2.0
    for l in range(args.n_layers):
        bb = block_of(l, args.n_layers, args.n_unique_blocks, args.block_map)
        pre = f"base_blocks.{bb}."
        lp = f"layer_loras.{l}."

        def proj(x, name, sub):
            W = p[f"{pre}{sub}.{name}.weight"].float()
            A = p[f"{lp}{name}.w_a.weight"].float()
            Bm = p[f"{lp}{name}.w_b.weight"].float()
            return reference_lora_linear(x, W, A, Bm, scale)

        x = _rms(h, p[pre + "attention_norm.weight"].float(), args.norm_eps)
        xq = proj(x, "wq", "attention").view(b, s, args.n_heads, args.head_dim)
        xk = proj(x, "wk", "attention").view(b, s, args.n_kv_heads, args.head_dim)
        xv = proj(x, "wv", "attention").view(b, s, args.n_kv_heads, args.head_dim)
        xq = _rms(xq, p[pre + "attention.q_norm.weight"].float(), args.norm_eps)
        xk = _rms(xk, p[pre + "attention.k_norm.weight"].float(), args.norm_eps)
        xq, xk = _rope(xq, rc), _rope(xk, rc)
        rep = args.n_heads // args.n_kv_heads
        xk = xk.repeat_interleave(rep, dim=2)
        xv = xv.repeat_interleave(rep, dim=2)
        o = F.scaled_dot_product_attention(xq.transpose(1, 2), xk.transpose(1, 2), xv.transpose(1, 2),
                                           is_causal=True)
        o = o.transpose(1, 2).reshape(b, s, -1)
        h = h + proj(o, "wo", "attention")
        x = _rms(h, p[pre + "ffn_norm.weight"].float(), args.norm_eps)
        g = proj(x, "w1", "feed_forward")
        u = proj(x, "w3", "feed_forward")
        h = h + proj(F.silu(g) * u, "w2", "feed_forward")
    h = _rms(h, p["norm.weight"].float(), args.norm_eps)
    return (h @ P) @ E.T


def reference_generate(p: dict, args, prompt: torch.Tensor, n_new: int) -> torch.Tensor:
    """Greedy decoding that re-runs the whole prefix each step.

    scripts/generate/_generation.py:49-80 (generate) with top_k = 1, which makes
    logits_to_probs keep one finite logit (:26-29) so sampling is the argmax.
    Pinned by: tests/test_model_cpu.py (first generated token = argmax of
    reference_forward on the prompt).
    """
    toks = prompt.clone()
    for _ in range(n_new):
        logits = reference_forward(p, args, toks)[:, -1]
        nxt = logits.argmax(dim=-1, keepdim=True)
        toks = torch.cat([toks, nxt], dim=1)
    return toks[:, prompt.shape[1]:]
