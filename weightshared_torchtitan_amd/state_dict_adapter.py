"""On-disk mapping of the weight-shared Qwen3 state dict.

The reference converts its native state dict to and from the HuggingFace layout with a
``StateDictAdapter`` (``to_hf`` / ``from_hf``, torchtitan/protocols/state_dict_adapter.py:19-55;
the Llama-3 one at torchtitan/models/llama3/model/state_dict_adapter.py:18-128, whose key map
still names the pre-LoRA attention). The weight-shared model keeps one copy of each unique
block's base weights (``base_blocks.{b}.*``) and per-layer adapters (``layer_loras.{l}.*``);
on disk the layout is flat and per layer, as every HuggingFace Qwen3 checkpoint is:

lossless (``to_hf(sd)``), PEFT-style LoRA names, the base weight repeated per layer:
    model.layers.{l}.self_attn.q_proj.base_layer.weight   base_blocks.{b(l)}.attention.wq.weight
    model.layers.{l}.self_attn.q_proj.lora_A.weight       layer_loras.{l}.wq.w_a.weight
    model.layers.{l}.self_attn.q_proj.lora_B.weight       layer_loras.{l}.wq.w_b.weight
    (k_proj/v_proj/o_proj = wk/wv/wo; mlp.gate_proj/up_proj/down_proj = w1/w3/w2)
    model.layers.{l}.self_attn.q_norm.weight / k_norm     base_blocks.{b(l)}.attention.q_norm / k_norm
    model.layers.{l}.input_layernorm.weight               base_blocks.{b(l)}.attention_norm.weight
    model.layers.{l}.post_attention_layernorm.weight      base_blocks.{b(l)}.ffn_norm.weight
    model.embed_tokens.emb_factor  [vocab, k]              tok_embeddings.emb
    model.embed_tokens.proj_factor [dim, k]                tok_embeddings.proj.weight
    model.norm.weight                                      norm.weight
``from_hf`` inverts it exactly; the layers of one block must carry identical base weights and
norms (the shared layout cannot hold anything else), or it raises.

merged (``to_hf(sd, merged=True)``): a plain dense Qwen3 checkpoint, loadable by any model
without LoRA or sharing: ``q_proj.weight = W_b(l) + s * B_l . A_l`` (computed in fp32, stored in
the source dtype), ``embed_tokens.weight = E . P^T`` and ``lm_head.weight`` the same tensor (the
head is tied). It cannot be split back into shared bases and adapters; ``from_hf`` refuses it.

Qwen3 uses rotate-half RoPE like HuggingFace (torchtitan/experiments/qwen3/model/model.py:73-90),
so q/k need none of the row permutation the Llama adapter applies.
"""
from __future__ import annotations

import re
from typing import Any, Dict

import torch

# (our projection name, module holding it, HF module path, HF projection name)
_PROJ_MAP = (
    ("wq", "attention", "self_attn", "q_proj"),
    ("wk", "attention", "self_attn", "k_proj"),
    ("wv", "attention", "self_attn", "v_proj"),
    ("wo", "attention", "self_attn", "o_proj"),
    ("w1", "feed_forward", "mlp", "gate_proj"),
    ("w3", "feed_forward", "mlp", "up_proj"),
    ("w2", "feed_forward", "mlp", "down_proj"),
)
# per-block tensors that are not projections: ours -> HF per-layer name
_NORM_MAP = (
    ("attention.q_norm.weight", "self_attn.q_norm.weight"),
    ("attention.k_norm.weight", "self_attn.k_norm.weight"),
    ("attention_norm.weight", "input_layernorm.weight"),
    ("ffn_norm.weight", "post_attention_layernorm.weight"),
)


class SharedQwen3StateDictAdapter:
    """``to_hf`` / ``from_hf`` for :class:`~weightshared_torchtitan_amd.qwen3_shared.SharedQwen3`.

    Same constructor and method names as the reference's adapters
    (torchtitan/protocols/state_dict_adapter.py:29-55); ``hf_assets_path`` is accepted and
    unused (no safetensors index is read: the build has no network or HF assets)."""

    def __init__(self, model_args, hf_assets_path: str | None = None):
        self.model_args = model_args
        self.hf_assets_path = hf_assets_path

    # ------------------------------------------------------------------ helpers
    def _scale(self) -> float:
        a = self.model_args
        return float(a.lora_scale) if a.lora_scale is not None else 2.0  # alpha = 2 * rank

    def _layers_of(self, b: int):
        a = self.model_args
        return [l for l in range(a.n_layers) if a.block_of(l) == b]

    # ------------------------------------------------------------------ export
    def to_hf(self, state_dict: Dict[str, Any], merged: bool = False) -> Dict[str, Any]:
        a = self.model_args
        sd = state_dict
        out: Dict[str, Any] = {}
        s = self._scale()
        for l in range(a.n_layers):
            b = a.block_of(l)
            base = f"base_blocks.{b}."
            for ours, sub, hf_mod, hf_name in _PROJ_MAP:
                W = sd[f"{base}{sub}.{ours}.weight"]
                A = sd[f"layer_loras.{l}.{ours}.w_a.weight"]
                B = sd[f"layer_loras.{l}.{ours}.w_b.weight"]
                key = f"model.layers.{l}.{hf_mod}.{hf_name}"
                if merged:
                    dense = W.float() + s * (B.float() @ A.float())
                    out[f"{key}.weight"] = dense.to(W.dtype)
                else:
                    out[f"{key}.base_layer.weight"] = W
                    out[f"{key}.lora_A.weight"] = A
                    out[f"{key}.lora_B.weight"] = B
            for ours, hf in _NORM_MAP:
                out[f"model.layers.{l}.{hf}"] = sd[base + ours]
        E = sd["tok_embeddings.emb"]
        P = sd["tok_embeddings.proj.weight"]
        if merged:
            emb = (E.float() @ P.float().t()).to(E.dtype)
            out["model.embed_tokens.weight"] = emb
            out["lm_head.weight"] = emb  # tied: (h . P) . E^T = h . (E . P^T)^T
        else:
            out["model.embed_tokens.emb_factor"] = E
            out["model.embed_tokens.proj_factor"] = P
        out["model.norm.weight"] = sd["norm.weight"]
        return out

    # ------------------------------------------------------------------ import
    def from_hf(self, hf_state_dict: Dict[str, Any]) -> Dict[str, Any]:
        a = self.model_args
        hf = hf_state_dict
        if "model.embed_tokens.weight" in hf or any(re.search(r"_proj\.weight$", k) for k in hf):
            raise ValueError("a merged (dense) checkpoint cannot be split back into shared base blocks and "
                             "per-layer LoRA adapters; from_hf takes the lossless layout (to_hf(sd))")
        out: Dict[str, Any] = {}
        for b in range(a.n_unique_blocks):
            layers = self._layers_of(b)
            if not layers:
                raise ValueError(f"block {b} is used by no layer")
            base = f"base_blocks.{b}."
            pairs = [(f"{sub}.{ours}.weight", f"{hf_mod}.{hf_name}.base_layer.weight")
                     for ours, sub, hf_mod, hf_name in _PROJ_MAP] + list(_NORM_MAP)
            for ours, hf_name in pairs:
                first = hf[f"model.layers.{layers[0]}.{hf_name}"]
                for l in layers[1:]:
                    other = hf[f"model.layers.{l}.{hf_name}"]
                    if other.shape != first.shape or not torch.equal(other, first):
                        raise ValueError(f"layers {layers[0]} and {l} carry different {hf_name}, but both use "
                                         f"base block {b}: the shared layout cannot represent them")
                out[base + ours] = first
        for l in range(a.n_layers):
            for ours, _, hf_mod, hf_name in _PROJ_MAP:
                key = f"model.layers.{l}.{hf_mod}.{hf_name}"
                out[f"layer_loras.{l}.{ours}.w_a.weight"] = hf[f"{key}.lora_A.weight"]
                out[f"layer_loras.{l}.{ours}.w_b.weight"] = hf[f"{key}.lora_B.weight"]
        out["tok_embeddings.emb"] = hf["model.embed_tokens.emb_factor"]
        out["tok_embeddings.proj.weight"] = hf["model.embed_tokens.proj_factor"]
        out["norm.weight"] = hf["model.norm.weight"]
        return out
