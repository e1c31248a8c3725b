"""CPU round trips of the weight-shared Qwen3 state-dict adapter (on-disk layout)."""
import pytest
import torch

from oracle import qwen3_ref as Q
from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3, SharedQwen3Args
from weightshared_torchtitan_amd.state_dict_adapter import SharedQwen3StateDictAdapter


def tiny_args(**kw):
    a = SharedQwen3Args(dim=32, n_layers=6, n_unique_blocks=2, n_heads=4, n_kv_heads=2, head_dim=8,
                        hidden_dim=48, vocab_size=50, embed_rank=16, lora_rank=4, max_seq_len=16)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def model_of(a, seed=0):
    m = SharedQwen3(a)  # construction only: no op runs on the CPU
    m.init_random(seed=seed, std=0.2)
    with torch.no_grad():
        g = torch.Generator().manual_seed(seed + 1)
        for n, p in m.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
    return m


@pytest.mark.parametrize("block_map", ["cyclic", "contiguous"])
def test_lossless_round_trip(block_map):
    a = tiny_args(block_map=block_map)
    m = model_of(a)
    ad = SharedQwen3StateDictAdapter(a)
    sd = m.state_dict()
    hf = ad.to_hf(sd)
    # a flat per-layer layout: every layer carries its block's base weights and its own adapters
    assert "model.layers.5.self_attn.q_proj.base_layer.weight" in hf
    assert "model.layers.5.mlp.down_proj.lora_B.weight" in hf
    assert not any(k.startswith(("base_blocks", "layer_loras")) for k in hf)
    b5 = a.block_of(5)
    assert torch.equal(hf["model.layers.5.self_attn.q_proj.base_layer.weight"],
                       sd[f"base_blocks.{b5}.attention.wq.weight"])
    assert torch.equal(hf["model.layers.5.post_attention_layernorm.weight"], sd[f"base_blocks.{b5}.ffn_norm.weight"])
    back = ad.from_hf(hf)
    assert set(back) == set(sd)
    for k in sd:
        assert torch.equal(back[k], sd[k]), k
    m2 = SharedQwen3(a)
    m2.load_state_dict(back, strict=True)


def test_from_hf_rejects_unshared_bases():
    a = tiny_args()
    ad = SharedQwen3StateDictAdapter(a)
    hf = ad.to_hf(model_of(a).state_dict())
    # layers 0 and 2 share block 0 (cyclic); make layer 2's o_proj base differ
    hf["model.layers.2.self_attn.o_proj.base_layer.weight"] = hf["model.layers.2.self_attn.o_proj.base_layer.weight"] + 1
    with pytest.raises(ValueError, match="base block 0"):
        ad.from_hf(hf)


def test_from_hf_rejects_merged_checkpoints():
    a = tiny_args()
    ad = SharedQwen3StateDictAdapter(a)
    with pytest.raises(ValueError, match="merged"):
        ad.from_hf(ad.to_hf(model_of(a).state_dict(), merged=True))


def test_merged_export_reproduces_the_shared_model():
    """The dense checkpoint, run as a plain Qwen3 (every layer its own block, no adapter, an
    identity embedding projection over the materialised table), gives the shared model's
    logits: the merge W + s B.A, the tied E.P^T table and the per-layer norms are all right
    (a dropped scale or a transposed B.A fails)."""
    a = tiny_args(lora_scale=1.5)
    m = model_of(a, seed=3)
    sd = {k: v.detach().float() for k, v in m.state_dict().items()}
    hf = SharedQwen3StateDictAdapter(a).to_hf(sd, merged=True)
    assert hf["lm_head.weight"] is hf["model.embed_tokens.weight"]
    dense = SharedQwen3Args(**{**a.__dict__, "n_unique_blocks": a.n_layers, "block_map": "cyclic",
                               "embed_rank": a.dim})
    p = {"tok_embeddings.emb": hf["model.embed_tokens.weight"], "tok_embeddings.proj.weight": torch.eye(a.dim),
         "norm.weight": hf["model.norm.weight"]}
    names = {"wq": ("attention", "self_attn.q_proj"), "wk": ("attention", "self_attn.k_proj"),
             "wv": ("attention", "self_attn.v_proj"), "wo": ("attention", "self_attn.o_proj"),
             "w1": ("feed_forward", "mlp.gate_proj"), "w3": ("feed_forward", "mlp.up_proj"),
             "w2": ("feed_forward", "mlp.down_proj")}
    for l in range(a.n_layers):
        for ours, (sub, hfn) in names.items():
            W = hf[f"model.layers.{l}.{hfn}.weight"]
            p[f"base_blocks.{l}.{sub}.{ours}.weight"] = W
            p[f"layer_loras.{l}.{ours}.w_a.weight"] = torch.zeros(a.lora_rank, W.shape[1])
            p[f"layer_loras.{l}.{ours}.w_b.weight"] = torch.zeros(W.shape[0], a.lora_rank)
        p[f"base_blocks.{l}.attention.q_norm.weight"] = hf[f"model.layers.{l}.self_attn.q_norm.weight"]
        p[f"base_blocks.{l}.attention.k_norm.weight"] = hf[f"model.layers.{l}.self_attn.k_norm.weight"]
        p[f"base_blocks.{l}.attention_norm.weight"] = hf[f"model.layers.{l}.input_layernorm.weight"]
        p[f"base_blocks.{l}.ffn_norm.weight"] = hf[f"model.layers.{l}.post_attention_layernorm.weight"]
    toks = torch.randint(0, a.vocab_size, (2, 9), generator=torch.Generator().manual_seed(5))
    ref = Q.reference_forward(sd, a, toks)
    got = Q.reference_forward(p, dense, toks)
    assert (got - ref).abs().max() <= 1e-4 * ref.abs().max()
    # and the scale matters: merged with the wrong scale does not match
    bad = SharedQwen3StateDictAdapter(tiny_args(lora_scale=2.0)).to_hf(sd, merged=True)
    assert not torch.allclose(bad["model.layers.0.self_attn.q_proj.weight"],
                              hf["model.layers.0.self_attn.q_proj.weight"])
