"""CPU checks of the weight-shared Qwen3 oracle (oracle/qwen3_ref.py) and of the model's
host-side structure (parameter names, block map), on a tiny configuration.

The oracle's full-sequence forward is compared with an independent float64 restatement
written with explicit loops (causal attention, GQA head mapping, RMSNorm, complex-number
RoPE), so a dropped scale, a wrong mask or a transposed head mapping fails here."""
import math

import numpy as np
import pytest
import torch

from oracle import lora_oracle as O
from oracle import qwen3_ref as Q
from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3, SharedQwen3Args


def tiny_args(**kw):
    a = SharedQwen3Args(dim=32, n_layers=4, n_unique_blocks=2, n_heads=4, n_kv_heads=2, head_dim=8,
                        hidden_dim=48, vocab_size=50, embed_rank=16, lora_rank=4, max_seq_len=16)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def tiny_params(a, seed=0):
    """State dict of the product model's parameter names, filled on the CPU."""
    with torch.device("meta"):
        m = SharedQwen3(a)
    g = torch.Generator().manual_seed(seed)
    p = {}
    for name, t in m.named_parameters():
        if name.endswith("norm.weight"):
            p[name] = 1.0 + 0.1 * torch.randn(t.shape, generator=g)
        else:
            p[name] = torch.randn(t.shape, generator=g) * 0.2
    return p


# ------------------------------------------------------------------ RoPE
def test_rope_identity_at_position_zero():
    rc = Q.rope_cache(8, 4, 1e6)
    assert torch.equal(rc[0, :8], torch.ones(8))
    assert torch.equal(rc[0, 8:], torch.zeros(8))


def test_rope_is_the_complex_rotation_of_half_pairs():
    hd, s, theta = 8, 5, 1e4
    x = torch.randn(1, s, 3, hd, dtype=torch.float64)
    y = Q._rope(x.float(), Q.rope_cache(hd, s, theta)).double()
    h = hd // 2
    for t in range(s):
        for i in range(h):
            ang = t * theta ** (-2.0 * i / hd)
            z = (x[0, t, :, i].numpy() + 1j * x[0, t, :, i + h].numpy()) * np.exp(1j * ang)
            np.testing.assert_allclose(y[0, t, :, i].numpy(), np.real(z), rtol=1e-5, atol=1e-5)
            np.testing.assert_allclose(y[0, t, :, i + h].numpy(), np.imag(z), rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ block map
@pytest.mark.parametrize("block_map", ["cyclic", "contiguous"])
def test_block_map_matches_oracle_and_uses_each_block_equally(block_map):
    a = SharedQwen3Args(n_layers=28, n_unique_blocks=4, block_map=block_map)
    got = [a.block_of(l) for l in range(28)]
    assert got == [Q.block_of(l, 28, 4, block_map) for l in range(28)]
    assert sorted(got.count(b) for b in range(4)) == [7, 7, 7, 7]
    if block_map == "cyclic":
        assert got[:5] == [0, 1, 2, 3, 0]
    else:
        assert got[:8] == [0] * 7 + [1]


def test_model_parameter_names_cover_what_the_oracle_reads():
    a = tiny_args()
    p = tiny_params(a)
    assert p["tok_embeddings.emb"].shape == (50, 16)
    assert p["tok_embeddings.proj.weight"].shape == (32, 16)
    for l in range(a.n_layers):
        for name, (out, inp) in a.proj_shapes().items():
            assert p[f"layer_loras.{l}.{name}.w_a.weight"].shape == (4, inp)
            assert p[f"layer_loras.{l}.{name}.w_b.weight"].shape == (out, 4)
    for b in range(a.n_unique_blocks):
        assert p[f"base_blocks.{b}.attention.wq.weight"].shape == (32, 32)
        assert p[f"base_blocks.{b}.feed_forward.w2.weight"].shape == (32, 48)
    # exactly n_unique_blocks base sets, n_layers adapter sets
    assert not any(k.startswith(f"base_blocks.{a.n_unique_blocks}.") for k in p)


# ------------------------------------------------------------------ forward
def explicit_forward(p, a, tokens):
    """float64 loops: embedding gather + projection, per layer pre-norm attention with
    q/k RMSNorm, RoPE as complex rotation, GQA (query head h reads kv head h // rep),
    causal softmax(q.k / sqrt(hd)) v, SwiGLU, tied head."""
    d = {k: v.double().numpy() for k, v in p.items()}
    b, s = tokens.shape
    E, P = d["tok_embeddings.emb"], d["tok_embeddings.proj.weight"]
    h = np.stack([[E[t] @ P.T for t in row] for row in tokens.tolist()])  # [b, s, dim]

    def rms(x, w):
        return x / np.sqrt((x * x).mean(-1, keepdims=True) + a.norm_eps) * w

    def rope(v, t):
        hd = v.shape[-1]
        half = hd // 2
        out = v.copy()
        for i in range(half):
            ang = t * a.rope_theta ** (-2.0 * i / hd)
            c, sn = math.cos(ang), math.sin(ang)
            out[..., i] = v[..., i] * c - v[..., i + half] * sn
            out[..., i + half] = v[..., i] * sn + v[..., i + half] * c
        return out

    sc = 2.0 if a.lora_scale is None else a.lora_scale
    rep = a.n_heads // a.n_kv_heads
    for l in range(a.n_layers):
        bb = Q.block_of(l, a.n_layers, a.n_unique_blocks, a.block_map)
        pre, lp = f"base_blocks.{bb}.", f"layer_loras.{l}."

        def proj(x, name, sub):
            return O.lora_linear(x.reshape(-1, x.shape[-1]), d[f"{pre}{sub}.{name}.weight"],
                                 d[f"{lp}{name}.w_a.weight"], d[f"{lp}{name}.w_b.weight"], sc
                                 ).reshape(*x.shape[:-1], -1)

        x = rms(h, d[pre + "attention_norm.weight"])
        q = proj(x, "wq", "attention").reshape(b, s, a.n_heads, a.head_dim)
        k = proj(x, "wk", "attention").reshape(b, s, a.n_kv_heads, a.head_dim)
        v = proj(x, "wv", "attention").reshape(b, s, a.n_kv_heads, a.head_dim)
        q = rms(q, d[pre + "attention.q_norm.weight"])
        k = rms(k, d[pre + "attention.k_norm.weight"])
        for t in range(s):
            q[:, t] = rope(q[:, t], t)
            k[:, t] = rope(k[:, t], t)
        o = np.zeros_like(q)
        for bi in range(b):
            for hq in range(a.n_heads):
                hk = hq // rep
                for t in range(s):
                    sco = np.array([q[bi, t, hq] @ k[bi, u, hk] for u in range(t + 1)]) / math.sqrt(a.head_dim)
                    w = np.exp(sco - sco.max())
                    w /= w.sum()
                    o[bi, t, hq] = sum(w[u] * v[bi, u, hk] for u in range(t + 1))
        h = h + proj(o.reshape(b, s, -1), "wo", "attention")
        x = rms(h, d[pre + "ffn_norm.weight"])
        g = proj(x, "w1", "feed_forward")
        u = proj(x, "w3", "feed_forward")
        h = h + proj(g / (1.0 + np.exp(-g)) * u, "w2", "feed_forward")
    h = rms(h, d["norm.weight"])
    return (h @ P) @ E.T


@pytest.mark.parametrize("block_map", ["cyclic", "contiguous"])
def test_reference_forward_equals_explicit_restatement(block_map):
    a = tiny_args(block_map=block_map)
    p = tiny_params(a, seed=1)
    tokens = torch.tensor([[3, 17, 42, 5], [49, 0, 8, 8]])
    got = Q.reference_forward(p, a, tokens).double().numpy()
    want = explicit_forward(p, a, tokens)
    np.testing.assert_allclose(got, want, rtol=2e-4, atol=2e-4 * np.abs(want).max())


def test_reference_forward_is_causal():
    a = tiny_args()
    p = tiny_params(a, seed=2)
    toks = torch.tensor([[1, 2, 3, 4, 5]])
    full = Q.reference_forward(p, a, toks)
    for s in (1, 3):
        part = Q.reference_forward(p, a, toks[:, :s])
        torch.testing.assert_close(full[:, :s], part, rtol=1e-5, atol=1e-5)


def test_lora_scale_enters_linearly():
    # With the LoRA scale set to 0 the forward equals the forward with every B zeroed.
    a = tiny_args(lora_scale=0.0)
    p = tiny_params(a, seed=3)
    toks = torch.tensor([[7, 9, 11]])
    p0 = {k: (torch.zeros_like(v) if k.endswith("w_b.weight") else v) for k, v in p.items()}
    torch.testing.assert_close(Q.reference_forward(p, a, toks), Q.reference_forward(p0, tiny_args(), toks))


def test_reference_generate_is_greedy_over_full_prefix():
    a = tiny_args()
    p = tiny_params(a, seed=4)
    prompt = torch.tensor([[4, 8, 15], [16, 23, 42]])
    new = Q.reference_generate(p, a, prompt, 3)
    assert new.shape == (2, 3)
    toks = prompt
    for i in range(3):
        nxt = Q.reference_forward(p, a, toks)[:, -1].argmax(-1)
        assert torch.equal(new[:, i], nxt)
        toks = torch.cat([toks, nxt[:, None]], 1)
