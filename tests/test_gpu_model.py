"""The weight-shared Qwen3 model on the GPU against the CPU oracle (oracle/qwen3_ref.py)
on a small configuration whose shapes reach the prefill, decode and embedding kernels.

Whole-model bf16 logits are compared with the fp32 oracle by max|d| / max|ref|. Greedy
tokens are checked step by step against the oracle's no-cache forward of the same prefix
(scripts/generate/_generation.py:43 re-runs the prefix): the model's token must be one
whose oracle logit is within the bf16 tolerance of the oracle's maximum, so near-ties do
not make the test flaky and a wrong cache or position fails it."""
import pytest
import torch

from oracle import qwen3_ref as Q

pytestmark = pytest.mark.gpu

LOGIT_TOL = 3e-2  # whole-model bf16 vs fp32, max|d| / max|ref|


def small_args():
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3Args
    return SharedQwen3Args(dim=256, n_layers=4, n_unique_blocks=2, n_heads=4, n_kv_heads=2, head_dim=64,
                           hidden_dim=512, vocab_size=1000, embed_rank=64, lora_rank=16, max_seq_len=128)


def build(gpu, seed=0):
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3
    a = small_args()
    m = SharedQwen3(a)
    m.init_random(seed=seed, std=0.05)
    m = m.to(gpu).to(torch.bfloat16)
    p = {k: v.detach().float().cpu() for k, v in m.named_parameters()}
    return a, m, p


def rel(x, ref):
    return ((x.float().cpu() - ref).abs().max() / ref.abs().max()).item()


@pytest.mark.parametrize("seq", [12, 40])  # M = 24 (decode kernels) and 80 (prefill kernels)
def test_forward_logits_match_oracle(gpu, seq):
    a, m, p = build(gpu, seed=1)
    g = torch.Generator().manual_seed(seq)
    toks = torch.randint(0, a.vocab_size, (2, seq), generator=g)
    with torch.no_grad():
        got = m(toks.to(gpu))
    ref = Q.reference_forward(p, a, toks)
    assert rel(got, ref) <= LOGIT_TOL


def test_cached_decode_matches_no_cache_greedy(gpu):
    a, m, p = build(gpu, seed=2)
    g = torch.Generator().manual_seed(5)
    prompt = torch.randint(0, a.vocab_size, (2, 9), generator=g)
    n_new = 6
    with torch.no_grad():
        new, _ = m.generate(prompt.to(gpu), n_new, use_graph=True)
    new = new.cpu()
    toks = prompt
    for i in range(n_new):
        ref = Q.reference_forward(p, a, toks)[:, -1]  # [b, vocab]
        tol = LOGIT_TOL * ref.abs().max(dim=-1).values
        chosen = ref.gather(1, new[:, i:i + 1])[:, 0]
        assert bool((chosen >= ref.max(dim=-1).values - tol).all()), f"step {i}"
        toks = torch.cat([toks, new[:, i:i + 1]], 1)


def test_decode_step_logits_match_oracle(gpu):
    # One cached step (graph-free) against the oracle's full-prefix forward.
    from weightshared_torchtitan_amd.qwen3_shared import KVCache
    a, m, p = build(gpu, seed=3)
    g = torch.Generator().manual_seed(6)
    toks = torch.randint(0, a.vocab_size, (2, 11), generator=g)
    cache = KVCache(a, 2, 16, gpu)
    with torch.no_grad():
        m(toks[:, :10].to(gpu), cache)
        pos = torch.full((), 10, dtype=torch.int64, device=gpu)
        got = m.decode_step(toks[:, 10:11].to(gpu), pos, cache)
    ref = Q.reference_forward(p, a, toks)[:, -1]
    assert rel(got, ref) <= LOGIT_TOL


def fused_args():
    """A configuration the fused decode-step launches cover (K >= 1024 on every projection)."""
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3Args
    return SharedQwen3Args(dim=1024, n_layers=4, n_unique_blocks=2, n_heads=8, n_kv_heads=4, head_dim=128,
                           hidden_dim=2048, vocab_size=1000, embed_rank=64, lora_rank=16, max_seq_len=64)


def test_fused_decode_step_matches_oracle_and_unfused(gpu):
    from weightshared_torchtitan_amd.qwen3_shared import KVCache, SharedQwen3
    a = fused_args()
    m = SharedQwen3(a)
    m.init_random(seed=4, std=0.03)
    m = m.to(gpu).to(torch.bfloat16)
    p = {k: v.detach().float().cpu() for k, v in m.named_parameters()}
    g = torch.Generator().manual_seed(8)
    toks = torch.randint(0, a.vocab_size, (2, 11), generator=g)
    plan = m._fusion_plan(2, m._decode_pack())
    assert plan["on"], "the fused launches should cover this configuration"
    outs = {}
    for mode in ("fused", "separate"):
        m.decode_fusion = mode != "separate"
        cache = KVCache(a, 2, 16, gpu)
        with torch.no_grad():
            m(toks[:, :10].to(gpu), cache)
            pos = torch.full((), 10, dtype=torch.int64, device=gpu)
            outs[mode] = m.decode_step(toks[:, 10:11].to(gpu), pos, cache)
    m.decode_fusion = True
    ref = Q.reference_forward(p, a, toks)[:, -1]
    assert rel(outs["fused"], ref) <= LOGIT_TOL
    assert rel(outs["fused"], outs["separate"].float().cpu()) <= LOGIT_TOL


def test_fused_decode_graph_greedy_matches_oracle(gpu):
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3
    a = fused_args()
    m = SharedQwen3(a)
    m.init_random(seed=5, std=0.03)
    m = m.to(gpu).to(torch.bfloat16)
    p = {k: v.detach().float().cpu() for k, v in m.named_parameters()}
    g = torch.Generator().manual_seed(9)
    prompt = torch.randint(0, a.vocab_size, (2, 7), generator=g)
    n_new = 5
    with torch.no_grad():
        new, _ = m.generate(prompt.to(gpu), n_new, use_graph=True)
    new = new.cpu()
    toks = prompt
    for i in range(n_new):
        ref = Q.reference_forward(p, a, toks)[:, -1]
        tol = LOGIT_TOL * ref.abs().max(dim=-1).values
        chosen = ref.gather(1, new[:, i:i + 1])[:, 0]
        assert bool((chosen >= ref.max(dim=-1).values - tol).all()), f"step {i}"
        toks = torch.cat([toks, new[:, i:i + 1]], 1)


def test_greedy_tokens_with_and_without_the_fused_head(gpu):
    """generate() with the head fused into the argmax (no logits written) picks the same tokens
    as with the unfused head + separate argmax, step for step (the fused config covers it)."""
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3
    from weightshared_torchtitan_amd import ops
    a = fused_args()
    a.embed_rank = 256
    a.vocab_size = 40000
    m = SharedQwen3(a)
    m.init_random(seed=11, std=0.03)
    m = m.to(gpu).to(torch.bfloat16)
    assert ops.tied_head_argmax_supported(2, a.vocab_size, a.embed_rank)
    g = torch.Generator().manual_seed(12)
    prompt = torch.randint(0, a.vocab_size, (2, 9), generator=g).to(gpu)
    with torch.no_grad():
        m.head_argmax_fusion = True
        fused, _ = m.generate(prompt, 6, use_graph=True)
        m.head_argmax_fusion = False
        plain, _ = m.generate(prompt, 6, use_graph=True)
        m.head_argmax_fusion = True
    assert torch.equal(fused, plain)


@pytest.mark.parametrize("seq", [12, 40, 100])
def test_grouped_prefill_matches_per_projection(gpu, seq):
    """Inference prefill with q|k|v and gate|up as grouped launches gives the same logits,
    bit for bit, as one launch per projection (each group's block is the single op's)."""
    a, m, p = build(gpu, seed=2)
    g = torch.Generator().manual_seed(100 + seq)
    toks = torch.randint(0, a.vocab_size, (2, seq), generator=g).to(gpu)
    with torch.no_grad():
        m.prefill_grouped = True
        grouped = m(toks)
        m.prefill_grouped = False
        single = m(toks)
    assert torch.equal(grouped, single)
    ref = Q.reference_forward(p, a, toks.cpu())
    assert rel(grouped, ref) <= LOGIT_TOL
