"""Config 4 at its real size on the GPU: the weight-shared Qwen3-0.6B decoder (28 layers
from 4 cyclic blocks, 16/8 heads of 128, hidden 1024, SwiGLU 3072, vocab 151936 through a
rank-256 factorized embedding with tied output, rank-32 LoRA on every projection), a
batch-8, 512-token random prompt, greedy decoding through the HIP-graph decode step.

The reference re-runs the whole prefix every step (scripts/generate/_generation.py:43,
69-78), so the full-prefix forward is the oracle:
- two of the eight sequences go through the fp32 CPU oracle (oracle/qwen3_ref.py) over the
  prompt and the generated tokens; every generated token must be one whose oracle logit is
  within the bf16 tolerance of the oracle's maximum at its position (near-ties do not make
  the test flaky; a wrong cache slot, position or head fails it);
- for all eight, the logits the graph-replayed decode steps chose from must match the GPU
  full-prefix forward of the same tokens (no KV cache) within the same tolerance."""
import sys
import time

import pytest
import torch

from oracle import qwen3_ref as Q

pytestmark = pytest.mark.gpu

LOGIT_TOL = 3e-2  # whole-model bf16 vs fp32, max|d| / max|ref|
N_NEW = 4


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def c4(gpu):
    from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3, qwen3_0p6b_shared
    a = qwen3_0p6b_shared()
    assert (a.n_layers, a.n_unique_blocks, a.n_heads, a.n_kv_heads, a.head_dim, a.dim, a.hidden_dim,
            a.vocab_size, a.embed_rank, a.lora_rank) == (28, 4, 16, 8, 128, 1024, 3072, 151936, 256, 32)
    m = SharedQwen3(a)
    m.init_random(seed=4)
    m = m.to(gpu).to(torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, a.vocab_size, (8, 512), generator=g)
    _say("[c4] generate b=8 s=512 n_new=4 (graph)")
    with torch.no_grad():
        new, res = m.generate(prompt.to(gpu), N_NEW, use_graph=True, return_logits=True)
    torch.cuda.synchronize()
    return a, m, prompt, new.cpu(), res["logits"]


def test_c4_graph_steps_match_gpu_full_prefix(gpu, c4):
    a, m, prompt, new, logits = c4
    toks = torch.cat([prompt, new[:, :N_NEW - 1]], 1).to(gpu)
    _say("[c4] GPU full-prefix forward, 8 x 515")
    with torch.no_grad():
        full = m(toks)  # no KV cache: every position recomputed
    for i in range(N_NEW):
        ref = full[:, 511 + i].float()
        got = logits[:, i].float()
        err = ((got - ref).abs().max() / ref.abs().max()).item()
        assert err <= LOGIT_TOL, f"step {i}: {err}"
        assert torch.equal(new[:, i].to(gpu), got.argmax(-1)), f"step {i}: token is not the argmax of its logits"


def test_c4_greedy_tokens_match_cpu_oracle(c4):
    a, m, prompt, new, _ = c4
    p = {k: v.detach().float().cpu() for k, v in m.named_parameters()}
    seqs = [0, 5]
    toks = torch.cat([prompt[seqs], new[seqs, :N_NEW - 1]], 1)
    torch.set_num_threads(max(1, min(16, torch.get_num_threads())))
    t0 = time.time()
    _say(f"[c4] CPU oracle forward, {len(seqs)} x {toks.shape[1]}")
    with torch.no_grad():
        ref = Q.reference_forward(p, a, toks)  # [2, 515, vocab] fp32
    _say(f"[c4] oracle done in {time.time() - t0:.1f} s")
    for i in range(N_NEW):
        r = ref[:, 511 + i]
        tol = LOGIT_TOL * r.abs().max(dim=-1).values
        chosen = r.gather(1, new[seqs, i:i + 1])[:, 0]
        assert bool((chosen >= r.max(dim=-1).values - tol).all()), f"step {i}"


def test_c4_chain_decode_equals_separate_launches(gpu, c4):
    """The same generation with the decode step's chains (one launch for each layer's o,
    gate|up, down and the next layer's q|k|v): the chains compute what the separate fused
    launches do bit for bit, so the tokens and the logits they were chosen from are equal."""
    from weightshared_torchtitan_amd import ops
    a, m, prompt, new, logits = c4
    _say("[c4] generate with chains")
    m.decode_chain = True
    try:
        with torch.no_grad():
            new2, res = m.generate(prompt.to(gpu), N_NEW, use_graph=True, return_logits=True)
        torch.cuda.synchronize()
        assert not ops.chain_status(gpu)
    finally:
        m.decode_chain = False
    assert torch.equal(new2.cpu(), new)
    assert torch.equal(res["logits"], logits)
