"""The wsl_lora converter on the GPU: a converted reference-style block gives the outputs
and gradients of the unconverted one (plain torch, fp32 on the CPU), to the bf16 bar."""
import copy

import pytest
import torch

from oracle import lora_oracle as O
from tests._ref_style import RefAttentionProjections

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def test_converted_block_matches_reference_forward_and_backward(gpu):
    from weightshared_torchtitan_amd import converter as C
    print("[converter] reference-style block, fused q pair + converted k offset", flush=True)
    torch.manual_seed(3)
    ref = RefAttentionProjections()
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0, 0.02)
    ref = ref.bfloat16()
    x = torch.randn(384, 512).bfloat16()
    gq = torch.randn(384, 512).bfloat16()
    gk = torch.randn(384, 256).bfloat16()
    # the reference in fp32 on the CPU
    ref32 = copy.deepcopy(ref).float()
    x32 = x.float().requires_grad_(True)
    q_ref, k_ref = ref32(x32)
    torch.autograd.backward([q_ref, k_ref], [gq.float(), gk.float()])
    # converted, on the GPU
    model = copy.deepcopy(ref).to(gpu)
    C.WslLoRAConverter().convert(model)
    xg = x.to(gpu).requires_grad_(True)
    q, k = model(xg)
    torch.autograd.backward([q, k], [gq.to(gpu), gk.to(gpu)])
    torch.cuda.synchronize()
    assert O.max_rel_err(q.detach().float().cpu().numpy(), q_ref.detach().numpy()) <= BF16_TOL
    assert O.max_rel_err(k.detach().float().cpu().numpy(), k_ref.detach().numpy()) <= BF16_TOL
    assert O.max_rel_err(xg.grad.float().cpu().numpy(), x32.grad.numpy()) <= BF16_TOL
    ref_params = dict(ref32.named_parameters())
    for n, p in model.named_parameters():
        assert p.grad is not None, n
        err = O.max_rel_err(p.grad.float().cpu().numpy(), ref_params[n].grad.numpy())
        assert err <= BF16_TOL, (n, err)


SHARING_MODES = [
    ("default", dict()),
    ("head_sharing g=2", dict(head_sharing=True, grouping=2)),           # the reference's 40M preset
    ("qkv_sharing [q,k,v]", dict(qkv_sharing=[["q", "k", "v"]])),
    ("qkv_sharing [q,k],[v] + head_sharing g=4", dict(qkv_sharing=[["q", "k"], ["v"]], head_sharing=True,
                                                       grouping=4)),
    ("two_step", dict(two_step=True)),
    ("two_step + qkv_sharing [q,k,v]", dict(two_step=True, qkv_sharing=[["q", "k", "v"]])),
    ("two_step + qkv_sharing [q,k],[v] + head_sharing g=4", dict(two_step=True, qkv_sharing=[["q", "k"], ["v"]],
                                                                   head_sharing=True, grouping=4)),
]


@pytest.mark.parametrize("mode,kw", SHARING_MODES, ids=[m for m, _ in SHARING_MODES])
@pytest.mark.parametrize("M", [384, 24])  # prefill and decode paths
def test_sharing_modes_match_reference_forward_and_backward(gpu, mode, kw, M):
    """Each sharing switch of the reference's attention (tests/_ref_style.RefSharedAttention,
    40M dims: dim 512, 16 heads of 32, 8 kv heads, rank 8): the converted block's q, k, v and
    every gradient match the unconverted block in fp32 on the CPU."""
    import tests._ref_style as R
    from weightshared_torchtitan_amd import converter as C
    print(f"[converter] {mode} M={M}", flush=True)
    torch.manual_seed(7)
    ref = R.RefSharedAttention(**kw)
    with torch.no_grad():
        for p in ref.parameters():
            p.normal_(0, 0.05)
    ref = ref.bfloat16()
    x = torch.randn(M, 512).bfloat16()
    ref32 = copy.deepcopy(ref).float()
    x32 = x.float().requires_grad_(True)
    outs_ref = ref32(x32)
    grads = [torch.randn_like(o).bfloat16() for o in outs_ref]
    torch.autograd.backward(list(outs_ref), [g.float() for g in grads])
    model = copy.deepcopy(ref).to(gpu)
    conv = C.WslLoRAConverter()
    conv.convert(model)
    assert len(conv.fused) == (4 if kw.get("two_step") else 3)  # two_step: head_offset and 3 only-offsets
    assert conv.converted == []
    xg = x.to(gpu).requires_grad_(True)
    outs = model(xg)
    torch.autograd.backward(list(outs), [g.to(gpu) for g in grads])
    torch.cuda.synchronize()
    for o, o_ref in zip(outs, outs_ref):
        assert O.max_rel_err(o.detach().float().cpu().numpy(), o_ref.detach().numpy()) <= BF16_TOL
    assert O.max_rel_err(xg.grad.float().cpu().numpy(), x32.grad.numpy()) <= BF16_TOL
    ref_params = dict(ref32.named_parameters())
    for n, p in model.named_parameters():
        assert p.grad is not None, n
        err = O.max_rel_err(p.grad.float().cpu().numpy(), ref_params[n].grad.numpy())
        assert err <= BF16_TOL, (mode, n, err)


@pytest.mark.parametrize("mode,kw,launches", [
    ("head_sharing g=2", dict(head_sharing=True, grouping=2), 3),
    ("qkv_sharing [q,k,v]", dict(qkv_sharing=[["q", "k", "v"]]), 1),
    ("two_step", dict(two_step=True), 3),
    ("two_step + qkv_sharing [q,k,v]", dict(two_step=True, qkv_sharing=[["q", "k", "v"]]), 1),
])
def test_converted_projections_are_one_launch_each(gpu, mode, kw, launches):
    """Inference forward of a converted block: one fused-LoRA kernel per projection (one per
    shared q/k/v group) and nothing else on the device: no separate base, delta, expand or
    add kernels."""
    import tests._ref_style as R
    from torch.profiler import ProfilerActivity, profile
    from weightshared_torchtitan_amd import converter as C
    print(f"[converter launches] {mode}", flush=True)
    torch.manual_seed(8)
    model = R.RefSharedAttention(**kw).bfloat16().to(gpu)
    C.WslLoRAConverter().convert(model)
    x = torch.randn(384, 512, device=gpu).bfloat16()
    with torch.no_grad():
        model(x)  # warm-up: workspaces, stacked factors
        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            model(x)
            torch.cuda.synchronize()
    kernels = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    if not kernels:
        pytest.skip("the profiler recorded no device activity on this build")
    wsl = [k for k in kernels if "wsl::" in k]
    assert len(wsl) == launches, kernels
    assert len(kernels) == launches, kernels


@pytest.mark.parametrize("M,N,K,r,base_n,g,G,fp8", [
    (384, 512, 512, 8, 64, 2, 1, False),     # q of the 40M head-sharing preset (prefill path)
    (24, 256, 512, 8, 32, 2, 1, False),      # k of the same (decode path), 16-wide templates
    (256, 1024, 1024, 16, 1024, 1, 3, False),  # one base for q, k, v
    (200, 512, 520, 8, 128, 4, 2, False),    # K off the 64 grid: generic path
    (512, 2048, 1024, 32, 512, 4, 3, True),  # fp8 base, shared by 3 groups, 4 templates (fp8 MFMA path)
    (16, 2048, 1024, 32, 512, 4, 3, True),   # the same at decode shape
])
def test_bcast_op_matches_broadcast_add_oracle(gpu, M, N, K, r, base_n, g, G, fp8):
    """wsl::lora_linear_bcast against the float64 oracle of the reference composition
    broadcast_add(x . W^T, s (x . A_j^T) . B_j^T, g) (oracle.broadcast_add, pinned by golden
    vectors), on every path."""
    from weightshared_torchtitan_amd import ops, quantize_fp8_per_channel
    print(f"[bcast] M={M} N={N} K={K} r={r} base_n={base_n} g={g} groups={G} fp8={fp8}", flush=True)
    gen = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=gen).bfloat16()
    Wf = torch.randn(base_n, K, generator=gen) * 0.02
    A = (torch.randn(G * r, K, generator=gen) * 0.02).bfloat16()
    B = (torch.randn(G * N, r, generator=gen) * 0.02).bfloat16()
    if fp8:
        q, sc = quantize_fp8_per_channel(Wf)
        W, ws = q, sc
        Wref = O.dequantize_fp8(q.view(torch.uint8).numpy(), sc.numpy())
    else:
        W, ws = Wf.bfloat16(), None
        Wref = W.float().numpy()
    y = ops.lora_linear_bcast_op(x.to(gpu), W.to(gpu), None if ws is None else ws.to(gpu), A.to(gpu), B.to(gpu),
                                 2.0, g, G).float().cpu().numpy()
    xn, An, Bn = x.float().numpy(), A.float().numpy(), B.float().numpy()
    base = xn.astype("float64") @ Wref.T
    for j in range(G):
        delta = O.lora_delta(xn, An[j * r:(j + 1) * r], Bn[j * N:(j + 1) * N], 2.0)
        ref = O.broadcast_add(base, delta, dim=-1, g=g)
        err = O.max_rel_err(y[:, j * N:(j + 1) * N], ref)
        assert err <= BF16_TOL, (j, err)
