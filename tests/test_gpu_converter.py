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
