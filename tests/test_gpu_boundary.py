"""The torch-facing boundary on the GPU: autocast rules registered on the ops (called
directly through torch.ops.wsl.*), and the decode-step kernels' guard for a position past
the cache (forced from the host: the kernels exit normally, write NaN outputs and leave
the cache untouched)."""
import sys

import numpy as np
import pytest
import torch

from oracle import lora_oracle as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_autocast_on_the_op_itself(gpu):
    """torch.ops.wsl.lora_linear with fp32 operands inside torch.autocast("cuda", bf16): the
    op's own autocast rule casts them (the reference's AMP path,
    torchtitan/distributed/utils.py:219-239), and the result is the bf16 call's, bit for bit."""
    _say("[autocast] lora_linear fp32 operands")
    g = torch.Generator().manual_seed(3)
    M, N, K, r = 96, 512, 256, 16
    x = torch.randn(M, K, generator=g).to(gpu)
    W = (torch.randn(N, K, generator=g) * 0.02).to(gpu)
    A = (torch.randn(r, K, generator=g) * 0.02).to(gpu)
    B = (torch.randn(N, r, generator=g) * 0.02).to(gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = torch.ops.wsl.lora_linear(x, W, None, A, B, 2.0)
    want = torch.ops.wsl.lora_linear(x.bfloat16(), W.bfloat16(), None, A.bfloat16(), B.bfloat16(), 2.0)
    assert y.dtype == torch.bfloat16
    assert torch.equal(y, want)
    ref = O.lora_linear(x.bfloat16().float().cpu().numpy(), W.bfloat16().float().cpu().numpy(),
                        A.bfloat16().float().cpu().numpy(), B.bfloat16().float().cpu().numpy(), 2.0)
    assert O.max_rel_err(y.float().cpu().numpy(), ref) <= 1e-2
    with pytest.raises(TypeError):  # outside autocast an fp32 x is refused
        torch.ops.wsl.lora_linear(x, W.bfloat16(), None, None, None, 0.0)


def test_autocast_keeps_fp8_base_and_scale(gpu):
    from weightshared_torchtitan_amd import quantize_fp8_per_channel
    _say("[autocast] fp8 base")
    g = torch.Generator().manual_seed(4)
    M, N, K = 8, 256, 512
    x = torch.randn(M, K, generator=g).to(gpu)
    q, sc = quantize_fp8_per_channel(torch.randn(N, K, generator=g) * 0.02)
    q, sc = q.to(gpu), sc.to(gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = torch.ops.wsl.lora_linear(x, q, sc, None, None, 0.0)
    assert torch.equal(y, torch.ops.wsl.lora_linear(x.bfloat16(), q, sc, None, None, 0.0))


def test_autocast_factorized_embedding(gpu):
    _say("[autocast] factorized_embedding")
    g = torch.Generator().manual_seed(5)
    E = (torch.randn(1000, 64, generator=g) * 0.1).to(gpu)
    P = (torch.randn(256, 64, generator=g) * 0.1).to(gpu)
    ids = torch.randint(0, 1000, (3, 7), generator=g).to(gpu)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = torch.ops.wsl.factorized_embedding(ids, E, P)
    assert torch.equal(out, torch.ops.wsl.factorized_embedding(ids, E.bfloat16(), P.bfloat16()))


@pytest.mark.parametrize("fused", [True, False])
def test_position_past_the_cache_writes_nothing(gpu, fused):
    """pos = cache_len (a device value the host does not read): the attention kernels return
    NaN outputs and leave the cache untouched, instead of reading and writing past it."""
    from weightshared_torchtitan_amd import ops
    _say(f"[pos guard] fused={fused}")
    b, nh, nkv, hd, L = 2, 8, 4, 128, 64
    g = torch.Generator().manual_seed(6)
    qkv = torch.randn(b, (nh + 2 * nkv) * hd, generator=g).bfloat16().to(gpu)
    kc = torch.randn(b, nkv, L, hd, generator=g).bfloat16().to(gpu)
    vc = torch.randn(b, nkv, L, hd, generator=g).bfloat16().to(gpu)
    k0, v0 = kc.clone(), vc.clone()
    ones = torch.ones(hd, dtype=torch.bfloat16, device=gpu)
    rope = torch.zeros(L, 2 * hd, device=gpu)
    rope[:, :hd] = 1.0
    pos = torch.full((), L, dtype=torch.int64, device=gpu)
    if fused:
        out = ops.decode_attention_step_op(qkv, ones, ones, 1e-6, rope, pos, kc, vc, nh, nkv, hd ** -0.5)
    else:
        q = ops.qk_norm_rope_op(qkv, ones, ones, 1e-6, rope, pos, kc, vc, nh, nkv)
        assert bool(torch.isnan(q.float()).all())
        out = ops.decode_attention_op(q, kc, vc, pos, hd ** -0.5)
    torch.cuda.synchronize()
    assert bool(torch.isnan(out.float()).all())
    assert torch.equal(kc, k0) and torch.equal(vc, v0)
    # and the last valid position still works after it
    pos.fill_(L - 1)
    out = ops.decode_attention_step_op(qkv, ones, ones, 1e-6, rope, pos, kc, vc, nh, nkv, hd ** -0.5)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
