"""The op boundary under the reference's compile and meta-init contract. The reference
compiles every transformer block with torch.compile(..., fullgraph=True)
(torchtitan/models/llama3/infra/parallelize.py:348-357) and builds its model on the meta
device before materialising it (torchtitan/train.py:156-157). Here:

- torch.library.opcheck on wsl::lora_linear, wsl::lora_linear_grouped, wsl::lora_linear_bcast,
  wsl::factorized_embedding and wsl::lora_linear_bwd_input: schema, fake (meta) kernels,
  autograd registration and AOT dispatch, forward and backward;
- a block of LoRALinear projections (grouped q|k|v, o, SwiGLU MLP) under
  torch.compile(fullgraph=True): no graph break, outputs and every gradient equal to eager;
- the same block built on the meta device, materialised with to_empty and initialised, runs
  on the GPU."""
import sys

import pytest
import torch
import torch.nn as nn

import weightshared_torchtitan_amd  # noqa: F401  (registers torch.ops.wsl.*)

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _t(*shape, g, scale=1.0, grad=True, dev="cuda"):
    t = (torch.randn(*shape, generator=g) * scale).bfloat16().to(dev)
    return t.requires_grad_(grad)


OPCHECK_UTILS = ("test_schema", "test_autograd_registration", "test_faketensor", "test_aot_dispatch_dynamic")


@pytest.mark.parametrize("M", [300, 16])  # prefill and decode paths
def test_opcheck_lora_linear(gpu, M):
    _say(f"[opcheck] wsl::lora_linear M={M}")
    g = torch.Generator().manual_seed(M)
    K, N, r = 256, 512, 16
    args = (_t(M, K, g=g), _t(N, K, g=g, scale=0.02), None, _t(r, K, g=g, scale=0.02), _t(N, r, g=g, scale=0.02), 2.0)
    torch.library.opcheck(torch.ops.wsl.lora_linear.default, args, test_utils=OPCHECK_UTILS)
    # the delta alone (the reference's LoRAModule.forward)
    args = (_t(M, K, g=g), None, None, _t(r, K, g=g, scale=0.02), _t(N, r, g=g, scale=0.02), 2.0)
    torch.library.opcheck(torch.ops.wsl.lora_linear.default, args, test_utils=OPCHECK_UTILS)


def test_opcheck_lora_linear_grouped(gpu):
    _say("[opcheck] wsl::lora_linear_grouped")
    g = torch.Generator().manual_seed(2)
    M, K, r, gn = 256, 256, 16, [256, 128, 128]
    N = sum(gn)
    args = (_t(M, K, g=g), _t(N, K, g=g, scale=0.02), None, _t(len(gn) * r, K, g=g, scale=0.02),
            _t(N, r, g=g, scale=0.02), 2.0, gn)
    torch.library.opcheck(torch.ops.wsl.lora_linear_grouped.default, args, test_utils=OPCHECK_UTILS)


def test_opcheck_lora_linear_bcast(gpu):
    _say("[opcheck] wsl::lora_linear_bcast")
    g = torch.Generator().manual_seed(3)
    M, K, N, r, base_n, hs, G = 192, 256, 512, 8, 128, 2, 3
    args = (_t(M, K, g=g), _t(base_n, K, g=g, scale=0.02), None, _t(G * r, K, g=g, scale=0.02),
            _t(G * N, r, g=g, scale=0.02), 2.0, hs, G)
    torch.library.opcheck(torch.ops.wsl.lora_linear_bcast.default, args, test_utils=OPCHECK_UTILS)


def test_opcheck_factorized_embedding(gpu):
    _say("[opcheck] wsl::factorized_embedding")
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 1000, (4, 33), generator=g).to(gpu)
    args = (ids, _t(1000, 64, g=g, grad=False), _t(256, 64, g=g, grad=False))
    torch.library.opcheck(torch.ops.wsl.factorized_embedding.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))


def test_opcheck_lora_linear_bwd_input(gpu):
    """The input-gradient op the backward formulas call (no autograd of its own)."""
    _say("[opcheck] wsl::lora_linear_bwd_input")
    g = torch.Generator().manual_seed(5)
    M, N, K, r = 256, 512, 256, 16
    args = (_t(M, N, g=g, grad=False), _t(N, K, g=g, scale=0.02, grad=False), None,
            _t(r, K, g=g, scale=0.02, grad=False), _t(N, r, g=g, scale=0.02, grad=False), 2.0)
    torch.library.opcheck(torch.ops.wsl.lora_linear_bwd_input.default, args,
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))


class Block(nn.Module):
    """q|k|v as one grouped LoRA linear, o, and a SwiGLU MLP of LoRA linears, with the
    residuals: the projection part of a Qwen3 block (qwen3/model/model.py:184,218,250-251)."""

    def __init__(self, dim=256, qkv=(256, 128, 128), hidden=512, r=16):
        super().__init__()
        from weightshared_torchtitan_amd.lora import LoRALinear, LoRAModule
        self.qkv_n = list(qkv)
        self.wqkv = nn.Linear(dim, sum(qkv), bias=False)
        self.qkv_a = nn.Parameter(torch.empty(len(qkv) * r, dim))
        self.qkv_b = nn.Parameter(torch.empty(sum(qkv), r))
        self.wo = LoRALinear(nn.Linear(qkv[0], dim, bias=False), LoRAModule(qkv[0], dim, r))
        self.w1 = LoRALinear(nn.Linear(dim, hidden, bias=False), LoRAModule(dim, hidden, r))
        self.w3 = LoRALinear(nn.Linear(dim, hidden, bias=False), LoRAModule(dim, hidden, r))
        self.w2 = LoRALinear(nn.Linear(hidden, dim, bias=False), LoRAModule(hidden, dim, r))

    def init(self, seed):
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * 0.05)

    def forward(self, x):
        # the glue between the projections is one elementwise op at a time (each rounds to
        # bf16 once, compiled or not), so compiled and eager differ only in how the backward
        # sums the gradients that fan out of x and h
        from weightshared_torchtitan_amd import ops
        qkv = ops.lora_linear_grouped_op(x, self.wqkv.weight, None, self.qkv_a, self.qkv_b, 2.0, self.qkv_n)
        q, k, v = qkv.split(self.qkv_n, dim=-1)
        h = x + self.wo(q + torch.cat([k, v], -1))
        return h + self.w2(self.w1(h) * self.w3(h))


def _run(model, x, gy):
    y = model(x)
    y.backward(gy)
    grads = {n.removeprefix("_orig_mod."): p.grad.detach().clone() for n, p in model.named_parameters()}
    return y.detach(), x.grad.detach().clone(), grads


def test_compiled_block_matches_eager(gpu):
    """torch.compile(fullgraph=True) over the block: no graph break (fullgraph raises on one),
    and the compiled forward and backward give the eager results."""
    import copy
    _say("[compile] fullgraph block, forward + backward")
    torch._dynamo.reset()
    torch.manual_seed(0)
    eager = Block().bfloat16().to(gpu)
    eager.init(1)
    comp = copy.deepcopy(eager)
    cfn = torch.compile(comp, fullgraph=True)
    g = torch.Generator().manual_seed(9)
    x0 = torch.randn(384, 256, generator=g).bfloat16().to(gpu)
    gy = torch.randn(384, 256, generator=g).bfloat16().to(gpu)
    y_e, gx_e, gp_e = _run(eager, x0.clone().requires_grad_(True), gy)
    y_c, gx_c, gp_c = _run(cfn, x0.clone().requires_grad_(True), gy)
    torch.cuda.synchronize()
    assert torch.equal(y_c, y_e), "the compiled forward runs the same kernels on the same inputs"

    def err(a, b):
        return ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp_min(1e-30)).item()

    _say(f"   dx max_rel_err {err(gx_c, gx_e):.2e}")
    assert err(gx_c, gx_e) <= 1e-2
    for n in gp_e:
        assert err(gp_c[n], gp_e[n]) <= 1e-2, n


def test_meta_init_then_materialise(gpu):
    """Built on the meta device (the fake kernels give every shape), then to_empty on the GPU,
    initialised and run: the output matches a block built on the GPU directly with the same
    weights, bit for bit."""
    _say("[meta init] block")
    with torch.device("meta"):
        m = Block().bfloat16()
        y_meta = m(torch.empty(8, 256, dtype=torch.bfloat16))
    assert y_meta.device.type == "meta" and y_meta.shape == (8, 256)
    m = m.to_empty(device=gpu)
    m.init(3)
    ref = Block().bfloat16().to(gpu)
    ref.init(3)
    x = torch.randn(40, 256, generator=torch.Generator().manual_seed(1)).bfloat16().to(gpu)
    with torch.no_grad():
        assert torch.equal(m(x), ref(x))
