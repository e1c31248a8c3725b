"""Host-side logic of the torch layer, on the CPU: workspace lifetime, bounds checks of the
decode path, the autocast rules registered on the ops, the embedding id check, and the
product broadcast_add against the committed golden vectors."""
import os

import numpy as np
import pytest
import torch

from weightshared_torchtitan_amd import lora, ops
from weightshared_torchtitan_amd.qwen3_shared import SharedQwen3, SharedQwen3Args

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------ workspaces
def test_grown_workspace_keeps_the_old_buffer_alive():
    """A graph captured while a workspace was current addresses it on every replay: growing
    (or dropping after a failed launch) must retire the buffer, never free it."""
    dev = torch.device("cpu")
    key_stream = 12345
    a = ops.workspace(dev, key_stream, 1 << 10, kind="test")
    a_ptr = a.data_ptr()
    n_retired = len(ops._retired)
    b = ops.workspace(dev, key_stream, (ops._WS_MIN_BYTES) + 1, kind="test")  # must grow
    assert b.data_ptr() != a_ptr
    assert len(ops._retired) == n_retired + 1
    assert ops._retired[-1].data_ptr() == a_ptr  # still referenced: its memory cannot be reused
    assert ops.workspace(dev, key_stream, 16, kind="test") is b  # no growth: same buffer
    ops._retire((dev.index, key_stream, "test"))  # the failed-launch path
    assert ops._retired[-1] is b
    assert (dev.index, key_stream, "test") not in ops._workspaces


# ------------------------------------------------------------------ bounds of the decode path
def _tiny(**kw):
    a = SharedQwen3Args(dim=32, n_layers=2, n_unique_blocks=1, n_heads=4, n_kv_heads=2, head_dim=8,
                        hidden_dim=48, vocab_size=50, embed_rank=16, lora_rank=4, max_seq_len=16)
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_generate_rejects_positions_past_the_rope_table():
    m = SharedQwen3(_tiny())
    prompt = torch.zeros(1, 10, dtype=torch.int64)
    with pytest.raises(IndexError, match="max_seq_len"):
        m.generate(prompt, 8)  # needs positions up to 16 > 15
    with pytest.raises(IndexError, match="max_seq_len"):
        m(torch.zeros(1, 17, dtype=torch.int64))
    with pytest.raises(ValueError):
        m.generate(prompt, 0)


def test_rope_table_must_cover_the_cache():
    ops._check_rope(torch.zeros(16, 16), 16, 8)
    ops._check_rope(torch.zeros(20, 16), 16, 8)
    with pytest.raises(ValueError, match="rope"):
        ops._check_rope(torch.zeros(15, 16), 16, 8)
    with pytest.raises(ValueError, match="rope"):
        ops._check_rope(torch.zeros(16, 12), 16, 8)


# ------------------------------------------------------------------ autocast
@pytest.mark.parametrize("op", ["lora_linear", "lora_linear_grouped", "factorized_embedding"])
def test_autocast_rule_is_registered_on_the_op(op):
    assert torch._C._dispatch_has_kernel_for_dispatch_key(f"wsl::{op}", "AutocastCUDA")


def test_autocast_operand_casts():
    f32 = torch.zeros(2, 2)
    assert ops.autocast_operand(f32).dtype == torch.bfloat16
    assert ops.autocast_operand(f32.half()).dtype == torch.bfloat16
    bf = f32.bfloat16()
    assert ops.autocast_operand(bf) is bf
    q = f32.to(torch.float8_e4m3fn)
    assert ops.autocast_operand(q) is q  # an fp8 base keeps its storage type
    ids = torch.zeros(3, dtype=torch.int64)
    assert ops.autocast_operand(ids) is ids
    assert ops.autocast_operand(None) is None


# ------------------------------------------------------------------ embedding ids
def test_embedding_id_check():
    ops.check_embedding_ids(torch.tensor([0, 5, 9]), 10)
    ops.check_embedding_ids(torch.zeros(0, dtype=torch.int64), 10)
    with pytest.raises(IndexError):
        ops.check_embedding_ids(torch.tensor([0, 10]), 10)
    with pytest.raises(IndexError):
        ops.check_embedding_ids(torch.tensor([-1, 3]), 10)


# ------------------------------------------------------------------ broadcast_add (product)
def test_product_broadcast_add_matches_golden():
    """lora.broadcast_add (the head-sharing composition the converter and models use) against
    the committed index-formula vectors: bit for bit in float64, to one rounding in float32."""
    g = np.load(os.path.join(GOLDEN, "broadcast_add.npz"))
    for name in g["names"]:
        base = torch.from_numpy(g[f"{name}_base"])
        delta = torch.from_numpy(g[f"{name}_delta"])
        out = lora.broadcast_add(base, delta, dim=-1, g=int(g[f"{name}_g"]))
        np.testing.assert_array_equal(out.numpy(), g[f"{name}_out"], err_msg=str(name))
        # in float32 each element is one rounded add of the same two operands
        out32 = lora.broadcast_add(base.float(), delta.float(), dim=-1, g=int(g[f"{name}_g"]))
        np.testing.assert_allclose(out32.double().numpy(), g[f"{name}_out"], rtol=3e-7, atol=1e-7, err_msg=str(name))


def test_product_broadcast_add_rejects_incompatible_widths():
    with pytest.raises(AssertionError):
        lora.broadcast_add(torch.zeros(2, 6), torch.zeros(2, 10))
