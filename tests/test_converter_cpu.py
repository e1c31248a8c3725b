"""The wsl_lora model converter on reference-style modules: structure only (the converted
forward runs on the GPU, in tests/test_gpu_converter.py)."""
import torch

from tests._ref_style import RefAttentionProjections, RefLoRA
from weightshared_torchtitan_amd import converter as C
from weightshared_torchtitan_amd.lora import LoRAModule


def test_registry_and_build():
    convs = C.build_model_converters(["wsl_lora"])
    assert len(convs) == 1 and isinstance(convs[0], C.WslLoRAConverter)
    try:
        C.register_model_converter(C.WslLoRAConverter, "wsl_lora")
    except ValueError:
        pass
    else:
        raise AssertionError("a second registration under one name must fail")


def test_convert_keeps_parameters_and_state_dict_keys():
    torch.manual_seed(0)
    m = torch.nn.Sequential(RefAttentionProjections(), RefAttentionProjections())
    keys = list(m.state_dict().keys())
    params = {n: p for n, p in m.named_parameters()}
    conv = C.WslLoRAConverter()
    conv.convert(m)
    assert list(m.state_dict().keys()) == keys
    for n, p in m.named_parameters():
        assert p is params[n], n
    # q (equal widths) and k (a base of g templates broadcast over the offset) both fold
    assert sorted(conv.fused) == ["0.wk_offset", "0.wq_offset", "1.wk_offset", "1.wq_offset"]
    assert conv.converted == []
    for i, blk in enumerate(m):
        assert isinstance(blk.wq_base, C.FusedBase) and blk.wq_base.weight is params[f"{i}.wq_base.weight"]
        assert isinstance(blk.wq_offset, LoRAModule) and blk.wq_offset.scale == 2.0
        assert isinstance(blk.wk_base, C.FusedBase) and blk.wk_base.weight is params[f"{i}.wk_base.weight"]
        assert type(blk.wo) is torch.nn.Linear


def test_convert_is_idempotent_and_keeps_unpaired_scale():
    m = torch.nn.ModuleDict({"lonely": RefLoRA(64, 32, rank=4), "proj": RefAttentionProjections()})
    m["lonely"].alpha = 12  # a non-default alpha: scale 3
    conv = C.WslLoRAConverter()
    conv.convert(m)
    assert type(m["lonely"]) is LoRAModule and m["lonely"].scale == 3.0
    before = [type(x) for x in m.modules()]
    conv2 = C.WslLoRAConverter()
    conv2.convert(m)
    assert conv2.fused == [] and conv2.converted == []
    assert [type(x) for x in m.modules()] == before


def test_shared_attention_modes_fold_and_keep_keys():
    """Every sharing switch of the reference's attention folds into fused bases; parameters and
    state-dict keys are kept; the module's broadcast_add is wrapped once, keeping its original."""
    import tests._ref_style as R
    orig = getattr(R.broadcast_add, "_wsl_original", R.broadcast_add)  # an earlier test may have wrapped it
    for kw, n_fused, n_shared in ((dict(), 3, 0), (dict(head_sharing=True, grouping=2), 3, 0),
                                  (dict(qkv_sharing=[["q", "k", "v"]]), 3, 1),
                                  (dict(qkv_sharing=[["q", "k"], ["v"]], head_sharing=True, grouping=4), 3, 2),
                                  (dict(two_step=True), 4, 0),
                                  (dict(two_step=True, qkv_sharing=[["q", "k", "v"]]), 4, 1),
                                  (dict(two_step=True, qkv_sharing=[["q", "k"], ["v"]], head_sharing=True,
                                        grouping=4), 4, 1)):
        m = R.RefSharedAttention(**kw)
        keys = list(m.state_dict().keys())
        params = {n: p for n, p in m.named_parameters()}
        conv = C.WslLoRAConverter()
        conv.convert(m)
        assert list(m.state_dict().keys()) == keys, kw
        for n, p in m.named_parameters():
            assert p is params[n], (kw, n)
        assert len(conv.fused) == n_fused and len(conv.shared) == n_shared, (kw, conv.fused, conv.shared)
        assert getattr(R.broadcast_add, "_wsl_original", None) is orig
    R.broadcast_add = orig  # leave the stand-in module as found


def test_folding_broadcast_add_keeps_original_semantics():
    """Calls without placeholders go to the original broadcast_add unchanged."""
    import numpy as np
    from weightshared_torchtitan_amd.lora import broadcast_add as ref_ba
    fn = C.folding_broadcast_add(ref_ba)
    g = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "broadcast_add.npz"))
    for name in g["names"]:
        out = fn(torch.from_numpy(g[f"{name}_base"]), torch.from_numpy(g[f"{name}_delta"]), g=int(g[f"{name}_g"]))
        np.testing.assert_array_equal(out.numpy(), g[f"{name}_out"])


def test_two_step_pair_is_one_lora_of_the_stacked_factors():
    """The folding identity of the two_step offsets (the reference's model.py:367-375):
    broadcast_add(s (x . A_p^T) . B_p^T, s (x . A_h^T) . B_h^T) with the D-wide B_p repeated over
    the heads equals s (x . A^T) . B^T for A = [A_h; A_p], B = [B_h | B_p repeated], in float64.
    A wrong repeat order (B_p tiled per column instead of per head) fails it."""
    import tests._ref_style as R
    torch.manual_seed(5)
    H, D, K, r = 8, 16, 64, 4
    head, only = R.RefLoRA(K, H * D, r).double(), R.RefLoRA(K, D, r).double()
    x = torch.randn(7, K, dtype=torch.float64)
    from weightshared_torchtitan_amd.lora import broadcast_add
    want = broadcast_add(only(x), head(x))
    pair = C._TwoStepPair(C._as_wsl(head), C._as_wsl(only))
    a, b = pair.factors()
    assert a.shape == (2 * r, K) and b.shape == (H * D, 2 * r) and pair.rank == 2 * r and pair.scale == 2.0
    got = (x @ a.t()) @ b.t() * pair.scale
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    wrong = torch.cat([head.w_b.weight, only.w_b.weight.repeat_interleave(H, 0)], 1)
    assert not torch.allclose((x @ a.t()) @ wrong.t() * 2.0, want)


def test_two_step_placeholders_compose():
    """The converted two_step forward's bookkeeping on the CPU: broadcast_add of an
    only-offset's and the head's placeholders gives a contiguous placeholder naming the pair's
    block ((j, width), kept by .contiguous()); unexpected pairings raise."""
    import tests._ref_style as R
    m = R.RefSharedAttention(two_step=True, qkv_sharing=[["q", "k", "v"]])
    orig = getattr(R.broadcast_add, "_wsl_original", R.broadcast_add)
    try:
        C.WslLoRAConverter().convert(m)
        x = torch.randn(3, 5, 512)
        h, k = m.head_offset(x), m.wk_only_offset(x)
        c = R.broadcast_add(k, h).contiguous()
        assert c.is_contiguous() and c.shape == (3, 5, 512) and getattr(c, C._FOLDED) == (1, 512)
        import pytest
        with pytest.raises(RuntimeError):
            R.broadcast_add(h, k)
    finally:
        R.broadcast_add = orig
