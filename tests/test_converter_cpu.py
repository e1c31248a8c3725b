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
    assert sorted(conv.fused) == ["0.wq_offset", "1.wq_offset"]
    assert sorted(conv.converted) == ["0.wk_offset", "1.wk_offset"]
    for i, blk in enumerate(m):
        assert isinstance(blk.wq_base, C.FusedBase) and blk.wq_base.weight is params[f"{i}.wq_base.weight"]
        assert isinstance(blk.wq_offset, LoRAModule) and blk.wq_offset.scale == 2.0
        assert type(blk.wk_offset) is LoRAModule and isinstance(blk.wk_base, torch.nn.Linear)
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
