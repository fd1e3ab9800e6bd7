"""Host-side LoRA bookkeeping (lucid_amd/peft): config validation (lucid/peft/_config.py:196-244),
target matching (lucid/peft/_targeting.py:35,88-93), the wrapped model's state-dict keys and
which parameters train, adding adapters, unload."""

from __future__ import annotations

import numpy as np
import pytest


def test_lora_config_validation():
    from lucid_amd.peft import LoraConfig

    with pytest.raises(ValueError, match="positive"):
        LoraConfig(r=0)
    with pytest.raises(TypeError):
        LoraConfig(r=True)
    with pytest.raises(ValueError, match=r"\[0, 1\)"):
        LoraConfig(lora_dropout=1.0)
    with pytest.raises(ValueError, match="init_lora_weights"):
        LoraConfig(init_lora_weights="eva")
    assert LoraConfig(r=4, lora_alpha=8).scaling == 2.0
    assert LoraConfig(r=4, lora_alpha=8, use_rslora=True).scaling == 4.0


def test_target_matching():
    from lucid_amd.peft import LoraConfig

    c = LoraConfig(target_modules=["q_proj", "fc"])
    assert c.matches("layers.0.q_proj") and c.matches("fc") and not c.matches("xfc")
    r = LoraConfig(target_modules=r".*\.(q|v)_proj")
    assert r.matches("layers.1.v_proj") and not r.matches("v_proj") and not r.matches("layers.1.k_proj")
    with pytest.raises(ValueError, match="target_modules"):
        LoraConfig().matches("fc")


def _mlp():
    import lucid_amd.nn as nn

    return nn.Sequential(nn.Linear(8, 16), nn.ReLU(), nn.Linear(16, 4))


def test_get_peft_model_keys_and_trainable():
    from lucid_amd.peft import LoraConfig, get_peft_model

    model = _mlp()
    first = model[0]
    peft = get_peft_model(model, LoraConfig(r=2, target_modules=["0"]))
    keys = list(peft.state_dict().keys())
    assert "base_model.model.0.base_layer.weight" in keys
    assert "base_model.model.0.lora_A.default.weight" in keys
    assert "base_model.model.0.lora_B.default.weight" in keys
    assert "base_model.model.2.weight" in keys
    trainable = {n for n, p in peft.named_parameters() if p.requires_grad}
    assert trainable == {"base_model.model.0.lora_A.default.weight", "base_model.model.0.lora_B.default.weight"}
    layer = peft.base_model.model[0]
    assert layer.base_layer is first
    assert np.all(layer.lora_B["default"].weight.numpy() == 0)
    peft.add_adapter("other", LoraConfig(r=3, target_modules=["0"]))
    assert "base_model.model.0.lora_A.other.weight" in peft.state_dict()
    assert layer.lora_A["other"].weight.shape == (3, 8)
    with pytest.raises(ValueError, match="already exists"):
        peft.add_adapter("other", LoraConfig(r=3, target_modules=["0"]))
    plain = peft.unload()
    assert plain[0] is first


def test_targets_must_exist_and_be_supported():
    import lucid_amd.nn as nn
    from lucid_amd.peft import LoraConfig, get_peft_model

    with pytest.raises(ValueError, match="not found"):
        get_peft_model(_mlp(), LoraConfig(target_modules=["nope"]))
    with pytest.raises(ValueError, match="no LoRA layer"):
        get_peft_model(nn.Sequential(nn.ReLU()), LoraConfig(target_modules=["0"]))
