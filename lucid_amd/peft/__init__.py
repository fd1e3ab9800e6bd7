"""Parameter-efficient adapters over the quantized layers (lucid.peft's LoRA path for
``nn.quantized.Linear``, ``nn.quantized.dynamic.Linear`` and ``QuantizedLinearMLX``)."""

from lucid_amd.peft.lora import Linear, LoraConfig, QuantizedLinear, lora_layer_for
from lucid_amd.peft.peft_model import LoraModel, PeftModel, get_peft_model

__all__ = ["Linear", "LoraConfig", "LoraModel", "PeftModel", "QuantizedLinear", "get_peft_model", "lora_layer_for"]
