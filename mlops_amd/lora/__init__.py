"""Expert LoRA over the MI355X block-FP8 MoE path (reference: ``src/mlops/lora``)."""

from .experts import expert_lora

__all__ = ["expert_lora"]
