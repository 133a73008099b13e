from .kernel import attention_core, fused_gate_forward, gate_out_forward, prep_forward, triangle_attn_forward
from .module import forward, precompute, triangle_attention

__all__ = [
    "triangle_attention",
    "precompute",
    "forward",
    "triangle_attn_forward",
    "fused_gate_forward",
    "prep_forward",
    "attention_core",
    "gate_out_forward",
]
