from .kernel import apb_forward, apb_forward_qkv, apb_qkn_prep
from .module import attention_pair_bias, attention_pair_bias_qknorm, forward, forward_qknorm, precompute

__all__ = [
    "attention_pair_bias",
    "precompute",
    "forward",
    "apb_forward",
    "attention_pair_bias_qknorm",
    "forward_qknorm",
    "apb_qkn_prep",
    "apb_forward_qkv",
]
