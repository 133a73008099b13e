"""Shared host-side helpers used by all three ops (weight folding, layouts, dtype codes)."""

from .dtype import TORCH_TO_TL, io_dtype_code, tl_io_dtype
from .layouts import interleave_kv, interleave_qkv, qkv_head_major
from .ln_absorption import absorb_ln, absorb_ln_matmul

__all__ = [
    "TORCH_TO_TL",
    "tl_io_dtype",
    "io_dtype_code",
    "absorb_ln",
    "absorb_ln_matmul",
    "interleave_qkv",
    "interleave_kv",
    "qkv_head_major",
]
