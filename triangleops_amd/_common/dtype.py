"""I/O dtype codes of the HIP kernels.

Mirrors `triangle_ops/_common/dtype.py:7-19` of the reference: the same names
(`TORCH_TO_TL`, `tl_io_dtype`) and the same ValueError for an unsupported dtype, but the
values are the C-ABI dtype codes of `include/triangleops_amd.h` instead of Triton types.
"""

import torch

DTYPE_F16 = 1
DTYPE_BF16 = 2
DTYPE_F32 = 3

# torch I/O dtype -> C-ABI dtype code (the reference maps to `tl.*` types).
TORCH_TO_TL = {
    torch.float16: DTYPE_F16,
    torch.bfloat16: DTYPE_BF16,
    torch.float32: DTYPE_F32,
}

# dtypes the tuned gfx950 kernels compute on (MFMA operands).  fp32 I/O is taken by the
# any-shape fp32 kernels where an op has them (`any_shape_dtype_code`).
KERNEL_DTYPES = (torch.bfloat16, torch.float16)


def tl_io_dtype(dtype: torch.dtype) -> int:
    """Return the C-ABI dtype code for a torch I/O dtype, raising ValueError on unsupported."""
    try:
        return TORCH_TO_TL[dtype]
    except KeyError as e:
        raise ValueError(f"unsupported IO dtype {dtype}; expected one of {list(TORCH_TO_TL)}") from e


def io_dtype_code(dtype: torch.dtype) -> int:
    """Like `tl_io_dtype`, but also rejects dtypes the HIP kernels do not compute in."""
    code = tl_io_dtype(dtype)
    if dtype not in KERNEL_DTYPES:
        raise ValueError(
            f"IO dtype {dtype} is not supported by the gfx950 kernels; use torch.bfloat16 or torch.float16"
        )
    return code


def any_shape_dtype_code(dtype: torch.dtype) -> int:
    """C-ABI dtype code for the any-shape kernels, which also take fp32 I/O."""
    return tl_io_dtype(dtype)
