"""ctypes binding of `libtriangleops_amd.so` (the C ABI declared in include/triangleops_amd.h).

The library is loaded on first use.  There is no fallback: if it is missing or cannot be
loaded, every op raises ImportError naming the build command.  Each call passes raw device
pointers and torch's current HIP stream; a non-zero return code becomes RuntimeError with
the library's message.
"""

from __future__ import annotations

import ctypes
import functools
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtriangleops_amd.so")
ABI_VERSION = 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (all return int status codes except where noted)
_SIGNATURES = {
    "tops_tmu_input_phase": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32, _f32, _i32, _p],
    "tops_tmu_einsum": [_p, _p, _i64, _i64, _i64, _i64, _i32, _p],
    "tops_tmu_output_phase": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p],
    "tops_tri_prep": [
        _p, _i64, _i64, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _p,
    ],
    "tops_tri_repack": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i32, _p],
    "tops_tri_attention": [_p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "tops_tri_attention_two_row": [_p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _p],
    "tops_gate_out": [
        _p, _i64, _i64, _p, _i64, _i64, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p,
    ],
    "tops_apb_forward": [
        _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _p,
    ],
    "tops_apb_forward_gated": [
        _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
        _f32, _i32, _p,
    ],
    "tops_apb_merge_gate": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _p],
    "tops_apb_forward_noalloc": [
        _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _p,
    ],
    "tops_apb_forward_qkv": [
        _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _p,
    ],
    "tops_apb_qkn_prep": [
        _p, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _f32, _i32, _p,
    ],
    "tops_tmu_output_phase_residual": [
        _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p,
    ],
    "tops_gate_out_residual": [
        _p, _i64, _i64, _p, _i64, _i64, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64,
        _i64, _i64, _i32, _p,
    ],
    "tops_gate_out_generic_residual": [
        _p, _i64, _i64, _p, _i64, _i64, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64,
        _i64, _i64, _i64, _i64, _i32, _p,
    ],
    "tops_tri_generic_prep": [
        _p, _i64, _i64, _p, _p, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _i32, _p,
    ],
    "tops_tri_generic_attention": [_p, _p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p],
    "tops_apb_generic_prep": [
        _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f32, _i32, _p,
    ],
    "tops_apb_generic_attention": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _i32, _p],
    "tops_gate_out_generic": [
        _p, _i64, _i64, _p, _i64, _i64, _p, _p, _f32, _i32, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i32,
        _p,
    ],
}
_OTHER = {
    "tops_last_error": ([], ctypes.c_char_p),
    "tops_abi_version": ([], ctypes.c_int),
    "tops_apb_workspace_bytes": ([_i64, _i64, _i64], ctypes.c_int64),
    "tops_apb_gated_workspace_bytes": ([_i64, _i64, _i64], ctypes.c_int64),
}

EXPORTED = tuple(_SIGNATURES) + tuple(_OTHER)

_lib = None


def load(path: str = LIB_PATH):
    """Loads the library (once) and declares the prototypes; raises ImportError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"triangleops_amd: HIP library not found at {path}; build it with "
            "`python -m triangleops_amd._build` (hipcc, gfx950)"
        )
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:
        raise ImportError(f"triangleops_amd: cannot load {path}: {e}") from e
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    for name, (argtypes, restype) in _OTHER.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    if lib.tops_abi_version() != ABI_VERSION:
        raise ImportError(f"triangleops_amd: ABI version mismatch ({lib.tops_abi_version()} != {ABI_VERSION})")
    _lib = lib
    return lib


_fns: dict = {}


def call(name: str, *args) -> None:
    """Calls C entry point `name`; raises RuntimeError with the library's message on failure."""
    fn = _fns.get(name)
    if fn is None:
        lib = _lib if _lib is not None else load()
        fn = _fns[name] = getattr(lib, name)
    rc = fn(*args)
    if rc != 0:
        msg = _lib.tops_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


@functools.lru_cache(maxsize=256)
def apb_workspace_bytes(M: int, H: int, D: int) -> int:
    lib = _lib if _lib is not None else load()
    return int(lib.tops_apb_workspace_bytes(M, H, D))


@functools.lru_cache(maxsize=256)
def apb_gated_workspace_bytes(M: int, H: int, D: int) -> int:
    lib = _lib if _lib is not None else load()
    return int(lib.tops_apb_gated_workspace_bytes(M, H, D))


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Raw hipStream_t of torch's current stream on `t`'s device (without building a Stream object)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def check_device(*tensors) -> None:
    """All tensors must be on one GPU (the kernels dereference raw device pointers)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        d = t.get_device()  # device index, -1 off the GPU
        if d < 0:
            raise ValueError(f"triangleops_amd kernels need GPU tensors (got a tensor on {t.device})")
        if dev is None:
            dev = d
        elif d != dev:
            raise ValueError(f"all tensors must be on one device (got cuda:{dev} and {t.device})")


def vec16_ok(t: torch.Tensor) -> bool:
    """True when the kernels' 16-byte vector accesses of `t` are valid: unit last stride, every
    other stride a multiple of 8 elements and a 16-byte aligned base."""
    return t.stride(-1) == 1 and all(st % 8 == 0 for st in t.stride()[:-1]) and t.data_ptr() % 16 == 0


def vec16(t: torch.Tensor) -> torch.Tensor:
    """`t` itself when vec16_ok(t), else a fresh contiguous copy (which is 16-byte aligned;
    `.contiguous()` alone would return a contiguous but misaligned view unchanged).  Only for
    tensors whose strides are passed to the kernel; see `dense` for the others."""
    return t if vec16_ok(t) else t.clone(memory_format=torch.contiguous_format)


def dense(t: torch.Tensor | None, dtype: torch.dtype | None = None) -> torch.Tensor | None:
    """`t` (cast to `dtype` if given) as a dense row-major tensor with a 16-byte aligned base:
    itself when it already is one, else a fresh contiguous copy.  For every tensor the kernels
    index without strides (activations such as X or a residual, weights, bias vectors): a
    column slice such as S[:, :128] of a wider tensor is not dense and is copied."""
    if t is None:
        return None
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t if (t.is_contiguous() and t.data_ptr() % 16 == 0) else t.clone(memory_format=torch.contiguous_format)


def mask_i8(mask: torch.Tensor | None) -> torch.Tensor | None:
    """Mask as int8 storage without a copy for bool/int8/uint8 contiguous masks."""
    if mask is None:
        return None
    m = mask if mask.is_contiguous() else mask.contiguous()
    if m.dtype in (torch.bool, torch.uint8):
        return m.view(torch.int8)
    if m.dtype == torch.int8:
        return m
    return m.to(torch.int8)
