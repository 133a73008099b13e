"""Low-level launchers of the gfx950 triangle-multiplicative-update kernels.

Same wrapper names, arguments and return layouts as the reference's Triton launchers
(`triangle_mul/kernel.py:235-326`): `input_phase` returns ab as (2C, B, L, L) channel-major,
any C and bf16 / fp16 / fp32 I/O (the library runs C = 128 in 16-bit types on the tuned
kernels, everything else on its any-shape kernels),
`output_phase` consumes y as (C, B, L, L) channel-major and returns (B, L, L, C).  The extra
keyword arguments (`transpose`, `ld`, `ldy`) expose the layout options the fused `forward`
uses; their defaults reproduce the reference layout exactly.
"""

import torch

from .. import _native
from .._common.dtype import any_shape_dtype_code


def _prep_weights(x, *ws):
    return [_native.dense(w, x.dtype) for w in ws]


def _f32(*vs):
    return [_native.dense(v, torch.float32) for v in vs]


def input_phase(
    x,
    mask,
    p_in_combined,
    g_in_combined,
    sum_W_p_in,
    sum_W_g_in,
    B_p_in_const,
    B_g_in_const,
    eps,
    *,
    transpose=False,
    ld=None,
):
    """LN_in + p_in * sigmoid(g_in) * mask -> ab, channel-major (2C, B, L, ld).

    With `transpose=True` each channel's L x L token grid is stored transposed (the layout
    the incoming einsum consumes).  `ld` must be a multiple of 64; columns [L, ld) are zero.
    With the defaults the result is the reference's contiguous (2C, B, L, L) tensor.
    """
    B, L, L2, C = x.shape
    assert L == L2, "x must be (B, L, L, C)"
    C_out = p_in_combined.shape[0]
    trim = ld is None and L % 64 != 0
    ld = max(64, (L + 63) // 64 * 64) if ld is None else int(ld)
    code = any_shape_dtype_code(x.dtype)
    _native.check_device(x, p_in_combined, g_in_combined, mask)
    x = _native.dense(x)
    Wp, Wg = _prep_weights(x, p_in_combined, g_in_combined)
    sWp, sWg, Bp, Bg = _f32(sum_W_p_in, sum_W_g_in, B_p_in_const, B_g_in_const)
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == B * L * L, "mask must have B*L*L elements"
    out = torch.empty(C_out, B, L, ld, device=x.device, dtype=x.dtype)
    _native.call(
        "tops_tmu_input_phase",
        x.data_ptr(),
        _native.ptr(m8),
        Wp.data_ptr(),
        Wg.data_ptr(),
        sWp.data_ptr(),
        sWg.data_ptr(),
        Bp.data_ptr(),
        Bg.data_ptr(),
        out.data_ptr(),
        B,
        L,
        C,
        C_out,
        ld,
        1 if transpose else 0,
        float(eps),
        code,
        _native.stream_of(x),
    )
    return out[..., :L].contiguous() if trim else out


def triangle_einsum(ab, L, ld, C, B):
    """y[d, b, i, j] = sum_k a[d, b, i, k] b[d, b, j, k] over the (2C, B, L, ld) tensor ab.

    `ld` must be a multiple of 64 with zero columns [L, ld) (as `input_phase(..., ld=ld)`
    writes them); only k < round_up(L, 64) is read, so ld may carry extra row padding.
    Returns y as (C, B, L, ld); columns [L, ld) are left unspecified.
    """
    y = torch.empty(C, B, L, ld, device=ab.device, dtype=ab.dtype)
    _native.call(
        "tops_tmu_einsum",
        ab.data_ptr(),
        y.data_ptr(),
        C * B,
        L,
        ld,
        ld,
        any_shape_dtype_code(ab.dtype),
        _native.stream_of(ab),
    )
    return y


def output_phase(
    y_t,
    x,
    p_out_combined,
    g_out_combined,
    sum_W_p_out,
    sum_W_g_out,
    B_p_out_const,
    B_g_out_const,
    eps,
    *,
    ldy=None,
    residual=None,
):
    """sigmoid(g_out(LN_in x)) * p_out(LN_out y) -> (B, L, L, C_out); y channel-major (C, B, L, ldy).

    The kernel reads y rows padded to a multiple of 64 (`ldy`); with the default (y as the
    reference's (C, B, L, L) tensor) a padded copy is made when L is not a multiple of 64.
    `residual` (B, L, L, C_out): returns residual + result, the add fused into the kernel's store
    (each sum rounded once, as `residual + result` would be).
    """
    B, L, _, C = x.shape
    C_out = p_out_combined.shape[0]
    code = any_shape_dtype_code(x.dtype)
    _native.check_device(x, y_t, p_out_combined, g_out_combined)
    x = _native.dense(x)
    if ldy is None:
        ldy = max(64, (L + 63) // 64 * 64)
        y_t = y_t.reshape(C, B, L, L)
        if ldy != L:
            y_t = torch.nn.functional.pad(y_t, (0, ldy - L))
    else:
        ldy = int(ldy)
        assert y_t.is_contiguous() and y_t.numel() == C * B * L * ldy
    y_t = _native.dense(y_t, x.dtype)
    Wp, Wg = _prep_weights(x, p_out_combined, g_out_combined)
    sWp, sWg, Bp, Bg = _f32(sum_W_p_out, sum_W_g_out, B_p_out_const, B_g_out_const)
    out = torch.empty(B, L, L, C_out, device=x.device, dtype=x.dtype)
    res = []
    if residual is not None:
        assert residual.shape == out.shape, "residual must have the output's shape (B, L, L, C_out)"
        _native.check_device(x, residual)
        res = [_native.dense(residual, x.dtype)]
    _native.call(
        "tops_tmu_output_phase_residual" if res else "tops_tmu_output_phase",
        y_t.data_ptr(),
        x.data_ptr(),
        Wp.data_ptr(),
        Wg.data_ptr(),
        sWp.data_ptr(),
        sWg.data_ptr(),
        Bp.data_ptr(),
        Bg.data_ptr(),
        *[r.data_ptr() for r in res],
        out.data_ptr(),
        B,
        L,
        C,
        C_out,
        ldy,
        float(eps),
        code,
        _native.stream_of(x),
    )
    return out
