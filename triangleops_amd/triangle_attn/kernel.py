"""Low-level launchers of the gfx950 triangle-attention kernels.

Same names and arguments as the reference's launchers (`triangle_attn/kernel.py:256-374`
`triangle_attn_forward`, `:438-470` `fused_gate_forward`), plus `ln_bias_forward`, the one
pass that produces x_ln = LN(x) and the row-shared bias together (the reference runs
F.layer_norm and then a separate bias kernel).
"""

import torch

from .. import _native
from .._common.dtype import io_dtype_code


def _as(x, t):
    if t is None:
        return None
    return t if (t.dtype == x.dtype and t.is_contiguous()) else t.to(x.dtype).contiguous()


def wqkv_from_layouts(WQ_c, WKV_c, H, D, WK_c=None, WV_c=None):
    """(H, 3, D, C) head-major weight the attention kernel loads, from the reference layouts."""
    C = WQ_c.shape[0]
    if WK_c is not None and WV_c is not None:
        WK, WV = WK_c.reshape(C, H, D), WV_c.reshape(C, H, D)
    else:
        kv = WKV_c.reshape(C, H, D, 2)
        WK, WV = kv[..., 0], kv[..., 1]
    w = torch.stack((WQ_c.reshape(C, H, D), WK, WV), dim=0)  # (3, C, H, D)
    return w.permute(2, 0, 3, 1).contiguous()


def ln_bias_forward(X, W_ln, B_ln, WZ_c, BZ, *, eps=1e-5, apply_ln=True, X_ln=None, Bias_buf=None):
    """x_ln = LN(X) (if apply_ln) and bias[h, q, k] = x_ln[q, k] . WZ_c[h] + BZ[h] in one pass.

    X may be any (N, N, C) view with unit channel stride (e.g. the transposed view of the
    ending node).  Returns (x_ln or None, bias (H, N, N)).
    """
    N, N2, C = X.shape
    assert N == N2, "X must be (N, N, C)"
    H = WZ_c.shape[0]
    code = io_dtype_code(X.dtype)
    _native.check_device(X, WZ_c, W_ln, B_ln)
    if X.stride(2) != 1 or X.stride(0) % 8 or X.stride(1) % 8:
        X = X.contiguous()
    if apply_ln and X_ln is None:
        X_ln = torch.empty(N, N, C, device=X.device, dtype=X.dtype)
    if Bias_buf is None:
        Bias_buf = torch.empty(H, N, N, device=X.device, dtype=X.dtype)
    WZ = _as(X, WZ_c)
    BZf = None if BZ is None else BZ.float().contiguous()
    _native.call(
        "tops_tri_ln_bias",
        X.data_ptr(),
        X.stride(0),
        X.stride(1),
        _native.ptr(_as(X, W_ln)) if apply_ln else None,
        _native.ptr(_as(X, B_ln)) if apply_ln else None,
        1 if apply_ln else 0,
        WZ.data_ptr(),
        _native.ptr(BZf),
        _native.ptr(X_ln) if apply_ln else None,
        Bias_buf.data_ptr(),
        N,
        C,
        H,
        float(eps),
        code,
        _native.stream_of(X),
    )
    return (X_ln if apply_ln else None), Bias_buf


def attention_core(X_ln, wqkv, bias, out, *, scale=1.0, mask=None):
    """O[i, q, h*D:(h+1)*D] = softmax_k(scale Q.K + bias - 1e9 [mask[i,k] == 0]) V, written into `out`."""
    N, _, C = X_ln.shape
    H, _, D, _ = wqkv.shape
    _native.check_device(X_ln, wqkv, bias, out, mask)
    assert out.shape == (N, N, H * D) and out.stride(2) == 1, "out must be (N, N, H*D) with unit last stride"
    m8 = None
    sm0 = sm1 = 0
    if mask is not None:
        m8 = mask.view(torch.int8) if mask.dtype in (torch.bool, torch.uint8) else mask.to(torch.int8)
        sm0, sm1 = m8.stride()
    _native.call(
        "tops_tri_attention",
        X_ln.data_ptr(),
        wqkv.data_ptr(),
        bias.data_ptr(),
        _native.ptr(m8),
        sm0,
        sm1,
        out.data_ptr(),
        out.stride(0),
        out.stride(1),
        N,
        C,
        H,
        D,
        float(scale),
        io_dtype_code(X_ln.dtype),
        _native.stream_of(X_ln),
    )
    return out


def triangle_attn_forward(
    X_ln,
    WQ_c,
    WKV_c,
    WZ_c,
    BZ,
    out,
    scale=1.0,
    mask=None,
    Bias_buf=None,
    *,
    WK_c=None,
    WV_c=None,
):
    """Bias projection + attention over a pre-normalized X_ln (N, N, C), written into out (N, N, H*D)."""
    N, N2, C = X_ln.shape
    assert N == N2
    H = WZ_c.shape[0]
    D = WQ_c.shape[1] // H
    assert WKV_c.shape == (C, 2 * H * D)
    assert out.shape == (N, N, H * D)
    X_ln = X_ln if X_ln.is_contiguous() else X_ln.contiguous()
    _, Bias_buf = ln_bias_forward(X_ln, None, None, WZ_c, BZ, apply_ln=False, Bias_buf=Bias_buf)
    wqkv = wqkv_from_layouts(_as(X_ln, WQ_c), _as(X_ln, WKV_c), H, D, _as(X_ln, WK_c), _as(X_ln, WV_c))
    return attention_core(X_ln, wqkv, Bias_buf, out, scale=scale, mask=mask)


def gate_out_forward(o, gin, W_g, b_g, W_o, b_o):
    """out = ((o * sigmoid(gin W_g^T + b_g)) -> io) W_o^T + b_o over (N1, N2, C) tokens."""
    N1, N2, C = o.shape
    _native.check_device(o, gin, W_g, W_o)
    if o.stride(2) != 1 or o.stride(0) % 4 or o.stride(1) % 4:
        o = o.contiguous()
    gin = gin if gin.is_contiguous() else gin.contiguous()
    assert gin.numel() == N1 * N2 * C
    out = torch.empty(N1, N2, C, device=o.device, dtype=o.dtype)
    _native.call(
        "tops_gate_out",
        o.data_ptr(),
        o.stride(0),
        o.stride(1),
        gin.data_ptr(),
        _as(o, W_g).data_ptr(),
        _native.ptr(_as(o, b_g)),
        _as(o, W_o).data_ptr(),
        _native.ptr(_as(o, b_o)),
        out.data_ptr(),
        N1,
        N2,
        C,
        io_dtype_code(o.dtype),
        _native.stream_of(o),
    )
    return out


def fused_gate_forward(o_attn, qx_ln, WG, WO):
    """Out = (o_attn * sigmoid(qx_ln @ WG^T)) @ WO^T; o_attn (N, N, H, D) at any strides, WG/WO (out, in)."""
    N1, N2, H, D = o_attn.shape
    if o_attn.stride(3) != 1 or o_attn.stride(2) != D:
        o_attn = o_attn.contiguous()
    o = o_attn.as_strided((N1, N2, H * D), (o_attn.stride(0), o_attn.stride(1), 1))
    return gate_out_forward(o, qx_ln, WG, None, WO, None)
