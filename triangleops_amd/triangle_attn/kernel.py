"""Low-level launchers of the gfx950 triangle-attention kernels.

Same names and arguments as the reference's launchers (`triangle_attn/kernel.py:256-374`
`triangle_attn_forward`, `:438-470` `fused_gate_forward`), plus the pieces `forward` uses:

    prep_forward      LN(x), the row-shared bias and Q/K/V of all heads in one pass over x
    attention_core    flash attention over the pre-pass outputs
    gate_out_forward  sigmoid gate (optionally on LN of its input) and output projection
"""

import torch

from .. import _native
from .._common.dtype import any_shape_dtype_code, io_dtype_code


def _as(x, t):
    """A weight or parameter vector as a dense, 16-byte aligned tensor of x's dtype."""
    return _native.dense(t, x.dtype)


def row_stride(N):
    """Padded key count of the pre-pass buffers: N rounded up to a multiple of 64."""
    return max(64, (N + 63) // 64 * 64)


def wqkv_from_layouts(WQ_c, WKV_c, H, D, WK_c=None, WV_c=None):
    """(H, 3, D, C) head-major weight the kernels load, from the reference layouts."""
    C = WQ_c.shape[0]
    if WK_c is not None and WV_c is not None:
        WK, WV = WK_c.reshape(C, H, D), WV_c.reshape(C, H, D)
    else:
        kv = WKV_c.reshape(C, H, D, 2)
        WK, WV = kv[..., 0], kv[..., 1]
    w = torch.stack((WQ_c.reshape(C, H, D), WK, WV), dim=0)  # (3, C, H, D)
    return w.permute(2, 0, 3, 1).contiguous()


def prep_forward(X, W_ln, B_ln, wqkv, WZ_c, BZ, *, scale=1.0, eps=1e-5, apply_ln=True):
    """One pass over X (N, N, C): returns (Qp, KV, bias, ldn) in the attention kernel's layouts.

    X may be any (N, N, C) view with unit channel stride (e.g. the transposed view of the
    ending node).  With apply_ln=False, X is taken as already normalized.
    """
    N, N2, C = X.shape
    assert N == N2, "X must be (N, N, C)"
    H, _, D, _ = wqkv.shape
    code = io_dtype_code(X.dtype)
    _native.check_device(X, wqkv, WZ_c, W_ln)
    X = _native.vec16(X)
    ldn = row_stride(N)
    # the attention kernel's 32-wide head layout; a head with D = 16 is zero-padded to 32
    Qp = torch.empty(N, H, ldn, 32, device=X.device, dtype=X.dtype)
    KV = torch.empty(N, H, ldn // 64, 4096, device=X.device, dtype=X.dtype)
    bias = torch.empty(H, (N + 31) // 32, ldn // 32, 1024, device=X.device, dtype=X.dtype)
    BZf = None if BZ is None else _native.dense(BZ, torch.float32)
    _native.call(
        "tops_tri_prep",
        X.data_ptr(),
        X.stride(0),
        X.stride(1),
        _native.ptr(_as(X, W_ln)) if apply_ln else None,
        _native.ptr(_as(X, B_ln)) if apply_ln else None,
        1 if apply_ln else 0,
        _as(X, wqkv).data_ptr(),
        _as(X, WZ_c).data_ptr(),
        _native.ptr(BZf),
        Qp.data_ptr(),
        KV.data_ptr(),
        bias.data_ptr(),
        N,
        ldn,
        C,
        H,
        D,
        float(eps),
        float(scale),
        code,
        _native.stream_of(X),
    )
    return Qp, KV, bias, ldn


LOG2E = 1.4426950408889634


TUNED_MAX_N = 16384  # largest N of tops_tri_prep / tops_tri_attention (per-row key-block tables in LDS)


def fast_shape(C, H, D, N=None):
    """True when the tuned pre-pass and attention kernels apply: C_in in (128, 64), H = 4, D in (32,
    16) (the Apo shape C_in = 64, D = 16 included: heads zero-padded to 32 lanes) and N within the
    tuned kernels' limit.  Other shapes run the any-shape pre-pass (then the MFMA attention kernel
    when `padded_ok`).  The gate picks its own kernel (`gate_fast_shape`)."""
    return C in (128, 64) and H == 4 and D in (32, 16) and (N is None or N <= TUNED_MAX_N)


def gate_fast_shape(C_in, HD, C_out):
    """True when the tuned gate kernel applies: C_in = H*D = C_out in (128, 64)."""
    return C_in == HD == C_out and HD in (128, 64)


def generic_prep_forward(X, W_ln, B_ln, wqkv, WZ_c, BZ, *, eps=1e-5, apply_ln=True):
    """Any-shape pre-pass over X (N, N, C): (xln, q, k, v, bias) with q/k/v (N, N, H, D) in X's
    dtype and bias (H, N, N) fp32 (tops_tri_generic_prep)."""
    N, _, C = X.shape
    H, _, D, _ = wqkv.shape
    _native.check_device(X, wqkv, WZ_c, W_ln)
    if X.stride(2) != 1:
        X = X.contiguous()
    dt = X.dtype
    xln = torch.empty(N, N, C, device=X.device, dtype=dt)
    q, k, v = (torch.empty(N, N, H, D, device=X.device, dtype=dt) for _ in range(3))
    bias = torch.empty(H, N, N, device=X.device, dtype=torch.float32)
    BZf = None if BZ is None else _native.dense(BZ, torch.float32)
    _native.call(
        "tops_tri_generic_prep",
        X.data_ptr(),
        X.stride(0),
        X.stride(1),
        _native.ptr(_as(X, W_ln)) if apply_ln else None,
        _native.ptr(_as(X, B_ln)) if apply_ln else None,
        1 if apply_ln else 0,
        _as(X, wqkv).data_ptr(),
        _as(X, WZ_c).data_ptr(),
        _native.ptr(BZf),
        xln.data_ptr(),
        q.data_ptr(),
        k.data_ptr(),
        v.data_ptr(),
        bias.data_ptr(),
        N,
        C,
        H,
        D,
        float(eps),
        any_shape_dtype_code(dt),
        _native.stream_of(X),
    )
    return xln, q, k, v, bias


def padded_ok(N, H, D, dtype):
    """True when attention at a shape the pre-pass does not cover can run on the MFMA attention
    kernel after tops_tri_repack: D <= 32 (zero-padded to 32), H <= 64, 16-bit I/O, N within the
    tuned kernels' limit."""
    return D <= 32 and H <= 64 and dtype in (torch.bfloat16, torch.float16) and N <= TUNED_MAX_N


def padded_attention(q, k, v, bias, out, *, scale=1.0, mask=None):
    """generic_attention on the MFMA attention kernel: q, k, v (N, N, H, D) and the fp32 bias
    (H, N, N) of the any-shape pre-pass are repacked into the attention kernel's layouts with D
    zero-padded to 32 (tops_tri_repack), then tops_tri_attention runs; out (N, N, H*D)."""
    N, _, H, D = q.shape
    _native.check_device(q, k, v, bias, out, mask)
    assert padded_ok(N, H, D, q.dtype) and out.shape == (N, N, H * D) and out.stride(2) == 1
    ldn = row_stride(N)
    dev, dt = q.device, q.dtype
    Qp = torch.empty(N, H, ldn, 32, device=dev, dtype=dt)
    KV = torch.empty(N, H, ldn // 64, 4096, device=dev, dtype=dt)
    bt = torch.empty(H, (N + 31) // 32, ldn // 32, 1024, device=dev, dtype=dt)
    q, k, v = (_native.dense(t) for t in (q, k, v))
    bias = _native.dense(bias, torch.float32)
    _native.call("tops_tri_repack", q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                 Qp.data_ptr(), KV.data_ptr(), bt.data_ptr(), N, ldn, H, D, float(scale), io_dtype_code(dt),
                 _native.stream_of(q))
    if D % 8 == 0:  # the kernel writes heads of D in {8, 16, 24, 32} directly
        return attention_core(Qp, KV, bt, out, N=N, ldn=ldn, mask=mask)
    opad = torch.empty(N, N, H * 32, device=dev, dtype=dt)
    attention_core(Qp, KV, bt, opad, N=N, ldn=ldn, mask=mask)
    out.copy_(opad.view(N, N, H, 32)[..., :D].reshape(N, N, H * D))
    return out


def generic_attention(q, k, v, bias, out, *, scale=1.0, mask=None):
    """Any-shape attention core: out[i, q, h*D:(h+1)*D] = softmax_k(scale q.k + bias - 1e9 [masked]) v."""
    N, _, H, D = q.shape
    _native.check_device(q, k, v, bias, out, mask)
    assert out.shape == (N, N, H * D) and out.stride(2) == 1, "out must be (N, N, H*D) with unit last stride"
    m8 = None
    sm0 = sm1 = 0
    if mask is not None:
        m8 = mask.view(torch.int8) if mask.dtype in (torch.bool, torch.uint8) else mask.to(torch.int8)
        sm0, sm1 = m8.stride()
    _native.call(
        "tops_tri_generic_attention",
        q.data_ptr(),
        k.data_ptr(),
        v.data_ptr(),
        bias.data_ptr(),
        _native.ptr(m8),
        sm0,
        sm1,
        out.data_ptr(),
        out.stride(0),
        out.stride(1),
        N,
        H,
        D,
        float(scale),
        any_shape_dtype_code(q.dtype),
        _native.stream_of(q),
    )
    return out


def untile_bias(bias, N):
    """(H, N, N) view-copy of the pre-pass bias tiles (log2(e)-scaled, see tops_tri_prep)."""
    H, nqt, nkt, _ = bias.shape
    # element (32 qt + c, 32 kt + 16 j + 8 u + 4 hl + e) of a tile at (64 j + 32 hl + c) * 8 + 4 u + e
    t = bias.view(H, nqt, nkt, 2, 2, 32, 2, 4).permute(0, 1, 5, 2, 3, 6, 4, 7)  # h, qt, c, kt, j, u, hl, e
    return t.reshape(H, nqt * 32, nkt * 32)[:, :N, :N]


def attention_core(Qp, KV, bias, out, *, N, ldn, mask=None):
    """O[i, q, h*D:(h+1)*D] = softmax_k(scale Q.K + bias - 1e9 [mask[i,k] == 0]) V, written into `out`
    (N, N, H*D); Qp / KV hold 32-wide heads, of which the first D = out.shape[2] / H are written."""
    _, H, _, D32 = Qp.shape
    assert D32 == 32, "Qp must have the kernel's 32-wide head layout"
    D = out.shape[2] // H
    _native.check_device(Qp, KV, bias, out, mask)
    assert out.shape == (N, N, H * D) and out.stride(2) == 1, "out must be (N, N, H*D) with unit last stride"
    m8 = None
    sm0 = sm1 = 0
    if mask is not None:
        m8 = mask.view(torch.int8) if mask.dtype in (torch.bool, torch.uint8) else mask.to(torch.int8)
        if m8.stride(1) != 1:
            # every block reads its row's whole key mask a byte per key: with keys N bytes apart (the
            # ending node's mask.T) each byte is its own cache line, so copy to key-contiguous rows
            m8 = m8.contiguous()
        sm0, sm1 = m8.stride()
    _native.call(
        "tops_tri_attention",
        Qp.data_ptr(),
        KV.data_ptr(),
        bias.data_ptr(),
        _native.ptr(m8),
        sm0,
        sm1,
        out.data_ptr(),
        out.stride(0),
        out.stride(1),
        N,
        ldn,
        H,
        D,
        io_dtype_code(Qp.dtype),
        _native.stream_of(Qp),
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
    """Bias projection + attention over a pre-normalized X_ln (N, N, C), written into out (N, N, H*D).

    `Bias_buf` (optional (H, N, N) scratch) receives the pair bias, as in the reference.
    """
    N, N2, C = X_ln.shape
    assert N == N2
    H = WZ_c.shape[0]
    D = WQ_c.shape[1] // H
    assert WKV_c.shape == (C, 2 * H * D)
    assert out.shape == (N, N, H * D)
    wqkv = wqkv_from_layouts(_as(X_ln, WQ_c), _as(X_ln, WKV_c), H, D, _as(X_ln, WK_c), _as(X_ln, WV_c))
    if not fast_shape(C, H, D, N=N) or X_ln.dtype == torch.float32:
        xln, q, k, v, bias = generic_prep_forward(X_ln, None, None, wqkv, WZ_c, BZ, apply_ln=False)
        if Bias_buf is not None:
            Bias_buf.copy_(bias)
        if padded_ok(N, H, D, X_ln.dtype):
            return padded_attention(q, k, v, bias, out, scale=scale, mask=mask)
        return generic_attention(q, k, v, bias, out, scale=scale, mask=mask)
    Qp, KV, bias, ldn = prep_forward(X_ln, None, None, wqkv, WZ_c, BZ, scale=scale, apply_ln=False)
    if Bias_buf is not None:
        Bias_buf.copy_(untile_bias(bias, N).float() * (1.0 / LOG2E))
    return attention_core(Qp, KV, bias, out, N=N, ldn=ldn, mask=mask)


def _residual_views(o, residual, out, Cout, aligned):
    """The residual and destination of a fused residual add: (N1, N2, C_out) views with unit channel
    stride (`out` defaults to a new contiguous tensor; a residual that does not meet the kernel's
    stride / alignment rules is copied)."""
    N1, N2 = o.shape[0], o.shape[1]
    assert residual.shape == (N1, N2, Cout), "residual must be (N1, N2, C_out)"
    _native.check_device(o, residual, out)
    if residual.dtype != o.dtype or not aligned(residual):
        residual = residual.to(o.dtype).clone(memory_format=torch.contiguous_format)
    if out is None:
        out = torch.empty(N1, N2, Cout, device=o.device, dtype=o.dtype)
    assert out.shape == (N1, N2, Cout) and out.dtype == o.dtype, "out must be (N1, N2, C_out) of the I/O dtype"
    assert aligned(out), "out must have unit channel stride (and, at the tuned shape, 16-byte aligned tokens)"
    return residual, out


def gate_out_forward(o, gin, W_g, b_g, W_o, b_o, *, ln=None, residual=None, out=None):
    """out = ((o * sigmoid(g W_g^T + b_g)) -> io) W_o^T + b_o over (N1, N2, C) tokens.

    g = gin, or LN(gin) with ln = (w_ln, b_ln, eps).  o and gin may be strided views with unit
    channel stride.  With `residual` ((N1, N2, C_out), any token strides, unit channel stride) the
    result is residual + out, the add fused into the store; `out` (optional, with `residual`)
    is the destination view, e.g. a transposed view of a contiguous tensor.
    """
    N1, N2, C = o.shape
    _native.check_device(o, gin, W_g, W_o)
    Cin = gin.shape[-1]
    assert out is None or residual is not None, "out= is supported together with residual="
    if not gate_fast_shape(Cin, C, W_o.shape[0]) or o.dtype == torch.float32:
        return _gate_out_generic(o, gin, W_g, b_g, W_o, b_o, ln=ln, residual=residual, out=out)
    o = _native.vec16(o)
    gin = _native.vec16(gin.reshape(N1, N2, C) if gin.dim() != 3 else gin)
    w_ln = b_ln = None
    eps = 1e-5
    if ln is not None:
        w_ln, b_ln, eps = ln
    args = [o.data_ptr(), o.stride(0), o.stride(1), gin.data_ptr(), gin.stride(0), gin.stride(1),
            _native.ptr(_as(o, w_ln)), _native.ptr(_as(o, b_ln)), float(eps), 1 if ln is not None else 0,
            _as(o, W_g).data_ptr(), _native.ptr(_as(o, b_g)), _as(o, W_o).data_ptr(), _native.ptr(_as(o, b_o))]
    if residual is None:
        out = torch.empty(N1, N2, C, device=o.device, dtype=o.dtype)
        _native.call("tops_gate_out", *args, out.data_ptr(), N1, N2, C, io_dtype_code(o.dtype), _native.stream_of(o))
        return out

    residual, out = _residual_views(o, residual, out, C, _native.vec16_ok)
    _native.call("tops_gate_out_residual", *args, residual.data_ptr(), residual.stride(0), residual.stride(1),
                 out.data_ptr(), out.stride(0), out.stride(1), N1, N2, C, io_dtype_code(o.dtype), _native.stream_of(o))
    return out


def _gate_out_generic(o, gin, W_g, b_g, W_o, b_o, *, ln=None, residual=None, out=None):
    """gate_out_forward for any (C_in, H*D, C_out) (tops_gate_out_generic[_residual])."""
    N1, N2, HD = o.shape
    Cin, Cout = gin.shape[-1], W_o.shape[0]
    assert W_g.shape == (HD, Cin) and W_o.shape == (Cout, HD), "W_g (H*D, C_in) and W_o (C_out, H*D) expected"
    gin = gin.reshape(N1, N2, Cin) if gin.dim() != 3 else gin
    if o.stride(2) != 1:
        o = o.contiguous()
    if gin.stride(2) != 1:
        gin = gin.contiguous()
    w_ln = b_ln = None
    eps = 1e-5
    if ln is not None:
        w_ln, b_ln, eps = ln
    args = [o.data_ptr(), o.stride(0), o.stride(1), gin.data_ptr(), gin.stride(0), gin.stride(1),
            _native.ptr(_as(o, w_ln)), _native.ptr(_as(o, b_ln)), float(eps), 1 if ln is not None else 0,
            _as(o, W_g).data_ptr(), _native.ptr(_as(o, b_g)), _as(o, W_o).data_ptr(), _native.ptr(_as(o, b_o))]
    code = any_shape_dtype_code(o.dtype)
    if residual is None:
        out = torch.empty(N1, N2, Cout, device=o.device, dtype=o.dtype)
        _native.call("tops_gate_out_generic", *args, out.data_ptr(), N1, N2, Cin, HD, Cout, code, _native.stream_of(o))
        return out
    residual, out = _residual_views(o, residual, out, Cout, lambda t: t.stride(2) == 1)
    _native.call("tops_gate_out_generic_residual", *args, residual.data_ptr(), residual.stride(0), residual.stride(1),
                 out.data_ptr(), out.stride(0), out.stride(1), N1, N2, Cin, HD, Cout, code, _native.stream_of(o))
    return out


def fused_gate_forward(o_attn, qx_ln, WG, WO):
    """Out = (o_attn * sigmoid(qx_ln @ WG^T)) @ WO^T; o_attn (N, N, H, D) at any strides, WG/WO (out, in)."""
    N1, N2, H, D = o_attn.shape
    if o_attn.stride(3) != 1 or o_attn.stride(2) != D:
        o_attn = o_attn.contiguous()
    o = o_attn.as_strided((N1, N2, H * D), (o_attn.stride(0), o_attn.stride(1), 1))
    return gate_out_forward(o, qx_ln, WG, None, WO, None)
