"""Low-level launcher of the gfx950 attention-pair-bias kernel.

Same name and arguments as the reference's `apb_forward` (`attn_pair_bias/kernel.py:205-257`),
with two keyword-only additions: `mask` (an optional (M,) key mask, masked keys -> -inf) and
`wqkv_hm`, the head-major (H, 3, D, C) weight the kernel loads (derived from W_QKV when absent).
"""

import torch

from .. import _native
from .._common.dtype import any_shape_dtype_code, io_dtype_code


def wqkv_from_interleaved(W_QKV, H, D):
    """(C, 3*H*D) per-head [Q_h | K_h | V_h] columns -> (H, 3, D, C)."""
    C = W_QKV.shape[0]
    return W_QKV.reshape(C, H, 3, D).permute(1, 2, 3, 0).contiguous()


def apb_forward(X, W_QKV, Z, W_combined, sum_W_combined, B_const, Og, scale=1.0, eps=1e-5, *, mask=None,
                wqkv_hm=None):
    """Fused QKV projection + LN(Z) bias projection + attention into Og (M, H*D)."""
    M, C = X.shape
    H = sum_W_combined.shape[0]
    D = W_QKV.shape[1] // (3 * H)
    assert W_QKV.shape == (C, 3 * H * D)
    assert Z.shape[:2] == (M, M)
    Cz = Z.shape[2]
    assert W_combined.shape == (H, Cz)
    assert B_const.shape == (H,)
    assert Og.shape == (M, H * D)
    if not (C == 128 and Cz == 128 and H == 4 and D == 32) or X.dtype == torch.float32:
        return _apb_generic(X, W_QKV, Z, W_combined, B_const, Og, scale, eps, mask, wqkv_hm, H, D)
    code = io_dtype_code(X.dtype)
    _native.check_device(X, W_QKV, Z, W_combined, Og, mask)
    X = _native.dense(X)  # the kernels index X rows without a stride
    Z = _native.vec16(Z)  # Z's strides are passed
    if wqkv_hm is None:
        wqkv_hm = wqkv_from_interleaved(W_QKV, H, D)
    wqkv_hm = _native.dense(wqkv_hm, X.dtype)
    Wc = _native.dense(W_combined, torch.float32)
    sWc = _native.dense(sum_W_combined, torch.float32)
    Bc = _native.dense(B_const, torch.float32)
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == M, "mask must be (M,)"
    assert Og.is_contiguous() and Og.data_ptr() % 16 == 0, "Og must be contiguous and 16-byte aligned"
    nbytes = _native.apb_workspace_bytes(M, H, D)
    work = torch.empty(max(nbytes, 1), device=X.device, dtype=torch.uint8) if nbytes else None
    _native.call(
        "tops_apb_forward",
        X.data_ptr(),
        wqkv_hm.data_ptr(),
        Z.data_ptr(),
        Z.stride(0),
        Z.stride(1),
        Wc.data_ptr(),
        sWc.data_ptr(),
        Bc.data_ptr(),
        _native.ptr(m8),
        Og.data_ptr(),
        _native.ptr(work),
        M,
        C,
        Cz,
        H,
        D,
        float(scale),
        float(eps),
        code,
        _native.stream_of(X),
    )
    return Og


def gated_ok(X, Z, W_combined, W_g, W_o, residual=None):
    """True when apb_forward_gated applies: the tuned shape (C_s = C_z = 128, H = 4, D = 32) with
    C_out = 128 and 16-bit I/O (the residual, if any, (M, 128) with unit channel stride)."""
    M, C = X.shape
    H = W_combined.shape[0]
    ok = (C == 128 and Z.shape[2] == 128 and H == 4 and W_combined.shape[1] == 128 and X.dtype != torch.float32
          and tuple(W_g.shape) == (128, 128) and tuple(W_o.shape) == (128, 128))
    return ok and (residual is None or tuple(residual.shape) == (M, 128))


def apb_forward_gated(X, Z, W_combined, sum_W_combined, B_const, wqkv_hm, W_g, b_g, W_o, b_o, *, scale=1.0,
                      eps=1e-5, mask=None, residual=None):
    """out = ((Og * sigmoid(X W_g^T + b_g)) -> io) W_o^T + b_o (+ residual), Og = apb_forward(...):
    the attention with the gate and output projection of attn_pair_bias/module.py:69-70 fused.  With
    split keys: tops_apb_forward (Og = NULL) then tops_apb_merge_gate (the split merge, gate and W_o in
    one kernel); otherwise tops_apb_forward_gated.  Requires gated_ok(...); returns (M, 128)."""
    assert gated_ok(X, Z, W_combined, W_g, W_o, residual) and wqkv_hm.shape[2] == 32
    return gated_forward(X, Z, W_combined, sum_W_combined, B_const, wqkv_hm, W_g, b_g, W_o, b_o, scale, eps, mask,
                         residual)


def _dense_as(t, dt):
    """_native.dense(t, dt) with the common case (already dense, aligned, of dtype dt) tested inline."""
    if t is None or (t.dtype is dt and t.is_contiguous() and t.data_ptr() % 16 == 0):
        return t
    return _native.dense(t, dt)


def gated_forward(X, Z, Wc, sWc, Bc, wqkv_hm, W_g, b_g, W_o, b_o, scale, eps, mask, residual):
    """apb_forward_gated after gated_ok(...) has been established by the caller.  Everything the
    first launch reads is checked and prepared before it; the gate's operands (W_g, b_g, W_o, b_o,
    residual) while the attention runs."""
    M = X.shape[0]
    dt = X.dtype
    code = io_dtype_code(dt)
    f32 = torch.float32
    nqkv = (3 * M * 4 * 32 * 2 + 255) // 256 * 256
    nbytes = _native.apb_workspace_bytes(M, 4, 32)
    if nbytes > nqkv:
        # split keys: three launches, each issued once its own operands are checked, the next one's
        # prepared while the previous runs: the Q / K / V pre-pass (tops_apb_qkn_prep without Q bias
        # or norm runs tops_apb_forward's first kernel), the attention (tops_apb_forward_qkv with
        # Og = NULL leaves the split partials after Q / K / V, where tops_apb_forward leaves them),
        # then tops_apb_merge_gate; the same kernels and bits as tops_apb_forward_gated
        _native.check_device(X, wqkv_hm)
        X = _dense_as(X, dt)  # X, the weights, biases and residual are indexed without strides
        wqkv_hm = _dense_as(wqkv_hm, dt)
        st = _native.stream_of(X)
        work = torch.empty(nbytes, device=X.device, dtype=torch.uint8)
        w0 = work.data_ptr()
        q, k, v = w0, w0 + M * 256, w0 + 2 * M * 256
        _native.call("tops_apb_qkn_prep", X.data_ptr(), wqkv_hm.data_ptr(), None, 0, None, None, None, None, q, k, v,
                     M, 128, 4, 32, float(scale), float(eps), code, st)
        _native.check_device(X, Z, Wc, sWc, Bc, mask)
        Z = _native.vec16(Z)  # Z's strides are passed
        Wc, sWc, Bc = _dense_as(Wc, f32), _dense_as(sWc, f32), _dense_as(Bc, f32)
        m8 = _native.mask_i8(mask)
        if m8 is not None:
            assert m8.numel() == M, "mask must be (M,)"
        _native.call("tops_apb_forward_qkv", q, k, v, Z.data_ptr(), Z.stride(0), Z.stride(1), Wc.data_ptr(),
                     sWc.data_ptr(), Bc.data_ptr(), None if m8 is None else m8.data_ptr(), None, w0 + nqkv, M, 128,
                     128, 4, 32, 1.0, float(eps), code, st)
        _native.check_device(X, W_g, b_g, W_o, b_o, residual)
        W_g, b_g, W_o, b_o, res = (_dense_as(W_g, dt), _dense_as(b_g, dt), _dense_as(W_o, dt), _dense_as(b_o, dt),
                                   _dense_as(residual, dt))
        out = torch.empty(M, 128, device=X.device, dtype=dt)
        _native.call("tops_apb_merge_gate", w0 + nqkv, X.data_ptr(), W_g.data_ptr(), _native.ptr(b_g),
                     W_o.data_ptr(), _native.ptr(b_o), _native.ptr(res), out.data_ptr(), M, 4, 32, code, st)
        return out
    _native.check_device(X, Z, wqkv_hm, Wc, sWc, Bc, mask, W_g, b_g, W_o, b_o, residual)
    X = _dense_as(X, dt)
    Z = _native.vec16(Z)
    wqkv_hm = _dense_as(wqkv_hm, dt)
    Wc, sWc, Bc = _dense_as(Wc, f32), _dense_as(sWc, f32), _dense_as(Bc, f32)
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == M, "mask must be (M,)"
    st = _native.stream_of(X)
    W_g, b_g, W_o, b_o, res = (_dense_as(W_g, dt), _dense_as(b_g, dt), _dense_as(W_o, dt), _dense_as(b_o, dt),
                               _dense_as(residual, dt))
    out = torch.empty(M, 128, device=X.device, dtype=dt)
    nbytes = _native.apb_gated_workspace_bytes(M, 4, 32)
    work = torch.empty(max(nbytes, 1), device=X.device, dtype=torch.uint8) if nbytes else None
    _native.call("tops_apb_forward_gated", X.data_ptr(), wqkv_hm.data_ptr(), Z.data_ptr(), Z.stride(0), Z.stride(1),
                 Wc.data_ptr(), sWc.data_ptr(), Bc.data_ptr(), _native.ptr(m8), W_g.data_ptr(), _native.ptr(b_g),
                 W_o.data_ptr(), _native.ptr(b_o), _native.ptr(res), out.data_ptr(), _native.ptr(work), M, 128,
                 128, 4, 32, 128, float(scale), float(eps), code, st)
    return out


def _apb_generic(X, W_QKV, Z, W_combined, B_const, Og, scale, eps, mask, wqkv_hm, H, D):
    """apb_forward at any (C_s, C_z, H, D) or with fp32 I/O (tops_apb_generic_prep / _attention);
    the Q/K/V and bias scratch is allocated here."""
    M, C = X.shape
    Cz = Z.shape[2]
    code = any_shape_dtype_code(X.dtype)
    _native.check_device(X, W_QKV, Z, W_combined, Og, mask)
    X = _native.dense(X)
    if Z.stride(2) != 1:
        Z = Z.contiguous()
    if wqkv_hm is None:
        wqkv_hm = wqkv_from_interleaved(W_QKV, H, D)
    wqkv_hm = _native.dense(wqkv_hm, X.dtype)
    Wc = _native.dense(W_combined, torch.float32)
    Bc = _native.dense(B_const, torch.float32)
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == M, "mask must be (M,)"
    assert Og.is_contiguous() and Og.data_ptr() % 16 == 0, "Og must be contiguous and 16-byte aligned"
    q, k, v = (torch.empty(M, H, D, device=X.device, dtype=X.dtype) for _ in range(3))
    bias = torch.empty(H, M, M, device=X.device, dtype=torch.float32)
    st = _native.stream_of(X)
    _native.call("tops_apb_generic_prep", X.data_ptr(), wqkv_hm.data_ptr(), Z.data_ptr(), Z.stride(0), Z.stride(1),
                 Wc.data_ptr(), Bc.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(), M, C, Cz, H,
                 D, float(eps), code, st)
    _native.call("tops_apb_generic_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                 _native.ptr(m8), Og.data_ptr(), M, H, D, float(scale), code, st)
    return Og



def _io(t, dtype):
    """A per-channel parameter as a dense, aligned vector of the I/O dtype (no copy when it already is)."""
    return _native.dense(t, dtype)


def apb_qkn_prep(X, wqkv_hm, b_q=None, qkn=None, eps=1e-5, qscale=1.0):
    """q = qscale * (X.Wq + b_q), k = X.Wk, v = X.Wv as (M, H*D) io tensors; with qkn = (w_q, b_q_ln,
    w_k, b_k_ln) q and k are LayerNormed over the full H*D channel first (before the scale)
    (benchmarks/references.py:258-264)."""
    M, C = X.shape
    H, three, D, C2 = wqkv_hm.shape
    assert three == 3 and C2 == C, "wqkv_hm must be (H, 3, D, C)"
    code = any_shape_dtype_code(X.dtype)
    _native.check_device(X, wqkv_hm, b_q, *(qkn or ()))
    X = _native.dense(X)
    w = _native.dense(wqkv_hm, X.dtype)
    bq = _io(b_q, X.dtype)
    gq, bqn, gk, bkn = (_io(t, X.dtype) for t in (qkn or (None,) * 4))
    for t in (bq, gq, bqn, gk, bkn):
        assert t is None or t.numel() == H * D, "Q bias and qk-norm parameters must have H*D elements"
    q, k, v = (torch.empty(M, H * D, device=X.device, dtype=X.dtype) for _ in range(3))
    _native.call("tops_apb_qkn_prep", X.data_ptr(), w.data_ptr(), _native.ptr(bq), 1 if qkn is not None else 0,
                 _native.ptr(gq), _native.ptr(bqn), _native.ptr(gk), _native.ptr(bkn), q.data_ptr(), k.data_ptr(),
                 v.data_ptr(), M, C, H, D, float(qscale), float(eps), code, _native.stream_of(X))
    return q, k, v


def apb_forward_qkv(q, k, v, Z, W_combined, sum_W_combined, B_const, Og, scale=1.0, eps=1e-5, *, mask=None):
    """LN(Z) bias + attention into Og (M, H*D) with q, k, v (M, H*D) given (from `apb_qkn_prep`;
    pass scale=1.0 when q is already scaled there)."""
    M, HD = q.shape
    H = sum_W_combined.shape[0]
    D = HD // H
    assert k.shape == v.shape == (M, HD) and Og.shape == (M, HD)
    assert Z.shape[:2] == (M, M)
    Cz = Z.shape[2]
    assert W_combined.shape == (H, Cz) and B_const.shape == (H,)
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == M, "mask must be (M,)"
    assert Og.is_contiguous() and Og.data_ptr() % 16 == 0, "Og must be contiguous and 16-byte aligned"
    Wc, sWc, Bc = (_native.dense(t, torch.float32) for t in (W_combined, sum_W_combined, B_const))
    q, k, v = (_native.dense(t) for t in (q, k, v))
    _native.check_device(q, k, v, Z, W_combined, Og, mask)
    st = _native.stream_of(q)
    if HD == 128 and Cz == 128 and H == 4 and D == 32 and q.dtype != torch.float32:
        Z = _native.vec16(Z)
        nbytes = _native.apb_workspace_bytes(M, H, D)
        work = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8) if nbytes else None
        _native.call("tops_apb_forward_qkv", q.data_ptr(), k.data_ptr(), v.data_ptr(), Z.data_ptr(), Z.stride(0),
                     Z.stride(1), Wc.data_ptr(), sWc.data_ptr(), Bc.data_ptr(), _native.ptr(m8), Og.data_ptr(),
                     _native.ptr(work), M, HD, Cz, H, D, float(scale), float(eps), io_dtype_code(q.dtype), st)
        return Og
    # any shape / fp32: the generic LN(Z) bias (its own Q/K/V outputs are discarded) and attention
    code = any_shape_dtype_code(q.dtype)
    if Z.stride(2) != 1:
        Z = Z.contiguous()
    wid = torch.eye(HD, device=q.device, dtype=q.dtype).reshape(H, 1, D, HD).expand(H, 3, D, HD).contiguous()
    scratch = torch.empty(3, M, HD, device=q.device, dtype=q.dtype)
    bias = torch.empty(H, M, M, device=q.device, dtype=torch.float32)
    _native.call("tops_apb_generic_prep", q.data_ptr(), wid.data_ptr(), Z.data_ptr(), Z.stride(0), Z.stride(1),
                 Wc.data_ptr(), Bc.data_ptr(), scratch[0].data_ptr(), scratch[1].data_ptr(), scratch[2].data_ptr(),
                 bias.data_ptr(), M, HD, Cz, H, D, float(eps), code, st)
    _native.call("tops_apb_generic_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                 _native.ptr(m8), Og.data_ptr(), M, H, D, float(scale), code, st)
    return Og
