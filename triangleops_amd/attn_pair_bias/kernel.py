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
    X = X if X.is_contiguous() else X.contiguous()
    if Z.stride(2) != 1 or Z.stride(0) % 8 or Z.stride(1) % 8:
        Z = Z.contiguous()
    if wqkv_hm is None:
        wqkv_hm = wqkv_from_interleaved(W_QKV, H, D)
    if wqkv_hm.dtype != X.dtype:
        wqkv_hm = wqkv_hm.to(X.dtype)
    Wc = W_combined.float().contiguous()
    sWc = sum_W_combined.float().contiguous()
    Bc = B_const.float().contiguous()
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == M, "mask must be (M,)"
    assert Og.is_contiguous()
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


def _apb_generic(X, W_QKV, Z, W_combined, B_const, Og, scale, eps, mask, wqkv_hm, H, D):
    """apb_forward at any (C_s, C_z, H, D) or with fp32 I/O (tops_apb_generic_prep / _attention);
    the Q/K/V and bias scratch is allocated here."""
    M, C = X.shape
    Cz = Z.shape[2]
    code = any_shape_dtype_code(X.dtype)
    _native.check_device(X, W_QKV, Z, W_combined, Og, mask)
    X = X if X.is_contiguous() else X.contiguous()
    if Z.stride(2) != 1:
        Z = Z.contiguous()
    if wqkv_hm is None:
        wqkv_hm = wqkv_from_interleaved(W_QKV, H, D)
    if wqkv_hm.dtype != X.dtype:
        wqkv_hm = wqkv_hm.to(X.dtype)
    wqkv_hm = wqkv_hm.contiguous()
    Wc = W_combined.float().contiguous()
    Bc = B_const.float().contiguous()
    m8 = _native.mask_i8(mask)
    if m8 is not None:
        assert m8.numel() == M, "mask must be (M,)"
    assert Og.is_contiguous()
    q, k, v = (torch.empty(M, H, D, device=X.device, dtype=X.dtype) for _ in range(3))
    bias = torch.empty(H, M, M, device=X.device, dtype=torch.float32)
    st = _native.stream_of(X)
    _native.call("tops_apb_generic_prep", X.data_ptr(), wqkv_hm.data_ptr(), Z.data_ptr(), Z.stride(0), Z.stride(1),
                 Wc.data_ptr(), Bc.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(), M, C, Cz, H,
                 D, float(eps), code, st)
    _native.call("tops_apb_generic_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                 _native.ptr(m8), Og.data_ptr(), M, H, D, float(scale), code, st)
    return Og
