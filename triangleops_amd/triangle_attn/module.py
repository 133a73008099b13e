"""Public API of triangle attention (AlphaFold-3 starting node) on gfx950.

Drop-in for `triangle_ops/triangle_attn/module.py` of the reference: same `precompute`,
`forward` and one-shot signatures and precompute keys (WQ_c, WKV_c, WK_c, WV_c, WZ_c, BZ,
W_ln, B_ln), plus `wqkv_hm`, the head-major weight the kernels load.  Three launches per
call:

    prep        LN(x), the row-shared bias and Q/K/V of all heads in one pass over x
    attention   per (row, head, query chunk): flash attention over the row's keys
    gate_out    sigmoid(LN(x) W_g^T) gate (LN recomputed from x) and W_o projection

The ending node is the same op on X.transpose(0, 1) (and mask.T): the pre-pass and the gate
read the transposed view in place, so no transpose copy is made.  Any N is handled natively:
`pad_to` is accepted for signature compatibility and ignored.
"""

import torch

from .._common.layouts import interleave_kv, qkv_head_major
from .kernel import (attention_core, fast_shape, gate_out_forward, generic_attention, generic_prep_forward,
                     padded_attention, padded_ok, prep_forward)


def precompute(W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, H, D):
    """One-time layout prep.  WQ/WK/WV (C_in, H*D), W_proj_z (C_in, H) (matmul convention)."""
    WQ_c = WQ.contiguous()
    WKV_c = interleave_kv(WK, WV, H, D)
    WK_c = WK.contiguous() if D == 16 else None
    WV_c = WV.contiguous() if D == 16 else None
    WZ_c = W_proj_z.t().contiguous()
    if B_proj_z is None:
        BZ = torch.zeros(H, device=WQ.device, dtype=torch.float32)
    else:
        BZ = B_proj_z.float().contiguous()
    return {
        "WQ_c": WQ_c,
        "WKV_c": WKV_c,
        "WK_c": WK_c,
        "WV_c": WV_c,
        "WZ_c": WZ_c,
        "BZ": BZ,
        "W_ln": W_ln,
        "B_ln": B_ln,
        "wqkv_hm": qkv_head_major(WQ, WK, WV, H, D),
    }


def forward(X, pre, *, mask=None, scale=1.0, eps=1e-5, W_proj_g, B_proj_g, W_proj_o, B_proj_o, pad_to=32,
            residual=None, out=None):
    """Per-call forward.  X (N, N, C_in) -> (N, N, C_out); mask (N, N), nonzero = valid key.

    Optional extras for composing a Pairformer block: `residual` (N, N, C_out) returns
    residual + result with the add fused into the gate kernel's store; `out` is then the
    destination view (for the ending node, a transposed view of the untransposed pair tensor)."""
    assert B_proj_g is None and B_proj_o is None, (
        "fused gate path assumes bias-free linear_g / linear_o (K-Fold LinearNoBias)"
    )
    N = X.shape[0]
    wqkv = pre["wqkv_hm"]
    if wqkv.dtype != X.dtype:
        wqkv = wqkv.to(X.dtype)
    H, _, D, C = wqkv.shape
    if not fast_shape(C, H, D, N) or X.dtype == torch.float32:
        # any-shape pre-pass: other shapes, N above the tuned limit, fp32 I/O
        xln, q, k, v, bias = generic_prep_forward(X, pre["W_ln"], pre["B_ln"], wqkv, pre["WZ_c"], pre["BZ"], eps=eps)
        O = torch.empty(N, N, H * D, device=X.device, dtype=X.dtype)
        if padded_ok(N, H, D, X.dtype):  # D <= 32 in 16-bit I/O: the MFMA attention kernel, D padded
            padded_attention(q, k, v, bias, O, scale=scale, mask=mask)
        else:
            generic_attention(q, k, v, bias, O, scale=scale, mask=mask)
        return gate_out_forward(O, xln, W_proj_g, None, W_proj_o, None, residual=residual, out=out)
    Qp, KV, bias, ldn = prep_forward(X, pre["W_ln"], pre["B_ln"], wqkv, pre["WZ_c"], pre["BZ"], scale=scale, eps=eps)
    O = torch.empty(N, N, H * D, device=X.device, dtype=X.dtype)
    attention_core(Qp, KV, bias, O, N=N, ldn=ldn, mask=mask)
    # the gate reads LN(X); it is recomputed from X inside the gate kernel (the tuned one when
    # C_in = H*D = C_out, e.g. 128 / 128 / 128 or the Apo shape's 64 / 64 / 64)
    return gate_out_forward(O, X, W_proj_g, None, W_proj_o, None, ln=(pre["W_ln"], pre["B_ln"], eps),
                            residual=residual, out=out)


def triangle_attention(
    X,
    W_ln,
    B_ln,
    WQ,
    WK,
    WV,
    W_proj_z,
    B_proj_z,
    W_proj_g,
    B_proj_g,
    W_proj_o,
    B_proj_o,
    H,
    D,
    scale=1.0,
    eps=1e-5,
    mask=None,
):
    """One-shot (precompute included).  For amortized latency call `precompute` once, then `forward`."""
    pre = precompute(W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, H, D)
    return forward(
        X,
        pre,
        mask=mask,
        scale=scale,
        eps=eps,
        W_proj_g=W_proj_g,
        B_proj_g=B_proj_g,
        W_proj_o=W_proj_o,
        B_proj_o=B_proj_o,
    )
