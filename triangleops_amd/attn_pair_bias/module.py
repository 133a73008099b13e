"""Public API of attention with pair bias on gfx950.

Drop-in for `triangle_ops/attn_pair_bias/module.py` of the reference: same `precompute`,
`forward` and one-shot signatures and precompute keys (W_QKV, W_combined, sum_W_combined,
B_const), plus `wqkv_hm` (the head-major weight the kernel loads).  Three launches per call at the
tuned shape (C_s = C_z = C_out = 128, H = 4, D = 32): the Q / K / V pre-pass, the LN(Z) bias +
attention kernel, and the split merge fused with the gate + W_o (tops_apb_forward_gated; the gate
kernel itself when the keys are not split); other shapes run `apb_forward` then the gate.

Additive extension: `forward(..., mask=None)` / `attention_pair_bias(..., mask=None)` take an
optional (M,) key mask (masked keys -> -inf, as the reference's K-Fold variant does at
`benchmarks/references.py:273-274`); without it the behaviour is the reference's.

qk-norm variant: `attention_pair_bias_qknorm` has the signature of the reference's
`torch_attn_pair_bias_qknorm` (`benchmarks/references.py:230-277`: Q bias, optional LayerNorm over
the full H*D channel of Q and K before the head split, key mask, bias-free gate and output
projections); `forward_qknorm` is its per-call half over the same `precompute` dict.  Three
launches plus the gate: the Q/K/V pre-pass (Q bias, qk-norm and the softmax scale applied
there), the LN(Z) bias + attention kernel fed with those Q/K/V (and its split combine), the
gate + W_o kernel.
"""

import torch

from .._common.layouts import interleave_qkv, qkv_head_major
from .._common.ln_absorption import absorb_ln_matmul
from ..triangle_attn.kernel import gate_out_forward
from .kernel import apb_forward, apb_forward_qkv, apb_qkn_prep, gated_forward, gated_ok


def precompute(WQ, WK, WV, W_ln, B_ln, W_proj_z, B_proj_z, H, D):
    """One-time weight fusion.  Returns W_QKV (C, 3HD), W_combined (H, Cz) fp32, sum_W_combined (H,), B_const (H,)."""
    W_QKV = interleave_qkv(WQ, WK, WV, H, D)
    W_combined, sum_W_combined, B_const = absorb_ln_matmul(W_proj_z, W_ln, B_ln, weight_dtype=torch.float32)
    W_combined = W_combined.t().contiguous()
    if B_proj_z is not None:
        B_const = B_const + B_proj_z.float()
    return {
        "W_QKV": W_QKV,
        "W_combined": W_combined,
        "sum_W_combined": sum_W_combined,
        "B_const": B_const.contiguous(),
        "wqkv_hm": qkv_head_major(WQ, WK, WV, H, D),
    }


def forward(X, Z, pre, *, scale=1.0, eps=1e-5, W_proj_g, B_proj_g, W_proj_o, B_proj_o, mask=None, residual=None):
    """Per-call forward.  X (M, C_s), Z (M, M, C_z) -> (M, C_out); `residual` (M, C_out) returns
    residual + result, the add fused into the gate kernel's store (Pairformer single update)."""
    wq, Wc = pre.get("wqkv_hm"), pre["W_combined"]
    if wq is not None and wq.shape[2] == 32 and gated_ok(X, Z, Wc, W_proj_g, W_proj_o, residual):
        return gated_forward(X, Z, Wc, pre["sum_W_combined"], pre["B_const"], wq, W_proj_g, B_proj_g, W_proj_o,
                             B_proj_o, scale, eps, mask, residual)
    M = X.shape[0]
    H = pre["sum_W_combined"].shape[0]
    D = pre["W_QKV"].shape[1] // (3 * H)
    Og = torch.empty(M, H * D, device=X.device, dtype=X.dtype)
    apb_forward(
        X,
        pre["W_QKV"],
        Z,
        pre["W_combined"],
        pre["sum_W_combined"],
        pre["B_const"],
        Og,
        scale=scale,
        eps=eps,
        mask=mask,
        wqkv_hm=pre.get("wqkv_hm"),
    )
    res = None if residual is None else residual.view(M, 1, -1)
    return gate_out_forward(Og.view(M, 1, H * D), X, W_proj_g, B_proj_g, W_proj_o, B_proj_o,
                            residual=res).view(M, -1)


def attention_pair_bias(
    X,
    WQ,
    WK,
    WV,
    Z,
    W_ln,
    B_ln,
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
    pre = precompute(WQ, WK, WV, W_ln, B_ln, W_proj_z, B_proj_z, H, D)
    return forward(
        X,
        Z,
        pre,
        scale=scale,
        eps=eps,
        W_proj_g=W_proj_g,
        B_proj_g=B_proj_g,
        W_proj_o=W_proj_o,
        B_proj_o=B_proj_o,
        mask=mask,
    )


def forward_qknorm(X, Z, pre, *, b_q=None, qkn_w_q=None, qkn_b_q=None, qkn_w_k=None, qkn_b_k=None, key_mask=None,
                   scale=1.0, eps=1e-5, W_proj_g, W_proj_o):
    """Per-call forward of the qk-norm variant over a `precompute` dict.  X (M, C_s), Z (M, M, C_z) ->
    (M, C_out).  qk-norm is on when `qkn_w_q` is given (q with (qkn_w_q, qkn_b_q), k with
    (qkn_w_k, qkn_b_k); a None weight / bias acts as 1 / 0), as in references.py:262-264."""
    M = X.shape[0]
    H = pre["sum_W_combined"].shape[0]
    D = pre["W_QKV"].shape[1] // (3 * H)
    qkn = None if qkn_w_q is None else (qkn_w_q, qkn_b_q, qkn_w_k, qkn_b_k)
    q, k, v = apb_qkn_prep(X, pre["wqkv_hm"], b_q, qkn, eps, qscale=scale)
    Og = torch.empty(M, H * D, device=X.device, dtype=X.dtype)
    apb_forward_qkv(q, k, v, Z, pre["W_combined"], pre["sum_W_combined"], pre["B_const"], Og, scale=1.0, eps=eps,
                    mask=key_mask)
    return gate_out_forward(Og.view(M, 1, H * D), X, W_proj_g, None, W_proj_o, None).view(M, -1)


def attention_pair_bias_qknorm(
    X,
    WQ,
    b_q,
    WK,
    WV,
    Z,
    W_ln,
    B_ln,
    W_proj_z,
    B_proj_z,
    W_proj_g,
    W_proj_o,
    H,
    D,
    *,
    qkn_w_q=None,
    qkn_b_q=None,
    qkn_w_k=None,
    qkn_b_k=None,
    key_mask=None,
    scale=1.0,
    eps=1e-5,
):
    """One-shot qk-norm variant (precompute included); arguments as the reference's
    `torch_attn_pair_bias_qknorm` (benchmarks/references.py:230-250)."""
    pre = precompute(WQ, WK, WV, W_ln, B_ln, W_proj_z, B_proj_z, H, D)
    return forward_qknorm(
        X,
        Z,
        pre,
        b_q=b_q,
        qkn_w_q=qkn_w_q,
        qkn_b_q=qkn_b_q,
        qkn_w_k=qkn_w_k,
        qkn_b_k=qkn_b_k,
        key_mask=key_mask,
        scale=scale,
        eps=eps,
        W_proj_g=W_proj_g,
        W_proj_o=W_proj_o,
    )
