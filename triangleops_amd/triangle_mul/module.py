"""Public API of the triangle multiplicative update (outgoing / incoming) on gfx950.

Drop-in for `triangle_ops/triangle_mul/module.py` of the reference: same `precompute`,
`forward` and one-shot signatures, the same 12-key precompute dict and the same
LayerNorm-affine folding (g_out folds LN_in because it gates on x, reference `:48`).
The per-call path is three HIP launches:

    input phase  (LN_in + gated projection + mask, channel-major; incoming transposed)
    einsum       (batched MFMA GEMM, y = A . B^T per channel)
    output phase (LN_out(y) projection gated by LN_in(x) projection, token-major)

x is (B, L, L, C) with C = 128; B > 1 is supported.
"""

from .._common.ln_absorption import absorb_ln
from .kernel import input_phase, output_phase, triangle_einsum

_DIRECTIONS = ("outgoing", "incoming")


def precompute(
    norm_in_weight,
    norm_in_bias,
    p_in_weight,
    g_in_weight,
    norm_out_weight,
    norm_out_bias,
    p_out_weight,
    g_out_weight,
):
    """One-time fold of the LN affines into the four projections (nn.Linear (out, in) weights).

    p_in/g_in: (2C, C); p_out/g_out: (C, C).  g_out absorbs LN_in (it gates on x).
    """
    dt = p_in_weight.dtype
    p_in_c, sWp_in, Bp_in = absorb_ln(p_in_weight, norm_in_weight, norm_in_bias, weight_dtype=dt)
    g_in_c, sWg_in, Bg_in = absorb_ln(g_in_weight, norm_in_weight, norm_in_bias, weight_dtype=dt)
    p_out_c, sWp_out, Bp_out = absorb_ln(p_out_weight, norm_out_weight, norm_out_bias, weight_dtype=dt)
    g_out_c, sWg_out, Bg_out = absorb_ln(g_out_weight, norm_in_weight, norm_in_bias, weight_dtype=dt)
    return {
        "p_in_combined": p_in_c,
        "g_in_combined": g_in_c,
        "p_out_combined": p_out_c,
        "g_out_combined": g_out_c,
        "sum_W_p_in": sWp_in,
        "sum_W_g_in": sWg_in,
        "sum_W_p_out": sWp_out,
        "sum_W_g_out": sWg_out,
        "B_p_in_const": Bp_in,
        "B_g_in_const": Bg_in,
        "B_p_out_const": Bp_out,
        "B_g_out_const": Bg_out,
    }


def forward(x, pre, *, direction, mask=None, eps=1e-5, residual=None):
    """Per-call forward with precomputed weights.  x (B, L, L, C) -> (B, L, L, C).

    `residual` (optional extra, e.g. x itself in a Pairformer block): returns residual + result
    with the add fused into the output phase's store."""
    if direction not in _DIRECTIONS:
        raise ValueError(f"unknown direction: {direction!r} (expected 'outgoing'/'incoming')")
    B, L, _, C = x.shape
    ld = max(64, (L + 63) // 64 * 64)
    ab = input_phase(
        x,
        mask,
        pre["p_in_combined"],
        pre["g_in_combined"],
        pre["sum_W_p_in"],
        pre["sum_W_g_in"],
        pre["B_p_in_const"],
        pre["B_g_in_const"],
        eps,
        transpose=direction == "incoming",
        ld=ld,
    )
    y = triangle_einsum(ab, L, ld, C, B)
    return output_phase(
        y,
        x,
        pre["p_out_combined"],
        pre["g_out_combined"],
        pre["sum_W_p_out"],
        pre["sum_W_g_out"],
        pre["B_p_out_const"],
        pre["B_g_out_const"],
        eps,
        ldy=ld,
        residual=residual,
    )


def triangle_multiplicative_update(
    x,
    *,
    direction,
    mask=None,
    eps=1e-5,
    norm_in_weight,
    norm_in_bias,
    p_in_weight,
    g_in_weight,
    norm_out_weight,
    norm_out_bias,
    p_out_weight,
    g_out_weight,
):
    """One-shot (precompute included).  For amortized latency call `precompute` once, then `forward`."""
    pre = precompute(
        norm_in_weight,
        norm_in_bias,
        p_in_weight,
        g_in_weight,
        norm_out_weight,
        norm_out_bias,
        p_out_weight,
        g_out_weight,
    )
    return forward(x, pre, direction=direction, mask=mask, eps=eps)
