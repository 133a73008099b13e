"""Pairformer block composition over the three ops (the step after each op on the hot path).

The reference ships the three AlphaFold-3 Pairformer primitives but no block; a caller writes the
residual stream around them.  This module does it with the residual add fused into each op's
output kernel, so z is not read and written once more per update:

    pair_stack:     z <- z + tmu(z, outgoing)
                    z <- z + tmu(z, incoming)
                    z <- z + triangle_attention(z)                       (starting node)
                    z <- z + triangle_attention(z^T)^T                   (ending node; written straight
                                                                          into z's layout)
    single_update:  s <- s + attention_pair_bias(s, z)

Each sum is rounded once to the I/O type from the op's rounded result, so the fused block equals
the unfused sequence `z + op(z)` bit for bit.  The pair and single transitions of a full
Pairformer block are plain two-layer MLPs and are not part of these ops.

Weights are passed as the keyword dicts of the ops' own signatures:
  tmu_out, tmu_in        norm_in_weight, norm_in_bias, p_in_weight, g_in_weight, norm_out_weight,
                         norm_out_bias, p_out_weight, g_out_weight
  tri_start, tri_end     W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, W_proj_g, W_proj_o
  apb                    WQ, WK, WV, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, B_proj_g, W_proj_o, B_proj_o
"""

from __future__ import annotations

import torch

from . import attn_pair_bias, triangle_attn, triangle_mul

_TMU_KEYS = ("norm_in_weight", "norm_in_bias", "p_in_weight", "g_in_weight", "norm_out_weight", "norm_out_bias",
             "p_out_weight", "g_out_weight")


def precompute(tmu_out, tmu_in, tri_start, tri_end, apb=None, *, H=4, D=32):
    """One-time weight folding of every op of the block -> dict of the ops' precompute dicts."""
    pre = {
        "tmu_out": triangle_mul.precompute(*(tmu_out[k] for k in _TMU_KEYS)),
        "tmu_in": triangle_mul.precompute(*(tmu_in[k] for k in _TMU_KEYS)),
        "H": H,
        "D": D,
    }
    for name, w in (("tri_start", tri_start), ("tri_end", tri_end)):
        pre[name] = triangle_attn.precompute(w["W_ln"], w["B_ln"], w["WQ"], w["WK"], w["WV"], w["W_proj_z"],
                                             w["B_proj_z"], H, D)
        pre[name + "_proj"] = (w["W_proj_g"], w["W_proj_o"])
    if apb is not None:
        pre["apb"] = attn_pair_bias.precompute(apb["WQ"], apb["WK"], apb["WV"], apb["W_ln"], apb["B_ln"],
                                               apb["W_proj_z"], apb["B_proj_z"], H, D)
        pre["apb_proj"] = (apb["W_proj_g"], apb.get("B_proj_g"), apb["W_proj_o"], apb.get("B_proj_o"))
    return pre


def pair_stack(z, pre, *, pair_mask=None, eps=1e-5, scale=None):
    """The four pair updates with residuals.  z (N, N, C) -> new (N, N, C) tensor; pair_mask (N, N)
    (nonzero = valid pair) masks the triangle updates' tokens and the attentions' keys (transposed
    for the ending node).  scale defaults to D**-0.5."""
    N = z.shape[0]
    assert z.dim() == 3 and z.shape[1] == N, "z must be (N, N, C)"
    scale = pre["D"] ** -0.5 if scale is None else scale
    m3 = None if pair_mask is None else pair_mask.reshape(1, N, N)
    z1 = triangle_mul.forward(z[None], pre["tmu_out"], direction="outgoing", mask=m3, eps=eps, residual=z[None])
    z2 = triangle_mul.forward(z1, pre["tmu_in"], direction="incoming", mask=m3, eps=eps, residual=z1)[0]
    wg, wo = pre["tri_start_proj"]
    z3 = triangle_attn.forward(z2, pre["tri_start"], mask=pair_mask, scale=scale, eps=eps, W_proj_g=wg,
                               B_proj_g=None, W_proj_o=wo, B_proj_o=None, residual=z2)
    z4 = torch.empty_like(z3)
    wg, wo = pre["tri_end_proj"]
    z3t = z3.transpose(0, 1)
    triangle_attn.forward(z3t, pre["tri_end"], mask=None if pair_mask is None else pair_mask.T, scale=scale,
                          eps=eps, W_proj_g=wg, B_proj_g=None, W_proj_o=wo, B_proj_o=None, residual=z3t,
                          out=z4.transpose(0, 1))
    return z4


def single_update(s, z, pre, *, key_mask=None, eps=1e-5, scale=None):
    """s (M, C_s) + attention_pair_bias(s, z) -> new (M, C_s) tensor; key_mask (M,) optional."""
    scale = pre["D"] ** -0.5 if scale is None else scale
    wg, bg, wo, bo = pre["apb_proj"]
    return attn_pair_bias.forward(s, z, pre["apb"], scale=scale, eps=eps, W_proj_g=wg, B_proj_g=bg, W_proj_o=wo,
                                  B_proj_o=bo, mask=key_mask, residual=s)


def pairformer_block(z, s, pre, *, pair_mask=None, single_mask=None, eps=1e-5, scale=None):
    """pair_stack, then single_update on the updated z (when s is given).  Returns (z, s)."""
    z = pair_stack(z, pre, pair_mask=pair_mask, eps=eps, scale=scale)
    if s is not None:
        s = single_update(s, z, pre, key_mask=single_mask, eps=eps, scale=scale)
    return z, s
