"""LayerNorm-affine absorption (one-time, model-init fold).

A LayerNorm followed by a linear projection satisfies, per token with C features,
    LN(x) . W^T = rstd * (x . Wc^T - mean * sum_i Wc[:, i]) + W . beta,   Wc = W * gamma,
so a kernel that already has the token's (mean, rstd) applies the affine with only the
folded weight Wc, the fp32 row sums of Wc and the fp32 constant W . beta.  Same contract as
the reference (`triangle_ops/_common/ln_absorption.py:28-63`): the sums come from the
unrounded fp32 Wc, and Wc is cast to `weight_dtype` (default: the weight's dtype).
"""

import torch


def absorb_ln(weight: torch.Tensor, w_ln: torch.Tensor, b_ln: torch.Tensor, *, weight_dtype=None):
    """Fold for an (out, in) nn.Linear weight: returns Wc (out, in), sum_W (out,) fp32, B_const (out,) fp32."""
    W = weight.float()
    Wc = W * w_ln.float()[None, :]
    sum_W = Wc.sum(dim=1)
    B_const = torch.mv(W, b_ln.float())
    dt = weight.dtype if weight_dtype is None else weight_dtype
    return Wc.to(dt).contiguous(), sum_W.contiguous(), B_const.contiguous()


def absorb_ln_matmul(weight: torch.Tensor, w_ln: torch.Tensor, b_ln: torch.Tensor, *, weight_dtype=None):
    """Fold for an (in, out) matmul weight (y = LN(x) @ W): returns Wc (in, out), sum_W (out,), B_const (out,)."""
    W = weight.float()
    Wc = W * w_ln.float()[:, None]
    sum_W = Wc.sum(dim=0)
    B_const = torch.mv(W.t(), b_ln.float())
    dt = weight.dtype if weight_dtype is None else weight_dtype
    return Wc.to(dt).contiguous(), sum_W.contiguous(), B_const.contiguous()
