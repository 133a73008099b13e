"""CPU fp32 oracle for the three Pairformer ops — TEST INFRASTRUCTURE ONLY.

This module restates, in plain PyTorch on the CPU, the mathematics of the
reference's pure-torch formulations.  It is the checker the HIP kernels are
compared against; it is never the thing measured or shipped.  Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it.  The product package (`triangleops_amd`) never does.

Reference files followed (paths relative to the reference repository root):

* `benchmarks/references.py:208-221`  triangle_multiplicative_update
  (LN_in -> p_in * sigmoid(g_in) -> mask -> chunk -> triangle einsum ->
  LN_out -> p_out * sigmoid(g_out(LN_in x))).  `triangle_mul/module.py:48`
  confirms g_out gates on LN_in(x).
* `benchmarks/references.py:174-205`  triangle_attention (starting node).
  The additive pair mask is -1e9 (`triangle_attn/kernel.py:230-237,369`);
  here it is added in fp32, which is what the reference's masked torch path
  does in fp32.
* `benchmarks/references.py:143-171`  attention_pair_bias, plus the optional
  key mask semantics of `benchmarks/references.py:273-274` (masked keys are
  filled with -inf before the softmax).
* `benchmarks/references.py:230-277`  attention_pair_bias_qknorm (the K-Fold
  variant: Q bias, optional LayerNorm over the full H*D channel of Q and K
  before the head split, key mask, bias-free gate and output projections).
* Pairformer-block composition (no counterpart in the reference, which ships
  the ops only): the pair stack z += tmu_out(z), z += tmu_in(z),
  z += tri_start(z), z += tri_end(z) = tri(z^T)^T, and the single update
  s += apb(s, z), composed from the functions above.

How each function is pinned (tests/test_oracle.py):
* every op is compared with the pure-Python loop restatement in
  `oracle/brute.py` at tiny shapes in float64;
* the LayerNorm-affine fold is checked against its closed-form identity;
* the einsum direction identity  y_in(a, b) == y_out(a^T, b^T);
* attention invariants: masked keys carry exactly zero weight, a fully masked
  row is the uniform average of V, and a padded+masked problem restricted to
  its valid block equals the cropped problem;
* planted-mistake variants of the oracle fail these checks.

All functions take float tensors (any float dtype), compute in `dtype`
(float32 by default, float64 for pinning) and return results in that dtype.
Rows of the attention ops are independent, so `rows=` selects a subset of
rows (query rows for apb, pair rows i for triangle attention) so that full
configuration sizes can be spot-checked on the CPU in seconds.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = [
    "layer_norm",
    "tmu_gated_input",
    "tmu_einsum",
    "tmu_output",
    "triangle_multiplicative_update",
    "tri_layer_norm_bias",
    "tri_attention_core",
    "tri_gate_out",
    "triangle_attention",
    "apb_bias",
    "apb_attention_core",
    "apb_gate_out",
    "attention_pair_bias",
    "apb_qknorm_qkv",
    "attention_pair_bias_qknorm",
    "pair_stack",
    "single_update",
]


def _f(t, dtype):
    return None if t is None else t.detach().to("cpu", dtype)


def layer_norm(x, w, b, eps, dtype=torch.float32):
    """LayerNorm over the last dim (library routine, `F.layer_norm`)."""
    x = _f(x, dtype)
    return F.layer_norm(x, (x.shape[-1],), _f(w, dtype), _f(b, dtype), eps)


# --------------------------------------------------------------------------- #
# triangle_multiplicative_update   (references.py:208-221)
# --------------------------------------------------------------------------- #
def tmu_gated_input(x, mask, norm_in_weight, norm_in_bias, p_in_weight, g_in_weight, eps=1e-5,
                    dtype=torch.float32):
    """Input phase: ab = (LN_in(x) p_in^T) * sigmoid(LN_in(x) g_in^T) * mask.

    x (B, L, L, C) -> ab (B, L, L, 2C) in token-major order (references.py:210-214).
    """
    xln = layer_norm(x, norm_in_weight, norm_in_bias, eps, dtype)
    g = F.linear(xln, _f(p_in_weight, dtype)) * torch.sigmoid(F.linear(xln, _f(g_in_weight, dtype)))
    if mask is not None:
        g = g * _f(mask, dtype).unsqueeze(-1)
    return g


def tmu_einsum(a, b, direction, dtype=torch.float32, rows=None):
    """Triangle einsum over token-major a, b (B, L, L, C) -> y (B, L, L, C).

    outgoing: y[b,i,j,d] = sum_k a[b,i,k,d] b[b,j,k,d]
    incoming: y[b,i,j,d] = sum_k a[b,k,i,d] b[b,k,j,d]   (references.py:216-219)
    `rows` restricts the output rows i (the result then has len(rows) rows).
    """
    a, b = _f(a, dtype), _f(b, dtype)
    if direction == "outgoing":
        A = a if rows is None else a[:, rows]
        return torch.einsum("bikd,bjkd->bijd", A, b)
    if direction == "incoming":
        A = a if rows is None else a[:, :, rows]
        return torch.einsum("bkid,bkjd->bijd", A, b)
    raise ValueError(f"unknown direction: {direction!r} (expected 'outgoing'/'incoming')")


def tmu_output(y, x, norm_in_weight, norm_in_bias, norm_out_weight, norm_out_bias, p_out_weight, g_out_weight,
               eps=1e-5, dtype=torch.float32):
    """Output phase: p_out(LN_out(y)) * sigmoid(g_out(LN_in(x))) (references.py:220-221)."""
    yln = layer_norm(y, norm_out_weight, norm_out_bias, eps, dtype)
    xln = layer_norm(x, norm_in_weight, norm_in_bias, eps, dtype)
    return F.linear(yln, _f(p_out_weight, dtype)) * torch.sigmoid(F.linear(xln, _f(g_out_weight, dtype)))


def triangle_multiplicative_update(x, *, direction, mask=None, eps=1e-5, dtype=torch.float32, rows=None, **w):
    """Whole op (references.py:208-221).  x (B, L, L, C) -> (B, L, L, C).

    With `rows`, only output rows i in `rows` are produced: (B, len(rows), L, C).
    """
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"unknown direction: {direction!r} (expected 'outgoing'/'incoming')")
    g = tmu_gated_input(x, mask, w["norm_in_weight"], w["norm_in_bias"], w["p_in_weight"], w["g_in_weight"],
                        eps, dtype)
    a, b = torch.chunk(g, 2, dim=-1)
    y = tmu_einsum(a, b, direction, dtype, rows)
    xs = x if rows is None else x[:, rows]
    return tmu_output(y, xs, w["norm_in_weight"], w["norm_in_bias"], w["norm_out_weight"], w["norm_out_bias"],
                      w["p_out_weight"], w["g_out_weight"], eps, dtype)


# --------------------------------------------------------------------------- #
# triangle_attention   (references.py:174-205, mask as triangle_attn/kernel.py:230-237)
# --------------------------------------------------------------------------- #
def tri_layer_norm_bias(X, W_ln, B_ln, W_proj_z, B_proj_z, eps=1e-5, dtype=torch.float32):
    """x_ln = LN(X) (N, N, C) and the row-shared bias (H, N, N):
    bias[h, q, k] = x_ln[q, k, :] . W_proj_z[:, h] + B_proj_z[h]  (references.py:194,198)."""
    xln = layer_norm(X, W_ln, B_ln, eps, dtype)
    bp = xln @ _f(W_proj_z, dtype)
    if B_proj_z is not None:
        bp = bp + _f(B_proj_z, dtype)
    return xln, bp.permute(2, 0, 1).contiguous()


def tri_attention_core(xln, WQ, WK, WV, bias, H, D, scale=1.0, mask=None, dtype=torch.float32, rows=None,
                       chunk=8):
    """Attention over each pair row i (references.py:195-202).

    xln (N, N, C), bias (H, N, N), mask (N, N) (nonzero = valid key) ->
    O (R, N, H*D) for rows i in `rows` (all rows by default), before gating.
    Masked keys get -1e9 added to their scores in fp32, as the reference kernel does.
    """
    xln, bias = _f(xln, dtype), _f(bias, dtype)
    WQ, WK, WV = _f(WQ, dtype), _f(WK, dtype), _f(WV, dtype)
    N = xln.shape[0]
    rows = torch.arange(N) if rows is None else torch.as_tensor(rows)
    outs = []
    for s in range(0, len(rows), chunk):
        r = rows[s : s + chunk]
        xr = xln[r]  # (R, N, C)
        R = xr.shape[0]
        q = (xr @ WQ).view(R, N, H, D).permute(0, 2, 1, 3)
        k = (xr @ WK).view(R, N, H, D).permute(0, 2, 1, 3)
        v = (xr @ WV).view(R, N, H, D).permute(0, 2, 1, 3)
        scores = torch.matmul(q * scale, k.transpose(-1, -2)) + bias.unsqueeze(0)
        if mask is not None:
            # -1e9 is added in fp32, as the reference does, also when checking in float64:
            # a row without valid keys then has all scores == -1e9 (uniform weights).
            valid = (_f(mask, dtype)[r] != 0)[:, None, None, :]  # (R, 1, 1, N) over keys
            masked = (scores.float() + torch.tensor(-1e9, dtype=torch.float32)).to(dtype)
            scores = torch.where(valid, scores, masked)
        o = torch.matmul(torch.softmax(scores, -1), v)  # (R, H, N, D)
        outs.append(o.permute(0, 2, 1, 3).reshape(R, N, H * D))
    return torch.cat(outs, 0)


def tri_gate_out(o, xln, W_proj_g, B_proj_g, W_proj_o, B_proj_o, dtype=torch.float32):
    """out = (o * sigmoid(linear(x_ln, W_g, b_g))) W_o^T + b_o (references.py:203-205)."""
    o, xln = _f(o, dtype), _f(xln, dtype)
    g = torch.sigmoid(F.linear(xln, _f(W_proj_g, dtype), _f(B_proj_g, dtype)))
    return F.linear(o * g, _f(W_proj_o, dtype), _f(B_proj_o, dtype))


def triangle_attention(X, W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, W_proj_g, B_proj_g, W_proj_o, B_proj_o, H, D,
                       scale=1.0, eps=1e-5, mask=None, dtype=torch.float32, rows=None):
    """Whole op, starting node (references.py:174-205).  X (N, N, C) -> (N, N, C_out).

    The ending node is this op applied to X.transpose(0, 1) with mask.T and the
    output transposed back (the reference leaves that to the caller).
    """
    xln, bias = tri_layer_norm_bias(X, W_ln, B_ln, W_proj_z, B_proj_z, eps, dtype)
    o = tri_attention_core(xln, WQ, WK, WV, bias, H, D, scale, mask, dtype, rows)
    xs = xln if rows is None else xln[torch.as_tensor(rows)]
    return tri_gate_out(o, xs, W_proj_g, B_proj_g, W_proj_o, B_proj_o, dtype)


# --------------------------------------------------------------------------- #
# attention_pair_bias   (references.py:143-171, key mask as references.py:273-274)
# --------------------------------------------------------------------------- #
def apb_bias(Z, W_ln, B_ln, W_proj_z, B_proj_z, eps=1e-5, dtype=torch.float32, rows=None):
    """bias[h, q, k] = LN(Z[q, k, :]) . W_proj_z[:, h] + B_proj_z[h]  (references.py:167)."""
    Zs = Z if rows is None else Z[torch.as_tensor(rows)]
    zb = layer_norm(Zs, W_ln, B_ln, eps, dtype) @ _f(W_proj_z, dtype)
    if B_proj_z is not None:
        zb = zb + _f(B_proj_z, dtype)
    return zb.permute(2, 0, 1)


def apb_attention_core(X, WQ, WK, WV, bias, H, D, scale=1.0, mask=None, dtype=torch.float32, rows=None):
    """o[q, h*D+d] = softmax_k((q.k)*scale + bias[h,q,k]) v  (references.py:164-169).

    bias is (H, R, M) for the R query rows selected by `rows`.  mask (M,) over
    keys: masked keys are filled with -inf (references.py:273-274).
    """
    X = _f(X, dtype)
    M = X.shape[0]
    Xq = X if rows is None else X[torch.as_tensor(rows)]
    R = Xq.shape[0]
    q = (Xq @ _f(WQ, dtype)).reshape(R, H, D).permute(1, 0, 2)
    k = (X @ _f(WK, dtype)).reshape(M, H, D).permute(1, 0, 2)
    v = (X @ _f(WV, dtype)).reshape(M, H, D).permute(1, 0, 2)
    scores = torch.matmul(q * scale, k.transpose(-1, -2)) + _f(bias, dtype)
    if mask is not None:
        scores = scores.masked_fill(~(_f(mask, dtype) != 0)[None, None, :], float("-inf"))
    o = torch.matmul(torch.softmax(scores, -1), v)
    return o.permute(1, 0, 2).reshape(R, H * D)


def apb_gate_out(o, X, W_proj_g, B_proj_g, W_proj_o, B_proj_o, dtype=torch.float32):
    """out = (sigmoid(linear(X, W_g, b_g)) * o) W_o^T + b_o, gate on raw X (references.py:170-171)."""
    X, o = _f(X, dtype), _f(o, dtype)
    g = torch.sigmoid(F.linear(X, _f(W_proj_g, dtype), _f(B_proj_g, dtype)))
    return F.linear(g * o, _f(W_proj_o, dtype), _f(B_proj_o, dtype))


def attention_pair_bias(X, WQ, WK, WV, Z, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, B_proj_g, W_proj_o, B_proj_o,
                        H, D, scale=1.0, eps=1e-5, mask=None, dtype=torch.float32, rows=None, chunk=256):
    """Whole op (references.py:143-171).  X (M, C_s), Z (M, M, C_z) -> (M, C_out)."""
    M = X.shape[0]
    rows = torch.arange(M) if rows is None else torch.as_tensor(rows)
    outs = []
    for s in range(0, len(rows), chunk):
        r = rows[s : s + chunk]
        bias = apb_bias(Z, W_ln, B_ln, W_proj_z, B_proj_z, eps, dtype, r)
        o = apb_attention_core(X, WQ, WK, WV, bias, H, D, scale, mask, dtype, r)
        outs.append(apb_gate_out(o, _f(X, dtype)[r], W_proj_g, B_proj_g, W_proj_o, B_proj_o, dtype))
    return torch.cat(outs, 0)


def apb_qknorm_qkv(X, WQ, b_q, WK, WV, H, D, qkn_w_q=None, qkn_b_q=None, qkn_w_k=None, qkn_b_k=None, eps=1e-5,
                   dtype=torch.float32):
    """q = X WQ + b_q, k = X WK, v = X WV (M, H*D); with qkn_w_q given, q and k are LayerNormed over
    the full H*D channel with (qkn_w_q, qkn_b_q) / (qkn_w_k, qkn_b_k) before the head split
    (references.py:258-264)."""
    X = _f(X, dtype)
    q = X @ _f(WQ, dtype)
    if b_q is not None:
        q = q + _f(b_q, dtype)
    k = X @ _f(WK, dtype)
    v = X @ _f(WV, dtype)
    if qkn_w_q is not None:
        q = F.layer_norm(q, (H * D,), _f(qkn_w_q, dtype), _f(qkn_b_q, dtype), eps=eps)
        k = F.layer_norm(k, (H * D,), _f(qkn_w_k, dtype), _f(qkn_b_k, dtype), eps=eps)
    return q, k, v


def attention_pair_bias_qknorm(X, WQ, b_q, WK, WV, Z, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, W_proj_o, H, D, *,
                               qkn_w_q=None, qkn_b_q=None, qkn_w_k=None, qkn_b_k=None, key_mask=None, scale=1.0,
                               eps=1e-5, dtype=torch.float32, rows=None, chunk=256):
    """Whole K-Fold variant (references.py:230-277).  X (M, C_s), Z (M, M, C_z) -> (M, C_out);
    gate sigmoid(X W_g^T) and output projection without biases."""
    M = X.shape[0]
    q, k, v = apb_qknorm_qkv(X, WQ, b_q, WK, WV, H, D, qkn_w_q, qkn_b_q, qkn_w_k, qkn_b_k, eps, dtype)
    kh = k.reshape(M, H, D).permute(1, 0, 2)
    vh = v.reshape(M, H, D).permute(1, 0, 2)
    rows = torch.arange(M) if rows is None else torch.as_tensor(rows)
    outs = []
    for s in range(0, len(rows), chunk):
        r = rows[s : s + chunk]
        bias = apb_bias(Z, W_ln, B_ln, W_proj_z, B_proj_z, eps, dtype, r)
        qh = q[r].reshape(len(r), H, D).permute(1, 0, 2)
        scores = torch.matmul(qh * scale, kh.transpose(-1, -2)) + bias
        if key_mask is not None:
            scores = scores.masked_fill(~(_f(key_mask, dtype) != 0)[None, None, :], float("-inf"))
        o = torch.matmul(torch.softmax(scores, -1), vh).permute(1, 0, 2).reshape(len(r), H * D)
        outs.append(apb_gate_out(o, _f(X, dtype)[r], W_proj_g, None, W_proj_o, None, dtype))
    return torch.cat(outs, 0)


def pair_stack(z, tmu_out, tmu_in, tri_start, tri_end, H, D, pair_mask=None, eps=1e-5, scale=None,
               dtype=torch.float32):
    """The four pair updates with residuals; z (N, N, C).  tmu_* are the 8-weight keyword dicts of
    triangle_multiplicative_update, tri_* dicts with W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z,
    W_proj_g, W_proj_o (bias-free gate / output).  The ending node is the op on z^T, transposed back."""
    z = _f(z, dtype)
    N = z.shape[0]
    scale = D**-0.5 if scale is None else scale
    m3 = None if pair_mask is None else pair_mask.reshape(1, N, N)
    z = z + triangle_multiplicative_update(z[None], direction="outgoing", mask=m3, eps=eps, dtype=dtype, **tmu_out)[0]
    z = z + triangle_multiplicative_update(z[None], direction="incoming", mask=m3, eps=eps, dtype=dtype, **tmu_in)[0]

    def tri(x, w, mask):
        return triangle_attention(x, w["W_ln"], w["B_ln"], w["WQ"], w["WK"], w["WV"], w["W_proj_z"], w["B_proj_z"],
                                  w["W_proj_g"], None, w["W_proj_o"], None, H, D, scale=scale, eps=eps, mask=mask,
                                  dtype=dtype)

    z = z + tri(z, tri_start, pair_mask)
    z = z + tri(z.transpose(0, 1), tri_end, None if pair_mask is None else pair_mask.T).transpose(0, 1)
    return z


def single_update(s, z, apb, H, D, key_mask=None, eps=1e-5, scale=None, dtype=torch.float32):
    """s + attention_pair_bias(s, z); apb: dict of the op's weights (gate / output biases optional)."""
    scale = D**-0.5 if scale is None else scale
    out = attention_pair_bias(s, apb["WQ"], apb["WK"], apb["WV"], z, apb["W_ln"], apb["B_ln"], apb["W_proj_z"],
                              apb["B_proj_z"], apb["W_proj_g"], apb.get("B_proj_g"), apb["W_proj_o"],
                              apb.get("B_proj_o"), H, D, scale=scale, eps=eps, mask=key_mask, dtype=dtype)
    return _f(s, dtype) + out
