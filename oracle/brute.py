"""Pure-Python loop restatement of the three ops — TEST INFRASTRUCTURE ONLY.

Independent of `oracle/reference.py`: no torch ops, no einsum, no library
LayerNorm or softmax; every sum is an explicit Python loop in float64 over
nested lists.  Used only at tiny shapes (L, N, M <= ~8) to pin the torch
oracle.  Formulas follow the same reference lines as `oracle/reference.py`:
`benchmarks/references.py:143-221` and `:273-274`, the -1e9 pair mask of
`triangle_attn/kernel.py:230-237,369`.

Tensors are accepted as anything with `.tolist()` and converted to nested
Python lists of floats.
"""

from __future__ import annotations

import math
import struct


def _l(t):
    return None if t is None else (t.tolist() if hasattr(t, "tolist") else t)


def _ln(v, w, b, eps):
    n = len(v)
    mean = sum(v) / n
    var = sum((e - mean) ** 2 for e in v) / n
    r = 1.0 / math.sqrt(var + eps)
    return [(v[c] - mean) * r * (w[c] if w is not None else 1.0) + (b[c] if b is not None else 0.0) for c in range(n)]


def _lin(v, W, bias=None):
    """v (in,) . W (out, in)^T  (+ bias)."""
    return [sum(W[o][c] * v[c] for c in range(len(v))) + (bias[o] if bias is not None else 0.0) for o in range(len(W))]


def _matvec_in_out(v, W):
    """v (in,) @ W (in, out)."""
    return [sum(v[c] * W[c][o] for c in range(len(v))) for o in range(len(W[0]))]


def _f32(v):
    """Round a Python float to the nearest float32 value."""
    return struct.unpack("f", struct.pack("f", v))[0]


def _masked_score(s):
    """The reference adds -1e9 to a masked score in fp32 (triangle_attn/kernel.py:230-237)."""
    return _f32(_f32(s) + _f32(-1e9))


def _sig(z):
    return 1.0 / (1.0 + math.exp(-z))


def triangle_multiplicative_update(x, *, direction, mask=None, eps=1e-5, **w):
    x = _l(x)
    mask = _l(mask)
    w = {k: _l(v) for k, v in w.items()}
    B, L, C = len(x), len(x[0]), len(x[0][0][0])
    xln = [[[_ln(x[b][i][j], w["norm_in_weight"], w["norm_in_bias"], eps) for j in range(L)] for i in range(L)]
           for b in range(B)]
    ab = [[[None] * L for _ in range(L)] for _ in range(B)]
    for b in range(B):
        for i in range(L):
            for j in range(L):
                p = _lin(xln[b][i][j], w["p_in_weight"])
                g = _lin(xln[b][i][j], w["g_in_weight"])
                m = 1.0 if mask is None else float(mask[b][i][j])
                ab[b][i][j] = [p[o] * _sig(g[o]) * m for o in range(len(p))]
    out = [[[None] * L for _ in range(L)] for _ in range(B)]
    for b in range(B):
        for i in range(L):
            for j in range(L):
                y = []
                for d in range(C):
                    s = 0.0
                    for k in range(L):
                        if direction == "outgoing":
                            s += ab[b][i][k][d] * ab[b][j][k][C + d]
                        else:
                            s += ab[b][k][i][d] * ab[b][k][j][C + d]
                    y.append(s)
                yln = _ln(y, w["norm_out_weight"], w["norm_out_bias"], eps)
                p = _lin(yln, w["p_out_weight"])
                g = _lin(xln[b][i][j], w["g_out_weight"])
                out[b][i][j] = [p[o] * _sig(g[o]) for o in range(len(p))]
    return out


def _softmax_weights(scores):
    m = max(scores)
    if m == -math.inf:
        return [math.nan] * len(scores)
    e = [math.exp(s - m) for s in scores]
    t = sum(e)
    return [v / t for v in e]


def triangle_attention(X, W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, W_proj_g, B_proj_g, W_proj_o, B_proj_o, H, D,
                       scale=1.0, eps=1e-5, mask=None):
    X, W_ln, B_ln = _l(X), _l(W_ln), _l(B_ln)
    WQ, WK, WV, Wz, Bz = _l(WQ), _l(WK), _l(WV), _l(W_proj_z), _l(B_proj_z)
    Wg, Bg, Wo, Bo, mask = _l(W_proj_g), _l(B_proj_g), _l(W_proj_o), _l(B_proj_o), _l(mask)
    N = len(X)
    xln = [[_ln(X[q][k], W_ln, B_ln, eps) for k in range(N)] for q in range(N)]
    bias = [[[sum(xln[q][k][c] * Wz[c][h] for c in range(len(xln[q][k]))) + (Bz[h] if Bz is not None else 0.0)
              for k in range(N)] for q in range(N)] for h in range(H)]
    out = [[None] * N for _ in range(N)]
    for i in range(N):
        qv = [_matvec_in_out(xln[i][q], WQ) for q in range(N)]
        kv = [_matvec_in_out(xln[i][k], WK) for k in range(N)]
        vv = [_matvec_in_out(xln[i][k], WV) for k in range(N)]
        for q in range(N):
            o = []
            for h in range(H):
                sc = []
                for k in range(N):
                    s = sum(qv[q][h * D + d] * scale * kv[k][h * D + d] for d in range(D)) + bias[h][q][k]
                    if mask is not None and not mask[i][k]:
                        s = _masked_score(s)
                    sc.append(s)
                p = _softmax_weights(sc)
                o.extend(sum(p[k] * vv[k][h * D + d] for k in range(N)) for d in range(D))
            g = [_sig(z) for z in _lin(xln[i][q], Wg, Bg)]
            out[i][q] = _lin([o[c] * g[c] for c in range(len(o))], Wo, Bo)
    return out


def attention_pair_bias(X, WQ, WK, WV, Z, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, B_proj_g, W_proj_o, B_proj_o,
                        H, D, scale=1.0, eps=1e-5, mask=None):
    X, WQ, WK, WV, Z = _l(X), _l(WQ), _l(WK), _l(WV), _l(Z)
    W_ln, B_ln, Wz, Bz = _l(W_ln), _l(B_ln), _l(W_proj_z), _l(B_proj_z)
    Wg, Bg, Wo, Bo, mask = _l(W_proj_g), _l(B_proj_g), _l(W_proj_o), _l(B_proj_o), _l(mask)
    M = len(X)
    qv = [_matvec_in_out(X[m], WQ) for m in range(M)]
    kv = [_matvec_in_out(X[m], WK) for m in range(M)]
    vv = [_matvec_in_out(X[m], WV) for m in range(M)]
    out = []
    for q in range(M):
        zb = [_matvec_in_out(_ln(Z[q][k], W_ln, B_ln, eps), Wz) for k in range(M)]
        o = []
        for h in range(H):
            sc = []
            for k in range(M):
                s = sum(qv[q][h * D + d] * scale * kv[k][h * D + d] for d in range(D)) + zb[k][h]
                s += Bz[h] if Bz is not None else 0.0
                if mask is not None and not mask[k]:
                    s = -math.inf
                sc.append(s)
            p = _softmax_weights(sc)
            o.extend(sum(p[k] * vv[k][h * D + d] for k in range(M)) for d in range(D))
        g = [_sig(z) for z in _lin(X[q], Wg, Bg)]
        out.append(_lin([g[c] * o[c] for c in range(len(o))], Wo, Bo))
    return out


def attention_pair_bias_qknorm(X, WQ, b_q, WK, WV, Z, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, W_proj_o, H, D, *,
                               qkn_w_q=None, qkn_b_q=None, qkn_w_k=None, qkn_b_k=None, key_mask=None, scale=1.0,
                               eps=1e-5):
    """Loop restatement of benchmarks/references.py:230-277 (per token, per head, per key)."""
    X, WQ, WK, WV, Z = _l(X), _l(WQ), _l(WK), _l(WV), _l(Z)
    W_ln, B_ln, Wz, Bz = _l(W_ln), _l(B_ln), _l(W_proj_z), _l(B_proj_z)
    Wg, Wo, mask, bq = _l(W_proj_g), _l(W_proj_o), _l(key_mask), _l(b_q)
    gq, bqn, gk, bkn = _l(qkn_w_q), _l(qkn_b_q), _l(qkn_w_k), _l(qkn_b_k)
    M, HD = len(X), H * D
    qv = [_matvec_in_out(X[m], WQ) for m in range(M)]
    if bq is not None:
        qv = [[qv[m][c] + bq[c] for c in range(HD)] for m in range(M)]
    kv = [_matvec_in_out(X[m], WK) for m in range(M)]
    vv = [_matvec_in_out(X[m], WV) for m in range(M)]
    if gq is not None:  # one LayerNorm over all H*D channels of each token's q and k
        qv = [_ln(qv[m], gq, bqn, eps) for m in range(M)]
        kv = [_ln(kv[m], gk, bkn, eps) for m in range(M)]
    out = []
    for q in range(M):
        zb = [_matvec_in_out(_ln(Z[q][k], W_ln, B_ln, eps), Wz) for k in range(M)]
        o = []
        for h in range(H):
            sc = []
            for k in range(M):
                s = sum(qv[q][h * D + d] * scale * kv[k][h * D + d] for d in range(D)) + zb[k][h]
                s += Bz[h] if Bz is not None else 0.0
                if mask is not None and not mask[k]:
                    s = -math.inf
                sc.append(s)
            p = _softmax_weights(sc)
            o.extend(sum(p[k] * vv[k][h * D + d] for k in range(M)) for d in range(D))
        g = [_sig(z) for z in _lin(X[q], Wg)]
        out.append(_lin([g[c] * o[c] for c in range(len(o))], Wo))
    return out
