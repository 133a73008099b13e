"""Seeded synthetic inputs for the three ops (CPU generator, fixed draw order).

Shapes and distributions restate the benchmark configurations: x ~ N(0, 1), weights
~ N(0, 1/fan_in), LayerNorm gamma = 1 + 0.1 N(0, 1), beta = 0.1 N(0, 1); padding masks
mark the last rows/cols (pair masks) or keys (apb) as invalid.  Every tensor is rounded
to the I/O dtype once; the fp32 oracle consumes the same rounded values upcast, so input
quantisation is not counted as kernel error.
"""

import torch


def _g(seed):
    return torch.Generator().manual_seed(seed)


def pad_pair_mask(n, frac=10, batch=None):
    """valid = (i < n - n // frac) & (j < n - n // frac)."""
    v = n - n // frac
    idx = torch.arange(n)
    m = (idx[:, None] < v) & (idx[None, :] < v)
    return m if batch is None else m.expand(batch, n, n).contiguous()


def random_mask(shape, seed, p_valid=0.8):
    return torch.rand(*shape, generator=_g(seed)) < p_valid


def tmu_inputs(L, *, B=1, C=128, seed=0, dtype=torch.bfloat16, mask="pad", affine=True):
    g = _g(seed)
    x = torch.randn(B, L, L, C, generator=g)
    s = C**-0.5
    w = {
        "p_in_weight": torch.randn(2 * C, C, generator=g) * s,
        "g_in_weight": torch.randn(2 * C, C, generator=g) * s,
        "p_out_weight": torch.randn(C, C, generator=g) * s,
        "g_out_weight": torch.randn(C, C, generator=g) * s,
    }
    if affine:
        w["norm_in_weight"] = 1 + 0.1 * torch.randn(C, generator=g)
        w["norm_in_bias"] = 0.1 * torch.randn(C, generator=g)
        w["norm_out_weight"] = 1 + 0.1 * torch.randn(C, generator=g)
        w["norm_out_bias"] = 0.1 * torch.randn(C, generator=g)
    else:
        w["norm_in_weight"], w["norm_in_bias"] = torch.ones(C), torch.zeros(C)
        w["norm_out_weight"], w["norm_out_bias"] = torch.ones(C), torch.zeros(C)
    if mask == "pad":
        m = pad_pair_mask(L, 10, B)
    elif mask == "random":
        m = random_mask((B, L, L), seed + 1)
    elif mask == "ones":
        m = torch.ones(B, L, L, dtype=torch.bool)
    else:
        m = None
    x = x.to(dtype)
    w = {k: v.to(dtype) for k, v in w.items()}
    return x, m, w


def tri_inputs(N, *, C=128, H=4, D=32, seed=0, dtype=torch.bfloat16, mask="pad", bias_z=False):
    g = _g(seed)
    X = torch.randn(N, N, C, generator=g)
    s = C**-0.5
    W_ln = 1 + 0.1 * torch.randn(C, generator=g)
    B_ln = 0.1 * torch.randn(C, generator=g)
    WQ = torch.randn(C, H * D, generator=g) * s
    WK = torch.randn(C, H * D, generator=g) * s
    WV = torch.randn(C, H * D, generator=g) * s
    W_pz = torch.randn(C, H, generator=g) * s
    B_pz = 0.1 * torch.randn(H, generator=g) if bias_z else torch.zeros(H)
    W_pg = torch.randn(H * D, C, generator=g) * s
    W_po = torch.randn(C, H * D, generator=g) * (H * D) ** -0.5
    if mask == "pad":
        m = pad_pair_mask(N, 10)
    elif mask == "random":
        m = random_mask((N, N), seed + 1)
    else:
        m = None
    t = [X, W_ln, B_ln, WQ, WK, WV, W_pz, B_pz, W_pg, W_po]
    X, W_ln, B_ln, WQ, WK, WV, W_pz, B_pz, W_pg, W_po = [v.to(dtype) for v in t]
    return dict(X=X, W_ln=W_ln, B_ln=B_ln, WQ=WQ, WK=WK, WV=WV, W_proj_z=W_pz, B_proj_z=B_pz, W_proj_g=W_pg,
                B_proj_g=None, W_proj_o=W_po, B_proj_o=None, H=H, D=D, scale=D**-0.5, mask=m)


def apb_inputs(M, *, C=128, Cz=128, H=4, D=32, seed=0, dtype=torch.bfloat16, mask="pad", biases=False):
    g = _g(seed)
    X = torch.randn(M, C, generator=g)
    Z = torch.randn(M, M, Cz, generator=g)
    s = C**-0.5
    WQ = torch.randn(C, H * D, generator=g) * s
    WK = torch.randn(C, H * D, generator=g) * s
    WV = torch.randn(C, H * D, generator=g) * s
    W_ln = 1 + 0.1 * torch.randn(Cz, generator=g)
    B_ln = 0.1 * torch.randn(Cz, generator=g)
    W_pz = torch.randn(Cz, H, generator=g) * Cz**-0.5
    W_pg = torch.randn(H * D, C, generator=g) * s
    W_po = torch.randn(C, H * D, generator=g) * (H * D) ** -0.5
    if biases:
        B_pz = 0.1 * torch.randn(H, generator=g)
        B_pg = 0.1 * torch.randn(H * D, generator=g)
        B_po = 0.1 * torch.randn(C, generator=g)
    else:
        B_pz, B_pg, B_po = torch.zeros(H), torch.zeros(H * D), torch.zeros(C)
    if mask == "pad":
        m = torch.arange(M) < M - M // 20
    elif mask == "random":
        m = random_mask((M,), seed + 1, 0.9)
    else:
        m = None
    t = [X, Z, WQ, WK, WV, W_ln, B_ln, W_pz, B_pz, W_pg, B_pg, W_po, B_po]
    X, Z, WQ, WK, WV, W_ln, B_ln, W_pz, B_pz, W_pg, B_pg, W_po, B_po = [v.to(dtype) for v in t]
    return dict(X=X, WQ=WQ, WK=WK, WV=WV, Z=Z, W_ln=W_ln, B_ln=B_ln, W_proj_z=W_pz, B_proj_z=B_pz, W_proj_g=W_pg,
                B_proj_g=B_pg, W_proj_o=W_po, B_proj_o=B_po, H=H, D=D, scale=D**-0.5, mask=m)


def apb_qkn_inputs(M, *, C=128, Cz=128, H=4, D=32, seed=0, dtype=torch.bfloat16, mask="pad", qkn=True):
    """Inputs of the qk-norm variant (benchmarks/references.py:230-250): apb_inputs plus a Q bias and
    the qk-norm affine parameters (None when qkn is False); the gate / output projections are
    bias-free, and the key mask goes by `key_mask`."""
    d = apb_inputs(M, C=C, Cz=Cz, H=H, D=D, seed=seed, dtype=dtype, mask=mask, biases=True)
    g = _g(seed + 1000)
    HD = H * D
    d["b_q"] = (0.5 * torch.randn(HD, generator=g)).to(dtype)
    for name, base in (("qkn_w_q", 1.0), ("qkn_b_q", 0.0), ("qkn_w_k", 1.0), ("qkn_b_k", 0.0)):
        d[name] = (base + 0.2 * torch.randn(HD, generator=g)).to(dtype) if qkn else None
    d["key_mask"] = d.pop("mask")
    for k in ("B_proj_g", "B_proj_o"):
        d.pop(k)
    return d


def to_dev(d, device):
    if isinstance(d, dict):
        return {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in d.items()}
    return d.to(device)


# Parity bar for bf16 / fp16 outputs against the fp32 oracle.
TOL_MAX_ABS = {torch.bfloat16: 3e-2, torch.float16: 1e-2, torch.float32: 1e-4}
TOL_COS = 0.9999


def compare(out, ref):
    """(max |out - ref|, cosine similarity) over all elements, in float64."""
    o = out.detach().double().cpu().flatten()
    r = ref.detach().double().cpu().flatten()
    diff = (o - r).abs().max().item() if o.numel() else 0.0
    cos = torch.nn.functional.cosine_similarity(o, r, dim=0).item() if o.numel() else 1.0
    return diff, cos
