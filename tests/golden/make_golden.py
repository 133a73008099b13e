"""Writes the golden fixtures of tests/golden/*.npz.

Each fixture holds tiny seeded inputs (rounded to bf16 once, stored exactly as float32) and
the expected output computed by `oracle/brute.py` (pure-Python loops in float64, independent
of the torch oracle), stored as float64.  Shapes use the kernels' real channel widths
(C = Cz = 128, H = 4, D = 32) so the same fixtures check the HIP path on the GPU.

The reference repository ships no golden vectors for these ops (its tests compare live
against cuequivariance), so these fixtures are this build's own known-answer vectors.

    python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute  # noqa: E402

C, H, D = 128, 4, 32


def _bf(t):
    return t.to(torch.bfloat16).to(torch.float32)


def _save(name, inputs, expected, meta):
    arrays = {f"in_{k}": v.numpy() for k, v in inputs.items() if torch.is_tensor(v)}
    arrays["expected"] = np.asarray(expected, dtype=np.float64)
    for k, v in meta.items():
        arrays[f"meta_{k}"] = np.asarray(v)
    np.savez_compressed(os.path.join(HERE, name), **arrays)
    print("wrote", name, arrays["expected"].shape)


def tmu(direction, L=6, seed=101):
    g = torch.Generator().manual_seed(seed)
    s = C**-0.5
    x = _bf(torch.randn(1, L, L, C, generator=g))
    w = {
        "norm_in_weight": _bf(1 + 0.1 * torch.randn(C, generator=g)),
        "norm_in_bias": _bf(0.1 * torch.randn(C, generator=g)),
        "p_in_weight": _bf(torch.randn(2 * C, C, generator=g) * s),
        "g_in_weight": _bf(torch.randn(2 * C, C, generator=g) * s),
        "norm_out_weight": _bf(1 + 0.1 * torch.randn(C, generator=g)),
        "norm_out_bias": _bf(0.1 * torch.randn(C, generator=g)),
        "p_out_weight": _bf(torch.randn(C, C, generator=g) * s),
        "g_out_weight": _bf(torch.randn(C, C, generator=g) * s),
    }
    mask = (torch.rand(1, L, L, generator=g) < 0.75).to(torch.float32)
    out = brute.triangle_multiplicative_update(x, direction=direction, mask=mask, eps=1e-5, **w)
    _save(f"tmu_{direction}.npz", dict(x=x, mask=mask, **w), out, {"direction": direction, "eps": 1e-5})


def tri(N=5, seed=202):
    g = torch.Generator().manual_seed(seed)
    s = C**-0.5
    inp = dict(
        X=_bf(torch.randn(N, N, C, generator=g)),
        W_ln=_bf(1 + 0.1 * torch.randn(C, generator=g)),
        B_ln=_bf(0.1 * torch.randn(C, generator=g)),
        WQ=_bf(torch.randn(C, H * D, generator=g) * s),
        WK=_bf(torch.randn(C, H * D, generator=g) * s),
        WV=_bf(torch.randn(C, H * D, generator=g) * s),
        W_proj_z=_bf(torch.randn(C, H, generator=g) * s),
        B_proj_z=_bf(0.1 * torch.randn(H, generator=g)),
        W_proj_g=_bf(torch.randn(H * D, C, generator=g) * s),
        W_proj_o=_bf(torch.randn(C, H * D, generator=g) * (H * D) ** -0.5),
    )
    mask = torch.rand(N, N, generator=g) < 0.7
    mask[N - 1, :] = False  # one fully masked row: uniform average of V
    inp["mask"] = mask.to(torch.float32)
    out = brute.triangle_attention(inp["X"], inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"], inp["WV"],
                                   inp["W_proj_z"], inp["B_proj_z"], inp["W_proj_g"], None, inp["W_proj_o"], None, H,
                                   D, scale=D**-0.5, eps=1e-5, mask=mask)
    _save("tri_attn.npz", inp, out, {"scale": D**-0.5, "eps": 1e-5})


def apb(M=6, seed=303):
    g = torch.Generator().manual_seed(seed)
    s = C**-0.5
    inp = dict(
        X=_bf(torch.randn(M, C, generator=g)),
        WQ=_bf(torch.randn(C, H * D, generator=g) * s),
        WK=_bf(torch.randn(C, H * D, generator=g) * s),
        WV=_bf(torch.randn(C, H * D, generator=g) * s),
        Z=_bf(torch.randn(M, M, C, generator=g)),
        W_ln=_bf(1 + 0.1 * torch.randn(C, generator=g)),
        B_ln=_bf(0.1 * torch.randn(C, generator=g)),
        W_proj_z=_bf(torch.randn(C, H, generator=g) * s),
        B_proj_z=_bf(0.1 * torch.randn(H, generator=g)),
        W_proj_g=_bf(torch.randn(H * D, C, generator=g) * s),
        B_proj_g=_bf(0.1 * torch.randn(H * D, generator=g)),
        W_proj_o=_bf(torch.randn(C, H * D, generator=g) * (H * D) ** -0.5),
        B_proj_o=_bf(0.1 * torch.randn(C, generator=g)),
    )
    mask = torch.ones(M, dtype=torch.bool)
    mask[1] = False
    mask[M - 1] = False
    inp["mask"] = mask.to(torch.float32)
    out = brute.attention_pair_bias(inp["X"], inp["WQ"], inp["WK"], inp["WV"], inp["Z"], inp["W_ln"], inp["B_ln"],
                                    inp["W_proj_z"], inp["B_proj_z"], inp["W_proj_g"], inp["B_proj_g"],
                                    inp["W_proj_o"], inp["B_proj_o"], H, D, scale=D**-0.5, eps=1e-5, mask=mask)
    _save("apb.npz", inp, out, {"scale": D**-0.5, "eps": 1e-5})


if __name__ == "__main__":
    tmu("outgoing")
    tmu("incoming")
    tri()
    apb()
