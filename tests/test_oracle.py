"""Pins the CPU oracle (`oracle/reference.py`) — CPU only.

Checks, each chosen so a plausible mistake (dropped term, wrong sign or index, transposed
operand, wrong gate input, mask on the wrong axis) fails at least one of them:
  * oracle == pure-Python loop restatement (`oracle/brute.py`) at tiny shapes in float64;
  * oracle == the committed golden fixtures (written by brute force, tests/golden);
  * closed forms: the LayerNorm-affine fold identity; the weight layout permutations;
  * identities: incoming einsum == outgoing einsum on transposed token grids;
  * attention invariants: masked keys carry zero weight, a fully masked triangle-attention
    row is the uniform average of V, padded+masked == cropped;
  * planted mistakes: mutated copies of the oracle fail the brute-force comparison.
"""

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import reference as ref
from triangleops_amd._common import absorb_ln, absorb_ln_matmul, interleave_kv, interleave_qkv, qkv_head_major

F64 = torch.float64
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _tmu_small(B=1, L=4, C=6, seed=0, mask=True):
    g = _g(seed)
    x = torch.randn(B, L, L, C, generator=g, dtype=F64)
    w = {
        "norm_in_weight": 1 + 0.2 * torch.randn(C, generator=g, dtype=F64),
        "norm_in_bias": 0.2 * torch.randn(C, generator=g, dtype=F64),
        "p_in_weight": torch.randn(2 * C, C, generator=g, dtype=F64),
        "g_in_weight": torch.randn(2 * C, C, generator=g, dtype=F64),
        "norm_out_weight": 1 + 0.2 * torch.randn(C, generator=g, dtype=F64),
        "norm_out_bias": 0.2 * torch.randn(C, generator=g, dtype=F64),
        "p_out_weight": torch.randn(C, C, generator=g, dtype=F64),
        "g_out_weight": torch.randn(C, C, generator=g, dtype=F64),
    }
    m = (torch.rand(B, L, L, generator=g) < 0.7).to(F64) if mask else None
    return x, m, w


def _tri_small(N=4, C=6, H=2, D=3, seed=0, full_masked_row=True):
    g = _g(seed)
    r = lambda *s, sd=1.0: torch.randn(*s, generator=g, dtype=F64) * sd  # noqa: E731
    d = dict(X=r(N, N, C), W_ln=1 + 0.2 * r(C), B_ln=0.2 * r(C), WQ=r(C, H * D), WK=r(C, H * D), WV=r(C, H * D),
             W_proj_z=r(C, H), B_proj_z=0.3 * r(H), W_proj_g=r(H * D, C), B_proj_g=0.1 * r(H * D),
             W_proj_o=r(C, H * D), B_proj_o=0.1 * r(C), H=H, D=D, scale=0.4)
    m = torch.rand(N, N, generator=g) < 0.6
    m[0, 0] = True
    if full_masked_row:
        m[N - 1] = False
    d["mask"] = m
    return d


def _apb_small(M=5, C=6, Cz=5, H=2, D=3, seed=0):
    g = _g(seed)
    r = lambda *s, sd=1.0: torch.randn(*s, generator=g, dtype=F64) * sd  # noqa: E731
    d = dict(X=r(M, C), WQ=r(C, H * D), WK=r(C, H * D), WV=r(C, H * D), Z=r(M, M, Cz), W_ln=1 + 0.2 * r(Cz),
             B_ln=0.2 * r(Cz), W_proj_z=r(Cz, H), B_proj_z=0.3 * r(H), W_proj_g=r(H * D, C), B_proj_g=0.1 * r(H * D),
             W_proj_o=r(C, H * D), B_proj_o=0.1 * r(C), H=H, D=D, scale=0.4)
    m = torch.ones(M, dtype=torch.bool)
    m[1] = False
    d["mask"] = m
    return d


def _tri_args(d):
    return (d["X"], d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"], d["B_proj_z"], d["W_proj_g"],
            d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], d["H"], d["D"])


def _apb_args(d):
    return (d["X"], d["WQ"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"],
            d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], d["H"], d["D"])


def _close(a, b, tol=1e-9):
    a = torch.as_tensor(a, dtype=F64)
    b = torch.as_tensor(b, dtype=F64)
    return a.shape == b.shape and torch.allclose(a, b, atol=tol, rtol=tol, equal_nan=True)


# --------------------------------------------------------------------------- #
# oracle vs brute force
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("B", [1, 2])
def test_tmu_oracle_matches_brute(direction, B):
    x, m, w = _tmu_small(B=B, seed=B)
    got = ref.triangle_multiplicative_update(x, direction=direction, mask=m, dtype=F64, **w)
    assert _close(got, brute.triangle_multiplicative_update(x, direction=direction, mask=m, **w))


def test_tmu_oracle_rows_subset():
    x, m, w = _tmu_small(L=5, seed=3)
    for direction in ("outgoing", "incoming"):
        full = ref.triangle_multiplicative_update(x, direction=direction, mask=m, dtype=F64, **w)
        rows = torch.tensor([0, 3])
        part = ref.triangle_multiplicative_update(x, direction=direction, mask=m, dtype=F64, rows=rows, **w)
        assert _close(part, full[:, rows])


def test_tri_oracle_matches_brute():
    d = _tri_small()
    got = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"], dtype=F64)
    assert _close(got, brute.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"]))
    got = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=None, dtype=F64)
    assert _close(got, brute.triangle_attention(*_tri_args(d), scale=d["scale"], mask=None))
    rows = torch.tensor([1, 3])
    part = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"], dtype=F64, rows=rows)
    full = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"], dtype=F64)
    assert _close(part, full[rows])


def test_apb_oracle_matches_brute():
    d = _apb_small()
    for mask in (d["mask"], None):
        got = ref.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=mask, dtype=F64)
        assert _close(got, brute.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=mask))
    part = ref.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=d["mask"], dtype=F64, rows=[0, 4], chunk=1)
    full = ref.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=d["mask"], dtype=F64)
    assert _close(part, full[[0, 4]])


def _qkn_small(seed=3):
    d = _apb_small(seed=seed)
    g = _g(seed + 100)
    HD = d["H"] * d["D"]
    r = lambda *s, sd=1.0: torch.randn(*s, generator=g, dtype=F64) * sd  # noqa: E731
    d.update(b_q=0.5 * r(HD), qkn_w_q=1 + 0.2 * r(HD), qkn_b_q=0.2 * r(HD), qkn_w_k=1 + 0.2 * r(HD),
             qkn_b_k=0.2 * r(HD))
    return d


def _qkn(d, fn=None, qkn=True, **over):
    """Call the qk-norm variant (oracle or brute force) on the dict d with overrides."""
    a = dict(d, **over)
    fn = fn or (lambda *x, **k: ref.attention_pair_bias_qknorm(*x, dtype=F64, **k))
    kw = dict(key_mask=a["mask"], scale=a["scale"])
    if qkn:
        kw.update(qkn_w_q=a["qkn_w_q"], qkn_b_q=a["qkn_b_q"], qkn_w_k=a["qkn_w_k"], qkn_b_k=a["qkn_b_k"])
    return fn(a["X"], a["WQ"], a["b_q"], a["WK"], a["WV"], a["Z"], a["W_ln"], a["B_ln"], a["W_proj_z"], a["B_proj_z"],
              a["W_proj_g"], a["W_proj_o"], a["H"], a["D"], **kw)


@pytest.mark.parametrize("qkn", [False, True])
def test_apb_qknorm_oracle_matches_brute(qkn):
    d = _qkn_small()
    for mask in (d["mask"], None):
        got = _qkn(d, qkn=qkn, mask=mask)
        assert _close(got, _qkn(d, fn=brute.attention_pair_bias_qknorm, qkn=qkn, mask=mask))
    part = ref.attention_pair_bias_qknorm(d["X"], d["WQ"], d["b_q"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"],
                                          d["W_proj_z"], d["B_proj_z"], d["W_proj_g"], d["W_proj_o"], 2, 3,
                                          key_mask=d["mask"], scale=d["scale"], dtype=F64, rows=[0, 3], chunk=1)
    full = ref.attention_pair_bias_qknorm(d["X"], d["WQ"], d["b_q"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"],
                                          d["W_proj_z"], d["B_proj_z"], d["W_proj_g"], d["W_proj_o"], 2, 3,
                                          key_mask=d["mask"], scale=d["scale"], dtype=F64)
    assert _close(part, full[[0, 3]])


def test_apb_qknorm_without_norm_is_apb():
    """qk-norm off, no Q bias: the plain op with bias-free gate / output projections (pinned above)."""
    d = _qkn_small()
    got = _qkn(d, qkn=False, b_q=None)
    want = ref.attention_pair_bias(d["X"], d["WQ"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                   d["B_proj_z"], d["W_proj_g"], None, d["W_proj_o"], None, 2, 3, scale=d["scale"],
                                   mask=d["mask"], dtype=F64)
    assert _close(got, want)


def test_apb_qknorm_norm_spans_all_heads_after_the_bias():
    """LN over the full H*D channel, applied after the Q bias: a constant added to every channel of
    b_q cancels; a constant that differs between heads does not (a per-head LN would cancel it)."""
    d = _qkn_small()
    base = _qkn(d)
    assert _close(base, _qkn(d, b_q=d["b_q"] + 0.7))
    per_head = torch.cat([torch.full((3,), 0.9, dtype=F64), torch.full((3,), -0.4, dtype=F64)])
    assert not _close(base, _qkn(d, b_q=d["b_q"] + per_head), tol=1e-4)
    # and without the norm the same per-channel constant is not removed
    assert not _close(_qkn(d, qkn=False), _qkn(d, qkn=False, b_q=d["b_q"] + 0.7), tol=1e-4)


def test_apb_qknorm_key_mask_crop():
    """Rows of the key-masked op equal the op on the cropped problem (valid keys first)."""
    d = _qkn_small()
    m = torch.tensor([True, True, True, False, False])
    full = _qkn(d, mask=m)
    crop = dict(d, X=d["X"][:3], Z=d["Z"][:3, :3], mask=None)
    assert _close(full[:3], _qkn(crop))


def _block_small(N=4, C=4, H=2, D=2, seed=11):
    """Weights of a tiny Pairformer pair stack (C = H*D so the attention output feeds the residual)."""
    _, _, tmu_out = _tmu_small(L=N, C=C, seed=seed)
    _, _, tmu_in = _tmu_small(L=N, C=C, seed=seed + 1)
    tri = []
    for k in (2, 3):
        d = _tri_small(N=N, C=C, H=H, D=D, seed=seed + k)
        tri.append({n: d[n] for n in ("W_ln", "B_ln", "WQ", "WK", "WV", "W_proj_z", "B_proj_z", "W_proj_g",
                                      "W_proj_o")})
    z = torch.randn(N, N, C, generator=_g(seed + 9), dtype=F64)
    m = torch.rand(N, N, generator=_g(seed + 10)) < 0.75
    m[:, 0] = True
    return z, m, tmu_out, tmu_in, tri[0], tri[1], H, D


def test_pair_stack_oracle_matches_brute_composition():
    """The oracle's pair stack == the same four residual updates built from the loop restatements
    (ending node = the op on z^T, transposed back)."""
    z, m, tmu_out, tmu_in, t0, t1, H, D = _block_small()
    got = ref.pair_stack(z, tmu_out, tmu_in, t0, t1, H, D, pair_mask=m, scale=0.5, dtype=F64)
    N = z.shape[0]
    zb = z.clone()
    zb = zb + torch.tensor(brute.triangle_multiplicative_update(zb[None], direction="outgoing",
                                                                mask=m.reshape(1, N, N).double(), **tmu_out),
                           dtype=F64)[0]
    zb = zb + torch.tensor(brute.triangle_multiplicative_update(zb[None], direction="incoming",
                                                                mask=m.reshape(1, N, N).double(), **tmu_in),
                           dtype=F64)[0]

    def tri(x, w, mask):
        return torch.tensor(brute.triangle_attention(x, w["W_ln"], w["B_ln"], w["WQ"], w["WK"], w["WV"],
                                                     w["W_proj_z"], w["B_proj_z"], w["W_proj_g"], None,
                                                     w["W_proj_o"], None, H, D, scale=0.5, mask=mask),
                            dtype=F64)

    zb = zb + tri(zb, t0, m)
    zb = zb + tri(zb.transpose(0, 1), t1, m.T).transpose(0, 1)
    assert _close(got, zb)
    # the ending node is not the starting node: swapping the transposes changes the result
    wrong = ref.pair_stack(z, tmu_out, tmu_in, t0, t0, H, D, pair_mask=m, scale=0.5, dtype=F64)
    assert not _close(got, wrong, tol=1e-6)


def test_single_update_oracle_is_residual_of_apb():
    d = _apb_small()
    apb = {k: d[k] for k in ("WQ", "WK", "WV", "W_ln", "B_ln", "W_proj_z", "B_proj_z", "W_proj_g", "B_proj_g",
                             "W_proj_o", "B_proj_o")}
    s = d["X"]
    got = ref.single_update(s, d["Z"], apb, 2, 3, key_mask=d["mask"], scale=d["scale"], dtype=F64)
    want = s + torch.tensor(brute.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=d["mask"]), dtype=F64)
    assert _close(got, want)


# --------------------------------------------------------------------------- #
# golden fixtures (written by brute force at the kernels' real widths)
# --------------------------------------------------------------------------- #
def _load(name):
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    inp = {k[3:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("in_")}
    meta = {k[5:]: z[k] for k in z.files if k.startswith("meta_")}
    return inp, torch.from_numpy(z["expected"]), meta


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_golden_tmu(direction):
    inp, expected, meta = _load(f"tmu_{direction}.npz")
    x, m = inp.pop("x"), inp.pop("mask")
    got = ref.triangle_multiplicative_update(x, direction=direction, mask=m, eps=float(meta["eps"]), **inp)
    assert (got.double() - expected).abs().max() < 2e-4


def test_golden_tri():
    inp, expected, meta = _load("tri_attn.npz")
    got = ref.triangle_attention(inp["X"], inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"], inp["WV"], inp["W_proj_z"],
                                 inp["B_proj_z"], inp["W_proj_g"], None, inp["W_proj_o"], None, 4, 32,
                                 scale=float(meta["scale"]), eps=float(meta["eps"]), mask=inp["mask"])
    assert (got.double() - expected).abs().max() < 2e-4


def test_golden_apb():
    inp, expected, meta = _load("apb.npz")
    got = ref.attention_pair_bias(inp["X"], inp["WQ"], inp["WK"], inp["WV"], inp["Z"], inp["W_ln"], inp["B_ln"],
                                  inp["W_proj_z"], inp["B_proj_z"], inp["W_proj_g"], inp["B_proj_g"],
                                  inp["W_proj_o"], inp["B_proj_o"], 4, 32, scale=float(meta["scale"]),
                                  eps=float(meta["eps"]), mask=inp["mask"])
    assert (got.double() - expected).abs().max() < 2e-4


# --------------------------------------------------------------------------- #
# closed forms and layouts
# --------------------------------------------------------------------------- #
def test_ln_fold_identity():
    """LN(x) W^T == rstd (x Wc^T - mean sum(Wc)) + W beta, both weight conventions."""
    g = _g(5)
    C, O = 16, 7
    x = torch.randn(9, C, generator=g, dtype=F64) * 3 + 1.5
    gam, bet = 1 + 0.3 * torch.randn(C, generator=g, dtype=F64), 0.3 * torch.randn(C, generator=g, dtype=F64)
    W = torch.randn(O, C, generator=g, dtype=F64)
    mean = x.mean(-1, keepdim=True)
    rstd = 1 / torch.sqrt(x.var(-1, unbiased=False, keepdim=True) + 1e-5)
    expect = F.layer_norm(x, (C,), gam, bet, 1e-5) @ W.t()
    # the fold is computed in fp32 by contract, so compare at fp32 accuracy
    Wc, sW, Bc = absorb_ln(W, gam, bet)
    assert _close(rstd * (x @ Wc.double().t() - mean * sW.double()) + Bc.double(), expect, tol=2e-5)
    Wc2, sW2, Bc2 = absorb_ln_matmul(W.t(), gam, bet)
    assert _close(rstd * (x @ Wc2.double() - mean * sW2.double()) + Bc2.double(), expect, tol=2e-5)
    # a dropped term (the mean correction) is far outside that tolerance
    assert not _close(rstd * (x @ Wc.double().t()) + Bc.double(), expect, tol=2e-5)
    # fold keeps fp32 sums of the unrounded folded weight and casts Wc to weight_dtype
    Wc3, sW3, _ = absorb_ln(W.float(), gam.float(), bet.float(), weight_dtype=torch.bfloat16)
    assert Wc3.dtype == torch.bfloat16 and sW3.dtype == torch.float32
    assert _close(sW3, (W.float() * gam.float()).sum(1), tol=1e-5)


def test_layout_permutations():
    C, H, D = 5, 3, 4
    WQ, WK, WV = (torch.arange(C * H * D, dtype=F64).reshape(C, H * D) + 1000 * r for r in range(3))
    qkv = interleave_qkv(WQ, WK, WV, H, D)
    kv = interleave_kv(WK, WV, H, D)
    hm = qkv_head_major(WQ, WK, WV, H, D)
    for h in range(H):
        for d in range(D):
            for r, W in enumerate((WQ, WK, WV)):
                assert torch.equal(qkv[:, 3 * h * D + r * D + d], W[:, h * D + d])
                assert torch.equal(hm[h, r, d, :], W[:, h * D + d])
            assert torch.equal(kv[:, 2 * h * D + 2 * d], WK[:, h * D + d])
            assert torch.equal(kv[:, 2 * h * D + 2 * d + 1], WV[:, h * D + d])


def test_einsum_direction_identity():
    g = _g(7)
    a = torch.randn(2, 5, 5, 3, generator=g, dtype=F64)
    b = torch.randn(2, 5, 5, 3, generator=g, dtype=F64)
    yin = ref.tmu_einsum(a, b, "incoming", F64)
    yout = ref.tmu_einsum(a.transpose(1, 2), b.transpose(1, 2), "outgoing", F64)
    assert _close(yin, yout)
    # and against an explicit loop on one element
    s = sum(a[1, k, 2, 1] * b[1, k, 4, 1] for k in range(5))
    assert abs(yin[1, 2, 4, 1].item() - s.item()) < 1e-12


# --------------------------------------------------------------------------- #
# attention invariants
# --------------------------------------------------------------------------- #
def test_tri_masked_keys_zero_weight_and_uniform_rows():
    d = _tri_small(N=5, full_masked_row=True)
    base = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"], dtype=F64)
    # perturbing x at (i, k) changes only row i's K/V of key k; masked keys must not matter
    m = d["mask"]
    i, k = next((i, k) for i in range(4) for k in range(5) if not m[i, k])
    X2 = d["X"].clone()
    X2[i, k] += 3.0
    xln2, bias2 = ref.tri_layer_norm_bias(X2, d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"], dtype=F64)
    xln, bias = ref.tri_layer_norm_bias(d["X"], d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"], dtype=F64)
    o1 = ref.tri_attention_core(xln, d["WQ"], d["WK"], d["WV"], bias, 2, 3, d["scale"], m, F64, rows=[i])
    o2 = ref.tri_attention_core(xln2, d["WQ"], d["WK"], d["WV"], bias, 2, 3, d["scale"], m, F64, rows=[i])
    q_other = [q for q in range(5) if q != k]
    assert _close(o1[0, q_other], o2[0, q_other])
    # fully masked row N-1: every query gets the uniform average of V over all N keys
    o = ref.tri_attention_core(xln, d["WQ"], d["WK"], d["WV"], bias, 2, 3, d["scale"], m, F64, rows=[4])
    v = xln[4] @ d["WV"]
    assert _close(o[0], v.mean(0, keepdim=True).expand(5, -1))
    assert torch.isfinite(base).all()


def test_tri_pad_crop_equivalence():
    d = _tri_small(N=6, full_masked_row=False)
    Nv = 4
    idx = torch.arange(6)
    m = (idx[:, None] < Nv) & (idx[None, :] < Nv)
    full = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=m, dtype=F64)
    dc = dict(d, X=d["X"][:Nv, :Nv])
    crop = ref.triangle_attention(*_tri_args(dc), scale=d["scale"], mask=None, dtype=F64)
    assert _close(full[:Nv, :Nv], crop)


def test_apb_masked_keys_and_all_masked():
    d = _apb_small()
    out = ref.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=d["mask"], dtype=F64)
    d2 = dict(d)
    d2["X"] = d["X"].clone()
    Z2 = d["Z"].clone()
    Z2[:, 1] += 5.0  # key 1 is masked: its pair features must not matter
    d2["Z"] = Z2
    assert _close(out, ref.attention_pair_bias(*_apb_args(d2), scale=d["scale"], mask=d["mask"], dtype=F64))
    allm = torch.zeros(5, dtype=torch.bool)
    o = ref.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=allm, dtype=F64)
    assert torch.isnan(o).all(), "all keys masked: softmax of all -inf is NaN, as in torch"


def test_tmu_masked_tokens_contribute_nothing():
    x, m, w = _tmu_small(L=5, seed=9)
    out = ref.triangle_multiplicative_update(x, direction="outgoing", mask=m, dtype=F64, **w)
    x2 = x.clone()
    b, i, k = map(int, (m == 0).nonzero()[0])
    x2[b, i, k] += 4.0
    out2 = ref.triangle_multiplicative_update(x2, direction="outgoing", mask=m, dtype=F64, **w)
    # token (i, k) feeds the einsum only through a[i,k] / b[i,k] (masked -> 0), but it is its own
    # output position's gate input, so every other output position is unchanged
    keep = torch.ones_like(out[..., 0], dtype=torch.bool)
    keep[b, i, k] = False
    assert _close(out[keep], out2[keep])


# --------------------------------------------------------------------------- #
# planted mistakes: each mutated oracle must fail the brute-force check
# --------------------------------------------------------------------------- #
def _mut_tmu_gate_on_y(x, *, direction, mask=None, eps=1e-5, dtype=torch.float32, rows=None, **w):
    g = ref.tmu_gated_input(x, mask, w["norm_in_weight"], w["norm_in_bias"], w["p_in_weight"], w["g_in_weight"],
                            eps, dtype)
    a, b = torch.chunk(g, 2, dim=-1)
    y = ref.tmu_einsum(a, b, direction, dtype)
    yln = ref.layer_norm(y, w["norm_out_weight"], w["norm_out_bias"], eps, dtype)
    return F.linear(yln, w["p_out_weight"].to(dtype)) * torch.sigmoid(F.linear(yln, w["g_out_weight"].to(dtype)))


def _mut_tmu_transposed_einsum(x, *, direction, mask=None, eps=1e-5, dtype=torch.float32, rows=None, **w):
    other = "incoming" if direction == "outgoing" else "outgoing"
    return ref.triangle_multiplicative_update(x, direction=other, mask=mask, eps=eps, dtype=dtype, **w)


def _mut_tmu_no_out_affine(x, *, direction, mask=None, eps=1e-5, dtype=torch.float32, rows=None, **w):
    w2 = dict(w, norm_out_bias=torch.zeros_like(w["norm_out_bias"]))
    return ref.triangle_multiplicative_update(x, direction=direction, mask=mask, eps=eps, dtype=dtype, **w2)


@pytest.mark.parametrize("mut", [_mut_tmu_gate_on_y, _mut_tmu_transposed_einsum, _mut_tmu_no_out_affine])
def test_planted_tmu_mistakes_are_caught(mut):
    x, m, w = _tmu_small(seed=11)
    expect = brute.triangle_multiplicative_update(x, direction="outgoing", mask=m, **w)
    assert not _close(mut(x, direction="outgoing", mask=m, dtype=F64, **w), expect)


def test_planted_tri_mistakes_are_caught():
    d = _tri_small(full_masked_row=False)
    expect = brute.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"])
    # mask on the query axis instead of the key axis
    wrong = ref.triangle_attention(*_tri_args(d), scale=d["scale"], mask=d["mask"].T, dtype=F64)
    assert not _close(wrong, expect)
    # bias indexed [h, k, q] instead of [h, q, k]
    xln, bias = ref.tri_layer_norm_bias(d["X"], d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"], dtype=F64)
    o = ref.tri_attention_core(xln, d["WQ"], d["WK"], d["WV"], bias.transpose(1, 2), 2, 3, d["scale"], d["mask"],
                               F64)
    wrong = ref.tri_gate_out(o, xln, d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], F64)
    assert not _close(wrong, expect)
    # gate on raw x instead of LN(x)
    o = ref.tri_attention_core(xln, d["WQ"], d["WK"], d["WV"], bias, 2, 3, d["scale"], d["mask"], F64)
    wrong = ref.tri_gate_out(o, d["X"], d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], F64)
    assert not _close(wrong, expect)


def test_planted_apb_mistakes_are_caught():
    d = _apb_small()
    expect = brute.attention_pair_bias(*_apb_args(d), scale=d["scale"], mask=d["mask"])
    # gate on LN(X) instead of raw X
    xln = F.layer_norm(d["X"], (6,))
    bias = ref.apb_bias(d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"], dtype=F64)
    o = ref.apb_attention_core(d["X"], d["WQ"], d["WK"], d["WV"], bias, 2, 3, d["scale"], d["mask"], F64)
    wrong = ref.apb_gate_out(o, xln, d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], F64)
    assert not _close(wrong, expect)
    # scale applied after the bias instead of to Q.K only
    o = ref.apb_attention_core(d["X"], d["WQ"], d["WK"], d["WV"], bias / d["scale"], 2, 3, d["scale"], d["mask"],
                               F64)
    wrong = ref.apb_gate_out(o, d["X"], d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], F64)
    assert not _close(wrong, expect)


def test_brute_softmax_matches_math():
    w = brute._softmax_weights([0.0, math.log(3.0)])
    assert abs(w[0] - 0.25) < 1e-15 and abs(w[1] - 0.75) < 1e-15
