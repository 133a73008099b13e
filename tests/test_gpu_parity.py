"""GPU parity: each op through the HIP library vs the CPU fp32 oracle on the same seeded inputs.

Bar (written here, applied to every output element): bf16 max|out - oracle| <= 3e-2 and
cosine >= 0.9999 (fp16: max|diff| <= 1e-2).  Masking is checked bit-exactly where the
semantics fix it: masked tokens give exact zeros in the triangle_mul gated projection, and a
padded+masked problem restricted to its valid block equals the cropped problem bitwise.
Large configurations are checked on a sample of output rows (rows are independent).
"""

import math

import pytest
import torch
from _inputs import (TOL_COS, TOL_MAX_ABS, apb_inputs, apb_qkn_inputs, compare, pad_pair_mask, tmu_inputs, to_dev,
                     tri_inputs)

import triangleops_amd as tops
from oracle import reference as ref

pytestmark = pytest.mark.gpu

TMU_W = ("norm_in_weight", "norm_in_bias", "p_in_weight", "g_in_weight", "norm_out_weight", "norm_out_bias",
         "p_out_weight", "g_out_weight")


def _check(out, expect, dtype, what):
    diff, cos = compare(out, expect)
    assert torch.isfinite(out.float()).all(), f"{what}: non-finite output"
    assert diff <= TOL_MAX_ABS[dtype] and cos >= TOL_COS, f"{what}: max|d|={diff:.3e} cos={cos:.6f}"
    return diff, cos


# --------------------------------------------------------------------------- #
# triangle_multiplicative_update
# --------------------------------------------------------------------------- #
@pytest.mark.parametrize("L", [33, 64, 130, 256])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
@pytest.mark.parametrize("mask", ["none", "pad", "random"])
def test_tmu_matches_oracle(device, L, direction, mask):
    x, m, w = tmu_inputs(L, seed=L, mask=mask)
    out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction,
                                              mask=None if m is None else m.to(device), **to_dev(w, device))
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, torch.bfloat16, f"tmu L={L} {direction} mask={mask}")


def test_tmu_config0_all_ones_mask(device):
    """BASELINE config 0 through the HIP path: outgoing, L = 128, all-ones mask, seed 0, the whole
    output against the fp32 oracle; and an all-ones mask gives the same bits as no mask."""
    x, m, w = tmu_inputs(128, seed=0, mask="ones")
    xd, wd = to_dev(x, device), to_dev(w, device)
    out = tops.triangle_multiplicative_update(xd, direction="outgoing", mask=m.to(device), **wd)
    expect = ref.triangle_multiplicative_update(x, direction="outgoing", mask=m, **w)
    _check(out, expect, torch.bfloat16, "tmu config 0")
    assert torch.equal(out, tops.triangle_multiplicative_update(xd, direction="outgoing", mask=None, **wd))


@pytest.mark.parametrize("dtype", [torch.float16])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_fp16(device, dtype, direction):
    x, m, w = tmu_inputs(96, seed=5, mask="random", dtype=dtype)
    out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                              **to_dev(w, device))
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, dtype, f"tmu fp16 {direction}")


@pytest.mark.parametrize("C", [32, 64, 96, 192, 320])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_any_channels(device, C, direction):
    """C != 128 runs the any-shape input / output phases (tiled up to C = 256, per-token above);
    the einsum kernels take any channel count."""
    x, m, w = tmu_inputs(70 if C <= 256 else 24, C=C, seed=C, mask="random")
    out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                              **to_dev(w, device))
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, torch.bfloat16, f"tmu C={C} {direction}")


@pytest.mark.parametrize("C,L", [(128, 40), (64, 130)])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_fp32_io(device, C, L, direction):
    """fp32 I/O: any-shape phases and the fp32 batched product, every value fp32 (max |d| <= 1e-4)."""
    x, m, w = tmu_inputs(L, C=C, seed=L + C, mask="pad", dtype=torch.float32)
    out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                              **to_dev(w, device))
    assert out.dtype == torch.float32
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, torch.float32, f"tmu fp32 C={C} L={L} {direction}")


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_fp32_batch(device, direction):
    """fp32 I/O with B = 2 and a ragged L: the tiled any-shape phases index batch rows and tail tiles."""
    x, m, w = tmu_inputs(33, B=2, C=96, seed=5, mask="random", dtype=torch.float32)
    out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                              **to_dev(w, device))
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, torch.float32, f"tmu fp32 B=2 {direction}")


def test_tmu_batch(device):
    x, m, w = tmu_inputs(48, B=3, seed=7, mask="random")
    for direction in ("outgoing", "incoming"):
        out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                                  **to_dev(w, device))
        expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
        _check(out, expect, torch.bfloat16, f"tmu B=3 {direction}")


def test_tmu_batch_large(device):
    """B = 2 at L = 512: the persistent einsum over C * B slabs and the phases' batch indexing,
    on sampled output rows of both batch elements."""
    L = 512
    x, m, w = tmu_inputs(L, B=2, seed=13, mask="random")
    rows = torch.tensor([0, 77, L // 2, L - 1])
    for direction in ("outgoing", "incoming"):
        out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                                  **to_dev(w, device))
        expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, rows=rows, **w)
        _check(out[:, rows].cpu(), expect, torch.bfloat16, f"tmu B=2 L={L} {direction}")


@pytest.mark.parametrize("transpose", [False, True])
def test_tmu_input_phase_and_mask_zeros(device, transpose):
    """Gated projection vs oracle; masked tokens are exactly zero (bit-exact masking)."""
    L = 80
    x, m, w = tmu_inputs(L, seed=3, mask="random")
    pre = tops.triangle_mul.precompute(*[w[k].to(device) for k in TMU_W])
    ld = 128
    ab = tops.triangle_mul.input_phase(to_dev(x, device), m.to(device), pre["p_in_combined"], pre["g_in_combined"],
                                       pre["sum_W_p_in"], pre["sum_W_g_in"], pre["B_p_in_const"],
                                       pre["B_g_in_const"], 1e-5, transpose=transpose, ld=ld)
    ab = ab.cpu()
    assert torch.all(ab[..., L:] == 0), "padding columns must be zero"
    ab = ab[..., :L]
    if transpose:
        ab = ab.transpose(-1, -2)
    g = ref.tmu_gated_input(x, m, w["norm_in_weight"], w["norm_in_bias"], w["p_in_weight"], w["g_in_weight"])
    _check(ab.permute(1, 2, 3, 0), g, torch.bfloat16, "tmu input phase")
    masked = ~m
    assert torch.all(ab.permute(1, 2, 3, 0)[masked] == 0), "masked tokens must be exactly zero"


def test_tmu_default_layout_low_level(device):
    """Reference-layout low-level path: input_phase (2C,B,L,L) -> torch einsum -> output_phase."""
    L = 72
    x, m, w = tmu_inputs(L, seed=9, mask="pad")
    xd = to_dev(x, device)
    pre = tops.triangle_mul.precompute(*[w[k].to(device) for k in TMU_W])
    ab = tops.triangle_mul.input_phase(xd, m.to(device), pre["p_in_combined"], pre["g_in_combined"],
                                       pre["sum_W_p_in"], pre["sum_W_g_in"], pre["B_p_in_const"],
                                       pre["B_g_in_const"], 1e-5)
    assert ab.shape == (256, 1, L, L)
    a, b = torch.chunk(ab.float(), 2, 0)
    y = torch.einsum("dbik,dbjk->dbij", a, b).to(torch.bfloat16).contiguous()
    out = tops.triangle_mul.output_phase(y, xd, pre["p_out_combined"], pre["g_out_combined"], pre["sum_W_p_out"],
                                         pre["sum_W_g_out"], pre["B_p_out_const"], pre["B_g_out_const"], 1e-5)
    expect = ref.triangle_multiplicative_update(x, direction="outgoing", mask=m, **w)
    _check(out, expect, torch.bfloat16, "tmu low-level reference layout")


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_pad_crop_bitwise(device, direction):
    """op(x, padding mask)[valid block] == op(x[valid block]) bitwise."""
    L, Lv = 128, 100
    x, _, w = tmu_inputs(L, seed=11, mask="none")
    idx = torch.arange(L)
    m = ((idx[:, None] < Lv) & (idx[None, :] < Lv)).unsqueeze(0)
    wd = to_dev(w, device)
    full = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device), **wd)
    crop = tops.triangle_multiplicative_update(to_dev(x[:, :Lv, :Lv].contiguous(), device), direction=direction,
                                               mask=None, **wd)
    assert torch.equal(full[:, :Lv, :Lv], crop)


def test_tmu_precompute_forward_matches_oneshot(device):
    x, m, w = tmu_inputs(256, seed=1, mask="ones")
    xd, md, wd = to_dev(x, device), m.to(device), to_dev(w, device)
    pre = tops.triangle_mul.precompute(*[wd[k] for k in TMU_W])
    a = tops.triangle_mul.forward(xd, pre, direction="outgoing", mask=md)
    b = tops.triangle_multiplicative_update(xd, direction="outgoing", mask=md, **wd)
    assert torch.equal(a, b)
    assert torch.equal(a, tops.triangle_mul.forward(xd, pre, direction="outgoing", mask=md)), "not deterministic"


@pytest.mark.parametrize("L", [512, 1024])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_config_sizes_whole_output(device, L, direction):
    """BASELINE config 1 sizes (pad mask): the whole output against the fp32 oracle."""
    x, m, w = tmu_inputs(L, seed=0, mask="pad")
    out = tops.triangle_multiplicative_update(to_dev(x, device), direction=direction, mask=m.to(device),
                                              **to_dev(w, device)).cpu()
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, torch.bfloat16, f"tmu L={L} {direction}")


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_tmu_fp16_large_offset(device, direction):
    """fp16 tokens with a large common offset (x = 300 + N(0, 0.5), quantised to 0.25): the
    LayerNorm statistics must not cancel (E[x^2] - mean^2 in fp32 would lose the variance)."""
    x, m, w = tmu_inputs(64, seed=31, mask="random", dtype=torch.float32)
    x = (300.0 + 0.5 * x).to(torch.float16)
    w = {k: v.to(torch.float16) for k, v in w.items()}
    out = tops.triangle_multiplicative_update(x.to(device), direction=direction, mask=m.to(device),
                                              **to_dev(w, device))
    expect = ref.triangle_multiplicative_update(x, direction=direction, mask=m, **w)
    _check(out, expect, torch.float16, f"tmu fp16 offset {direction}")


@pytest.mark.parametrize("L,nslab,dtype", [(400, 8, torch.bfloat16), (600, 64, torch.bfloat16),
                                           (768, 4, torch.bfloat16), (1000, 32, torch.bfloat16),
                                           (1024, 40, torch.bfloat16), (600, 64, torch.float16),
                                           (768, 4, torch.float16), (512, 100, torch.bfloat16),
                                           (1280, 16, torch.bfloat16), (1536, 12, torch.bfloat16),
                                           (2048, 6, torch.bfloat16)])
def test_tmu_einsum_large_kernels(device, L, nslab, dtype):
    """The L > 384 einsum kernels against a torch fp32 product of the same 16-bit operands: odd
    k-tile counts (L = 400), rows past L in the last block tile (L = 600, 1000), and the
    persistent kernel (L % 256 == 0) with fewer block tiles than CUs (L = 768) and with several
    block tiles per block in an uneven split (L = 1024, 640 tiles), including each width of its
    staggered k order (k-tile kt ^ r, r < 2 / 4 / 8 at L = 512 / 1024-1536 / 2048; L = 1280 and
    1536 have 5 and 6 block tiles per slab side, not a power of two).  Each output is the fp32 sum
    rounded once: within half an ulp of the 16-bit type plus the fp32 summation-order difference."""
    ld = (L + 63) // 64 * 64
    g = torch.Generator().manual_seed(L + nslab)
    ab = torch.zeros(2 * nslab, 1, L, ld, dtype=dtype)
    ab[..., :L] = torch.randn(2 * nslab, 1, L, L, generator=g).to(dtype)
    ab = ab.to(device)
    y = tops.triangle_mul.triangle_einsum(ab, L, ld, nslab, 1)
    a, b = ab[:nslab, 0].float(), ab[nslab:, 0].float()
    expect = torch.bmm(a, b.transpose(1, 2).contiguous())  # fp32 on the GPU
    half_ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = (y[:, 0, :, :L].float() - expect[:, :, :L]).abs()
    bound = half_ulp * expect[:, :, :L].abs() + 1e-5 * expect.abs().max()
    assert bool((err <= bound).all()), f"L={L} nslab={nslab}: max excess {float((err - bound).max()):.3e}"
    assert bool(torch.isfinite(y[..., L:].float()).all()), "padding columns must be finite"


@pytest.mark.parametrize("L,nslab", [(40, 3), (128, 2), (130, 4), (300, 5), (1024, 2)])
def test_tmu_einsum_fp32(device, L, nslab):
    """The fp32 product (fp32 MFMA, fp32 sums) against a float64 product of the same operands:
    rows past L in the last 128-row tile (L = 40, 130, 300), an exact tile (L = 128) and L = 1024.
    Bound: 1e-5 of sum_k |a||b| (fp32 rounding of up to 1024 terms, random signs)."""
    ld = (L + 63) // 64 * 64
    g = torch.Generator().manual_seed(L + 3 * nslab)
    ab = torch.zeros(2 * nslab, 1, L, ld, dtype=torch.float32)
    ab[..., :L] = torch.randn(2 * nslab, 1, L, L, generator=g)
    y = tops.triangle_mul.triangle_einsum(ab.to(device), L, ld, nslab, 1)
    assert y.dtype == torch.float32
    a, b = ab[:nslab, 0, :, :L].double(), ab[nslab:, 0, :, :L].double()
    expect = torch.bmm(a, b.transpose(1, 2))
    scale = torch.bmm(a.abs(), b.abs().transpose(1, 2))
    err = (y[:, 0, :, :L].cpu().double() - expect).abs()
    assert bool((err <= 1e-5 * scale + 1e-30).all()), f"L={L}: max err/scale {float((err / scale).max()):.3e}"


@pytest.mark.parametrize("L,nslab,pad,dtype", [(1024, 8, 128, torch.bfloat16), (600, 16, 64, torch.bfloat16),
                                               (200, 8, 64, torch.float16), (100, 4, 64, torch.float32)])
def test_tmu_einsum_row_padding_not_read(device, L, nslab, pad, dtype):
    """The product reads k < round_up(L, 64) only: a row stride ld beyond that is pure padding,
    here filled with NaN, and the result equals the one with ld = round_up(L, 64) bit for bit
    (persistent, large, small and fp32 kernels)."""
    lr = (L + 63) // 64 * 64
    g = torch.Generator().manual_seed(L)
    vals = torch.randn(2 * nslab, 1, L, L, generator=g).to(dtype)
    tight = torch.zeros(2 * nslab, 1, L, lr, dtype=dtype)
    tight[..., :L] = vals
    padded = torch.full((2 * nslab, 1, L, lr + pad), float("nan"), dtype=dtype)
    padded[..., :lr] = tight
    y0 = tops.triangle_mul.triangle_einsum(tight.to(device), L, lr, nslab, 1)
    y1 = tops.triangle_mul.triangle_einsum(padded.to(device), L, lr + pad, nslab, 1)
    assert torch.equal(y0[..., :L], y1[..., :L])


# --------------------------------------------------------------------------- #
# triangle_attention
# --------------------------------------------------------------------------- #
def _tri_call(inp, device, X=None, mask="inp"):
    d = to_dev(inp, device)
    return tops.triangle_attention(d["X"] if X is None else X, d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"],
                                   d["W_proj_z"], d["B_proj_z"], d["W_proj_g"], None, d["W_proj_o"], None, d["H"],
                                   d["D"], scale=d["scale"], eps=1e-5, mask=d["mask"] if mask == "inp" else mask)


def _tri_ref(inp, X=None, mask="inp", rows=None):
    return ref.triangle_attention(inp["X"] if X is None else X, inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"],
                                  inp["WV"], inp["W_proj_z"], inp["B_proj_z"], inp["W_proj_g"], None, inp["W_proj_o"],
                                  None, inp["H"], inp["D"], scale=inp["scale"], eps=1e-5,
                                  mask=inp["mask"] if mask == "inp" else mask, rows=rows)


@pytest.mark.parametrize("N", [33, 128, 130, 256])
@pytest.mark.parametrize("mask", ["none", "pad", "random"])
def test_tri_matches_oracle(device, N, mask):
    inp = tri_inputs(N, seed=N, mask=mask, bias_z=True)
    out = _tri_call(inp, device)
    _check(out, _tri_ref(inp), torch.bfloat16, f"tri N={N} mask={mask}")


def test_tri_fp16(device):
    inp = tri_inputs(96, seed=4, mask="random", dtype=torch.float16)
    _check(_tri_call(inp, device), _tri_ref(inp), torch.float16, "tri fp16")


@pytest.mark.parametrize("N,mask,qk", [(260, "pad", 1.0), (520, "random", 1.0), (260, "random", 2.0)])
def test_tri_fp16_two_query_tiles(device, N, mask, qk):
    """fp16 triangle attention where each wave holds two query tiles (N > 128): the running row max
    enters the accumulator initialiser beside the bias, and with Q and K scaled up (qk = 2: scores
    spread over tens of log2 units, so later tiles' weights would overflow fp16 under the first
    tile's max) the max is raised mid-row and O / l rescaled.  (Much larger scores put the fp16
    rounding of Q and K, relative to the score, beyond the fp16 bar against the fp32 oracle, in any
    16-bit attention.)"""
    inp = tri_inputs(N, seed=N + 7, mask=mask, dtype=torch.float16, bias_z=True)
    inp["WQ"] = (inp["WQ"].float() * qk).to(torch.float16)
    inp["WK"] = (inp["WK"].float() * qk).to(torch.float16)
    _check(_tri_call(inp, device), _tri_ref(inp), torch.float16, f"tri fp16 N={N} mask={mask} qk={qk}")


def test_tri_ending_node(device):
    """Ending node = op on X^T (a strided view, no copy) with mask^T, output transposed back."""
    N = 160
    inp = tri_inputs(N, seed=21, mask="pad")
    Xd = inp["X"].to(device)
    out = _tri_call(inp, device, X=Xd.transpose(0, 1), mask=inp["mask"].to(device).T).transpose(0, 1)
    expect = _tri_ref(inp, X=inp["X"].transpose(0, 1), mask=inp["mask"].T).transpose(0, 1)
    _check(out, expect, torch.bfloat16, "tri ending node")


def test_tri_masked_rows_uniform_and_pad_crop(device):
    """Fully masked rows average V uniformly; valid block equals the cropped problem bitwise."""
    N, Nv = 128, 96
    inp = tri_inputs(N, seed=5, mask="none")
    idx = torch.arange(N)
    m = (idx[:, None] < Nv) & (idx[None, :] < Nv)
    full = _tri_call(inp, device, mask=m.to(device))
    crop_inp = dict(inp, X=inp["X"][:Nv, :Nv].contiguous(), mask=None)
    crop = _tri_call(crop_inp, device)
    assert torch.equal(full[:Nv, :Nv], crop)
    _check(full, _tri_ref(inp, mask=m), torch.bfloat16, "tri padded rows")


def test_tri_low_level_entry_points(device):
    """triangle_attn_forward + fused_gate_forward reproduce forward() (reference call sequence)."""
    N = 64
    inp = to_dev(tri_inputs(N, seed=8, mask="random"), device)
    H, D = inp["H"], inp["D"]
    pre = tops.triangle_attn.precompute(inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"], inp["WV"], inp["W_proj_z"],
                                        inp["B_proj_z"], H, D)
    X_ln = torch.nn.functional.layer_norm(inp["X"], (128,), inp["W_ln"], inp["B_ln"], 1e-5)
    O = torch.empty(N, N, H * D, device=device, dtype=torch.bfloat16)
    tops.triangle_attn.triangle_attn_forward(X_ln, pre["WQ_c"], pre["WKV_c"], pre["WZ_c"], pre["BZ"], O,
                                             scale=inp["scale"], mask=inp["mask"])
    out = tops.triangle_attn.fused_gate_forward(O.view(N, N, H, D), X_ln, inp["W_proj_g"], inp["W_proj_o"])
    _check(out, _tri_ref(to_dev(inp, "cpu")), torch.bfloat16, "tri low-level")


def _config_rows(n, k=32):
    """k rows spread over [0, n) plus the last valid / first padded row of the pad mask."""
    v = n - n // 10
    return torch.unique(torch.cat([torch.linspace(0, n - 1, k).round().long(), torch.tensor([v - 1, v])]))


@pytest.mark.parametrize("N", [512, 1024, 2048])
def test_tri_config_sizes(device, N):
    """BASELINE configs 3/4 sizes (pad mask), starting and ending node: the whole output at
    N <= 1024; at 2048 34 rows spread over the grid, every query of each."""
    inp = tri_inputs(N, seed=0, mask="pad")
    rows = None if N <= 1024 else _config_rows(N)
    out = _tri_call(inp, device)
    out = (out if rows is None else out[rows.to(device)]).cpu()
    _check(out, _tri_ref(inp, rows=rows), torch.bfloat16, f"tri N={N} start")
    del out
    Xd = inp["X"].to(device)
    out_e = _tri_call(inp, device, X=Xd.transpose(0, 1), mask=inp["mask"].to(device).T)
    out_e = (out_e if rows is None else out_e[rows.to(device)]).cpu()
    exp_e = _tri_ref(inp, X=inp["X"].transpose(0, 1), mask=inp["mask"].T, rows=rows)
    _check(out_e, exp_e, torch.bfloat16, f"tri N={N} end")


def test_tri_padded_heads_not_multiple_of_8(device):
    """Heads of D = 12 (not a multiple of 8) in bf16 run the MFMA attention kernel on 32-wide zero-padded
    heads written to a scratch output whose first D columns of each head are kept."""
    inp = tri_inputs(130, C=48, H=4, D=12, seed=12, mask="random", bias_z=True)
    _check(_tri_call(inp, device), _tri_ref(inp), torch.bfloat16, "tri D=12")


def _bias_rows_below_n(bias, N):
    """The pre-pass bias tiles (H, ceil(N/32), ldn/32, 1024) as fp32 with the rows of queries >= N
    (in the last query tile; the pre-pass never writes them and the attention never reads them) set
    to zero.  Element (q, k) = (32 qt + c, ...) of a tile sits at (64 j + 32 hl + c) * 8 + e."""
    b = bias.float()
    c = (torch.arange(1024, device=b.device) // 8) % 32
    q = 32 * torch.arange(b.shape[1], device=b.device)[:, None] + c[None, :]  # (qt, 1024)
    return torch.where((q < N)[None, :, None, :], b, torch.zeros_like(b))


@pytest.mark.parametrize("N,shift", [(200, 150.0), (200, -200.0), (520, 150.0), (2100, -200.0)])
def test_tri_shift_free_softmax_fallback(device, N, shift):
    """bf16 triangle attention takes the weights as 2^s without the row max and recomputes a wave's
    query tiles with an exact running max when its row sums leave [2^-60, 2^100].  Softmax is
    shift-invariant, so adding a constant to every score of a (head, query tile) must leave its
    output unchanged.  The pre-pass bias tiles (log2 units) are rounded to integers, which bf16 holds
    exactly up to 256, and head 0's tiles (every query tile) and head 2's tiles of query tiles 2 and 3
    are shifted by +150 (the shift-free weights overflow) or -200 (they underflow): those heads must
    match the unshifted run to the bf16 bar, while heads 1 and 3, which run the shift-free path in the
    same launch, must match it bitwise.  N = 2100 runs the ragged 4-wave blocks."""
    from triangleops_amd.triangle_attn.kernel import attention_core, prep_forward

    inp = to_dev(tri_inputs(N, seed=N + 7, mask="random", bias_z=True), device)
    pre = tops.triangle_attn.precompute(inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"], inp["WV"], inp["W_proj_z"],
                                        inp["B_proj_z"], 4, 32)
    Qp, KV, bias, ldn = prep_forward(inp["X"], pre["W_ln"], pre["B_ln"], pre["wqkv_hm"], pre["WZ_c"], pre["BZ"],
                                     scale=inp["scale"])
    b0 = _bias_rows_below_n(bias, N).round()
    b1 = b0.clone()
    b1[0] += shift
    b1[2, 2:4] += shift
    assert b1.abs().max().item() < 256
    outs = []
    for b in (b0, b1):
        o = torch.empty(N, N, 128, device=device, dtype=torch.bfloat16)
        attention_core(Qp, KV, b.to(torch.bfloat16), o, N=N, ldn=ldn, mask=inp["mask"])
        outs.append(o.view(N, N, 4, 32).cpu())
    a, b = outs
    assert torch.isfinite(b.float()).all(), "non-finite output after the fallback"
    assert torch.equal(a[:, :, 1], b[:, :, 1]) and torch.equal(a[:, :, 3], b[:, :, 3])
    for h in (0, 2):
        _check(b[:, :, h], a[:, :, h].float(), torch.bfloat16, f"tri fallback N={N} shift={shift} head {h}")


def _two_row_mask(N, seed):
    """Random mask (80 % valid) with a pair of rows without valid keys (rows 2, 3), and a pair in
    which only the first row has none (rows 4, 5)."""
    m = torch.rand(N, N, generator=torch.Generator().manual_seed(seed)) < 0.8
    if N >= 8:
        m[2:5] = False
    return m


# tri_attn2_kernel faulted the GPU in an earlier build, whose copies were inline-asm global_load_lds
# with a base address rebuilt from v_readfirstlane halves.  Its copies now go through the compiler's
# global_load_lds builtin (the compiler sets M0 and inserts the wait states), and its index
# arithmetic is checked on the CPU by tests/test_tri_two_row_model.py; these tests passed on their
# first GPU run after that rewrite.
@pytest.mark.parametrize("N,mask", [(8, "two_row"), (33, "pad"), (130, "two_row"), (256, "pad"), (520, "two_row"),
                                    (1024, "pad")])
def test_tri_two_row_kernel(device, N, mask):
    """tops_tri_attention_two_row against tops_tri_attention on the same pre-pass buffers (bf16
    rounding of the weights at the same points; rows without valid keys in pairs and mixed pairs),
    and through the gate against the fp32 oracle; masked keys carry no weight (perturbing them
    changes nothing)."""
    from triangleops_amd import _native
    from triangleops_amd.triangle_attn.kernel import attention_core, gate_out_forward, prep_forward

    inp = tri_inputs(N, seed=N + 17, mask="pad" if mask == "pad" else "none", bias_z=True)
    if mask == "two_row":
        inp["mask"] = _two_row_mask(N, N)
    d = to_dev(inp, device)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], 4, 32)
    Qp, KV, bias, ldn = prep_forward(d["X"], pre["W_ln"], pre["B_ln"], pre["wqkv_hm"], pre["WZ_c"], pre["BZ"],
                                     scale=d["scale"])
    one = torch.empty(N, N, 128, device=device, dtype=torch.bfloat16)
    attention_core(Qp, KV, bias, one, N=N, ldn=ldn, mask=d["mask"])
    m8 = d["mask"].to(torch.int8).contiguous()

    def two(kv):
        o = torch.full((N, N, 128), float("nan"), device=device, dtype=torch.bfloat16)
        _native.call("tops_tri_attention_two_row", Qp.data_ptr(), kv.data_ptr(), bias.data_ptr(), m8.data_ptr(),
                     m8.stride(0), m8.stride(1), o.data_ptr(), o.stride(0), o.stride(1), N, ldn, 4, 32, 2,
                     _native.stream_of(Qp))
        return o

    o2 = two(KV)
    torch.cuda.synchronize()
    assert torch.isfinite(o2.float()).all(), f"N={N}: unwritten or non-finite output"
    _check(o2.cpu(), one.float().cpu(), torch.bfloat16, f"two-row vs one-row N={N} {mask}")
    out = gate_out_forward(o2, d["X"], d["W_proj_g"], None, d["W_proj_o"], None, ln=(pre["W_ln"], pre["B_ln"], 1e-5))
    rows = None if N <= 520 else torch.tensor([0, 1, N // 2, N - N // 10 - 1, N - 1])
    expect = _tri_ref(inp, rows=rows)
    _check((out if rows is None else out[rows.to(device)]).cpu(), expect, torch.bfloat16, f"two-row oracle N={N}")
    # masked keys are inert: perturb every K / V row of a key masked in a row (pre-pass layout)
    if N <= 256:
        kv2 = KV.clone()
        kvv = kv2.view(N, 4, ldn // 64, 4096)
        g = torch.Generator().manual_seed(N)
        for i in range(N):
            for k in torch.nonzero(~inp["mask"][i]).flatten().tolist():
                kb, kk = divmod(k, 64)
                kvv[i, :, kb, kk * 32:(kk + 1) * 32] = (10 * torch.randn(4, 32, generator=g)).to(kvv.dtype).to(device)
                # V^T column of key kk: group kk // 32, position x with perm32(x) = kk % 32
                n = kk % 32
                j, rem = n >> 4, n & 15
                x = 32 * (kk // 32) + 16 * j + 8 * ((rem >> 2) & 1) + 4 * (rem >> 3) + (rem & 3)
                cols = 2048 + 64 * torch.arange(32) + x
                kvv[i, :, kb, cols.to(device)] = (10 * torch.randn(4, 32, generator=g)).to(kvv.dtype).to(device)
        o3 = two(kv2)
        valid_rows = inp["mask"].any(1)
        assert torch.equal(o3[valid_rows.to(device)], o2[valid_rows.to(device)]), "masked keys changed the output"


@pytest.mark.parametrize("shift", [150.0, -200.0])
def test_tri_two_row_fallback(device, shift):
    """The two-row kernel's exact-max recomputation: shifted bias tiles (see
    test_tri_shift_free_softmax_fallback) give the unshifted output to the bf16 bar."""
    from triangleops_amd import _native
    from triangleops_amd.triangle_attn.kernel import prep_forward

    N = 200
    d = to_dev(tri_inputs(N, seed=N + 9, mask="random", bias_z=True), device)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], 4, 32)
    Qp, KV, bias, ldn = prep_forward(d["X"], pre["W_ln"], pre["B_ln"], pre["wqkv_hm"], pre["WZ_c"], pre["BZ"],
                                     scale=d["scale"])
    b0 = _bias_rows_below_n(bias, N).round()
    b1 = b0.clone()
    b1[0] += shift
    b1[2, 2:4] += shift
    m8 = d["mask"].to(torch.int8).contiguous()
    outs = []
    for b in (b0, b1):
        o = torch.empty(N, N, 128, device=device, dtype=torch.bfloat16)
        bb = b.to(torch.bfloat16)
        _native.call("tops_tri_attention_two_row", Qp.data_ptr(), KV.data_ptr(), bb.data_ptr(), m8.data_ptr(),
                     m8.stride(0), m8.stride(1), o.data_ptr(), o.stride(0), o.stride(1), N, ldn, 4, 32, 2,
                     _native.stream_of(Qp))
        torch.cuda.synchronize()
        outs.append(o.view(N, N, 4, 32).cpu())
    a, b = outs
    assert torch.isfinite(b.float()).all()
    assert torch.equal(a[:, :, 1], b[:, :, 1]) and torch.equal(a[:, :, 3], b[:, :, 3])
    for h in (0, 2):
        _check(b[:, :, h], a[:, :, h].float(), torch.bfloat16, f"two-row fallback shift={shift} head {h}")


@pytest.mark.parametrize("N", [100, 384])
def test_tri_masked_keys_bitwise_invariant(device, N):
    """Masked keys contribute exactly nothing (weight exactly 0, benchmarks/references.py:198-201 with
    the reference kernel's -1e9 add, triangle_attn/kernel.py:230-238).
    (a) Kernel level, random pair mask: the attention core fed with K/V projected from x perturbed at
        every masked (i, k) returns the same bits as with the original K/V.
    (b) Op level, a key mask shared by all rows (mask[i, k] = valid[k]): perturbing x[:, k] at every
        masked k changes only output columns k (their own query, gate input and bias entries are
        perturbed); every other output element is bitwise unchanged."""
    from triangleops_amd.triangle_attn.kernel import attention_core, prep_forward

    inp = tri_inputs(N, seed=N + 3, mask="random", bias_z=True)
    d = to_dev(inp, device)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], 4, 32)
    m = d["mask"]
    g = torch.Generator().manual_seed(N)
    noise = torch.randn(N, N, 128, generator=g).to(torch.bfloat16).to(device)
    X2 = torch.where(m[..., None], d["X"], d["X"] + 3 * noise)
    args = (pre["W_ln"], pre["B_ln"], pre["wqkv_hm"], pre["WZ_c"], pre["BZ"])
    Qp, KV, bias, ldn = prep_forward(d["X"], *args, scale=inp["scale"])
    _, KV2, _, _ = prep_forward(X2, *args, scale=inp["scale"])
    o1 = torch.empty(N, N, 128, device=device, dtype=torch.bfloat16)
    o2 = torch.empty_like(o1)
    attention_core(Qp, KV, bias, o1, N=N, ldn=ldn, mask=m)
    attention_core(Qp, KV2, bias, o2, N=N, ldn=ldn, mask=m)
    rows = m.any(dim=1)  # a row without valid keys averages every key (uniform path)
    assert not torch.equal(KV, KV2)
    assert torch.equal(o1[rows], o2[rows]), "masked keys changed valid rows (kernel level)"

    valid = torch.rand(N, generator=g) < 0.8
    valid[0] = False
    km = valid[None, :].expand(N, N).contiguous().to(device)
    X3 = d["X"].clone()
    X3[:, ~valid.to(device)] += 3 * noise[:, ~valid.to(device)]
    kw = dict(mask=km, scale=inp["scale"], W_proj_g=d["W_proj_g"], B_proj_g=None, W_proj_o=d["W_proj_o"],
              B_proj_o=None)
    a = tops.triangle_attn.forward(d["X"], pre, **kw)
    b = tops.triangle_attn.forward(X3, pre, **kw)
    cols = valid.to(device)
    assert not torch.equal(a[:, ~cols], b[:, ~cols])
    assert torch.equal(a[:, cols], b[:, cols]), "masked keys changed the output (op level)"
    _check(a, _tri_ref(inp, mask=km.cpu()), torch.bfloat16, f"tri key mask N={N}")


@pytest.mark.parametrize("N", [257, 300, 520])
@pytest.mark.parametrize("mask", ["none", "pad", "random"])
def test_tri_large_n_kernel(device, N, mask):
    """N > 256 runs the two-group attention kernel: ragged N, random / padded masks, sampled rows
    (first, last, padded and interior rows)."""
    inp = tri_inputs(N, seed=N + 7, mask=mask, bias_z=True)
    out = _tri_call(inp, device)
    rows = torch.tensor([0, 1, N // 3, N // 2 + 5, N - N // 10 - 1, N - 2, N - 1])
    _check(out[rows].cpu(), _tri_ref(inp, rows=rows), torch.bfloat16, f"tri N={N} mask={mask}")


@pytest.mark.parametrize("N,mask,C", [(2100, "random", 128), (2049, "pad", 128), (4097, "pad", 64),
                                      (4100, "random", 64)])
def test_tri_large_ragged_blocks(device, N, mask, C):
    """Ragged N (the last block's query tiles lie partly or wholly past N) on sampled rows: 4-wave
    blocks of 256 queries at N = 2049 / 2100, and 8-wave blocks of 512 queries, which run from
    N = 4096 on, at N = 4097 / 4100 (C_in = 64 keeps the fp32 oracle's input small)."""
    inp = tri_inputs(N, C=C, seed=N + 3, mask=mask, bias_z=True)
    out = _tri_call(inp, device)
    rows = torch.tensor([0, N // 2, N - N // 10 - 1, N - 1])
    _check(out[rows].cpu(), _tri_ref(inp, rows=rows), torch.bfloat16, f"tri N={N} C={C} mask={mask}")


@pytest.mark.parametrize("masked", [False, True])
def test_tri_apo_d16(device, masked):
    """The Apo shape of the reference's tests/test_triangle_attn.py:137-192 (N=33, H=4, D=16, C_in=64)
    runs the tuned kernels (C = 64 pre-pass and gate, heads zero-padded to 32 in the attention
    kernel); precompute keeps separate WK_c / WV_c for D = 16."""
    inp = tri_inputs(33, C=64, H=4, D=16, seed=31, mask="random" if masked else "none", bias_z=True)
    d = to_dev(inp, device)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], 4, 16)
    assert pre["WK_c"] is not None and pre["WK_c"].data_ptr() != pre["WKV_c"].data_ptr()
    out = tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], scale=inp["scale"], eps=1e-5,
                                     W_proj_g=d["W_proj_g"], B_proj_g=None, W_proj_o=d["W_proj_o"], B_proj_o=None)
    assert out.shape == (33, 33, 64)
    _check(out, _tri_ref(inp), torch.bfloat16, f"tri Apo masked={masked}")


@pytest.mark.parametrize("N,mask", [(256, "pad"), (520, "random")])
def test_tri_apo_mfma_path_sampled_rows(device, N, mask):
    """The Apo shape (C_in = 64, H = 4, D = 16) at larger N on the tuned kernels: starting and ending
    node on sampled rows; and, on the any-shape pre-pass's outputs, the MFMA attention kernel after
    tops_tri_repack (D zero-padded to 32, heads of 16 written directly) equals the any-shape scalar
    attention within the bf16 bar."""
    from triangleops_amd.triangle_attn.kernel import (generic_attention, generic_prep_forward, padded_attention,
                                                      padded_ok)

    inp = tri_inputs(N, C=64, H=4, D=16, seed=N + 17, mask=mask, bias_z=True)
    assert padded_ok(N, 4, 16, torch.bfloat16)
    out = _tri_call(inp, device)
    rows = torch.tensor([0, N // 3, N // 2, N - 1])
    _check(out[rows].cpu(), _tri_ref(inp, rows=rows), torch.bfloat16, f"tri Apo N={N} start")
    Xd = inp["X"].to(device)
    out_e = _tri_call(inp, device, X=Xd.transpose(0, 1), mask=inp["mask"].to(device).T)
    exp_e = _tri_ref(inp, X=inp["X"].transpose(0, 1), mask=inp["mask"].T, rows=rows)
    _check(out_e[rows].cpu(), exp_e, torch.bfloat16, f"tri Apo N={N} end")
    d = to_dev(inp, device)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], 4, 16)
    xln, q, k, v, bias = generic_prep_forward(d["X"], pre["W_ln"], pre["B_ln"], pre["wqkv_hm"], pre["WZ_c"],
                                              pre["BZ"])
    a = padded_attention(q, k, v, bias, torch.empty(N, N, 64, device=device, dtype=torch.bfloat16),
                         scale=inp["scale"], mask=d["mask"])
    b = generic_attention(q, k, v, bias, torch.empty(N, N, 64, device=device, dtype=torch.bfloat16),
                          scale=inp["scale"], mask=d["mask"])
    _check(a[rows].cpu(), b[rows].float().cpu(), torch.bfloat16, f"tri Apo N={N} padded vs scalar attention")


@pytest.mark.parametrize("N,C,D,mask", [(100, 64, 16, "pad"), (200, 64, 16, "random"), (130, 128, 16, "random"),
                                        (96, 64, 32, "pad")])
def test_tri_tuned_other_shapes(device, N, C, D, mask):
    """The tuned pre-pass and attention at C_in in {64, 128} x D in {16, 32} beyond the default
    (128, 32), whole grids vs the oracle, starting and ending node: the Apo shape (64, 16) also on
    the tuned gate (C_in = H*D = C_out = 64); (128, 16) and (64, 32) on the any-shape gate."""
    inp = tri_inputs(N, C=C, H=4, D=D, seed=N + C + D, mask=mask, bias_z=True)
    _check(_tri_call(inp, device), _tri_ref(inp), torch.bfloat16, f"tri tuned N={N} C={C} D={D} start")
    Xd = inp["X"].to(device)
    out_e = _tri_call(inp, device, X=Xd.transpose(0, 1), mask=inp["mask"].to(device).T)
    exp_e = _tri_ref(inp, X=inp["X"].transpose(0, 1), mask=inp["mask"].T)
    _check(out_e, exp_e, torch.bfloat16, f"tri tuned N={N} C={C} D={D} end")


@pytest.mark.parametrize("C", [64, 128])
def test_gate_tuned_matches_generic(device, C):
    """The tuned gate (C = 64 and 128) against the any-shape gate on the same inputs: with and without
    the LayerNorm of its input, with the fused residual add into a transposed destination view.  The
    tuned kernel takes the gate's weights times -log2(e) in the 16-bit type (one more rounding than
    the any-shape kernel's fp32 scaling), so a sum with the residual (values up to ~5 here, one
    bf16 rounding of the total) may fall on the other side of a rounding step: that comparison
    allows half an ulp of the largest magnitude beyond the bar, as the Pairformer block check does."""
    from triangleops_amd.triangle_attn.kernel import _gate_out_generic, gate_out_forward

    g = torch.Generator().manual_seed(C)
    N1, N2 = 37, 70
    o = torch.randn(N1, N2, C, generator=g).to(torch.bfloat16).to(device)
    x = torch.randn(N1, N2, C, generator=g).to(torch.bfloat16).to(device)
    Wg = (torch.randn(C, C, generator=g) * C**-0.5).to(torch.bfloat16).to(device)
    Wo = (torch.randn(C, C, generator=g) * C**-0.5).to(torch.bfloat16).to(device)
    ln = ((1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(device),
          (0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(device), 1e-5)
    for lnv in (None, ln):
        a = gate_out_forward(o, x, Wg, None, Wo, None, ln=lnv)
        b = _gate_out_generic(o, x, Wg, None, Wo, None, ln=lnv)
        _check(a, b.float().cpu(), torch.bfloat16, f"gate C={C} ln={lnv is not None}")
    res = torch.randn(N2, N1, C, generator=g).to(torch.bfloat16).to(device)
    dst_a, dst_b = torch.zeros_like(res), torch.zeros_like(res)
    gate_out_forward(o, x, Wg, None, Wo, None, ln=ln, residual=res.transpose(0, 1), out=dst_a.transpose(0, 1))
    _gate_out_generic(o, x, Wg, None, Wo, None, ln=ln, residual=res.transpose(0, 1), out=dst_b.transpose(0, 1))
    diff, cos = compare(dst_a, dst_b.float().cpu())
    tol = TOL_MAX_ABS[torch.bfloat16] + 0.5 * _bf16_ulp(float(dst_b.float().abs().max()))
    assert torch.isfinite(dst_a.float()).all() and diff <= tol and cos >= TOL_COS, \
        f"gate C={C} residual: max|d|={diff:.3e} (bar {tol:.3e}) cos={cos:.6f}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gate_saturating_bias(device, dtype):
    """Gate biases far beyond where the sigmoid saturates (|bg| = 6e4, beyond fp16's range once
    scaled by log2(e)): the tuned gate clamps the scaled bias before splitting it into two 16-bit
    parts, so those features gate to exactly 0 or 1, as the any-shape gate's fp32 sigmoid does."""
    from triangleops_amd.triangle_attn.kernel import _gate_out_generic, gate_out_forward

    C = 128
    g = torch.Generator().manual_seed(5)
    o = torch.randn(9, 70, C, generator=g).to(dtype).to(device)
    x = torch.randn(9, 70, C, generator=g).to(dtype).to(device)
    Wg = (torch.randn(C, C, generator=g) * C**-0.5).to(dtype).to(device)
    Wo = (torch.randn(C, C, generator=g) * C**-0.5).to(dtype).to(device)
    bg = (0.1 * torch.randn(C, generator=g))
    bg[::4] = 6e4
    bg[1::4] = -6e4
    bg = bg.to(dtype).to(device)
    a = gate_out_forward(o, x, Wg, bg, Wo, None)
    b = _gate_out_generic(o, x, Wg, bg, Wo, None)
    _check(a, b.float().cpu(), dtype, f"gate saturating bias {dtype}")


@pytest.mark.parametrize("N,C,H,D", [(40, 96, 3, 24), (70, 64, 2, 64), (130, 32, 8, 8), (257, 64, 4, 16)])
@pytest.mark.parametrize("mask", ["pad", "random"])
def test_tri_any_shape(device, N, C, H, D, mask):
    """Shapes outside the tuned pre-pass run the any-shape pre-pass, then the MFMA attention kernel
    (D <= 32; D = 24 and 8 written directly, heads zero-padded to 32) or the scalar one (D = 64);
    (257, 64, 4, 16) is the Apo shape on the tuned kernels."""
    inp = tri_inputs(N, C=C, H=H, D=D, seed=N + C, mask=mask, bias_z=True)
    out = _tri_call(inp, device)
    _check(out, _tri_ref(inp), torch.bfloat16, f"tri any-shape N={N} C={C} H={H} D={D} mask={mask}")


def test_tri_any_shape_fp16_and_low_level(device):
    """fp16 any-shape op; the low-level triangle_attn_forward (separate WK_c / WV_c, D = 16) fills
    Bias_buf with the pair bias and matches forward() followed by the gate."""
    inp = tri_inputs(48, C=64, H=4, D=16, seed=3, mask="random", dtype=torch.float16, bias_z=True)
    _check(_tri_call(inp, device), _tri_ref(inp), torch.float16, "tri any-shape fp16")
    inp = to_dev(tri_inputs(48, C=64, H=4, D=16, seed=4, mask="random", bias_z=True), device)
    H, D, N = 4, 16, 48
    pre = tops.triangle_attn.precompute(inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"], inp["WV"], inp["W_proj_z"],
                                        inp["B_proj_z"], H, D)
    X_ln = torch.nn.functional.layer_norm(inp["X"], (64,), inp["W_ln"], inp["B_ln"], 1e-5)
    O = torch.empty(N, N, H * D, device=device, dtype=torch.bfloat16)
    Bias = torch.empty(H, N, N, device=device, dtype=torch.bfloat16)
    tops.triangle_attn.triangle_attn_forward(X_ln, pre["WQ_c"], pre["WKV_c"], pre["WZ_c"], pre["BZ"], O,
                                             scale=inp["scale"], mask=inp["mask"], Bias_buf=Bias, WK_c=pre["WK_c"],
                                             WV_c=pre["WV_c"])
    cpu = to_dev(inp, "cpu")
    bias_ref = (X_ln.cpu().float() @ cpu["W_proj_z"].float() + cpu["B_proj_z"].float()).permute(2, 0, 1)
    _check(Bias, bias_ref, torch.bfloat16, "tri low-level Bias_buf")
    out = tops.triangle_attn.fused_gate_forward(O.view(N, N, H, D), X_ln, inp["W_proj_g"], inp["W_proj_o"])
    _check(out, _tri_ref(cpu), torch.bfloat16, "tri any-shape low-level")


@pytest.mark.parametrize("C,H,D", [(128, 4, 32), (64, 4, 16)])
def test_tri_fp32_io(device, C, H, D):
    """fp32 I/O runs the any-shape kernels with every value in fp32 (max |d| <= 1e-4)."""
    inp = tri_inputs(40, C=C, H=H, D=D, seed=C + 1, mask="random", dtype=torch.float32, bias_z=True)
    out = _tri_call(inp, device)
    assert out.dtype == torch.float32
    _check(out, _tri_ref(inp), torch.float32, f"tri fp32 C={C}")


def test_tri_bias_buf_fast_shape(device):
    """Bias_buf holds the plain pair bias (not the kernels' log2(e)-scaled tiles) on the tuned path too."""
    N = 64
    inp = to_dev(tri_inputs(N, seed=9, mask="pad", bias_z=True), device)
    pre = tops.triangle_attn.precompute(inp["W_ln"], inp["B_ln"], inp["WQ"], inp["WK"], inp["WV"], inp["W_proj_z"],
                                        inp["B_proj_z"], 4, 32)
    X_ln = torch.nn.functional.layer_norm(inp["X"], (128,), inp["W_ln"], inp["B_ln"], 1e-5)
    O = torch.empty(N, N, 128, device=device, dtype=torch.bfloat16)
    Bias = torch.empty(4, N, N, device=device, dtype=torch.bfloat16)
    tops.triangle_attn.triangle_attn_forward(X_ln, pre["WQ_c"], pre["WKV_c"], pre["WZ_c"], pre["BZ"], O,
                                             scale=inp["scale"], mask=inp["mask"], Bias_buf=Bias)
    cpu = to_dev(inp, "cpu")
    bias_ref = (X_ln.cpu().float() @ cpu["W_proj_z"].float() + cpu["B_proj_z"].float()).permute(2, 0, 1)
    _check(Bias, bias_ref, torch.bfloat16, "tri Bias_buf")


# --------------------------------------------------------------------------- #
# attention_pair_bias
# --------------------------------------------------------------------------- #
def _apb_call(inp, device, mask="inp"):
    d = to_dev(inp, device)
    return tops.attention_pair_bias(d["X"], d["WQ"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                    d["B_proj_z"], d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], d["H"],
                                    d["D"], scale=d["scale"], eps=1e-5, mask=d["mask"] if mask == "inp" else mask)


def _apb_ref(inp, rows=None):
    return ref.attention_pair_bias(inp["X"], inp["WQ"], inp["WK"], inp["WV"], inp["Z"], inp["W_ln"], inp["B_ln"],
                                   inp["W_proj_z"], inp["B_proj_z"], inp["W_proj_g"], inp["B_proj_g"],
                                   inp["W_proj_o"], inp["B_proj_o"], inp["H"], inp["D"], scale=inp["scale"], eps=1e-5,
                                   mask=inp["mask"], rows=rows)


@pytest.mark.parametrize("M,C,Cz,H,D", [(40, 96, 64, 3, 24), (130, 64, 32, 2, 64), (70, 128, 128, 8, 16)])
@pytest.mark.parametrize("mask", ["none", "pad"])
def test_apb_any_shape(device, M, C, Cz, H, D, mask):
    """Shapes outside (C_s, C_z, H, D) = (128, 128, 4, 32) run the any-shape kernels (with biases)."""
    inp = apb_inputs(M, C=C, Cz=Cz, H=H, D=D, seed=M + C, mask=mask, biases=True)
    _check(_apb_call(inp, device), _apb_ref(inp), torch.bfloat16, f"apb any-shape M={M} C={C} Cz={Cz} H={H} D={D}")


@pytest.mark.parametrize("M", [40, 96])
def test_apb_fp32_io(device, M):
    """fp32 I/O: every value fp32 (max |d| <= 1e-4)."""
    inp = apb_inputs(M, seed=M, mask="pad", biases=True, dtype=torch.float32)
    out = _apb_call(inp, device)
    assert out.dtype == torch.float32
    _check(out, _apb_ref(inp), torch.float32, f"apb fp32 M={M}")


@pytest.mark.parametrize("M", [40, 128, 200, 512])
@pytest.mark.parametrize("mask", ["none", "pad", "random"])
@pytest.mark.parametrize("biases", [False, True])
def test_apb_matches_oracle(device, M, mask, biases):
    inp = apb_inputs(M, seed=M, mask=mask, biases=biases)
    _check(_apb_call(inp, device), _apb_ref(inp), torch.bfloat16, f"apb M={M} mask={mask} biases={biases}")


def test_apb_fp16(device):
    inp = apb_inputs(160, seed=6, mask="random", biases=True, dtype=torch.float16)
    _check(_apb_call(inp, device), _apb_ref(inp), torch.float16, "apb fp16")


def test_apb_precompute_forward_matches_oneshot(device):
    inp = to_dev(apb_inputs(256, seed=2, mask="none"), device)
    pre = tops.attn_pair_bias.precompute(inp["WQ"], inp["WK"], inp["WV"], inp["W_ln"], inp["B_ln"], inp["W_proj_z"],
                                         inp["B_proj_z"], inp["H"], inp["D"])
    a = tops.attn_pair_bias.forward(inp["X"], inp["Z"], pre, scale=1.0, W_proj_g=inp["W_proj_g"],
                                    B_proj_g=inp["B_proj_g"], W_proj_o=inp["W_proj_o"], B_proj_o=inp["B_proj_o"])
    b = tops.attention_pair_bias(inp["X"], inp["WQ"], inp["WK"], inp["WV"], inp["Z"], inp["W_ln"], inp["B_ln"],
                                 inp["W_proj_z"], inp["B_proj_z"], inp["W_proj_g"], inp["B_proj_g"], inp["W_proj_o"],
                                 inp["B_proj_o"], inp["H"], inp["D"], scale=1.0)
    assert torch.equal(a, b)


@pytest.mark.parametrize("M,mask", [(40, "pad"), (200, "random"), (1024, "pad"), (2048, "random")])
def test_apb_forward_matches_forward_qkv_bitwise(device, M, mask):
    """tops_apb_forward (its own Q / K / V pre-pass) and tops_apb_forward_qkv on the Q / K / V of that
    pre-pass (tops_apb_qkn_prep at the tuned shape) give the same bits, split-key merge included
    (M = 40 .. 2048: 1 to 16 key splits), and consecutive calls repeat them."""
    from triangleops_amd.attn_pair_bias.kernel import apb_forward, apb_forward_qkv, apb_qkn_prep

    inp = apb_inputs(M, seed=M + 3, mask=mask, biases=True)
    d = to_dev(inp, device)
    H, D = 4, 32
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], H, D)
    scale = D**-0.5
    og_fused = torch.empty(M, H * D, device=device, dtype=torch.bfloat16)
    apb_forward(d["X"], pre["W_QKV"], d["Z"], pre["W_combined"], pre["sum_W_combined"], pre["B_const"], og_fused,
                scale=scale, mask=d["mask"], wqkv_hm=pre["wqkv_hm"])
    q, k, v = apb_qkn_prep(d["X"], pre["wqkv_hm"], None, None, qscale=scale)
    og_comb = torch.empty_like(og_fused)
    apb_forward_qkv(q, k, v, d["Z"], pre["W_combined"], pre["sum_W_combined"], pre["B_const"], og_comb, scale=1.0,
                    mask=d["mask"])
    assert torch.equal(og_fused, og_comb), f"M={M}: tops_apb_forward differs from tops_apb_forward_qkv"
    for _ in range(2):
        again = torch.empty_like(og_fused)
        apb_forward(d["X"], pre["W_QKV"], d["Z"], pre["W_combined"], pre["sum_W_combined"], pre["B_const"], again,
                    scale=scale, mask=d["mask"], wqkv_hm=pre["wqkv_hm"])
        assert torch.equal(again, og_fused), f"M={M}: repeated call differs"


def _apb_unfused(d, pre, mask, residual=None):
    """apb_forward then the gate kernel: the composition tops_apb_forward_gated replaces"""
    from triangleops_amd.attn_pair_bias.kernel import apb_forward
    from triangleops_amd.triangle_attn.kernel import gate_out_forward

    M = d["X"].shape[0]
    og = torch.empty(M, 128, device=d["X"].device, dtype=d["X"].dtype)
    apb_forward(d["X"], pre["W_QKV"], d["Z"], pre["W_combined"], pre["sum_W_combined"], pre["B_const"], og,
                scale=d["scale"], mask=mask, wqkv_hm=pre["wqkv_hm"])
    res = None if residual is None else residual.view(M, 1, -1)
    return gate_out_forward(og.view(M, 1, 128), d["X"], d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"],
                            residual=res).view(M, -1)


@pytest.mark.parametrize("M,mask,biases", [(40, "pad", True), (200, "random", False), (1024, "pad", True),
                                           (2048, "random", True)])
@pytest.mark.parametrize("residual", [False, True])
def test_apb_gated_matches_unfused_bitwise(device, M, mask, biases, residual):
    """forward() at the tuned shape runs tops_apb_forward_gated (split merge + gate + W_o in one kernel):
    bitwise equal to apb_forward followed by the gate kernel, with and without the residual add."""
    from triangleops_amd.attn_pair_bias.kernel import apb_forward_gated, gated_ok

    inp = apb_inputs(M, seed=M + 11, mask=mask, biases=biases)
    d = to_dev(inp, device)
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], 4, 32)
    res = torch.randn(M, 128, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(device) if residual \
        else None
    assert gated_ok(d["X"], d["Z"], pre["W_combined"], d["W_proj_g"], d["W_proj_o"], res)
    a = tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=d["scale"], W_proj_g=d["W_proj_g"],
                                    B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"], B_proj_o=d["B_proj_o"],
                                    mask=d["mask"], residual=res)
    b = apb_forward_gated(d["X"], d["Z"], pre["W_combined"], pre["sum_W_combined"], pre["B_const"], pre["wqkv_hm"],
                          d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], scale=d["scale"],
                          mask=d["mask"], residual=res)
    ref_ = _apb_unfused(d, pre, d["mask"], residual=res)
    assert torch.equal(a, b) and torch.equal(a, ref_), f"M={M}: fused gate path differs from the unfused one"


def test_apb_merge_gate_entry_points(device):
    """The fused call's launches one by one through the C ABI (the pre-pass, tops_apb_forward_qkv with Og =
    NULL leaving the split partials, tops_apb_merge_gate) give forward()'s bits; the entry points refuse
    what they cannot do (NULL Og without split keys, merge on unsplit keys)."""
    from triangleops_amd import _native
    from triangleops_amd.attn_pair_bias.kernel import apb_qkn_prep

    M = 512
    inp = apb_inputs(M, seed=13, mask="random", biases=True)
    d = to_dev(inp, device)
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], 4, 32)
    want = tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=d["scale"], W_proj_g=d["W_proj_g"],
                                       B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"], B_proj_o=d["B_proj_o"],
                                       mask=d["mask"])
    q, k, v = apb_qkn_prep(d["X"], pre["wqkv_hm"], None, None, qscale=d["scale"])
    work = torch.empty(_native.apb_workspace_bytes(M, 4, 32), device=device, dtype=torch.uint8)
    Wc, sWc, Bc = (pre[n].float().contiguous() for n in ("W_combined", "sum_W_combined", "B_const"))
    m8 = d["mask"].view(torch.int8)
    st = _native.stream_of(q)
    _native.call("tops_apb_forward_qkv", q.data_ptr(), k.data_ptr(), v.data_ptr(), d["Z"].data_ptr(), d["Z"].stride(0),
                 d["Z"].stride(1), Wc.data_ptr(), sWc.data_ptr(), Bc.data_ptr(), m8.data_ptr(), None, work.data_ptr(),
                 M, 128, 128, 4, 32, 1.0, 1e-5, 2, st)
    out = torch.empty(M, 128, device=device, dtype=torch.bfloat16)
    _native.call("tops_apb_merge_gate", work.data_ptr(), d["X"].data_ptr(), d["W_proj_g"].data_ptr(),
                 d["B_proj_g"].data_ptr(), d["W_proj_o"].data_ptr(), d["B_proj_o"].data_ptr(), None, out.data_ptr(), M,
                 4, 32, 2, st)
    assert torch.equal(out, want)
    # the one-call entry point (all three launches inside the library)
    gwork = torch.empty(_native.apb_gated_workspace_bytes(M, 4, 32), device=device, dtype=torch.uint8)
    out1 = torch.empty_like(out)
    _native.call("tops_apb_forward_gated", d["X"].data_ptr(), pre["wqkv_hm"].data_ptr(), d["Z"].data_ptr(),
                 d["Z"].stride(0), d["Z"].stride(1), Wc.data_ptr(), sWc.data_ptr(), Bc.data_ptr(), m8.data_ptr(),
                 d["W_proj_g"].data_ptr(), d["B_proj_g"].data_ptr(), d["W_proj_o"].data_ptr(), d["B_proj_o"].data_ptr(),
                 None, out1.data_ptr(), gwork.data_ptr(), M, 128, 128, 4, 32, 128, d["scale"], 1e-5, 2, st)
    assert torch.equal(out1, want)
    with pytest.raises(RuntimeError, match="keys unsplit"):
        _native.call("tops_apb_merge_gate", work.data_ptr(), d["X"].data_ptr(), d["W_proj_g"].data_ptr(), None,
                     d["W_proj_o"].data_ptr(), None, None, out.data_ptr(), 20000, 4, 32, 2, st)
    with pytest.raises(RuntimeError, match="Og may be NULL only"):
        _native.call("tops_apb_forward_qkv", q.data_ptr(), k.data_ptr(), v.data_ptr(), d["Z"].data_ptr(), 0, 0,
                     Wc.data_ptr(), sWc.data_ptr(), Bc.data_ptr(), None, None, work.data_ptr(), 20000, 128, 128, 4, 32,
                     1.0, 1e-5, 2, st)


def test_apb_gated_unsplit_keys_bitwise(device):
    """M = 16400 (at least 512 query blocks: no key split, so the fused path writes Og to its workspace and
    runs the gate kernel) on a broadcast Z (every pair shares one 128-channel row: strides (0, 0, 1)),
    bitwise against the unfused composition, with the residual."""
    M = 16400
    inp = apb_inputs(8, seed=5, mask="none", biases=True)
    g = torch.Generator().manual_seed(6)
    d = to_dev(inp, device)
    d["X"] = torch.randn(M, 128, generator=g).to(torch.bfloat16).to(device)
    d["Z"] = torch.randn(1, 1, 128, generator=g).to(torch.bfloat16).to(device).expand(M, M, 128)
    kmask = (torch.arange(M) < M - 37).to(device)
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], 4, 32)
    from triangleops_amd import _native

    assert _native.apb_gated_workspace_bytes(M, 4, 32) > _native.apb_workspace_bytes(M, 4, 32)  # unsplit: Og region
    res = torch.randn(M, 128, generator=g).to(torch.bfloat16).to(device)
    a = tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=d["scale"], W_proj_g=d["W_proj_g"],
                                    B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"], B_proj_o=d["B_proj_o"],
                                    mask=kmask, residual=res)
    ref_ = _apb_unfused(d, pre, kmask, residual=res)
    assert torch.isfinite(a.float()).all() and torch.equal(a, ref_), "unsplit fused path differs from the unfused one"


def _apb_perturbed(inp, kmask, seed):
    """inputs with X rows and Z key columns replaced at the masked keys"""
    g = torch.Generator().manual_seed(seed)
    X, Z = inp["X"].clone(), inp["Z"].clone()
    bad = ~kmask
    X[bad] = torch.randn(int(bad.sum()), X.shape[1], generator=g).to(X.dtype) * 3
    Z[:, bad] = torch.randn(Z.shape[0], int(bad.sum()), Z.shape[2], generator=g).to(Z.dtype) * 3
    return dict(inp, X=X, Z=Z, mask=kmask)


@pytest.mark.parametrize("M,shape,dtype", [(128, "tuned", torch.bfloat16), (200, "tuned", torch.bfloat16),
                                           (1024, "tuned", torch.bfloat16), (300, "tuned", torch.float16),
                                           (70, (96, 64, 3, 24), torch.bfloat16), (64, "tuned", torch.float32)])
@pytest.mark.parametrize("mask", ["pad", "random", "first"])
def test_apb_masked_keys_bitwise_invariant(device, M, shape, dtype, mask):
    """Masked keys contribute exactly nothing (-inf before the softmax, benchmarks/references.py:273-274):
    replacing the X rows and Z columns of every masked key leaves every unmasked query row of the output
    bitwise unchanged (tuned kernels incl. the split-key combine at M = 1024, the any-shape kernels and
    fp32 I/O); "first" masks key 0, the key every online softmax starts from."""
    C, Cz, H, D = (128, 128, 4, 32) if shape == "tuned" else shape
    inp = apb_inputs(M, C=C, Cz=Cz, H=H, D=D, seed=M + 11, mask="none", biases=True, dtype=dtype)
    g = torch.Generator().manual_seed(M)
    if mask == "pad":
        km = torch.arange(M) < M - M // 20
    elif mask == "random":
        km = torch.rand(M, generator=g) < 0.7
    else:
        km = torch.ones(M, dtype=torch.bool)
        km[0] = False
        km[M // 2] = False
    a_inp, b_inp = dict(inp, mask=km), _apb_perturbed(inp, km, M + 1)
    a, b = _apb_call(a_inp, device), _apb_call(b_inp, device)
    assert not torch.equal(a[~km.to(device)], b[~km.to(device)])
    assert torch.equal(a[km.to(device)], b[km.to(device)]), f"apb M={M} {shape} {dtype} mask={mask}"
    _check(a, _apb_ref(a_inp), dtype, f"apb M={M} {shape} {dtype} mask={mask}")


@pytest.mark.parametrize("M,shape,dtype", [(96, "tuned", torch.bfloat16), (70, (96, 64, 3, 24), torch.bfloat16),
                                           (48, "tuned", torch.float32)])
def test_apb_qknorm_first_key_masked(device, M, shape, dtype):
    """The qk-norm variant with key 0 masked (and a random key mask) matches the oracle on the tuned,
    any-shape and fp32 paths."""
    C, Cz, H, D = (128, 128, 4, 32) if shape == "tuned" else shape
    inp = apb_qkn_inputs(M, C=C, Cz=Cz, H=H, D=D, seed=M + 5, mask="random", dtype=dtype)
    inp["key_mask"][0] = False
    _check(_qkn_call(inp, device), _qkn_ref(inp), dtype, f"apb qk-norm key0 masked M={M} {shape} {dtype}")


@pytest.mark.parametrize("M", [1024, 2048])
def test_apb_config_sizes(device, M):
    """BASELINE config 2 sizes (key padding mask): the whole output against the fp32 oracle."""
    inp = apb_inputs(M, seed=0, mask="pad")
    _check(_apb_call(inp, device).cpu(), _apb_ref(inp), torch.bfloat16, f"apb M={M}")


@pytest.mark.parametrize("M", [200, 1024])
@pytest.mark.parametrize("residual", [False, True])
def test_apb_column_sliced_inputs(device, M, residual):
    """X, the residual and W_g as column slices of wider tensors (row stride 256, not dense): the
    kernels that index them without strides must get dense copies.  Through forward() (the gated
    path at the tuned shape), against the fp32 oracle (+ residual)."""
    inp = apb_inputs(M, seed=M + 3, mask="pad", biases=True)
    d = to_dev(inp, device)
    g = torch.Generator().manual_seed(M)
    wide_x = torch.randn(M, 256, generator=g).to(torch.bfloat16).to(device)
    wide_x[:, :128] = d["X"]
    wide_g = torch.randn(128, 256, generator=g).to(torch.bfloat16).to(device)
    wide_g[:, :128] = d["W_proj_g"]
    X, W_g = wide_x[:, :128], wide_g[:, :128]
    assert not X.is_contiguous() and not W_g.is_contiguous()
    res_cpu = torch.randn(M, 128, generator=g).to(torch.bfloat16)
    res = None
    if residual:
        wide_r = torch.randn(M, 256, generator=g).to(torch.bfloat16).to(device)
        wide_r[:, 128:] = res_cpu.to(device)
        res = wide_r[:, 128:]
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], 4, 32)
    out = tops.attn_pair_bias.forward(X, d["Z"], pre, scale=d["scale"], W_proj_g=W_g, B_proj_g=d["B_proj_g"],
                                      W_proj_o=d["W_proj_o"], B_proj_o=d["B_proj_o"], mask=d["mask"], residual=res)
    expect = _apb_ref(inp)
    if not residual:
        _check(out.cpu(), expect, torch.bfloat16, f"apb sliced M={M}")
        return
    # residual + result rounded once in bf16: the bar plus half a bf16 step of the sum
    expect = expect + res_cpu.float()
    e = expect.double()
    ulp = torch.exp2(torch.floor(torch.log2(e.abs().clamp_min(1e-30))) - 7)  # bf16 step at |expect|
    diff = ((out.cpu().double() - e).abs() - 0.5 * ulp).max().item()
    cos = torch.nn.functional.cosine_similarity(out.cpu().double().flatten(), expect.double().flatten(), dim=0).item()
    assert diff <= TOL_MAX_ABS[torch.bfloat16] and cos >= TOL_COS, f"apb sliced M={M} residual: {diff:.3e} {cos:.6f}"


# --------------------------------------------------------------------------- #
# attention_pair_bias, qk-norm variant (benchmarks/references.py:230-277)
# --------------------------------------------------------------------------- #
_QKN_KW = ("qkn_w_q", "qkn_b_q", "qkn_w_k", "qkn_b_k", "key_mask")


def _qkn_args(d):
    return (d["X"], d["WQ"], d["b_q"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"],
            d["W_proj_g"], d["W_proj_o"], d["H"], d["D"])


def _qkn_call(inp, device):
    d = to_dev(inp, device)
    return tops.attn_pair_bias.attention_pair_bias_qknorm(*_qkn_args(d), scale=d["scale"], eps=1e-5,
                                                          **{k: d[k] for k in _QKN_KW})


def _qkn_ref(inp, rows=None):
    return ref.attention_pair_bias_qknorm(*_qkn_args(inp), scale=inp["scale"], eps=1e-5, rows=rows,
                                          **{k: inp[k] for k in _QKN_KW})


@pytest.mark.parametrize("M", [40, 128, 200, 512])
@pytest.mark.parametrize("mask", ["none", "pad", "random"])
@pytest.mark.parametrize("qkn", [False, True])
def test_apb_qknorm_matches_oracle(device, M, mask, qkn):
    inp = apb_qkn_inputs(M, seed=M + 7, mask=mask, qkn=qkn)
    _check(_qkn_call(inp, device), _qkn_ref(inp), torch.bfloat16, f"apb qk-norm M={M} mask={mask} qkn={qkn}")


@pytest.mark.parametrize("M,C,Cz,H,D", [(40, 96, 64, 3, 24), (130, 64, 32, 2, 64), (70, 128, 128, 8, 16)])
def test_apb_qknorm_any_shape(device, M, C, Cz, H, D):
    inp = apb_qkn_inputs(M, C=C, Cz=Cz, H=H, D=D, seed=M + C, mask="pad")
    _check(_qkn_call(inp, device), _qkn_ref(inp), torch.bfloat16, f"apb qk-norm any-shape M={M} C={C} H={H} D={D}")


@pytest.mark.parametrize("M", [40, 96])
def test_apb_qknorm_fp32_io(device, M):
    inp = apb_qkn_inputs(M, seed=M, mask="pad", dtype=torch.float32)
    out = _qkn_call(inp, device)
    assert out.dtype == torch.float32
    _check(out, _qkn_ref(inp), torch.float32, f"apb qk-norm fp32 M={M}")


def test_apb_qknorm_fp16(device):
    inp = apb_qkn_inputs(160, seed=6, mask="random", dtype=torch.float16)
    _check(_qkn_call(inp, device), _qkn_ref(inp), torch.float16, "apb qk-norm fp16")


def test_apb_qknorm_precompute_forward_matches_oneshot(device):
    d = to_dev(apb_qkn_inputs(256, seed=2, mask="pad"), device)
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], d["H"], d["D"])
    a = tops.attn_pair_bias.forward_qknorm(d["X"], d["Z"], pre, b_q=d["b_q"], scale=d["scale"],
                                           W_proj_g=d["W_proj_g"], W_proj_o=d["W_proj_o"],
                                           **{k: d[k] for k in _QKN_KW})
    b = _qkn_call(d, device)
    assert torch.equal(a, b)


@pytest.mark.parametrize("M", [1024, 2048])
def test_apb_qknorm_config_sizes_sampled_rows(device, M):
    inp = apb_qkn_inputs(M, seed=0, mask="pad")
    out = _qkn_call(inp, device)
    rows = torch.tensor([0, 1, M // 2, M - M // 20 - 1, M - 1])
    _check(out[rows].cpu(), _qkn_ref(inp, rows=rows), torch.bfloat16, f"apb qk-norm M={M}")


# --------------------------------------------------------------------------- #
# Pairformer block composition (residual adds fused into the output kernels)
# --------------------------------------------------------------------------- #
_TRI_KEYS = ("W_ln", "B_ln", "WQ", "WK", "WV", "W_proj_z", "B_proj_z", "W_proj_g", "W_proj_o")


def _block_inputs(N, *, C=128, H=4, D=32, seed=0, dtype=torch.bfloat16, mask="pad"):
    x, m, tmu_o = tmu_inputs(N, C=C, seed=seed, dtype=dtype, mask=mask)
    _, _, tmu_i = tmu_inputs(N, C=C, seed=seed + 1, dtype=dtype, mask="none")
    ts = tri_inputs(N, C=C, H=H, D=D, seed=seed + 2, dtype=dtype, mask="none", bias_z=True)
    te = tri_inputs(N, C=C, H=H, D=D, seed=seed + 3, dtype=dtype, mask="none", bias_z=True)
    return (x[0], None if m is None else m[0], tmu_o, tmu_i, {k: ts[k] for k in _TRI_KEYS},
            {k: te[k] for k in _TRI_KEYS}, H, D)


def _bf16_ulp(v):
    return 2.0 ** (math.floor(math.log2(max(v, 1e-30))) - 7)


def _unfused_pair_stack(z, pm, pre, dev):
    """The same four updates from the ops without residual fusion and torch adds in the I/O type."""
    N = z.shape[0]
    m3 = None if pm is None else pm.reshape(1, N, N)
    sc = pre["D"] ** -0.5
    z = z + tops.triangle_mul.forward(z[None], pre["tmu_out"], direction="outgoing", mask=m3)[0]
    z = z + tops.triangle_mul.forward(z[None], pre["tmu_in"], direction="incoming", mask=m3)[0]
    wg, wo = pre["tri_start_proj"]
    z = z + tops.triangle_attn.forward(z, pre["tri_start"], mask=pm, scale=sc, W_proj_g=wg, B_proj_g=None,
                                       W_proj_o=wo, B_proj_o=None)
    wg, wo = pre["tri_end_proj"]
    e = tops.triangle_attn.forward(z.transpose(0, 1), pre["tri_end"], mask=None if pm is None else pm.T, scale=sc,
                                   W_proj_g=wg, B_proj_g=None, W_proj_o=wo, B_proj_o=None)
    return z + e.transpose(0, 1)


def _check_block(out, expect, dtype, what):
    """Budget of four residual updates: the per-op bar four times, plus one rounding of the residual
    stream per update (half an ulp of its largest magnitude) in a 16-bit I/O type."""
    diff, cos = compare(out, expect)
    big = float(expect.abs().max())
    ulp = {torch.bfloat16: _bf16_ulp(big), torch.float16: _bf16_ulp(big) / 8, torch.float32: 0.0}[dtype]
    tol = 4 * TOL_MAX_ABS[dtype] + 4 * 0.5 * ulp
    assert torch.isfinite(out.float()).all(), f"{what}: non-finite output"
    assert diff <= tol and cos >= TOL_COS, f"{what}: max|d|={diff:.3e} (budget {tol:.3e}) cos={cos:.6f}"


@pytest.mark.parametrize("N", [64, 130])
@pytest.mark.parametrize("mask", ["none", "pad"])
def test_pair_stack_fused_equals_unfused(device, N, mask):
    z, pm, tmu_o, tmu_i, ts, te, H, D = _block_inputs(N, seed=N, mask=mask)
    d = lambda t: None if t is None else t.to(device)  # noqa: E731
    dd = lambda w: {k: d(v) for k, v in w.items()}  # noqa: E731
    pre = tops.pairformer.precompute(dd(tmu_o), dd(tmu_i), dd(ts), dd(te), H=H, D=D)
    fused = tops.pairformer.pair_stack(d(z), pre, pair_mask=d(pm))
    assert fused.is_contiguous() and fused.shape == z.shape
    assert torch.equal(fused, _unfused_pair_stack(d(z), d(pm), pre, device)), f"pair stack N={N} mask={mask}"


@pytest.mark.parametrize("N,C,H,D,dtype", [(64, 128, 4, 32, torch.bfloat16), (130, 128, 4, 32, torch.bfloat16),
                                           (48, 64, 4, 16, torch.bfloat16), (40, 128, 4, 32, torch.float32)])
def test_pair_stack_matches_oracle(device, N, C, H, D, dtype):
    z, pm, tmu_o, tmu_i, ts, te, H, D = _block_inputs(N, C=C, H=H, D=D, seed=N + C, dtype=dtype)
    d = lambda t: None if t is None else t.to(device)  # noqa: E731
    dd = lambda w: {k: d(v) for k, v in w.items()}  # noqa: E731
    pre = tops.pairformer.precompute(dd(tmu_o), dd(tmu_i), dd(ts), dd(te), H=H, D=D)
    out = tops.pairformer.pair_stack(d(z), pre, pair_mask=d(pm))
    expect = ref.pair_stack(z, tmu_o, tmu_i, ts, te, H, D, pair_mask=pm)
    _check_block(out, expect, dtype, f"pair stack N={N} C={C} H={H} D={D} {dtype}")


@pytest.mark.parametrize("M", [96, 256])
def test_single_update_fused_and_oracle(device, M):
    inp = apb_inputs(M, seed=M, mask="pad", biases=True)
    apb = {k: inp[k] for k in ("WQ", "WK", "WV", "W_ln", "B_ln", "W_proj_z", "B_proj_z", "W_proj_g", "B_proj_g",
                               "W_proj_o", "B_proj_o")}
    d = to_dev(inp, device)
    _, _, tmu_o = tmu_inputs(4)  # the pair-stack weights are not used by the single update
    tri = {k: v for k, v in tri_inputs(4).items() if k in _TRI_KEYS}
    pre = tops.pairformer.precompute(to_dev(tmu_o, device), to_dev(tmu_o, device), to_dev(tri, device),
                                     to_dev(tri, device), to_dev(apb, device), H=4, D=32)
    s = tops.pairformer.single_update(d["X"], d["Z"], pre, key_mask=d["mask"])
    plain = d["X"] + tops.attention_pair_bias(d["X"], d["WQ"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"],
                                              d["W_proj_z"], d["B_proj_z"], d["W_proj_g"], d["B_proj_g"],
                                              d["W_proj_o"], d["B_proj_o"], 4, 32, scale=32**-0.5, mask=d["mask"])
    assert torch.equal(s, plain), f"single update M={M}: fused != unfused"
    expect = ref.single_update(inp["X"], inp["Z"], apb, 4, 32, key_mask=inp["mask"])
    diff, cos = compare(s, expect)
    tol = TOL_MAX_ABS[torch.bfloat16] + 0.5 * _bf16_ulp(float(expect.abs().max()))
    assert diff <= tol and cos >= TOL_COS, f"single update M={M}: max|d|={diff:.3e} (budget {tol:.3e}) cos={cos}"


def test_pairformer_block(device):
    z, pm, tmu_o, tmu_i, ts, te, H, D = _block_inputs(96, seed=5)
    inp = apb_inputs(96, seed=6, mask="none", biases=True)
    apb = {k: inp[k] for k in ("WQ", "WK", "WV", "W_ln", "B_ln", "W_proj_z", "B_proj_z", "W_proj_g", "B_proj_g",
                               "W_proj_o", "B_proj_o")}
    d = lambda t: None if t is None else t.to(device)  # noqa: E731
    dd = lambda w: {k: d(v) for k, v in w.items()}  # noqa: E731
    pre = tops.pairformer.precompute(dd(tmu_o), dd(tmu_i), dd(ts), dd(te), dd(apb), H=H, D=D)
    zo, so = tops.pairformer.pairformer_block(d(z), d(inp["X"]), pre, pair_mask=d(pm))
    assert torch.equal(zo, tops.pairformer.pair_stack(d(z), pre, pair_mask=d(pm)))
    assert torch.equal(so, tops.pairformer.single_update(d(inp["X"]), zo, pre))


# --------------------------------------------------------------------------- #
# HIP graph replay of whole calls (launch-bound small sizes)
# --------------------------------------------------------------------------- #
def _graph_check(device, call, fresh, n_replays=3):
    """Capture call(*inputs), then per replay: copy fresh values into the captured inputs, replay,
    run the same call eagerly (work between the replays) and compare bitwise."""
    inputs = fresh(0)
    g = tops.graph.capture(call, *inputs)
    for r in range(1, n_replays + 1):
        new = fresh(r)
        for dst, src in zip(g.inputs, new):
            dst.copy_(src)
        out = g.replay().clone()
        torch.cuda.synchronize()
        eager = call(*new)
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager call"


@pytest.mark.parametrize("L", [96, 512])  # 512: the persistent einsum kernel
def test_graph_replay_tmu(device, L):
    x, m, w = tmu_inputs(L, mask="pad")
    w = to_dev(w, device)
    pre = tops.triangle_mul.precompute(*(w[k] for k in ("norm_in_weight", "norm_in_bias", "p_in_weight",
                                                        "g_in_weight", "norm_out_weight", "norm_out_bias",
                                                        "p_out_weight", "g_out_weight")))
    m = m.to(device)

    def call(xx):
        return tops.triangle_mul.forward(xx, pre, direction="incoming", mask=m)

    _graph_check(device, call, lambda r: [tmu_inputs(L, seed=100 + r)[0].to(device)])


def test_graph_replay_tri_and_apb(device):
    d = to_dev(tri_inputs(80, mask="pad"), device)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], d["H"], d["D"])

    def tri(X):
        return tops.triangle_attn.forward(X, pre, mask=d["mask"], scale=d["scale"], W_proj_g=d["W_proj_g"],
                                          B_proj_g=None, W_proj_o=d["W_proj_o"], B_proj_o=None)

    _graph_check(device, tri, lambda r: [tri_inputs(80, seed=200 + r)["X"].to(device)])
    a = to_dev(apb_inputs(96, mask="pad", biases=True), device)
    pa = tops.attn_pair_bias.precompute(a["WQ"], a["WK"], a["WV"], a["W_ln"], a["B_ln"], a["W_proj_z"],
                                        a["B_proj_z"], a["H"], a["D"])

    def apb(X, Z):
        return tops.attn_pair_bias.forward(X, Z, pa, scale=a["scale"], W_proj_g=a["W_proj_g"],
                                           B_proj_g=a["B_proj_g"], W_proj_o=a["W_proj_o"], B_proj_o=a["B_proj_o"],
                                           mask=a["mask"])

    def fresh(r):
        f = apb_inputs(96, seed=300 + r)
        return [f["X"].to(device), f["Z"].to(device)]

    _graph_check(device, apb, fresh)


def test_graph_replay_pair_stack(device):
    z, pm, tmu_o, tmu_i, ts, te, H, D = _block_inputs(64, seed=9)
    dd = lambda w: {k: v.to(device) for k, v in w.items()}  # noqa: E731
    pre = tops.pairformer.precompute(dd(tmu_o), dd(tmu_i), dd(ts), dd(te), H=H, D=D)
    pm = pm.to(device)

    def call(zz):
        return tops.pairformer.pair_stack(zz, pre, pair_mask=pm)

    _graph_check(device, call, lambda r: [_block_inputs(64, seed=40 + r)[0].to(device)])


# --------------------------------------------------------------------------- #
# golden fixtures (brute-force float64 expected outputs, tests/golden)
# --------------------------------------------------------------------------- #
def _golden(name):
    import os

    import numpy as np

    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name), allow_pickle=False)
    inp = {k[3:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("in_")}
    meta = {k[5:]: z[k] for k in z.files if k.startswith("meta_")}
    return inp, torch.from_numpy(z["expected"]), meta


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_golden_tmu_gpu(device, direction):
    inp, expected, meta = _golden(f"tmu_{direction}.npz")
    d = {k: v.to(torch.bfloat16).to(device) for k, v in inp.items() if k not in ("mask",)}
    x = d.pop("x")
    out = tops.triangle_multiplicative_update(x, direction=direction, mask=inp["mask"].to(device).bool(),
                                              eps=float(meta["eps"]), **d)
    _check(out, expected, torch.bfloat16, f"golden tmu {direction}")


def test_golden_tri_gpu(device):
    inp, expected, meta = _golden("tri_attn.npz")
    d = {k: v.to(torch.bfloat16).to(device) for k, v in inp.items()}
    out = tops.triangle_attention(d["X"], d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                  d["B_proj_z"], d["W_proj_g"], None, d["W_proj_o"], None, 4, 32,
                                  scale=float(meta["scale"]), eps=float(meta["eps"]),
                                  mask=inp["mask"].to(device).bool())
    _check(out, expected, torch.bfloat16, "golden tri")


def test_golden_apb_gpu(device):
    inp, expected, meta = _golden("apb.npz")
    d = {k: v.to(torch.bfloat16).to(device) for k, v in inp.items()}
    out = tops.attention_pair_bias(d["X"], d["WQ"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                   d["B_proj_z"], d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], 4, 32,
                                   scale=float(meta["scale"]), eps=float(meta["eps"]),
                                   mask=inp["mask"].to(device).bool())
    _check(out, expected, torch.bfloat16, "golden apb")
