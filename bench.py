"""Benchmark of the triangleops_amd hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep FILE] [--no-cpu-baseline]

Default workload (the configuration its metric is quoted on):
triangle_multiplicative_update in bf16 at L = 1024, C = 128, B = 1, pad mask zeroing the last
10% of rows/cols, random-init LayerNorm / projection weights.  One step = one outgoing call
plus one incoming call (the two directions a Pairformer block runs).  Inputs are resident in
HBM before timing; the precompute (weight folding) is outside the timed region.  Before the W
warmup steps the headline runs untimed steps for SETTLE_S seconds (`settle_steps` in the line), so
the K timed steps run at the clocks of a loaded chip, not during their ramp from idle.

Prints ONE JSON line with the contract fields plus:
  roofline      dominant kernel of the step (largest average launch time), its algorithmic
                work per launch over its average HIP-event-timed duration, vs the MI355X peak
                (bf16 dense MFMA 2.5 PFLOP/s, HBM 8 TB/s);
  kernels       the same figures for each kernel of the step;
  torch_path_ms the reference's pure-torch bf16 formulation on the same GPU;
  cpu_baseline  the fp32 CPU oracle on this host (one full outgoing call at the same size);
  ops           the metric's other two ops at size 1024 (BASELINE.json configs 2 and 4):
                triangle_attention (starting and ending node) and attention_pair_bias, each with
                ms per call, per-kernel figures, the dominant kernel's roofline (the attention
                kernel's MFMA fraction; apb's HBM fraction), the torch path on the same GPU and
                its own CPU baseline (the fp32 oracle; triangle attention timed on sampled rows
                and scaled, rows being independent);
  config0       BASELINE.json configs[0], the reference's CPU-runnable case (tmu outgoing,
                L = 128, all-ones mask): ms per call with bf16 and fp32 I/O and the fp32 oracle's
                calls/s on the host;
  size_sweep    the metric's other config sizes (tmu L = 512, 2048; triangle attention N = 256,
                512, 2048; apb M = 128, 512, 2048): ms per call, the dominant kernel's roofline
                fraction, every kernel's ms and fraction, the torch path on the same GPU, and the
                HIP-graph replay time at sizes <= 512.
`--sweep FILE` additionally times all three ops, the apb qk-norm variant and a Pairformer pair stack at sizes 128..2048 (ours, the torch path and
per-kernel roofline fractions) and writes one JSON line per (op, size) to FILE.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import triangleops_amd as tops  # noqa: E402
from triangleops_amd import _native  # noqa: E402
from triangleops_amd.attn_pair_bias.kernel import apb_forward_qkv, apb_qkn_prep  # noqa: E402
from triangleops_amd.triangle_attn.kernel import attention_core, gate_out_forward, prep_forward  # noqa: E402
from triangleops_amd.triangle_mul.kernel import input_phase, output_phase, triangle_einsum  # noqa: E402

METRIC = "per-call ms + MFMA util % for each op at N/L/M=128–2048 (bf16, 1 GPU)"
PEAK_MFMA_BF16 = 2500.0  # TFLOP/s, MI355X dense bf16
PEAK_HBM = 8000.0  # GB/s
C = 128
H, D = 4, 32

TMU_KEYS = ("norm_in_weight", "norm_in_bias", "p_in_weight", "g_in_weight", "norm_out_weight", "norm_out_bias",
            "p_out_weight", "g_out_weight")


# --------------------------------------------------------------------------- #
# inputs (CPU generator, seed 0, fixed draw order; rounded to bf16 once)
# --------------------------------------------------------------------------- #
def _gen(seed=0):
    return torch.Generator().manual_seed(seed)


def pad_mask2(n, frac=10):
    v = n - n // frac
    i = torch.arange(n)
    return (i[:, None] < v) & (i[None, :] < v)


def tmu_inputs(L, seed=0):
    g = _gen(seed)
    x = torch.randn(1, L, L, C, generator=g).to(torch.bfloat16)
    s = C**-0.5
    w = {
        "p_in_weight": torch.randn(2 * C, C, generator=g) * s,
        "g_in_weight": torch.randn(2 * C, C, generator=g) * s,
        "p_out_weight": torch.randn(C, C, generator=g) * s,
        "g_out_weight": torch.randn(C, C, generator=g) * s,
        "norm_in_weight": 1 + 0.1 * torch.randn(C, generator=g),
        "norm_in_bias": 0.1 * torch.randn(C, generator=g),
        "norm_out_weight": 1 + 0.1 * torch.randn(C, generator=g),
        "norm_out_bias": 0.1 * torch.randn(C, generator=g),
    }
    w = {k: v.to(torch.bfloat16) for k, v in w.items()}
    return x, pad_mask2(L).unsqueeze(0), w


def tri_inputs(N, seed=0):
    g = _gen(seed)
    s = C**-0.5
    d = dict(
        X=torch.randn(N, N, C, generator=g),
        W_ln=1 + 0.1 * torch.randn(C, generator=g),
        B_ln=0.1 * torch.randn(C, generator=g),
        WQ=torch.randn(C, H * D, generator=g) * s,
        WK=torch.randn(C, H * D, generator=g) * s,
        WV=torch.randn(C, H * D, generator=g) * s,
        W_proj_z=torch.randn(C, H, generator=g) * s,
        B_proj_z=torch.zeros(H),
        W_proj_g=torch.randn(H * D, C, generator=g) * s,
        W_proj_o=torch.randn(C, H * D, generator=g) * (H * D) ** -0.5,
    )
    d = {k: v.to(torch.bfloat16) for k, v in d.items()}
    d["mask"] = pad_mask2(N)
    return d


def apb_inputs(M, seed=0):
    g = _gen(seed)
    s = C**-0.5
    d = dict(
        X=torch.randn(M, C, generator=g),
        Z=torch.randn(M, M, C, generator=g),
        WQ=torch.randn(C, H * D, generator=g) * s,
        WK=torch.randn(C, H * D, generator=g) * s,
        WV=torch.randn(C, H * D, generator=g) * s,
        W_ln=1 + 0.1 * torch.randn(C, generator=g),
        B_ln=0.1 * torch.randn(C, generator=g),
        W_proj_z=torch.randn(C, H, generator=g) * s,
        B_proj_z=torch.zeros(H),
        W_proj_g=torch.randn(H * D, C, generator=g) * s,
        B_proj_g=torch.zeros(H * D),
        W_proj_o=torch.randn(C, H * D, generator=g) * (H * D) ** -0.5,
        B_proj_o=torch.zeros(C),
    )
    d = {k: v.to(torch.bfloat16) for k, v in d.items()}
    d["mask"] = torch.arange(M) < M - M // 20
    return d


def apb_qkn_params(seed=0):
    """Q bias and qk-norm affine parameters of the qk-norm variant (benchmarks/references.py:230-250)."""
    g = _gen(seed + 7)
    p = dict(b_q=0.5 * torch.randn(H * D, generator=g), qkn_w_q=1 + 0.2 * torch.randn(H * D, generator=g),
             qkn_b_q=0.2 * torch.randn(H * D, generator=g), qkn_w_k=1 + 0.2 * torch.randn(H * D, generator=g),
             qkn_b_k=0.2 * torch.randn(H * D, generator=g))
    return {k: v.to(torch.bfloat16) for k, v in p.items()}


def to_dev(d, dev):
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in d.items()}


# --------------------------------------------------------------------------- #
# the reference's pure-torch bf16 path (benchmarks/references.py:143-221), restated.
# Batched products use contiguous operands and matmul (no einsum over transposed views).
# The tri_attn mask add is cast to the scores dtype (the reference's fp32 add fails in bf16).
# --------------------------------------------------------------------------- #
def torch_tmu(x, direction, mask, eps=1e-5, **w):
    xln = F.layer_norm(x, (C,), w["norm_in_weight"], w["norm_in_bias"], eps=eps)
    g = F.linear(xln, w["p_in_weight"]) * F.linear(xln, w["g_in_weight"]).sigmoid()
    g = g * mask.unsqueeze(-1)
    a, b = torch.chunk(g, 2, dim=-1)
    if direction == "outgoing":
        A = a.permute(0, 3, 1, 2).contiguous()  # b d i k
        Bm = b.permute(0, 3, 2, 1).contiguous()  # b d k j
    else:
        A = a.permute(0, 3, 2, 1).contiguous()  # b d i k  (a[b,k,i,d])
        Bm = b.permute(0, 3, 1, 2).contiguous()  # b d k j  (b[b,k,j,d])
    y = torch.matmul(A, Bm).permute(0, 2, 3, 1)
    yln = F.layer_norm(y, (C,), w["norm_out_weight"], w["norm_out_bias"], eps=eps)
    return F.linear(yln, w["p_out_weight"]) * F.linear(xln, w["g_out_weight"]).sigmoid()


def torch_tri(d, eps=1e-5):
    X = d["X"]
    N = X.shape[0]
    xln = F.layer_norm(X, (C,), d["W_ln"], d["B_ln"], eps=eps)
    q = (xln @ d["WQ"]).view(N, N, H, D).permute(0, 2, 1, 3)
    k = (xln @ d["WK"]).view(N, N, H, D).permute(0, 2, 3, 1).contiguous()
    v = (xln @ d["WV"]).view(N, N, H, D).permute(0, 2, 1, 3).contiguous()
    bp = (xln @ d["W_proj_z"] + d["B_proj_z"]).permute(2, 0, 1).unsqueeze(0)
    scores = torch.matmul((q * D**-0.5).contiguous(), k) + bp
    scores = scores + torch.where(d["mask"][:, None, None, :], 0.0, -1e9).to(scores.dtype)
    o = torch.matmul(torch.softmax(scores, -1), v).permute(0, 2, 1, 3).reshape(N, N, H * D)
    g = torch.sigmoid(F.linear(xln, d["W_proj_g"]))
    return F.linear(o * g, d["W_proj_o"])


def tri_inputs_shape(N, Cin, Hh, Dd, seed=0):
    """triangle attention inputs at another shape (the Apo shape: C_in = 64, H = 4, D = 16)."""
    g = _gen(seed)
    s = Cin**-0.5
    d = dict(
        X=torch.randn(N, N, Cin, generator=g),
        W_ln=1 + 0.1 * torch.randn(Cin, generator=g),
        B_ln=0.1 * torch.randn(Cin, generator=g),
        WQ=torch.randn(Cin, Hh * Dd, generator=g) * s,
        WK=torch.randn(Cin, Hh * Dd, generator=g) * s,
        WV=torch.randn(Cin, Hh * Dd, generator=g) * s,
        W_proj_z=torch.randn(Cin, Hh, generator=g) * s,
        B_proj_z=torch.zeros(Hh),
        W_proj_g=torch.randn(Hh * Dd, Cin, generator=g) * s,
        W_proj_o=torch.randn(Cin, Hh * Dd, generator=g) * (Hh * Dd) ** -0.5,
    )
    d = {k: v.to(torch.bfloat16) for k, v in d.items()}
    d["mask"] = pad_mask2(N)
    return d


def torch_tri_shape(d, Hh, Dd, eps=1e-5):
    """torch_tri at any (C_in, H, D)."""
    X = d["X"]
    N, _, Cin = X.shape
    xln = F.layer_norm(X, (Cin,), d["W_ln"], d["B_ln"], eps=eps)
    q = (xln @ d["WQ"]).view(N, N, Hh, Dd).permute(0, 2, 1, 3)
    k = (xln @ d["WK"]).view(N, N, Hh, Dd).permute(0, 2, 3, 1).contiguous()
    v = (xln @ d["WV"]).view(N, N, Hh, Dd).permute(0, 2, 1, 3).contiguous()
    bp = (xln @ d["W_proj_z"] + d["B_proj_z"]).permute(2, 0, 1).unsqueeze(0)
    scores = torch.matmul((q * Dd**-0.5).contiguous(), k) + bp
    scores = scores + torch.where(d["mask"][:, None, None, :], 0.0, -1e9).to(scores.dtype)
    o = torch.matmul(torch.softmax(scores, -1), v).permute(0, 2, 1, 3).reshape(N, N, Hh * Dd)
    g = torch.sigmoid(F.linear(xln, d["W_proj_g"]))
    return F.linear(o * g, d["W_proj_o"])


def torch_apb(d, eps=1e-5):
    X, Z = d["X"], d["Z"]
    M = X.shape[0]
    q = (X @ d["WQ"]).reshape(M, H, D).permute(1, 0, 2)
    k = (X @ d["WK"]).reshape(M, H, D).permute(1, 2, 0).contiguous()
    v = (X @ d["WV"]).reshape(M, H, D).permute(1, 0, 2).contiguous()
    bp = (F.layer_norm(Z, (C,), d["W_ln"], d["B_ln"], eps=eps) @ d["W_proj_z"] + d["B_proj_z"]).permute(2, 0, 1)
    scores = torch.matmul((q * D**-0.5).contiguous(), k) + bp
    scores = scores.masked_fill(~d["mask"][None, None, :], float("-inf"))
    o = torch.matmul(torch.softmax(scores, -1), v).permute(1, 0, 2).reshape(M, H * D)
    g = torch.sigmoid(F.linear(X, d["W_proj_g"], d["B_proj_g"]))
    return F.linear(g * o, d["W_proj_o"], d["B_proj_o"])


def torch_apb_qknorm(d, p, eps=1e-5):
    """benchmarks/references.py:258-277 in bf16 (the key mask fill keeps the scores' dtype)."""
    X, Z = d["X"], d["Z"]
    M = X.shape[0]
    q = F.layer_norm(X @ d["WQ"] + p["b_q"], (H * D,), p["qkn_w_q"], p["qkn_b_q"], eps=eps)
    k = F.layer_norm(X @ d["WK"], (H * D,), p["qkn_w_k"], p["qkn_b_k"], eps=eps)
    q = q.reshape(M, H, D).permute(1, 0, 2)
    k = k.reshape(M, H, D).permute(1, 2, 0).contiguous()
    v = (X @ d["WV"]).reshape(M, H, D).permute(1, 0, 2).contiguous()
    bp = (F.layer_norm(Z, (C,), d["W_ln"], d["B_ln"], eps=eps) @ d["W_proj_z"] + d["B_proj_z"]).permute(2, 0, 1)
    scores = torch.matmul((q * D**-0.5).contiguous(), k) + bp
    scores = scores.masked_fill(~d["mask"][None, None, :], float("-inf"))
    o = torch.matmul(torch.softmax(scores, -1), v).permute(1, 0, 2).reshape(M, H * D)
    g = torch.sigmoid(F.linear(X, d["W_proj_g"]))
    return F.linear(g * o, d["W_proj_o"])


def torch_pair_stack(z, m, w_out, w_in, ts, te, eps=1e-5):
    """The four residual pair updates of a Pairformer block over the torch formulations above."""
    z = z + torch_tmu(z[None], "outgoing", m[None], eps, **w_out)[0]
    z = z + torch_tmu(z[None], "incoming", m[None], eps, **w_in)[0]
    z = z + torch_tri(dict(ts, X=z, mask=m), eps)
    zt = z.transpose(0, 1).contiguous()
    return z + torch_tri(dict(te, X=zt, mask=m.T.contiguous()), eps).transpose(0, 1)


# --------------------------------------------------------------------------- #
# timing helpers
# --------------------------------------------------------------------------- #
# per-call timing of the reference's benchmark harness (benchmarks/harness.py:18-40: 12 warmup
# calls, then 30 calls each bracketed by events and a synchronize, the median); the op entries use
# it where a call is short enough, so clocks have settled as they have in the reference's runs
REF_ITERS, REF_WARMUP = 30, 12
# seconds of untimed headline steps before its warmup steps (clocks at their loaded level)
SETTLE_S = 0.25


def time_ms(fn, iters, warmup):
    """Median per-call ms via HIP events on the current stream; NaN on OOM."""
    try:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(iters):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            ts.append(s.elapsed_time(e))
        return statistics.median(ts)
    except torch.OutOfMemoryError:
        torch.cuda.empty_cache()
        return float("nan")


_LEAD = {}


def gpu_lead(n=6):
    """Queues ~n ms of GPU work ahead of a timed block (bf16 8192^3 GEMMs, which load every CU), so
    the host has enqueued the block's launches and events before the GPU reaches them: the block's
    calls then run back to back and event intervals hold GPU work only, not the host's launch gaps
    (which otherwise dominate phases shorter than their Python overhead).  Loaded work rather than
    a spin of one wave, so the block starts at the clocks of a busy chip, not of an idle one."""
    if "a" not in _LEAD:
        _LEAD["a"] = torch.randn(8192, 8192, device="cuda", dtype=torch.bfloat16)
        _LEAD["c"] = torch.empty_like(_LEAD["a"])
    for _ in range(n):
        torch.matmul(_LEAD["a"], _LEAD["a"], out=_LEAD["c"])


class PhaseTimer:
    """Records HIP events between the launches of one call; averages each phase over calls."""

    def __init__(self, names):
        self.names = names
        self.events = []

    def run(self, phases):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)]
        ev[0].record()
        for i, ph in enumerate(phases):
            ph()
            ev[i + 1].record()
        self.events.append(ev)

    def averages(self):
        torch.cuda.synchronize()
        out = {}
        for i, n in enumerate(self.names):
            out[n] = statistics.fmean(ev[i].elapsed_time(ev[i + 1]) for ev in self.events)
        return out


def kernel_entry(name, ms, bound, work):
    """Roofline figures of one kernel: work = algorithmic bytes (hbm) or flops (mfma) per launch."""
    if bound == "mfma":
        achieved = work / (ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_MFMA_BF16, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_MFMA_BF16, 4), "ms": round(ms, 4), "work": work}
    achieved = work / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM, 4), "ms": round(ms, 4), "work": work}


# --------------------------------------------------------------------------- #
# per-op phase decompositions (exactly the launches forward() issues)
# --------------------------------------------------------------------------- #
def tmu_phases(x, m, pre, direction):
    L = x.shape[1]
    ld = max(64, (L + 63) // 64 * 64)
    st = {}

    def p_in():
        st["ab"] = input_phase(x, m, pre["p_in_combined"], pre["g_in_combined"], pre["sum_W_p_in"],
                               pre["sum_W_g_in"], pre["B_p_in_const"], pre["B_g_in_const"], 1e-5,
                               transpose=direction == "incoming", ld=ld)

    def p_ein():
        st["y"] = triangle_einsum(st["ab"], L, ld, C, 1)

    def p_out():
        st["out"] = output_phase(st["y"], x, pre["p_out_combined"], pre["g_out_combined"], pre["sum_W_p_out"],
                                 pre["sum_W_g_out"], pre["B_p_out_const"], pre["B_g_out_const"], 1e-5, ldy=ld)

    return [p_in, p_ein, p_out]


def tmu_work(L):
    M = L * L
    return {
        "tmu_input_phase": ("hbm", 2 * M * C + M + 2 * M * 2 * C),
        "tmu_einsum": ("mfma", 2 * C * L**3),
        "tmu_output_phase": ("hbm", 3 * 2 * M * C),
    }


def tri_phases(d, pre, hd=(H, D)):
    st = {}
    N = d["X"].shape[0]
    h, dh = hd

    def p_prep():
        st["qp"], st["kv"], st["bias"], st["ldn"] = prep_forward(d["X"], pre["W_ln"], pre["B_ln"], pre["wqkv_hm"],
                                                                 pre["WZ_c"], pre["BZ"], scale=dh**-0.5)

    def p_att():
        st["o"] = torch.empty(N, N, h * dh, device=d["X"].device, dtype=d["X"].dtype)
        attention_core(st["qp"], st["kv"], st["bias"], st["o"], N=N, ldn=st["ldn"], mask=d["mask"])

    def p_gate():
        st["out"] = gate_out_forward(st["o"], d["X"], d["W_proj_g"], None, d["W_proj_o"], None,
                                     ln=(pre["W_ln"], pre["B_ln"], 1e-5))

    return [p_prep, p_att, p_gate]


def tri_work(N, c=C, h=H, dh=D):
    """Algorithmic work per launch at (C_in, H, D); at D = 16 the kernels carry heads zero-padded to
    32 lanes (twice the Q / K / V bytes and attention flops counted here)."""
    return {
        "tri_prep": ("hbm", 2 * N * N * c + 6 * N * N * h * dh + 2 * h * N * N),
        "tri_attention": ("mfma", 4 * N**3 * h * dh),
        "tri_gate_out": ("hbm", 6 * N * N * c),
    }


def apb_phases(d, pre):
    """forward()'s three launches at the tuned shape (tops_apb_forward_gated), each as its own call on
    the same workspace layout: the Q / K / V pre-pass (apb_qkv_kernel, which tops_apb_qkn_prep runs
    at the tuned shape without a Q bias or qk-norm, exactly as the fused call does), the attention
    kernel alone (tops_apb_forward_qkv with Og = NULL leaves the split partials in the workspace),
    then the split merge fused with the gate and W_o (tops_apb_merge_gate)."""
    st = {}
    M = d["X"].shape[0]
    dev, dt = d["X"].device, d["X"].dtype
    m8 = d["mask"].view(torch.int8) if d["mask"].dtype == torch.bool else d["mask"]
    work = torch.empty(max(_native.apb_workspace_bytes(M, H, D), 1), device=dev, dtype=torch.uint8)
    Wc, sWc, Bc = (pre[k].float().contiguous() for k in ("W_combined", "sum_W_combined", "B_const"))
    wg, bg, wo, bo = (d[k].to(dt).contiguous() for k in ("W_proj_g", "B_proj_g", "W_proj_o", "B_proj_o"))
    out = torch.empty(M, C, device=dev, dtype=dt)
    code = 1 if dt == torch.float16 else 2

    def p_qkv():
        st["qkv"] = apb_qkn_prep(d["X"], pre["wqkv_hm"], None, None, qscale=D**-0.5)

    def p_att():
        q, k, v = st["qkv"]
        _native.call("tops_apb_forward_qkv", q.data_ptr(), k.data_ptr(), v.data_ptr(), d["Z"].data_ptr(),
                     d["Z"].stride(0), d["Z"].stride(1), Wc.data_ptr(), sWc.data_ptr(), Bc.data_ptr(), m8.data_ptr(),
                     None, work.data_ptr(), M, H * D, C, H, D, 1.0, 1e-5, code, _native.stream_of(q))

    def p_mg():
        _native.call("tops_apb_merge_gate", work.data_ptr(), d["X"].data_ptr(), wg.data_ptr(), bg.data_ptr(),
                     wo.data_ptr(), bo.data_ptr(), None, out.data_ptr(), M, H, D, code, _native.stream_of(out))
        st["out"] = out

    return [p_qkv, p_att, p_mg]


def apb_work(M):
    """apb_attention: Z read once (2 M^2 C bytes) by apb_attn_kernel; apb_merge_gate reads the split
    partials (nsplit M H (D + 2) fp32) and X and writes the output."""
    part = _native.apb_workspace_bytes(M, H, D) - ((3 * M * H * D * 2 + 255) // 256 * 256)
    return {"apb_qkv": ("hbm", 2 * M * C + 3 * 2 * M * H * D), "apb_attention": ("hbm", 2 * M * M * C),
            "apb_merge_gate": ("hbm", part + 2 * 2 * M * C)}


def apb_qkn_phases(d, pre, p):
    st = {}
    M = d["X"].shape[0]

    def p_prep():
        st["qkv"] = apb_qkn_prep(d["X"], pre["wqkv_hm"], p["b_q"],
                                 (p["qkn_w_q"], p["qkn_b_q"], p["qkn_w_k"], p["qkn_b_k"]))

    def p_att():
        st["og"] = torch.empty(M, H * D, device=d["X"].device, dtype=d["X"].dtype)
        apb_forward_qkv(*st["qkv"], d["Z"], pre["W_combined"], pre["sum_W_combined"], pre["B_const"], st["og"],
                        scale=D**-0.5, mask=d["mask"])

    def p_gate():
        st["out"] = gate_out_forward(st["og"].view(M, 1, H * D), d["X"], d["W_proj_g"], None, d["W_proj_o"], None)

    return [p_prep, p_att, p_gate]


def apb_qkn_work(M):
    return {"apb_qkn_prep": ("hbm", 2 * M * C + 3 * 2 * M * H * D), "apb_attention": ("hbm", 2 * M * M * C),
            "apb_gate_out": ("hbm", 3 * 2 * M * C)}


def run_phases(phase_lists, names, iters, warmup):
    """Times the phase lists (one list per call in a step); returns (avg ms per phase name)."""
    for _ in range(warmup):
        for pl in phase_lists:
            for ph in pl:
                ph()
    torch.cuda.synchronize()
    timers = [PhaseTimer(names) for _ in phase_lists]
    gpu_lead()
    for _ in range(iters):
        for t, pl in zip(timers, phase_lists):
            t.run(pl)
    torch.cuda.synchronize()
    avgs = [t.averages() for t in timers]
    return {n: statistics.fmean(a[n] for a in avgs) for n in names}


def graph_ms(call, *args, iters=50):
    """ms per replay of `call(*args)` captured as one HIP graph (triangleops_amd.graph)."""
    g = tops.graph.capture(call, *args)
    return time_ms(g.replay, iters, 3)


# --------------------------------------------------------------------------- #
# CPU baseline (fp32 oracle on this host)
# --------------------------------------------------------------------------- #
CPU_SHARE = 16  # host cores of one GPU's share on the GPU boxes (OMP_NUM_THREADS there)


def _cpu_threads():
    """(threads used, CPUs in this process's affinity mask): the oracle runs on the GPU's CPU share."""
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(aff, int(os.environ.get("OMP_NUM_THREADS", CPU_SHARE) or CPU_SHARE), CPU_SHARE))
    torch.set_num_threads(threads)
    return threads, aff


def _repeat(fn, min_s):
    calls, t0 = 0, time.perf_counter()
    while True:  # whole calls until at least min_s of CPU work has been timed
        fn()
        calls += 1
        dt = time.perf_counter() - t0
        if dt >= min_s:
            return calls, dt


def cpu_baseline_tmu(x, m, w, L, min_s=10.0):
    from oracle import reference as oracle  # the checker, timed here as the CPU baseline

    threads, aff = _cpu_threads()
    calls, dt = _repeat(lambda: oracle.triangle_multiplicative_update(x, direction="outgoing", mask=m, **w), min_s)
    return {"value": round(calls / dt, 5), "unit": "calls/s", "cores": threads, "affinity_cpus": aff, "kind": "port",
            "sample": f"{calls} full outgoing call(s) at L={L} (fp32 torch oracle), {dt:.1f} s"}


def config0_entry(dev, cpu):
    """BASELINE configs[0], the reference's CPU-runnable case: triangle_multiplicative_update
    outgoing at L = 128 with an all-ones mask (the seed-0 inputs of tmu_inputs).  The HIP path's ms
    per call with bf16 and with fp32 I/O (the config's dtype, on the any-shape fp32 path) beside the
    fp32 oracle on the host cores, whole calls on the same inputs."""
    L = 128
    x_c, _, w_c = tmu_inputs(L)
    m_c = torch.ones(1, L, L, dtype=torch.bool)
    x, m = x_c.to(dev), m_c.to(dev)
    e = {"workload": f"triangle_multiplicative_update outgoing, L={L}, C={C}, B=1, all-ones mask"}
    w = {k: v.to(dev) for k, v in w_c.items()}
    pre = tops.triangle_mul.precompute(*[w[k] for k in TMU_KEYS])
    e["ms_per_call_bf16"] = round(time_ms(lambda: tops.triangle_mul.forward(x, pre, direction="outgoing", mask=m),
                                          50, 10), 4)
    xf, wf = x.float(), {k: v.float() for k, v in w.items()}
    pref = tops.triangle_mul.precompute(*[wf[k] for k in TMU_KEYS])
    e["ms_per_call_fp32"] = round(time_ms(lambda: tops.triangle_mul.forward(xf, pref, direction="outgoing", mask=m),
                                          50, 10), 4)
    e["cpu_baseline"] = cpu_baseline_tmu(x_c, m_c, w_c, L, min_s=5.0) if cpu else None
    return e


def cpu_baseline_tri(d, N, min_s=8.0):
    """fp32 oracle triangle attention on sampled rows: rows are independent, so a call over R rows
    costs a + b R (a: LayerNorm and pair bias of the whole grid, b: one row's projections, attention
    and gate); a and b come from timing R and 2R rows, and the whole call is estimated as a + b N."""
    from oracle import reference as oracle

    threads, aff = _cpu_threads()
    R = 16
    args = (d["X"], d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"], d["B_proj_z"], d["W_proj_g"],
            None, d["W_proj_o"], None, H, D)
    t = {}
    for r in (R, 2 * R):
        rows = torch.arange(r) * (N // (2 * R))
        calls, dt = _repeat(lambda: oracle.triangle_attention(*args, scale=D**-0.5, mask=d["mask"], rows=rows),
                            min_s / 2)
        t[r] = dt / calls
    b = max(t[2 * R] - t[R], 1e-9) / R
    a = max(t[R] - b * R, 0.0)
    est = a + b * N
    return {"value": round(1.0 / est, 6), "unit": "calls/s", "cores": threads, "affinity_cpus": aff, "kind": "port",
            "sample": f"starting node at N={N} (fp32 torch oracle) timed on {R} and {2 * R} sampled rows "
                      f"({t[R]:.2f} s / {t[2 * R]:.2f} s per call); whole call estimated as "
                      f"{a:.3g} s + {N} x {b:.4g} s = {est:.4g} s"}


def cpu_baseline_apb(d, M, min_s=6.0):
    from oracle import reference as oracle

    threads, aff = _cpu_threads()
    args = (d["X"], d["WQ"], d["WK"], d["WV"], d["Z"], d["W_ln"], d["B_ln"], d["W_proj_z"], d["B_proj_z"],
            d["W_proj_g"], d["B_proj_g"], d["W_proj_o"], d["B_proj_o"], H, D)
    calls, dt = _repeat(lambda: oracle.attention_pair_bias(*args, scale=D**-0.5, mask=d["mask"]), min_s)
    return {"value": round(calls / dt, 5), "unit": "calls/s", "cores": threads, "affinity_cpus": aff, "kind": "port",
            "sample": f"{calls} full call(s) at M={M} (fp32 torch oracle), {dt:.1f} s"}


def op_entry_tri(N, dev, iters, warmup, cpu):
    """triangle_attention at N: starting and ending node per call, per-kernel
    HIP-event times of the starting node, the attention kernel's MFMA fraction, the torch path."""
    d_c = tri_inputs(N)
    d = to_dev(d_c, dev)
    pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                        d["B_proj_z"], H, D)
    kw = dict(scale=D**-0.5, W_proj_g=d["W_proj_g"], B_proj_g=None, W_proj_o=d["W_proj_o"], B_proj_o=None)
    ms = time_ms(lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], **kw), iters, warmup)
    ms_end = time_ms(lambda: tops.triangle_attn.forward(d["X"].transpose(0, 1), pre, mask=d["mask"].T, **kw), iters,
                     warmup)
    work = tri_work(N)
    ph = run_phases([tri_phases(d, pre)], list(work), iters, warmup)
    kern = {n: kernel_entry(n, ph[n], *work[n]) for n in ph}
    ka = kern["tri_attention"]
    e = {"config": f"triangle_attention bf16, N={N}, H={H}, D={D}, C={C}, pad mask (last 10% rows/cols)",
         "ms_per_call": round(ms, 4), "ms_per_call_ending_node": round(ms_end, 4), "calls_per_s": round(1e3 / ms, 2),
         "roofline": {"kernel": "tri_attention", "bound": "mfma", "achieved": ka["achieved"], "peak": ka["peak"],
                      "unit": ka["unit"], "frac": ka["frac"], "traffic": measured_traffic("tri_attention", N)},
         "kernels": kern}
    e["torch_path_ms"] = round(time_ms(lambda: torch_tri(d), REF_ITERS, REF_WARMUP), 4)
    del d, pre
    torch.cuda.empty_cache()
    e["cpu_baseline"] = cpu_baseline_tri(d_c, N) if cpu else None
    return e


def op_entry_apb(M, dev, iters, warmup, cpu):
    """attention_pair_bias at M: per-kernel times, the attention kernel's HBM
    fraction (Z is read once: 2 M^2 C bytes), the torch path."""
    d_c = apb_inputs(M)
    d = to_dev(d_c, dev)
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], H, D)
    ms = time_ms(lambda: tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=D**-0.5, W_proj_g=d["W_proj_g"],
                                                      B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"],
                                                      B_proj_o=d["B_proj_o"], mask=d["mask"]), iters, warmup)
    work = apb_work(M)
    ph = run_phases([apb_phases(d, pre)], list(work), iters, warmup)
    kern = {n: kernel_entry(n, ph[n], *work[n]) for n in ph}
    ka = kern["apb_attention"]
    e = {"config": f"attention_pair_bias bf16, M={M}, H={H}, D={D}, C_s=C_z={C}, key mask (last 5% padded)",
         "ms_per_call": round(ms, 4), "calls_per_s": round(1e3 / ms, 2),
         "roofline": {"kernel": "apb_attention (apb_attn_kernel)", "bound": "hbm", "achieved": ka["achieved"], "peak": ka["peak"],
                      "unit": ka["unit"], "frac": ka["frac"], "traffic": measured_traffic("apb_attention", M)},
         "kernels": kern}
    e["torch_path_ms"] = round(time_ms(lambda: torch_apb(d), REF_ITERS, REF_WARMUP), 4)
    del d, pre
    torch.cuda.empty_cache()
    e["cpu_baseline"] = cpu_baseline_apb(d_c, M) if cpu else None
    return e


SIZE_SWEEP = {"triangle_multiplicative_update": (512, 2048), "triangle_attention": (256, 512, 2048),
              "attention_pair_bias": (128, 512, 2048)}


def _compact(kern):
    """The dominant kernel of a call (largest average time) and every kernel's ms and roofline fraction."""
    dom = max(kern, key=lambda n: kern[n]["ms"])
    return {"dominant": dom, "frac": kern[dom]["frac"], "bound": kern[dom]["bound"],
            "kernels": {n: {"ms": k["ms"], "frac": k["frac"]} for n, k in kern.items()}}


def size_sweep_entries(dev):
    """BASELINE.json's metric across its config sizes other than the 1024 entries above (tmu
    L = 512, 2048; triangle attention N = 256, 512, 2048; apb M = 128, 512, 2048): per op and size the
    ms per call (both directions / nodes), the dominant kernel's roofline fraction, every kernel's
    ms and fraction, the reference's torch path on the same GPU (NaN = out of memory), and at sizes
    <= 512 the same call replayed as one HIP graph (host launch overhead removed)."""
    out = []
    for L in SIZE_SWEEP["triangle_multiplicative_update"]:
        torch.cuda.empty_cache()
        x, m, w = tmu_inputs(L)
        x, m, w = x.to(dev), m.to(dev), {k: v.to(dev) for k, v in w.items()}
        pre = tops.triangle_mul.precompute(*[w[k] for k in TMU_KEYS])
        it, wu = (REF_ITERS, REF_WARMUP) if L <= 1024 else (10, 4)
        e = {"op": "triangle_multiplicative_update", "size": L}
        for direction in ("outgoing", "incoming"):
            e[f"ms_per_call_{direction}"] = round(time_ms(
                lambda: tops.triangle_mul.forward(x, pre, direction=direction, mask=m), it, wu), 4)
        work = tmu_work(L)
        ph = run_phases([tmu_phases(x, m, pre, "outgoing"), tmu_phases(x, m, pre, "incoming")], list(work), it, wu)
        e.update(_compact({n: kernel_entry(n, ph[n], *work[n]) for n in ph}))
        e["torch_path_ms"] = round(time_ms(lambda: torch_tmu(x, "outgoing", m, **w), it, wu), 4)
        if L <= 512:
            e["ms_graph"] = round(graph_ms(lambda xx: tops.triangle_mul.forward(xx, pre, direction="outgoing",
                                                                                mask=m), x), 4)
        out.append(e)
        print(f"size sweep: tmu L={L} done", file=sys.stderr, flush=True)
        del x, m, w, pre
    for N in SIZE_SWEEP["triangle_attention"]:
        torch.cuda.empty_cache()
        d = to_dev(tri_inputs(N), dev)
        pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                            d["B_proj_z"], H, D)
        kw = dict(scale=D**-0.5, W_proj_g=d["W_proj_g"], B_proj_g=None, W_proj_o=d["W_proj_o"], B_proj_o=None)
        it, wu = REF_ITERS, REF_WARMUP
        e = {"op": "triangle_attention", "size": N,
             "ms_per_call": round(time_ms(lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], **kw), it,
                                          wu), 4),
             "ms_per_call_ending_node": round(time_ms(lambda: tops.triangle_attn.forward(
                 d["X"].transpose(0, 1), pre, mask=d["mask"].T, **kw), it, wu), 4)}
        work = tri_work(N)
        ph = run_phases([tri_phases(d, pre)], list(work), it, wu)
        e.update(_compact({n: kernel_entry(n, ph[n], *work[n]) for n in ph}))
        # N = 2048: the (N, H, N, N) bf16 scores are 64 GiB per intermediate; timed 5 times after two
        # warmup calls (out of memory is reported as NaN, not skipped)
        e["torch_path_ms"] = round(time_ms(lambda: torch_tri(d), *((it, wu) if N <= 1024 else (5, 2))), 4)
        torch.cuda.empty_cache()
        if N <= 512:
            e["ms_graph"] = round(graph_ms(lambda X: tops.triangle_attn.forward(X, pre, mask=d["mask"], **kw),
                                           d["X"]), 4)
        out.append(e)
        print(f"size sweep: tri N={N} done", file=sys.stderr, flush=True)
        del d, pre
    for M in SIZE_SWEEP["attention_pair_bias"]:
        torch.cuda.empty_cache()
        d = to_dev(apb_inputs(M), dev)
        pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                             d["B_proj_z"], H, D)
        kw = dict(scale=D**-0.5, W_proj_g=d["W_proj_g"], B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"],
                  B_proj_o=d["B_proj_o"], mask=d["mask"])
        e = {"op": "attention_pair_bias", "size": M,
             "ms_per_call": round(time_ms(lambda: tops.attn_pair_bias.forward(d["X"], d["Z"], pre, **kw), REF_ITERS,
                                          REF_WARMUP), 4)}
        work = apb_work(M)
        ph = run_phases([apb_phases(d, pre)], list(work), 20, 5)
        e.update(_compact({n: kernel_entry(n, ph[n], *work[n]) for n in ph}))
        e["torch_path_ms"] = round(time_ms(lambda: torch_apb(d), REF_ITERS, REF_WARMUP), 4)
        if M <= 512:
            e["ms_graph"] = round(graph_ms(lambda X, Z: tops.attn_pair_bias.forward(X, Z, pre, **kw), d["X"], d["Z"]),
                                  4)
        out.append(e)
        print(f"size sweep: apb M={M} done", file=sys.stderr, flush=True)
        del d, pre
    torch.cuda.empty_cache()
    return out


# --------------------------------------------------------------------------- #
def sweep(path, sizes, dev):
    rows = []
    with open(path, "w") as f:
        for L in sizes:
            torch.cuda.empty_cache()
            x, m, w = tmu_inputs(L)
            x, m, w = x.to(dev), m.to(dev), {k: v.to(dev) for k, v in w.items()}
            pre = tops.triangle_mul.precompute(*[w[k] for k in TMU_KEYS])
            it, wu = (20, 5) if L <= 1024 else (8, 3)
            for direction in ("outgoing", "incoming"):
                ms = time_ms(lambda: tops.triangle_mul.forward(x, pre, direction=direction, mask=m), it, wu)
                tms = time_ms(lambda: torch_tmu(x, direction, m, **w), it, wu) if L <= 2048 else float("nan")
                ph = run_phases([tmu_phases(x, m, pre, direction)], list(tmu_work(L)), it, wu)
                kern = {n: kernel_entry(n, ph[n], *tmu_work(L)[n]) for n in ph}
                r = {"op": "triangle_multiplicative_update", "direction": direction, "size": L, "ms": round(ms, 4),
                     "calls_per_s": round(1e3 / ms, 1), "torch_path_ms": round(tms, 4), "kernels": kern}
                if L <= 512:  # launch-bound sizes: the same call replayed as one HIP graph
                    r["ms_graph"] = round(graph_ms(
                        lambda xx: tops.triangle_mul.forward(xx, pre, direction=direction, mask=m), x), 4)
                f.write(json.dumps(r) + "\n")
                f.flush()
                rows.append(r)
            del x, m, w, pre
        for N in sizes:
            torch.cuda.empty_cache()
            d = to_dev(tri_inputs(N), dev)
            pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                                d["B_proj_z"], H, D)
            it, wu = (20, 5) if N <= 1024 else (6, 2)
            fwd = lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], scale=D**-0.5,  # noqa: E731
                                                     W_proj_g=d["W_proj_g"], B_proj_g=None,
                                                     W_proj_o=d["W_proj_o"], B_proj_o=None)
            ms = time_ms(fwd, it, wu)
            ms_end = time_ms(lambda: tops.triangle_attn.forward(
                d["X"].transpose(0, 1), pre, mask=d["mask"].T, scale=D**-0.5, W_proj_g=d["W_proj_g"],
                B_proj_g=None, W_proj_o=d["W_proj_o"], B_proj_o=None), it, wu)
            tms = time_ms(lambda: torch_tri(d), max(3, it // 4), 1) if N <= 1024 else float("nan")
            ph = run_phases([tri_phases(d, pre)], list(tri_work(N)), it, wu)
            kern = {n: kernel_entry(n, ph[n], *tri_work(N)[n]) for n in ph}
            r = {"op": "triangle_attention", "size": N, "ms": round(ms, 4), "ms_ending_node": round(ms_end, 4),
                 "calls_per_s": round(1e3 / ms, 1), "torch_path_ms": round(tms, 4), "kernels": kern}
            if N <= 512:
                r["ms_graph"] = round(graph_ms(lambda X: tops.triangle_attn.forward(
                    X, pre, mask=d["mask"], scale=D**-0.5, W_proj_g=d["W_proj_g"], B_proj_g=None,
                    W_proj_o=d["W_proj_o"], B_proj_o=None), d["X"]), 4)
            f.write(json.dumps(r) + "\n")
            f.flush()
            rows.append(r)
            del d, pre
        # the Apo shape (C_in = 64, H = 4, D = 16) on the tuned kernels (C = 64 pre-pass and gate, heads
        # zero-padded to 32 lanes in the attention kernel); the any-shape scalar attention timed beside
        for N in [n for n in sizes if n in (256, 1024)]:
            torch.cuda.empty_cache()
            from triangleops_amd.triangle_attn.kernel import generic_attention, generic_prep_forward
            d = to_dev(tri_inputs_shape(N, 64, 4, 16), dev)
            pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                                d["B_proj_z"], 4, 16)
            it, wu = (20, 5) if N <= 512 else (10, 3)
            fwd = lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], scale=16**-0.5,  # noqa: E731
                                                     W_proj_g=d["W_proj_g"], B_proj_g=None,
                                                     W_proj_o=d["W_proj_o"], B_proj_o=None)
            ms = time_ms(fwd, it, wu)
            tms = time_ms(lambda: torch_tri_shape(d, 4, 16), 3, 1)
            work = tri_work(N, 64, 4, 16)
            ph = run_phases([tri_phases(d, pre, (4, 16))], list(work), it, wu)
            kern = {n: kernel_entry(n, ph[n], *work[n]) for n in ph}
            xln, q, k, v, bias = generic_prep_forward(d["X"], pre["W_ln"], pre["B_ln"], pre["wqkv_hm"], pre["WZ_c"],
                                                      pre["BZ"])
            o = torch.empty(N, N, 64, device=dev, dtype=torch.bfloat16)
            ms_scalar = time_ms(lambda: generic_attention(q, k, v, bias, o, scale=16**-0.5, mask=d["mask"]), 2, 1)
            r = {"op": "triangle_attention_apo", "shape": "C_in=64 H=4 D=16", "size": N, "ms": round(ms, 4),
                 "calls_per_s": round(1e3 / ms, 1), "torch_path_ms": round(tms, 4),
                 "attention_ms_scalar": round(ms_scalar, 4), "kernels": kern}
            f.write(json.dumps(r) + "\n")
            f.flush()
            rows.append(r)
            del d, pre, xln, q, k, v, bias, o
        for M in sizes:
            torch.cuda.empty_cache()
            d = to_dev(apb_inputs(M), dev)
            pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                                 d["B_proj_z"], H, D)
            fwd = lambda: tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=D**-0.5,  # noqa: E731
                                                      W_proj_g=d["W_proj_g"], B_proj_g=d["B_proj_g"],
                                                      W_proj_o=d["W_proj_o"], B_proj_o=d["B_proj_o"], mask=d["mask"])
            ms = time_ms(fwd, 20, 5)
            tms = time_ms(lambda: torch_apb(d), 10, 2)
            ph = run_phases([apb_phases(d, pre)], list(apb_work(M)), 20, 5)
            kern = {n: kernel_entry(n, ph[n], *apb_work(M)[n]) for n in ph}
            r = {"op": "attention_pair_bias", "size": M, "ms": round(ms, 4), "calls_per_s": round(1e3 / ms, 1),
                 "torch_path_ms": round(tms, 4), "kernels": kern}
            if M <= 512:
                r["ms_graph"] = round(graph_ms(lambda X, Z: tops.attn_pair_bias.forward(
                    X, Z, pre, scale=D**-0.5, W_proj_g=d["W_proj_g"], B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"],
                    B_proj_o=d["B_proj_o"], mask=d["mask"]), d["X"], d["Z"]), 4)
            f.write(json.dumps(r) + "\n")
            f.flush()
            rows.append(r)
            # the qk-norm variant on the same inputs (Q bias, LN over H*D of Q and K, key mask)
            p = to_dev(apb_qkn_params(), dev)
            fwd = lambda: tops.attn_pair_bias.forward_qknorm(  # noqa: E731
                d["X"], d["Z"], pre, b_q=p["b_q"], qkn_w_q=p["qkn_w_q"], qkn_b_q=p["qkn_b_q"], qkn_w_k=p["qkn_w_k"],
                qkn_b_k=p["qkn_b_k"], key_mask=d["mask"], scale=D**-0.5, W_proj_g=d["W_proj_g"],
                W_proj_o=d["W_proj_o"])
            ms = time_ms(fwd, 20, 5)
            tms = time_ms(lambda: torch_apb_qknorm(d, p), 10, 2)
            ph = run_phases([apb_qkn_phases(d, pre, p)], list(apb_qkn_work(M)), 20, 5)
            kern = {n: kernel_entry(n, ph[n], *apb_qkn_work(M)[n]) for n in ph}
            r = {"op": "attention_pair_bias_qknorm", "size": M, "ms": round(ms, 4), "calls_per_s": round(1e3 / ms, 1),
                 "torch_path_ms": round(tms, 4), "kernels": kern}
            f.write(json.dumps(r) + "\n")
            f.flush()
            rows.append(r)
            del d, pre, p
        # Pairformer pair stack (z += tmu_out, tmu_in, tri_start, tri_end): fused residual adds vs
        # the same ops with separate adds vs the torch formulation
        for N in [n for n in sizes if n <= 1024]:
            torch.cuda.empty_cache()
            x, m, w_out = tmu_inputs(N)
            _, _, w_in = tmu_inputs(N, seed=1)
            ts, te = tri_inputs(N, seed=2), tri_inputs(N, seed=3)
            keys = ("W_ln", "B_ln", "WQ", "WK", "WV", "W_proj_z", "B_proj_z", "W_proj_g", "W_proj_o")
            ts, te = ({k: t[k].to(dev) for k in keys} for t in (ts, te))
            z, pm = x[0].to(dev), m[0].to(dev)
            w_out, w_in = ({k: v.to(dev) for k, v in w.items()} for w in (w_out, w_in))
            pre = tops.pairformer.precompute(w_out, w_in, ts, te, H=H, D=D)
            it = 20 if N <= 512 else 8
            ms = time_ms(lambda: tops.pairformer.pair_stack(z, pre, pair_mask=pm), it, 3)

            def unfused():
                m3 = pm[None]
                z1 = z + tops.triangle_mul.forward(z[None], pre["tmu_out"], direction="outgoing", mask=m3)[0]
                z2 = z1 + tops.triangle_mul.forward(z1[None], pre["tmu_in"], direction="incoming", mask=m3)[0]
                z3 = z2 + tops.triangle_attn.forward(z2, pre["tri_start"], mask=pm, scale=D**-0.5, W_proj_g=ts["W_proj_g"],
                                                     B_proj_g=None, W_proj_o=ts["W_proj_o"], B_proj_o=None)
                e = tops.triangle_attn.forward(z3.transpose(0, 1), pre["tri_end"], mask=pm.T, scale=D**-0.5,
                                               W_proj_g=te["W_proj_g"], B_proj_g=None, W_proj_o=te["W_proj_o"],
                                               B_proj_o=None)
                return z3 + e.transpose(0, 1)

            ms_unf = time_ms(unfused, it, 3)
            tms = time_ms(lambda: torch_pair_stack(z, pm, w_out, w_in, ts, te), max(3, it // 4), 1)
            r = {"op": "pairformer_pair_stack", "size": N, "ms": round(ms, 4), "ms_unfused_adds": round(ms_unf, 4),
                 "calls_per_s": round(1e3 / ms, 1), "torch_path_ms": round(tms, 4), "kernels": {}}
            if N <= 512:
                r["ms_graph"] = round(graph_ms(lambda zz: tops.pairformer.pair_stack(zz, pre, pair_mask=pm), z), 4)
            f.write(json.dumps(r) + "\n")
            f.flush()
            rows.append(r)
            del x, m, z, pm, pre, w_out, w_in, ts, te
        # fp32 I/O (every value fp32; the fp32 product on the fp32 MFMA, the tiled any-shape phases
        # and attention) against the torch formulation in fp32
        f32 = lambda dd: {k: (v.float() if torch.is_tensor(v) and v.is_floating_point() else v)  # noqa: E731
                          for k, v in dd.items()}
        for n in [s for s in sizes if s <= 1024]:
            torch.cuda.empty_cache()
            it = 10 if n <= 512 else 3
            x, m, w = tmu_inputs(n)
            x, m, w = x.float().to(dev), m.to(dev), {k: v.float().to(dev) for k, v in w.items()}
            pre = tops.triangle_mul.precompute(*[w[k] for k in TMU_KEYS])
            ms = time_ms(lambda: tops.triangle_mul.forward(x, pre, direction="outgoing", mask=m), it, 2)
            tms = time_ms(lambda: torch_tmu(x, "outgoing", m, **w), it, 2)
            rows.append({"op": "triangle_multiplicative_update_fp32", "size": n, "ms": round(ms, 4),
                         "torch_path_ms": round(tms, 4), "kernels": {}})
            f.write(json.dumps(rows[-1]) + "\n")
            del x, m, w, pre
            torch.cuda.empty_cache()
            d = to_dev(f32(tri_inputs(n)), dev)
            pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                                d["B_proj_z"], H, D)
            ms = time_ms(lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], scale=D**-0.5,
                                                            W_proj_g=d["W_proj_g"], B_proj_g=None,
                                                            W_proj_o=d["W_proj_o"], B_proj_o=None), it, 1)
            tms = time_ms(lambda: torch_tri(d), max(2, it // 3), 1)
            rows.append({"op": "triangle_attention_fp32", "size": n, "ms": round(ms, 4), "torch_path_ms": round(tms, 4),
                         "kernels": {}})
            f.write(json.dumps(rows[-1]) + "\n")
            del d, pre
            torch.cuda.empty_cache()
            d = to_dev(f32(apb_inputs(n)), dev)
            pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                                 d["B_proj_z"], H, D)
            ms = time_ms(lambda: tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=D**-0.5,
                                                             W_proj_g=d["W_proj_g"], B_proj_g=d["B_proj_g"],
                                                             W_proj_o=d["W_proj_o"], B_proj_o=d["B_proj_o"],
                                                             mask=d["mask"]), it, 2)
            tms = time_ms(lambda: torch_apb(d), it, 2)
            rows.append({"op": "attention_pair_bias_fp32", "size": n, "ms": round(ms, 4),
                         "torch_path_ms": round(tms, 4), "kernels": {}})
            f.write(json.dumps(rows[-1]) + "\n")
            f.flush()
            del d, pre
    return rows


TRAFFIC_PROFILES = [os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f)
                    for f in ("tmu_L1024_hbm_traffic.md", "ops_1024_hbm_traffic.md")]


def measured_traffic(kernel, n):
    """HBM bytes per launch of `kernel` at size 1024, from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summaries (2 x FETCH_SIZE + WRITE_SIZE, checked on kernels whose bytes are fixed);
    None otherwise."""
    if n != 1024:
        return None
    for path in TRAFFIC_PROFILES:
        if not os.path.exists(path):
            continue
        for line in open(path):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            if len(cells) >= 5 and cells[0] == kernel:
                try:
                    return int(cells[4])
                except ValueError:
                    return None
    return None


def _op_call(op, n, dev):
    """One call of an op at size n on seeded inputs (`tri`: starting-node triangle attention; `tri_apo`:
    the same at the Apo shape C_in = 64, H = 4, D = 16; `apb`: attention_pair_bias; `tmu`: outgoing
    tmu; `tmu2`: outgoing then incoming tmu)."""
    if op == "tri_apo":
        d = to_dev(tri_inputs_shape(n, 64, 4, 16), dev)
        pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                            d["B_proj_z"], 4, 16)
        return lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], scale=16**-0.5,
                                                  W_proj_g=d["W_proj_g"], B_proj_g=None, W_proj_o=d["W_proj_o"],
                                                  B_proj_o=None)
    if op == "tri":
        d = to_dev(tri_inputs(n), dev)
        pre = tops.triangle_attn.precompute(d["W_ln"], d["B_ln"], d["WQ"], d["WK"], d["WV"], d["W_proj_z"],
                                            d["B_proj_z"], H, D)
        return lambda: tops.triangle_attn.forward(d["X"], pre, mask=d["mask"], scale=D**-0.5,
                                                  W_proj_g=d["W_proj_g"], B_proj_g=None, W_proj_o=d["W_proj_o"],
                                                  B_proj_o=None)
    if op == "apb":
        d = to_dev(apb_inputs(n), dev)
        pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                             d["B_proj_z"], H, D)
        return lambda: tops.attn_pair_bias.forward(d["X"], d["Z"], pre, scale=D**-0.5, W_proj_g=d["W_proj_g"],
                                                   B_proj_g=d["B_proj_g"], W_proj_o=d["W_proj_o"],
                                                   B_proj_o=d["B_proj_o"], mask=d["mask"])
    x_c, m_c, w_c = tmu_inputs(n)
    x, m = x_c.to(dev), m_c.to(dev)
    w = {k: v.to(dev) for k, v in w_c.items()}
    pre = tops.triangle_mul.precompute(*[w[k] for k in TMU_KEYS])
    dirs = ("outgoing", "incoming") if op == "tmu2" else ("outgoing",)
    return lambda: [tops.triangle_mul.forward(x, pre, direction=dd, mask=m) for dd in dirs]


def traffic_run(n, op="tmu2"):
    """Workload of the HBM-traffic counter runs (no timing): a 256 MiB bf16 negation whose bytes are
    known (a reference point: FETCH_SIZE counts 64 bytes per 128-byte read request, so its reading
    depends on the access width torch picks for it), then two calls of `op` at size n (default: two
    tmu steps, outgoing + incoming; `tri` / `apb`: two calls of triangle attention /
    attention_pair_bias)."""
    dev = torch.device("cuda:0")
    src = torch.randn(128 * 1024 * 1024, device=dev).to(torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(2):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst
    fn = _op_call(op, n, dev)
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    print(f"traffic run {op} n={n} done", flush=True)


def op_run(op, n):
    """Workload of the counter runs (no timing): 7 calls of one op at size n (see _op_call)."""
    fn = _op_call(op, n, torch.device("cuda:0"))
    for _ in range(7):
        fn()
    torch.cuda.synchronize()
    print(f"op run {op} n={n} done", flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--size", type=int, default=1024, help="L of the headline workload")
    ap.add_argument("--sweep", default=None, help="also sweep all ops/sizes; JSON lines to this file")
    ap.add_argument("--sweep-sizes", default="128,256,512,1024,2048")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-torch", action="store_true", help="skip the torch-path reference timing")
    ap.add_argument("--no-ops", action="store_true", help="skip the triangle_attention / attention_pair_bias entries")
    ap.add_argument("--ops-size", type=int, default=1024, help="N = M of the triangle_attention / apb entries")
    ap.add_argument("--no-size-sweep", action="store_true",
                    help="skip the compact per-size entries (tmu 512/2048, tri 256/512/2048, apb 128/512/2048)")
    ap.add_argument("--op-run", choices=("tri", "tri_apo", "apb", "tmu"), default=None,
                    help="only run 7 calls of one op at --size (workload of rocprofv3 counter runs)")
    ap.add_argument("--traffic-run", nargs="?", const="tmu2", default=None, choices=("tmu2", "tri", "apb"),
                    help="only run the workload of the HBM-traffic counter runs (rocprofv3 --pmc FETCH_SIZE / "
                         "WRITE_SIZE): tmu2 (default, two tmu steps), tri or apb at --size")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the ops are "
              "single-GPU kernels and no multi-GPU path is part of it", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    L = args.size
    if args.traffic_run:
        traffic_run(L, args.traffic_run)
        return
    if args.op_run:
        op_run(args.op_run, L)
        return

    x_c, m_c, w_c = tmu_inputs(L)
    x, m = x_c.to(dev), m_c.to(dev)
    w = {k: v.to(dev) for k, v in w_c.items()}
    pre = tops.triangle_mul.precompute(*[w[k] for k in TMU_KEYS])
    steps = [tmu_phases(x, m, pre, "outgoing"), tmu_phases(x, m, pre, "incoming")]
    names = list(tmu_work(L))

    # settle: untimed steps until the chip has run the workload for SETTLE_S seconds.  On a GPU that
    # was idle, the first ~25 ms of this work ran ~8 % slower than every later 20-step block (the
    # clocks come up under load), so a timed region right after a few warmup steps measured the
    # ramp instead of the steady state
    settle_steps, t_settle = 0, time.perf_counter()
    while True:
        for _ in range(10):
            for pl in steps:
                for ph in pl:
                    ph()
        settle_steps += 10
        torch.cuda.synchronize()
        if time.perf_counter() - t_settle >= SETTLE_S:
            break
    # warmup
    for _ in range(args.warmup):
        for pl in steps:
            for ph in pl:
                ph()
    torch.cuda.synchronize()
    # timed region: exactly K steps (outgoing + incoming), per-launch HIP events inside
    timers = [PhaseTimer(names) for _ in steps]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        for t, pl in zip(timers, steps):
            t.run(pl)
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    ms_per_step = total_ms / args.steps
    per_dir = [t.averages() for t in timers]
    ph = {n: statistics.fmean(a[n] for a in per_dir) for n in names}
    work = tmu_work(L)
    kernels = {n: kernel_entry(n, ph[n], *work[n]) for n in names}
    dominant = max(names, key=lambda n: ph[n])
    kd = kernels[dominant]
    roofline = {"kernel": dominant, "bound": kd["bound"], "achieved": kd["achieved"], "peak": kd["peak"],
                "unit": kd["unit"], "frac": kd["frac"], "traffic": measured_traffic(dominant, L)}

    torch_ms = {} if args.no_torch else {d: time_ms(lambda: torch_tmu(x, d, m, **w), 5, 2)
                                          for d in ("outgoing", "incoming")}

    out = {
        "metric": METRIC,
        "value": round(2 * args.steps / (total_ms * 1e-3), 2),
        "unit": "calls/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_steps": settle_steps,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_call": round(ms_per_step / 2, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, random-init weights)",
        "config": {"workload": f"triangle_multiplicative_update bf16 outgoing+incoming, L={L}, C={C}, B=1, "
                               "pad mask (last 10% rows/cols), one step = one call per direction",
                   "L": L, "C": C, "B": 1},
        "roofline": roofline,
        "kernels": kernels,
        "torch_path_ms": {k: round(v, 4) for k, v in torch_ms.items()},
        "device": torch.cuda.get_device_name(dev),
    }
    del x, m, w, pre, steps, timers
    torch.cuda.empty_cache()
    cpu = not args.no_cpu_baseline
    # the other two ops of the metric at their BASELINE configurations (size 1024)
    if not args.no_ops:
        out["ops"] = {
            "triangle_attention": op_entry_tri(args.ops_size, dev, REF_ITERS, REF_WARMUP, cpu),
            "attention_pair_bias": op_entry_apb(args.ops_size, dev, REF_ITERS, REF_WARMUP, cpu),
        }
        out["config0"] = config0_entry(dev, cpu)
    if not args.no_size_sweep:
        out["size_sweep"] = size_sweep_entries(dev)
    if args.sweep:
        sweep(args.sweep, [int(s) for s in args.sweep_sizes.split(",")], dev)
    out["cpu_baseline"] = cpu_baseline_tmu(x_c, m_c, w_c, L) if cpu else None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
