"""Host-side checks (CPU only): drop-in API surface, precompute contents, error behaviour,
and that the C-ABI library exports every entry point the header declares."""

import ctypes
import inspect
import os
import re
import subprocess
import sys

import pytest
import torch

import triangleops_amd as tops
from triangleops_amd import _native
from triangleops_amd._common import tl_io_dtype

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "triangleops_amd.h")

# Public signatures of the reference API (triangle_ops/*/module.py and kernel.py), as
# (parameter name, default or None, keyword-only) lists; the drop-in must accept the same calls.
REF_SIGNATURES = {
    "triangle_mul.triangle_multiplicative_update": "x, *, direction, mask=None, eps=1e-05, norm_in_weight, "
    "norm_in_bias, p_in_weight, g_in_weight, norm_out_weight, norm_out_bias, p_out_weight, g_out_weight",
    "triangle_mul.precompute": "norm_in_weight, norm_in_bias, p_in_weight, g_in_weight, norm_out_weight, "
    "norm_out_bias, p_out_weight, g_out_weight",
    "triangle_mul.forward": "x, pre, *, direction, mask=None, eps=1e-05",
    "triangle_mul.input_phase": "x, mask, p_in_combined, g_in_combined, sum_W_p_in, sum_W_g_in, B_p_in_const, "
    "B_g_in_const, eps",
    "triangle_mul.output_phase": "y_t, x, p_out_combined, g_out_combined, sum_W_p_out, sum_W_g_out, B_p_out_const, "
    "B_g_out_const, eps",
    "triangle_attn.triangle_attention": "X, W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, W_proj_g, B_proj_g, W_proj_o, "
    "B_proj_o, H, D, scale=1.0, eps=1e-05, mask=None",
    "triangle_attn.precompute": "W_ln, B_ln, WQ, WK, WV, W_proj_z, B_proj_z, H, D",
    "triangle_attn.forward": "X, pre, *, mask=None, scale=1.0, eps=1e-05, W_proj_g, B_proj_g, W_proj_o, B_proj_o, "
    "pad_to=32",
    "triangle_attn.triangle_attn_forward": "X_ln, WQ_c, WKV_c, WZ_c, BZ, out, scale=1.0, mask=None, Bias_buf=None, *, "
    "WK_c=None, WV_c=None",
    "triangle_attn.fused_gate_forward": "o_attn, qx_ln, WG, WO",
    "attn_pair_bias.attention_pair_bias": "X, WQ, WK, WV, Z, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, B_proj_g, "
    "W_proj_o, B_proj_o, H, D, scale=1.0, eps=1e-05",
    "attn_pair_bias.precompute": "WQ, WK, WV, W_ln, B_ln, W_proj_z, B_proj_z, H, D",
    "attn_pair_bias.forward": "X, Z, pre, *, scale=1.0, eps=1e-05, W_proj_g, B_proj_g, W_proj_o, B_proj_o",
    "attn_pair_bias.apb_forward": "X, W_QKV, Z, W_combined, sum_W_combined, B_const, Og, scale=1.0, eps=1e-05",
    # the qk-norm variant, stated by the reference only as a torch function
    # (benchmarks/references.py:230-250, `torch_attn_pair_bias_qknorm`)
    "attn_pair_bias.attention_pair_bias_qknorm": "X, WQ, b_q, WK, WV, Z, W_ln, B_ln, W_proj_z, B_proj_z, W_proj_g, "
    "W_proj_o, H, D, *, qkn_w_q=None, qkn_b_q=None, qkn_w_k=None, qkn_b_k=None, key_mask=None, scale=1.0, eps=1e-05",
}


def _parse(spec):
    out, kwonly = [], False
    for p in [s.strip() for s in spec.split(",")]:
        if p == "*":
            kwonly = True
            continue
        name, _, default = p.partition("=")
        out.append((name, default or None, kwonly))
    return out


@pytest.mark.parametrize("qual", sorted(REF_SIGNATURES))
def test_reference_signature_accepted(qual):
    """Every reference parameter exists with the same kind and default (extra optional ones allowed)."""
    mod, fn = qual.split(".")
    sig = inspect.signature(getattr(getattr(tops, mod), fn))
    params = list(sig.parameters.values())
    ref = _parse(REF_SIGNATURES[qual])
    pos = [p for p in params if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]
    ref_pos = [r for r in ref if not r[2]]
    assert [p.name for p in pos[: len(ref_pos)]] == [r[0] for r in ref_pos], qual
    for name, default, kwonly in ref:
        p = sig.parameters[name]
        assert (p.kind == p.KEYWORD_ONLY) == kwonly or not kwonly, (qual, name)
        if default is not None:
            assert repr(p.default) == default or str(p.default) == default, (qual, name, p.default)
        else:
            assert p.default is inspect.Parameter.empty, (qual, name)
    for p in params[len(ref):]:
        if p.name not in dict((r[0], r) for r in ref):
            assert p.default is not inspect.Parameter.empty, f"{qual}: extra parameter {p.name} must be optional"


def test_package_exports_match_reference():
    assert set(tops.__all__) == {"attn_pair_bias", "triangle_attn", "triangle_mul", "attention_pair_bias",
                                 "triangle_attention", "triangle_multiplicative_update"}
    assert tops.triangle_multiplicative_update is tops.triangle_mul.triangle_multiplicative_update
    assert tops.triangle_attention is tops.triangle_attn.triangle_attention
    assert tops.attention_pair_bias is tops.attn_pair_bias.attention_pair_bias


def test_triangle_ops_alias_package():
    import triangle_ops

    assert triangle_ops.triangle_multiplicative_update is tops.triangle_multiplicative_update
    assert triangle_ops.triangle_mul.forward is tops.triangle_mul.forward
    from triangle_ops.triangle_attn import triangle_attn_forward  # noqa: F401
    from triangle_ops._common import absorb_ln  # noqa: F401


def _w(C=128, dt=torch.bfloat16):
    g = torch.Generator().manual_seed(0)
    r = lambda *s: torch.randn(*s, generator=g).to(dt)  # noqa: E731
    return r


def test_precompute_dicts_cpu():
    r = _w()
    C, H, D = 128, 4, 32
    pre = tops.triangle_mul.precompute(r(C), r(C), r(2 * C, C), r(2 * C, C), r(C), r(C), r(C, C), r(C, C))
    assert set(pre) == {"p_in_combined", "g_in_combined", "p_out_combined", "g_out_combined", "sum_W_p_in",
                        "sum_W_g_in", "sum_W_p_out", "sum_W_g_out", "B_p_in_const", "B_g_in_const", "B_p_out_const",
                        "B_g_out_const"}
    assert pre["p_in_combined"].dtype == torch.bfloat16 and pre["sum_W_p_in"].dtype == torch.float32
    WQ, WK, WV, Wz = r(C, H * D), r(C, H * D), r(C, H * D), r(C, H)
    pre = tops.triangle_attn.precompute(r(C), r(C), WQ, WK, WV, Wz, None, H, D)
    for k in ("WQ_c", "WKV_c", "WK_c", "WV_c", "WZ_c", "BZ", "W_ln", "B_ln"):
        assert k in pre
    assert pre["WK_c"] is None and pre["WZ_c"].shape == (H, C) and torch.equal(pre["BZ"], torch.zeros(H))
    pre16 = tops.triangle_attn.precompute(r(64), r(64), r(64, 64), r(64, 64), r(64, 64), r(64, 4), r(4), 4, 16)
    assert pre16["WK_c"].data_ptr() != pre16["WKV_c"].data_ptr()
    pre = tops.attn_pair_bias.precompute(WQ, WK, WV, r(C), r(C), Wz, r(H), H, D)
    for k in ("W_QKV", "W_combined", "sum_W_combined", "B_const"):
        assert k in pre
    assert pre["W_QKV"].shape == (C, 3 * H * D)
    assert pre["W_combined"].shape == (H, C) and pre["W_combined"].dtype == torch.float32


def test_dtype_codes_and_errors():
    assert tl_io_dtype(torch.bfloat16) == 2 and tl_io_dtype(torch.float16) == 1 and tl_io_dtype(torch.float32) == 3
    with pytest.raises(ValueError):
        tl_io_dtype(torch.int32)


def test_bad_direction_and_bias_asserts():
    r = _w()
    C = 128
    pre = tops.triangle_mul.precompute(r(C), r(C), r(2 * C, C), r(2 * C, C), r(C), r(C), r(C, C), r(C, C))
    with pytest.raises(ValueError, match="unknown direction"):
        tops.triangle_mul.forward(r(1, 4, 4, C), pre, direction="sideways")
    with pytest.raises(AssertionError):
        tops.triangle_attn.forward(r(4, 4, C), {}, W_proj_g=r(C, C), B_proj_g=r(C), W_proj_o=r(C, C), B_proj_o=None)


def test_cpu_tensors_rejected():
    r = _w()
    C = 128
    pre = tops.triangle_mul.precompute(r(C), r(C), r(2 * C, C), r(2 * C, C), r(C), r(C), r(C, C), r(C, C))
    with pytest.raises(ValueError, match="GPU tensors"):
        tops.triangle_mul.forward(r(1, 4, 4, C), pre, direction="outgoing")


def test_unsupported_io_dtype_rejected_clearly():
    """float64 I/O raises the reference's ValueError (`_common/dtype.py:19`) before any launch;
    bf16, fp16 and fp32 are accepted."""
    r = _w(dt=torch.float64)
    M, C, H, D = 8, 128, 4, 32
    pre = tops.attn_pair_bias.precompute(r(C, H * D), r(C, H * D), r(C, H * D), r(C), r(C), r(C, H), None, H, D)
    with pytest.raises(ValueError, match="unsupported IO dtype"):
        tops.attn_pair_bias.forward(r(M, C), r(M, M, C), pre, W_proj_g=r(C, C), B_proj_g=None, W_proj_o=r(C, C),
                                    B_proj_o=None)
    pre = tops.triangle_mul.precompute(r(C), r(C), r(2 * C, C), r(2 * C, C), r(C), r(C), r(C, C), r(C, C))
    with pytest.raises(ValueError, match="unsupported IO dtype"):
        tops.triangle_mul.forward(r(1, 4, 4, C), pre, direction="outgoing")


def test_missing_library_fresh_process(tmp_path):
    code = ("import triangleops_amd._native as n\n"
            "try:\n    n.load('/nonexistent/libtriangleops_amd.so')\n"
            "except ImportError as e:\n    print('IMPORTERROR', e)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=ROOT, capture_output=True, text=True, timeout=120)
    assert "IMPORTERROR" in r.stdout and "python -m triangleops_amd._build" in r.stdout


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(tops_[a-z_0-9]+)\s*\(([^;]*?)\)\s*;", text, re.M)
    return {name: [a.strip() for a in args.split(",") if a.strip() and a.strip() != "void"] for name, args in decls}


def test_header_declares_all_bound_symbols():
    decl = _header_functions()
    assert set(decl) == set(_native.EXPORTED), set(decl) ^ set(_native.EXPORTED)
    for name, args in decl.items():
        n_bound = len(_native._SIGNATURES[name]) if name in _native._SIGNATURES else len(_native._OTHER[name][0])
        assert len(args) == n_bound, f"{name}: header has {len(args)} args, binding has {n_bound}"


@pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="HIP library not built")
def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_native.LIB_PATH)
    for name in _header_functions():
        assert hasattr(lib, name), name
    lib.tops_abi_version.restype = ctypes.c_int
    assert lib.tops_abi_version() == _native.ABI_VERSION


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "one GPU" in r.stderr


@pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="HIP library not built")
@pytest.mark.parametrize("N,ldn", [(100, 8192), (100, 64), (100, 192), (4096, 4160), (16385, 16448), (0, 0)])
def test_tri_abi_rejects_bad_ldn_and_n(N, ldn):
    """tops_tri_prep / tops_tri_attention accept only ldn = max(64, round_up(N, 64)) and N <= 16384
    (the attention kernel's per-row key-block tables in LDS hold that many blocks); anything else
    returns TOPS_EINVAL before any launch (the pointers below are never dereferenced)."""
    lib = _native.load()
    fake = ctypes.c_void_p(1 << 20)
    rc = lib.tops_tri_attention(fake, fake, fake, None, 0, 0, fake, 0, 0, N, ldn, 4, 32, 2, None)
    assert rc == 1, (N, ldn, rc)
    assert b"tops_tri_attention" in lib.tops_last_error()
    rc = lib.tops_tri_prep(fake, 0, 0, None, None, 0, fake, fake, None, fake, fake, fake, N, ldn, 128, 4, 32, 1e-5,
                           1.0, 2, None)
    assert rc == 1, (N, ldn, rc)


@pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="HIP library not built")
def test_tri_abi_shape_limits():
    """Shapes outside the tuned kernels return TOPS_EINVAL before any launch: the pre-pass takes
    C in {128, 64}, H = 4, D in {32, 16}; the attention D in {8, 16, 24, 32}; the gate C in {128, 64}
    (the pointers below are never dereferenced)."""
    lib = _native.load()
    f = ctypes.c_void_p(1 << 20)
    for C, H, D in ((96, 4, 32), (128, 8, 32), (128, 4, 24), (64, 4, 8), (256, 4, 32)):
        rc = lib.tops_tri_prep(f, 0, 0, None, None, 0, f, f, None, f, f, f, 64, 64, C, H, D, 1e-5, 1.0, 2, None)
        assert rc == 1 and b"tops_tri_prep: supports" in lib.tops_last_error(), (C, H, D)
    for D in (12, 40, 64):
        rc = lib.tops_tri_attention(f, f, f, None, 0, 0, f, 0, 0, 64, 64, 4, D, 2, None)
        assert rc == 1 and b"supports D in" in lib.tops_last_error(), D
    for C in (96, 32, 256):
        rc = lib.tops_gate_out(f, 0, 0, f, 0, 0, None, None, 1e-5, 0, f, None, f, None, f, 8, 8, C, 2, None)
        assert rc == 1 and b"C must be 128 or 64" in lib.tops_last_error(), C


@pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="HIP library not built")
def test_apb_abi_rejects_misaligned_z():
    """tops_apb_forward refuses Z token strides that are not multiples of 8 and misaligned bases (the
    kernel reads Z, X and the workspace with 16-byte loads)."""
    lib = _native.load()
    a = ctypes.c_void_p(1 << 20)
    for sz0, sz1, z in ((128 * 100 + 4, 128, 1 << 20), (128 * 100, 132, 1 << 20), (128 * 100, 128, (1 << 20) + 2)):
        rc = lib.tops_apb_forward(a, a, ctypes.c_void_p(z), sz0, sz1, a, a, a, None, a, a, 100, 128, 128, 4, 32,
                                  1.0, 1e-5, 2, None)
        assert rc == 1 and b"16-byte" in lib.tops_last_error(), (sz0, sz1, z)


@pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="HIP library not built")
def test_apb_noalloc_size_ranges_cpu():
    """The M that fit tops_apb_forward_noalloc's 16 MiB workspace on a 256-CU part (the count the
    library assumes without a GPU): every M up to 6990, and 8161..9039, 16353..21845, where the keys
    are split into fewer parts; the bounds the header states."""
    lib = _native.load()
    lim = 16 << 20
    for M, fits in ((6990, True), (6991, False), (8160, False), (8161, True), (9039, True), (9040, False),
                    (16352, False), (16353, True), (21845, True), (21846, False)):
        assert (lib.tops_apb_workspace_bytes(M, 4, 32) <= lim) == fits, M


def test_tri_dispatch_decision():
    """The tuned pre-pass and attention serve C_in in {128, 64}, H = 4, D in {32, 16} up to N = 16384
    (the Apo shape C_in = 64, D = 16 included); other shapes and larger N go to the any-shape
    pre-pass.  The tuned gate serves C_in = H*D = C_out in {128, 64}."""
    from triangleops_amd.triangle_attn.kernel import TUNED_MAX_N, fast_shape, gate_fast_shape

    assert TUNED_MAX_N == 16384
    assert fast_shape(128, 4, 32, 1024) and fast_shape(128, 4, 32, 16384) and fast_shape(64, 4, 16, 128)
    assert fast_shape(128, 4, 16, 128) and fast_shape(64, 4, 32, 128)
    assert not fast_shape(128, 4, 32, 16385) and not fast_shape(96, 4, 32, 128)
    assert not fast_shape(128, 8, 16, 128) and not fast_shape(128, 4, 8, 128)
    assert gate_fast_shape(128, 128, 128) and gate_fast_shape(64, 64, 64)
    assert not gate_fast_shape(128, 64, 128) and not gate_fast_shape(128, 128, 64)


def test_vec16_copies_misaligned_views():
    """A contiguous view whose base is off a 16-byte boundary is copied (`.contiguous()` alone would
    return it unchanged); aligned views with strides that are multiples of 8 are passed through."""
    base = torch.zeros(1024, dtype=torch.bfloat16)
    v = base[1:129].view(1, 128)
    assert v.is_contiguous() and v.data_ptr() % 16 != 0 and not _native.vec16_ok(v)
    c = _native.vec16(v)
    assert c.data_ptr() % 16 == 0 and torch.equal(c, v) and c.data_ptr() != v.data_ptr()
    x = torch.zeros(8, 8, 128, dtype=torch.bfloat16)
    t = x.transpose(0, 1)
    assert _native.vec16_ok(t) and _native.vec16(t).data_ptr() == t.data_ptr()


def test_dense_copies_strided_and_misaligned_views():
    """dense(): the tensors the kernels index without strides are made dense and 16-byte aligned.
    A column slice (row stride 256, unit last stride) passes vec16_ok but is not dense."""
    wide = torch.arange(64 * 256, dtype=torch.float32).reshape(64, 256).to(torch.bfloat16)
    s = wide[:, :128]
    assert _native.vec16_ok(s) and not s.is_contiguous()
    d = _native.dense(s)
    assert d.is_contiguous() and d.data_ptr() % 16 == 0 and torch.equal(d, s)
    flat = torch.zeros(1000, dtype=torch.bfloat16)
    mis = flat[1:129]
    assert mis.is_contiguous() and mis.data_ptr() % 16 != 0
    assert _native.dense(mis).data_ptr() % 16 == 0
    ok = torch.zeros(64, 128, dtype=torch.bfloat16)
    assert _native.dense(ok).data_ptr() == ok.data_ptr()
    f = _native.dense(ok, torch.float32)
    assert f.dtype == torch.float32 and f.is_contiguous()
    assert _native.dense(None) is None


@pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="HIP library not built")
def test_apb_noalloc_rejects_oversized_call_cpu():
    """tops_apb_forward_noalloc refuses a call whose workspace exceeds its 16 MiB static array before
    touching the GPU (M = 65536 needs 48 MiB of Q/K/V alone)."""
    lib = _native.load()
    assert lib.tops_apb_workspace_bytes(65536, 4, 32) > 16 << 20
    fake = ctypes.c_void_p(1 << 20)
    rc = lib.tops_apb_forward_noalloc(fake, fake, fake, 128 * 65536, 128, fake, fake, fake, None, fake, 65536, 128, 128,
                                      4, 32, 1.0, 1e-5, 2, None)
    assert rc == 1 and b"static workspace" in lib.tops_last_error()
