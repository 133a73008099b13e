"""tops_apb_forward_noalloc (the allocation-free variant of tops_apb_forward) through the C ABI:
its output equals tops_apb_forward's bit for bit on two calls in a row, the second with a smaller
M (so the library's static workspace still holds the first call's contents), with a key mask and
with the split-key combine active at both sizes.  (Its refusal of workspaces past the static array
is a host-side check, tested on the CPU in test_host.py.)"""

import pytest
import torch
from _inputs import apb_inputs, to_dev

import triangleops_amd as tops
from triangleops_amd import _native
from triangleops_amd._common.dtype import io_dtype_code

pytestmark = pytest.mark.gpu


def _args(d, pre, M):
    X = _native.dense(d["X"])
    Z = _native.vec16(d["Z"])
    wqkv = pre["wqkv_hm"].to(X.dtype).contiguous()
    Wc = pre["W_combined"].float().contiguous()
    sWc = pre["sum_W_combined"].float().contiguous()
    Bc = pre["B_const"].float().contiguous()
    m8 = _native.mask_i8(d["mask"])
    keep = (X, Z, wqkv, Wc, sWc, Bc, m8)
    head = [X.data_ptr(), wqkv.data_ptr(), Z.data_ptr(), Z.stride(0), Z.stride(1), Wc.data_ptr(), sWc.data_ptr(),
            Bc.data_ptr(), _native.ptr(m8)]
    tail = [M, 128, 128, 4, 32, float(d["scale"]), 1e-5, io_dtype_code(X.dtype), _native.stream_of(X)]
    return keep, head, tail


def _both(device, M, seed):
    d = to_dev(apb_inputs(M, seed=seed, mask="random", biases=True), device)
    pre = tops.attn_pair_bias.precompute(d["WQ"], d["WK"], d["WV"], d["W_ln"], d["B_ln"], d["W_proj_z"],
                                         d["B_proj_z"], 4, 32)
    keep, head, tail = _args(d, pre, M)
    og_ref = torch.empty(M, 128, device=device, dtype=torch.bfloat16)
    work = torch.empty(max(_native.apb_workspace_bytes(M, 4, 32), 1), device=device, dtype=torch.uint8)
    _native.call("tops_apb_forward", *head, og_ref.data_ptr(), work.data_ptr(), *tail)
    og = torch.full((M, 128), float("nan"), device=device, dtype=torch.bfloat16)
    _native.call("tops_apb_forward_noalloc", *head, og.data_ptr(), *tail)
    torch.cuda.synchronize()
    del keep
    return og_ref, og


def test_apb_noalloc_matches_workspace_entry_point(device):
    for M, seed in ((1024, 3), (200, 4)):
        ref, out = _both(device, M, seed)
        assert torch.isfinite(out.float()).all(), f"M={M}: non-finite output"
        assert torch.equal(out, ref), f"M={M}: the no-alloc entry point differs from tops_apb_forward"

