"""CPU model of tri_attn2_kernel's memory accesses (the two-row triangle-attention kernel in
triangleops_amd/csrc/tri.hip), checked before the kernel runs on a GPU.

The model restates the kernel's index arithmetic in numpy -- block -> (head, row pair, query
chunk) with the XCD remap, the key-validity pass, the union visit list, every global load (Q,
mask, bias, the K / V^T copies and their clamped tails), every LDS access (copy destinations,
operand reads, the validity tables) and every output store -- and checks each address against
its buffer for 18 sizes N with pad and random masks.  It also replays one block's copy on
symbolic data: every LDS chunk of a slot is written exactly once, and the swizzled operand reads
return the K row / V^T row chunk the MFMA layout asks for.
"""

import os

import numpy as np
import pytest

KV_BLOCK = 4096  # elements of one (row, head, 64-key) KV block: K 64 x 32, then V^T 32 x 64
MAX_KB = 256  # kMaxN / 64 (per-row key-block tables in LDS)
D, NW, RING = 32, 4, 4
ESZ = 2  # bf16
SLOT_BYTES = 2 * 2 * KV_BLOCK  # one slot: 2 rows x 8 KB
SIZES = [1, 2, 31, 32, 33, 63, 64, 65, 100, 127, 129, 200, 255, 257, 520, 1000, 1025, 2048]


def ldn_of(n):
    return 64 if n <= 64 else (n + 63) // 64 * 64


def masks(n, kind, seed=0):
    if kind == "pad":
        v = n - n // 10
        i = np.arange(n)
        return (i[:, None] < v) & (i[None, :] < v)
    rng = np.random.default_rng(seed + n)
    m = rng.random((n, n)) < 0.8
    if n > 3:
        m[n // 2] = False  # a row without valid keys
    return m


def lane_ids():
    tid = np.arange(256)
    return tid, tid & 63, tid >> 6


def copy_offsets():
    """gofs[s][lane] (bytes) of the kernel's copy, for cpart 0 (K) and 1 (V^T)."""
    lane = np.arange(64)
    out = {}
    for cpart in (0, 1):
        g = []
        for s in range(4):
            p = 64 * s + lane
            if cpart == 0:
                c = (p & ~3) | ((p & 3) ^ ((p >> 4) & 3))
            else:
                c = (p & ~7) | ((p & 7) ^ ((p >> 4) & 7))
            g.append(16 * c)
        out[cpart] = np.stack(g)
    return out


def test_copy_swizzle_round_trip():
    """Each slot chunk is written once per block copy, and read_k / read_v return the requested
    (row, chunk) of K (64 B rows) and V^T (128 B rows)."""
    gofs = copy_offsets()
    lane = np.arange(64)
    for cpart in (0, 1):
        # LDS chunk 64 s + lane of part cpart receives global chunk gofs / 16
        lds = np.full(256, -1)
        for s in range(4):
            pos = 64 * s + lane
            assert (lds[pos] == -1).all()
            lds[pos] = gofs[cpart][s] // 16
        assert sorted(lds) == list(range(256)), "copy is not a permutation of the part's chunks"
        hl, col = lane >> 5, lane & 31
        if cpart == 0:  # K: row key = 32 kt + col, logical chunk 2 j + hl at (c ^ ((key >> 2) & 3))
            for kt in range(2):
                key = 32 * kt + col
                for j in range(2):
                    c = 2 * j + hl
                    pos = key * 4 + (c ^ ((key >> 2) & 3))
                    assert (lds[pos] == key * 4 + c).all()
        else:  # V^T: row d = col, logical chunk 4 kt + 2 j + hl at (c ^ ((d >> 1) & 7))
            for kt in range(2):
                for j in range(2):
                    c = 4 * kt + 2 * j + hl
                    pos = col * 8 + (c ^ ((col >> 1) & 7))
                    assert (lds[pos] == col * 8 + c).all()


def test_lds_accesses_in_bounds():
    """Copy destinations (M0 + 1024 s + 16 lane in the wave's quarter of a slot) and operand reads
    stay inside their slot; validity-table indices stay below kMaxKB for N <= 16384."""
    tid, lane, wave = lane_ids()
    crow, cpart = wave >> 1, wave & 1
    for s in range(4):
        dst = crow * 2 * KV_BLOCK + cpart * 4096 + 1024 * s + 16 * lane
        assert dst.min() >= 0 and (dst + 16).max() <= SLOT_BYTES
    hl, col = lane >> 5, lane & 31
    for r in range(2):
        for kt in range(2):
            key = 32 * kt + col
            for j in range(2):
                a = r * 2 * KV_BLOCK + key * 64 + (((2 * j + hl) ^ ((key >> 2) & 3)) << 4)
                assert a.min() >= 0 and (a + 16).max() <= SLOT_BYTES
                b = r * 2 * KV_BLOCK + 4096 + col * 128 + (((4 * kt + 2 * j + hl) ^ ((col >> 1) & 7)) << 4)
                assert b.min() >= 0 and (b + 16).max() <= SLOT_BYTES
    assert ldn_of(16384) // 64 <= MAX_KB


def _pair_blocks(N, m):
    """Per row pair (i0, i1 = min(i0 + 1, N - 1)): the first and last visited key block and the
    number of visits (union of the two rows' blocks with a valid key; a row without valid keys
    visits every block with keys < N)."""
    ldn = ldn_of(N)
    nkb = ldn // 64
    mp = np.zeros((N, nkb * 64), dtype=bool)
    mp[:, :N] = m
    has = mp.reshape(N, nkb, 64).any(-1)  # (row, kb): a valid key in the block
    uniform = ~has.any(-1)
    allk = np.arange(nkb) * 64 < N
    vis_row = np.where(uniform[:, None], allk[None, :], has)
    nrp = (N + 1) // 2
    i0 = 2 * np.arange(nrp)
    i1 = np.minimum(i0 + 1, N - 1)
    vis = vis_row[i0] | vis_row[i1]
    nv = vis.sum(-1)
    kb_idx = np.arange(nkb)
    kb_min = np.where(vis, kb_idx, nkb).min(-1)
    kb_max = np.where(vis, kb_idx, -1).max(-1)
    return nv, kb_min, kb_max


@pytest.mark.parametrize("N", SIZES)
@pytest.mark.parametrize("kind", ["pad", "random"])
def test_global_accesses_in_bounds(N, kind):
    """Every global address of every block and lane lies in its buffer (extremes over lanes taken
    exactly: each address is a block term plus a lane term that does not depend on the block)."""
    H = 4
    ldn = ldn_of(N)
    nkb, nkt, nqt = ldn // 64, ldn // 32, (N + 31) // 32
    nqc, nrp = (N + 127) // 128, (N + 1) // 2
    total = H * nrp * nqc
    m = masks(N, kind)
    n_qp = N * H * ldn * D  # elements (bf16)
    n_kv = N * H * nkb * KV_BLOCK
    n_bias = H * nqt * nkt * 1024
    n_out = N * N * H * D
    so0, so1 = N * H * D, H * D
    # block -> (qc, rp, h): the XCD remap is a permutation of the block ids
    bid = np.arange(total)
    idx = (bid % 8) * (total // 8) + bid // 8 if total % 8 == 0 else bid
    assert np.array_equal(np.sort(idx), bid)
    qc, rp, h = idx % nqc, (idx // nqc) % nrp, idx // (nqc * nrp)
    i0, i1v = 2 * rp, 2 * rp + 1
    i1 = np.minimum(i1v, N - 1)
    assert (h < H).all() and (i1 < N).all()
    nv, kb_min, kb_max = _pair_blocks(N, m)
    nv, kb_min, kb_max = nv[rp], kb_min[rp], kb_max[rp]
    assert (nv >= 1).all() and (kb_min >= 0).all() and (kb_max < min(nkb, MAX_KB)).all()
    # lane terms (extremes over the 256 threads)
    qt_max = 4 * qc + 3  # wave 3
    q_max = np.minimum(32 * qt_max + 31, N - 1)
    for i in (i0, i1):
        # mask loads of the validity pass: row i, keys k < N
        assert (i * N + N - 1 < N * N).all()
        # Q operands: two 16-byte loads at d offsets 8 hl and 8 hl + 16
        assert (((i * H + h) * ldn + q_max) * D + 8 + 16 + 8 <= n_qp).all()
        # K / V^T rows read by the exact-max recomputation and the uniform rows
        off = (i * H + h) * nkb * KV_BLOCK
        assert (off + kb_max * KV_BLOCK + 64 * D + 31 * 64 + 32 + 8 + 16 + 8 <= n_kv).all()
        assert (off + kb_max * KV_BLOCK + (32 + 31) * D + 8 + 16 + 8 <= n_kv).all()
    # bias operands: tile (min(qt, nqt - 1), 2 kb + kt), lane term (32 hl + col) 8 <= 504, halves +512
    qtc_max = np.minimum(qt_max, nqt - 1)
    assert ((h * nqt + qtc_max) * nkt * 1024 + (2 * kb_max + 1) * 1024 + 504 + 512 + 8 <= n_bias).all()
    assert (2 * kb_max + 1 < nkt).all()
    # copies: (row w >> 1, part w & 1) of the (row, head, block) KV block, lane term gofs <= 4080
    gofs = copy_offsets()
    gmax = max(gofs[0].max(), gofs[1].max())
    assert gmax + 16 <= 4096 and min(gofs[0].min(), gofs[1].min()) >= 0
    for row in (i0, i1):
        base = (row * H + h) * nkb * KV_BLOCK
        assert ((base + kb_max * KV_BLOCK + 2048) * ESZ + gmax + 16 <= n_kv * ESZ).all()
        assert (base >= 0).all()
    # output stores: rows i0 and (when inside the grid) i1, queries q < N, 4 stores of 8 bytes
    for i, live in ((i0, np.ones_like(i0, dtype=bool)), (i1, i1v < N)):
        qo_max = np.minimum(32 * qt_max + 31, N - 1)
        ok = live & (32 * (4 * qc) < N)
        a = i * so0 + qo_max * so1 + h * D + 4 + 8 * 3 + 4
        assert (a[ok] <= n_out).all()
    # every (row, query, head) of the output is written by exactly one (block, lane)
    cover = np.zeros((nrp * 2, nqc * 128, H), dtype=np.int64)
    rows = np.concatenate([2 * rp, 2 * rp + 1])
    qcs = np.concatenate([qc, qc])
    hs = np.concatenate([h, h])
    np.add.at(cover, (rows[:, None], qcs[:, None] * 128 + np.arange(128)[None, :], hs[:, None]), 1)
    assert (cover[:N, :N] == 1).all()


def _hipcc():
    import shutil

    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_two_row_copy_asm_hazards(tmp_path):
    """The two-row kernel's inline-asm loads, in the gfx950 assembly the build produces: every
    global_load_lds takes a 64-bit per-lane VGPR address (no SGPR base, so no VALU-written SGPR is
    read by the load) and sits right behind an `s_nop 4` or longer (the M0 write that precedes it
    gets at least 5 wait states); and no register a bias load writes is read before the next
    vmcnt wait (no copy of an in-flight load)."""
    import re
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = os.path.join(root, "triangleops_amd", "csrc", "tri.hip")
    asm = tmp_path / "tri.s"
    cmd = [_hipcc(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", str(asm), src]
    subprocess.run(cmd, check=True, capture_output=True)
    text = asm.read_text()
    m = re.search(r"\n(_ZN4tops16tri_attn2_kernel\w*):(.*?)s_endpgm", text, re.S)
    assert m, "tri_attn2_kernel not found in the assembly"
    body = [ln.strip() for ln in m.group(2).splitlines()
            if ln.strip() and not ln.strip().startswith((";", "."))]
    ndma = 0
    pending = set()
    for idx, ln in enumerate(body):
        op = ln.split()[0]
        if op == "global_load_lds_dwordx4":
            ndma += 1
            assert re.search(r"v\[\d+:\d+\], off$", ln), f"copy without a VGPR address: {ln}"
            prev = body[idx - 1]
            assert re.match(r"s_nop ([4-9]|1[0-5])$", prev), f"copy not behind s_nop >= 4: {prev} / {ln}"
            continue
        if op.startswith("s_waitcnt") and "vmcnt" in ln:
            pending.clear()
            continue
        if pending and " " in ln:
            for part in ln.split(None, 1)[1].split(",")[1:]:
                for mm in re.finditer(r"v\[(\d+):(\d+)\]|v(\d+)\b", part):
                    regs = range(int(mm.group(1)), int(mm.group(2)) + 1) if mm.group(1) else [int(mm.group(3))]
                    assert not (set(regs) & pending), f"in-flight load register read early: {ln}"
        if op == "global_load_dwordx4":
            mm = re.match(r"global_load_dwordx4 v\[(\d+):(\d+)\]", ln)
            pending.update(range(int(mm.group(1)), int(mm.group(2)) + 1))
    assert ndma >= 8
