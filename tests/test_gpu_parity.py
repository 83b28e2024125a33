"""GPU parity of the HIP LUT-GEMV path against the CPU oracle and the
reference's golden vectors, through the C ABI.

Bars (north star): bit-exact for plane packing, table build, FWHT-256 and
index generation; outputs within max |y - y_ref| <= 1e-5 * ||y_ref||_2
(fp32 accumulation-order differences only).
"""
import numpy as np
import pytest
import torch

import lutmac_amd as L
import oracle
from conftest import TOL, load_golden, rel_max_err
from lutmac_amd import synth

pytestmark = pytest.mark.gpu

FORMAT_FILES = {1: "ternary", 2: "binary", 3: "int2", 5: "int3", 6: "int4", 7: "int8"}
ZERO_CODE_PLANE = {1: 1, 5: 2, 6: 3}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def oracle_planes_gemv(fmt, planes, scales, rows, cols, group, x, rotate):
    """Oracle over the same padded weight the device holds (pad codes in the
    columns past `cols`, zero scales for groups past the source's)."""
    Kp = -(-cols // 256) * 256
    P, S = L.PLANES[fmt], L.STAGES[fmt]
    padded = np.zeros((P, rows, Kp // 8), np.uint8)
    if fmt in ZERO_CODE_PLANE:
        padded[ZERO_CODE_PLANE[fmt]] = 0xFF
    padded[:, :, :cols // 8] = planes.reshape(P, rows, cols // 8)
    G = group or Kp
    ng = Kp // G
    sc = np.zeros((S, rows, ng), np.float32)
    src = scales.reshape(S, rows, -1)
    sc[:, :, :src.shape[2]] = src[:, :, :ng]
    xp = np.zeros(Kp, np.float32)
    xp[:cols] = x
    if rotate == L.ROTATE_FWHT256:
        xp = oracle.fwht256(xp)
    elif rotate == L.ROTATE_FWHT_FULL:
        xp = oracle.fwht_full(xp)
    return oracle.planes_gemv(fmt, padded, sc, rows, Kp, G, xp)


# ---- bit-exact primitives -----------------------------------------------------

def test_fwht256_bitexact(cuda):
    g = load_golden("tables_fwht.npz")
    x = dev(g["x"])
    L.fwht256(x)
    torch.cuda.synchronize()
    assert np.array_equal(x.cpu().numpy().view(np.uint32), g["x_rot"].view(np.uint32))
    big = synth.make_activations(8192 * 4, seed=1)
    xb = dev(big)
    L.fwht256(xb)
    assert np.array_equal(xb.cpu().numpy().view(np.uint32), oracle.fwht256(big).view(np.uint32))


def test_precompute_luts_bitexact(cuda):
    g = load_golden("tables_fwht.npz")
    t = L.precompute_luts(dev(g["x"]))
    assert np.array_equal(t.cpu().numpy().view(np.uint32), g["luts"].view(np.uint32))
    t = L.precompute_luts(dev(g["x"]), rotate=True)   # the GEMV's fused FWHT + table path
    assert np.array_equal(t.cpu().numpy().view(np.uint32), g["luts_rot"].view(np.uint32))
    x = synth.make_activations(8192, seed=2, outliers=True)
    t = L.precompute_luts(dev(x), rotate=True)
    assert np.array_equal(t.cpu().numpy().view(np.uint32),
                          oracle.precompute_luts(oracle.fwht256(x)).view(np.uint32))
    x = np.array([1, 2, 3, 4, 5, 6], np.float32)     # ragged: whole groups only
    t = L.precompute_luts(dev(x))
    assert t.cpu().numpy().tolist() == [0, 4, 3, 7, 2, 6, 5, 9, 1, 5, 4, 8, 3, 7, 6, 10]


def test_extract_indices_bitexact(cuda):
    g = load_golden("indices.npz")
    pos, neg = L.extract_indices(dev(g["sign"]), dev(g["zero"]), 256)
    assert np.array_equal(pos.cpu().numpy(), g["pos"])
    assert np.array_equal(neg.cpu().numpy(), g["neg"])
    s = np.array([0b01000000, 0], np.uint8)
    z = np.array([0b00100000, 0], np.uint8)
    pos, neg = L.extract_indices(dev(s), dev(z), 1)
    assert (int(pos[0]), int(neg[0])) == (0b1001, 0b0100)     # test_lut_gemm.cpp:57-88


@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_device_tiles_bitexact(cuda, fmt):
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    w = L.Weight.from_blocks(fmt, g["blocks"], M, K)
    planes, _ = L.blocks_to_planes(fmt, g["blocks"], M, K)
    Kp = -(-K // 256) * 256
    assert np.array_equal(w.read_tiles(), L.tile_planes(fmt, planes, M, Kp))
    assert np.array_equal(L.planes_to_blocks(fmt, L.untile_planes(fmt, w.read_tiles(), M, Kp),
                                             L.blocks_to_planes(fmt, g["blocks"], M, K)[1], M, K),
                          g["blocks"])


# ---- GEMV parity ----------------------------------------------------------------

@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_linear_reference_blocks_golden(cuda, fmt):
    """lut_linear on the reference's own quantized blocks (bias, batch 2)
    against the reference's outputs."""
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    w = L.Weight.from_blocks(fmt, g["blocks"], M, K)
    y = w.linear(dev(g["x"]), bias=dev(g["bias"])).cpu().numpy()
    for b in range(2):
        assert rel_max_err(y[b * M:(b + 1) * M], g["y"][b * M:(b + 1) * M]) < TOL
    y0 = w.linear(dev(g["x"])).cpu().numpy()
    assert rel_max_err(y0[:M], g["y_nobias"][:M]) < TOL


@pytest.mark.parametrize("fmt", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("group", [0, 128, 256])
@pytest.mark.parametrize("rows,cols", [(300, 640), (64, 2048), (1, 8), (513, 1536)])
@pytest.mark.parametrize("rotate", [L.ROTATE_NONE, L.ROTATE_FWHT256])
def test_gemv_formats(cuda, fmt, group, rows, cols, rotate):
    planes, scales, _ = synth.make_weights(fmt, rows, cols, seed=rows + cols + fmt, group=group or 128)
    if group == 0:
        scales = np.ascontiguousarray(scales[:, :, :1])
    x = synth.make_activations(cols, seed=cols, outliers=True)
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, group)
    y = w.gemv(dev(x), flags=rotate).cpu().numpy()
    ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, group, x, rotate)
    assert rel_max_err(y, ref) < TOL


def test_config1_int4_2048(cuda):
    planes, scales, g = synth.make_weights(L.FMT_INT4, 2048, 2048, seed=1)
    x = synth.make_activations(2048, seed=101)
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, 2048, 2048, g)
    y = w.gemv(dev(x)).cpu().numpy()
    assert rel_max_err(y, oracle.planes_gemv(6, planes, scales, 2048, 2048, g, x)) < TOL
    W = synth.dequant_f64(6, planes, scales, 2048, 2048, g)
    assert rel_max_err(y, W @ x.astype(np.float64)) < TOL


@pytest.mark.parametrize("name", sorted(synth.LLAMA_TERNARY_SHAPES))
@pytest.mark.parametrize("rotate", [L.ROTATE_FWHT256, L.ROTATE_FWHT_FULL])
def test_config2_ternary_shapes(cuda, name, rotate):
    rows, cols = synth.LLAMA_TERNARY_SHAPES[name]
    planes, scales, g = synth.make_weights(L.FMT_TERNARY, rows, cols, seed=rows * 7 + cols, group=0)
    x = synth.make_activations(cols, seed=cols + 5, outliers=True)
    w = L.Weight.from_planes(L.FMT_TERNARY, planes, scales, rows, cols, 0)
    y = w.gemv(dev(x), flags=rotate).cpu().numpy()
    assert rel_max_err(y, oracle_planes_gemv(1, planes, scales, rows, cols, 0, x, rotate)) < TOL


@pytest.mark.parametrize("fmt", [L.FMT_BINARY, L.FMT_TERNARY, L.FMT_RRQ2, L.FMT_RRQ3, L.FMT_INT4, L.FMT_INT8])
def test_config3_8192(cuda, fmt):
    n = 8192
    planes, scales, g = synth.make_weights(fmt, n, n, seed=30 + fmt, group=128)
    x = synth.make_activations(n, seed=31)
    w = L.Weight.from_planes(fmt, planes, scales, n, n, g)
    xd = dev(x)
    y = w.gemv(xd, flags=L.ROTATE_FWHT256).cpu().numpy()
    assert rel_max_err(y, oracle.planes_gemv(fmt, planes, scales, n, n, g, oracle.fwht256(x))) < TOL
    # size-independent properties at the full shape
    y2 = w.gemv(xd, flags=L.ROTATE_FWHT256).cpu().numpy()
    assert np.array_equal(y.view(np.uint32), y2.view(np.uint32))          # deterministic split-K
    x2 = synth.make_activations(n, seed=32)
    ya = w.gemv(dev(2.0 * x - 3.0 * x2), flags=L.ROTATE_FWHT256).cpu().numpy()
    yb = w.gemv(dev(x2), flags=L.ROTATE_FWHT256).cpu().numpy()
    assert rel_max_err(ya, 2.0 * y.astype(np.float64) - 3.0 * yb) < 1e-5 * 4  # linearity
    assert not w.gemv(torch.zeros(n, device="cuda"), flags=L.ROTATE_FWHT256).any()
    # the bench's 4/8-bit workload: input rotated once on the device, kernel unrotated
    if fmt in (L.FMT_INT4, L.FMT_INT8):
        xr = dev(x)
        L.fwht256(xr)
        yr = w.gemv(xr, flags=L.ROTATE_NONE).cpu().numpy()
        assert rel_max_err(yr, oracle.planes_gemv(fmt, planes, scales, n, n, g, oracle.fwht256(x))) < TOL


def test_batch_rows_independent(cuda):
    rows, cols, B = 700, 1024, 3
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=77)
    xs = np.stack([synth.make_activations(cols, seed=s) for s in range(B)])
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, g)
    y = w.gemv(dev(xs.ravel())).cpu().numpy().reshape(B, rows)
    for b in range(B):
        assert rel_max_err(y[b], oracle.planes_gemv(6, planes, scales, rows, cols, g, xs[b])) < TOL


def test_qwen_ffn_shape(cuda):
    # K = 8960 (35 x 256): the k-slice must divide the padded K.
    rows, cols = 1536, 8960
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=88)
    x = synth.make_activations(cols, seed=89)
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, g)
    y = w.gemv(dev(x)).cpu().numpy()
    assert rel_max_err(y, oracle.planes_gemv(6, planes, scales, rows, cols, g, x)) < TOL


def test_gemv_rejects_bad_arguments(cuda):
    planes, scales, g = synth.make_weights(L.FMT_INT4, 64, 256, seed=3)
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, 64, 256, g)
    x = torch.zeros(256, device="cuda")
    with pytest.raises(L.LmxError) as e:
        w.gemv(x, flags=7)
    assert e.value.status == L.ERR_INVALID_ARGUMENT
    w2 = L.Weight.from_planes(L.FMT_INT4, *synth.make_weights(L.FMT_INT4, 8, 768, seed=4)[:2], 8, 768, 128)
    with pytest.raises(L.LmxError):
        w2.gemv(torch.zeros(768, device="cuda"), flags=L.ROTATE_FWHT_FULL)   # 768 not a power of 2


# ---- every kernel plan, forced ---------------------------------------------
# (full-K configuration, rows, cols): shapes each configuration covers.
PLAN_SHAPES = {
    0: (300, 2560),   # split-K kernel
    1: (96, 8192),    # 16 waves x 2 slices x 2 chunks
    2: (96, 9216),    # 16 x 2 x 3 (planes <= 2 only)
    3: (70, 2048),    # 8 x 2 x 1
    4: (130, 1536),   # 16 x 1 x 1
    5: (40, 8192),    # 16 x 4 x 1
    6: (33, 2048),    # 4 x 4 x 1
    7: (44, 7936),    # 8 x 8 x 1 (a ragged last workgroup, 62 of 64 slices used)
    8: (40, 8960),    # 8 x 8 x 2 layered (70 chunks on 64 slices; 4-bit, lean kernel only)
}


# family: 0 auto (interleaved where it applies, else lean, else generic),
# 1 the generic full-K kernel, 2 the lean one; staged only affects the generic.
@pytest.mark.parametrize("fmt", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("cfg", sorted(PLAN_SHAPES))
@pytest.mark.parametrize("staged,family", [(0, 1), (1, 1), (1, 0), (1, 2)])
def test_forced_kernel_plans(cuda, monkeypatch, fmt, cfg, staged, family):
    rows, cols = PLAN_SHAPES[cfg]
    monkeypatch.setenv("LMX_FULLK", str(cfg))
    monkeypatch.setenv("LMX_STAGED", str(staged))
    monkeypatch.setenv("LMX_KERNEL", str(family))
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=cfg * 10 + fmt, group=128)
    x = synth.make_activations(cols, seed=cfg + 40, outliers=True)
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, g)
    used, _, st = w.kernel_config()
    cps = {1: 2, 2: 3}.get(cfg, 1)
    fits = cfg == 0 or L.PLANES[fmt] * cps <= 8 or (cfg == 1 and family == 0 and L.PLANES[fmt] * cps <= 16)
    if cfg == 8:
        fits = fmt == L.FMT_INT4 and family != 1
    assert used == (cfg if fits else 0) and st == staged
    y = w.gemv(dev(x), flags=L.ROTATE_FWHT256).cpu().numpy()
    ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, x, L.ROTATE_FWHT256)
    assert rel_max_err(y, ref) < TOL


# The 4 x 4 x 1, 16 x 4 x 1 and layered plans of an unrotated 4-bit GEMV
# split each chunk's four planes over two lanes (LMX_PS=1, the default; 2
# splits only the 4 x 4 x 1 plan, 0 neither): every form against the oracle,
# ragged and full workgroups.  (K > 2048 with at most 2048 rows: 16 x 4 x 1
# at 8 rows per workgroup when it splits, else the 8 x 8 x 1 plan; K = 8960:
# the layered plan, launched as 16 waves x 4 slices x 2 chunks when split.)
@pytest.mark.parametrize("ps", ["0", "1", "2"])
@pytest.mark.parametrize("rows,cols", [(33, 2048), (300, 640), (2048, 2048), (3072, 2048), (1536, 1536),
                                       (2048, 8192), (300, 4096), (45, 7936), (1536, 8960), (40, 8960)])
def test_int4_plane_split(cuda, monkeypatch, ps, rows, cols):
    monkeypatch.setenv("LMX_PS", ps)
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=rows + cols, group=128)
    x = synth.make_activations(cols, seed=7, outliers=True)
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, g)
    want_plan = 6 if cols <= 2048 else 8 if cols > 8192 else (5 if ps == "1" else 7)
    assert w.kernel_config()[0] == want_plan
    y = w.gemv(dev(x), flags=L.ROTATE_NONE).cpu().numpy()
    ref = oracle_planes_gemv(L.FMT_INT4, planes, scales, rows, cols, g, x, L.ROTATE_NONE)
    assert rel_max_err(y, ref) < TOL
    w.close()


# ---- split-K reductions: last-workgroup ticket and two-pass ----------------
@pytest.mark.parametrize("reduce", [0, 2])
@pytest.mark.parametrize("kslice", [256, 512])
@pytest.mark.parametrize("fmt", [1, 6, 7])
def test_splitk_reductions(cuda, monkeypatch, reduce, kslice, fmt):
    import torch
    rows, cols = 1000, 4096
    monkeypatch.setenv("LMX_FULLK", "0")
    monkeypatch.setenv("LMX_REDUCE", str(reduce))
    monkeypatch.setenv("LMX_KSLICE", str(kslice))
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=60 + fmt, group=128)
    x = synth.make_activations(cols, seed=61, outliers=True)
    bias = np.random.default_rng(62).standard_normal(rows).astype(np.float32)
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, g)
    assert w.kernel_config()[:2] == (0, kslice)
    ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, x, L.ROTATE_FWHT256)
    xd, bd = dev(x), dev(bias)
    y1 = w.gemv(xd, flags=L.ROTATE_FWHT256).cpu().numpy()
    y2 = w.gemv(xd, flags=L.ROTATE_FWHT256).cpu().numpy()     # counters were reset by call 1
    assert rel_max_err(y1, ref) < TOL
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    # graph replays, with eager calls on the same handle in between
    out = torch.empty(rows, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w.gemv(xd, y=out, flags=L.ROTATE_FWHT256)             # warm up off the capture
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        w.gemv(xd, y=out, flags=L.ROTATE_FWHT256)
    for _ in range(3):
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), y1.view(np.uint32))
        w.gemv(xd, flags=L.ROTATE_FWHT256)
        torch.cuda.synchronize()
    yb = w.linear(xd, bias=bd).cpu().numpy()                  # lmx_linear rotates 1-2 bit formats only
    refb = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, x,
                              L.ROTATE_FWHT256 if fmt in (1, 2, 3, 4) else L.ROTATE_NONE) + bias
    assert rel_max_err(yb, refb) < TOL


# ---- batched GEMV (weights read once per group of 2/4/8/16 vectors) ----------
@pytest.mark.parametrize("fmt", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("batch", [4, 7, 8, 16, 21])
@pytest.mark.parametrize("rows,cols", [(300, 640), (513, 1536)])
def test_batched_gemv(cuda, fmt, batch, rows, cols):
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=fmt * 100 + batch, group=128)
    xs = np.stack([synth.make_activations(cols, seed=1000 + s, outliers=True) for s in range(batch)])
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, g)
    y = w.gemv(dev(xs.ravel()), flags=L.ROTATE_FWHT256).cpu().numpy().reshape(batch, rows)
    for b in range(batch):
        ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, xs[b], L.ROTATE_FWHT256)
        assert rel_max_err(y[b], ref) < TOL, f"vector {b}"


# Unrotated 4-bit groups of 8 and 16 vectors, and groups of 4 the
# four-vector kernel does not take (K past 2048 here), run on the matrix
# cores (LMX_MFMA=1, the default: 8 waves per workgroup, the codes from the
# handle's nibble copy; 2: two row tiles per wave; 3: the codes from the
# planes; 4: four waves; 0 the
# lookup-table kernel): 128- and 256-wide
# k-slices, K past the last whole 256 (640), group scales of 128 and 256
# and one per row, a last group of fewer vectors (9, 21), against the oracle.
@pytest.mark.parametrize("mfma", ["1", "2", "3", "4", "0"])
@pytest.mark.parametrize("group", [128, 256, 0])
@pytest.mark.parametrize("batch", [8, 16, 9, 21, 4, 12])
@pytest.mark.parametrize("rows,cols", [(300, 640), (513, 1536), (2048, 2048), (4160, 4096)])
def test_batched_int4_matrix_cores(cuda, monkeypatch, mfma, group, batch, rows, cols):
    monkeypatch.setenv("LMX_MFMA", mfma)
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=batch * 31 + rows, group=group or 128)
    if group == 0:
        scales = np.ascontiguousarray(scales[:, :, :1])
    xs = np.stack([synth.make_activations(cols, seed=3000 + s, outliers=True) for s in range(batch)])
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, group)
    y = w.gemv(dev(xs.ravel()), flags=L.ROTATE_NONE).cpu().numpy().reshape(batch, rows)
    for b in range(batch):
        ref = oracle_planes_gemv(L.FMT_INT4, planes, scales, rows, cols, group, xs[b], L.ROTATE_NONE)
        assert rel_max_err(y[b], ref) < TOL, f"vector {b}"
    w.close()


@pytest.mark.parametrize("fmt", [1, 3, 5, 6])
@pytest.mark.parametrize("batch", [7, 8, 16])
@pytest.mark.parametrize("rows,cols", [(4160, 4096), (2112, 4096)])
def test_batched_gemv_row_groups(cuda, fmt, batch, rows, cols):
    # 256 rows per workgroup (4160 x 4096) and 128 (2112 x 4096), each with a
    # last workgroup whose upper row groups lie past the matrix
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=fmt * 7 + batch, group=128)
    xs = np.stack([synth.make_activations(cols, seed=2000 + s, outliers=True) for s in range(batch)])
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, g)
    y = w.gemv(dev(xs.ravel()), flags=L.ROTATE_FWHT256).cpu().numpy().reshape(batch, rows)
    for b in range(batch):
        ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, xs[b], L.ROTATE_FWHT256)
        assert rel_max_err(y[b], ref) < TOL, f"vector {b}"


@pytest.mark.parametrize("fmt", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("cfg", [3, 6])
@pytest.mark.parametrize("rows,cols", [(70, 2048), (33, 640)])
@pytest.mark.parametrize("flags", [0, 1])
def test_four_vector_full_k(cuda, monkeypatch, fmt, cfg, rows, cols, flags):
    # 4 vectors on a full-K plan of K <= 2048 (8x2x1, 4x4x1) take the kernel
    # that holds the 4 vectors' tables side by side and sums in the
    # workgroup: the oracle for each vector, and the batched kernel's values
    # (LMX_NO_QUAD=1) to the same bar; 640 leaves the upper slices idle
    monkeypatch.setenv("LMX_FULLK", str(cfg))
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=cfg * 31 + fmt, group=128)
    xs = np.stack([synth.make_activations(cols, seed=3000 + s, outliers=True) for s in range(4)])
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, g)
    assert w.kernel_config()[0] == cfg
    y = w.gemv(dev(xs.ravel()), flags=flags).cpu().numpy().reshape(4, rows)
    monkeypatch.setenv("LMX_NO_QUAD", "1")
    yb = w.gemv(dev(xs.ravel()), flags=flags).cpu().numpy().reshape(4, rows)
    for b in range(4):
        ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, xs[b], flags)
        assert rel_max_err(y[b], ref) < TOL, f"vector {b}"
        assert rel_max_err(y[b], yb[b]) < TOL, f"vector {b}"


@pytest.mark.parametrize("qps", ["0", "1"])
@pytest.mark.parametrize("rows,cols", [(70, 2048), (2048, 1536), (1536, 1536), (33, 640)])
def test_four_vector_plane_split(cuda, monkeypatch, qps, rows, cols):
    # 4 unrotated 4-bit vectors on the 4x4x1 plan: the four-vector kernel
    # with a chunk's planes split over two lanes (where twice its workgroups
    # still make one round; LMX_QPS=0 keeps one lane per row and chunk),
    # against the oracle for each vector
    monkeypatch.setenv("LMX_QPS", qps)
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=rows + 5 * cols, group=128)
    xs = np.stack([synth.make_activations(cols, seed=4000 + s, outliers=True) for s in range(4)])
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, g)
    assert w.kernel_config()[0] == 6
    y = w.gemv(dev(xs.ravel()), flags=L.ROTATE_NONE).cpu().numpy().reshape(4, rows)
    for b in range(4):
        ref = oracle_planes_gemv(L.FMT_INT4, planes, scales, rows, cols, g, xs[b], L.ROTATE_NONE)
        assert rel_max_err(y[b], ref) < TOL, f"vector {b}"
    w.close()


@pytest.mark.parametrize("fmt", [L.FMT_INT4, L.FMT_TERNARY])
def test_four_vector_linear_bias(cuda, fmt):
    # lmx_linear on exactly 4 vectors of a 4 x 4 x 1 plan: the four-vector
    # kernel's bias epilogue (ternary: the FWHT-256 lut_linear applies)
    rows, cols = 2048, 1536
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=90 + fmt, group=128)
    xs = np.stack([synth.make_activations(cols, seed=900 + s, outliers=True) for s in range(4)])
    bias = np.random.default_rng(91).standard_normal(rows).astype(np.float32)
    w = L.Weight.from_planes(fmt, planes, scales, rows, cols, g)
    assert w.kernel_config()[0] == 6
    y = w.linear(dev(xs.ravel()), bias=dev(bias)).cpu().numpy().reshape(4, rows)
    rot = L.ROTATE_FWHT256 if fmt == L.FMT_TERNARY else L.ROTATE_NONE
    for b in range(4):
        ref = oracle_planes_gemv(fmt, planes, scales, rows, cols, g, xs[b], rot) + bias
        assert rel_max_err(y[b], ref) < TOL, b


def test_four_vector_graph_replays(cuda):
    # the four-vector launch captured in a graph: every replay equals the
    # eager call, with eager calls on the same handle in between
    rows, cols = 2048, 1536
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=95, group=128)
    xs = dev(np.stack([synth.make_activations(cols, seed=950 + s) for s in range(4)]).ravel())
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, g)
    eager = w.gemv(xs).cpu().numpy()
    out = torch.empty(4 * rows, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w.gemv(xs, y=out)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        w.gemv(xs, y=out)
    for _ in range(3):
        out.zero_()
        gr.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint32), eager.view(np.uint32))
        w.gemv(xs)
        torch.cuda.synchronize()


def test_batched_linear_bias_and_repeat(cuda):
    rows, cols, batch = 2048, 2048, 16
    planes, scales, g = synth.make_weights(L.FMT_INT4, rows, cols, seed=5)
    xs = np.stack([synth.make_activations(cols, seed=s) for s in range(batch)])
    bias = np.random.default_rng(3).standard_normal(rows).astype(np.float32)
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, g)
    y1 = w.linear(dev(xs.ravel()), bias=dev(bias)).cpu().numpy().reshape(batch, rows)
    y2 = w.linear(dev(xs.ravel()), bias=dev(bias)).cpu().numpy().reshape(batch, rows)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))            # deterministic
    for b in (0, 7, 15):
        ref = oracle.planes_gemv(6, planes, scales, rows, cols, g, xs[b]) + bias
        assert rel_max_err(y1[b], ref) < TOL
