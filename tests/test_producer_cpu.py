"""The producer side (lmx_quantize, include/lutmac_synth.h) on the CPU.

Pinned by: the reference quantizers' own block bytes (tests/golden/quantizers.npz,
written by tests/golden/gen_golden.py from the reference build, and the live
reference build where it exists) for ternary, binary and 2-bit at group 256,
plain and with the quantize tool's weight rotation, and for 3-bit and 8-bit
(never rotated) plain; the closed form of the uniform rules (scale =
absmax / 4 or / 127, codes within half a step of w / scale); the FWHT-256 of the
activation path (a rotated quantization equals quantizing the oracle-rotated
weights); and, for the residual stages that have no reference rule, the
stage definitions (each stage binarises what the earlier ones left: sign
bits, scale = mean |residual|), with the first stage equal to the binary
producer and the reconstruction error shrinking stage by stage."""
import numpy as np
import pytest

import lutmac_amd as L
import oracle
from conftest import load_golden
from lutmac_amd import synth

REF_FORMATS = [(L.FMT_TERNARY, "ternary"), (L.FMT_BINARY, "binary"), (L.FMT_RRQ2, "int2")]
# formats the quantize tool never rotates (tools/lutmac-quantize.cpp:385-425)
PLAIN_FORMATS = [(L.FMT_INT3, "int3"), (L.FMT_INT8, "int8")]


@pytest.mark.parametrize("fmt,name", REF_FORMATS)
@pytest.mark.parametrize("rot", [False, True])
def test_quantizers_match_reference_fixtures(fmt, name, rot):
    g = load_golden("quantizers.npz")
    w = g["w"]
    M, K = w.shape
    planes, scales, _ = L.quantize(fmt, w, 256, L.QUANT_ROTATE if rot else 0)
    blocks = L.planes_to_blocks(fmt, planes, scales, M, K)
    assert np.array_equal(blocks, g[name + ("_rot" if rot else "")])


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref/libref.so not built")
@pytest.mark.parametrize("fmt,name", REF_FORMATS)
@pytest.mark.parametrize("M,K,seed", [(300, 2048, 1), (64, 4096, 2), (8, 256, 3)])
def test_quantizers_match_reference_build(fmt, name, M, K, seed):
    R = oracle.ref()
    w = (np.random.default_rng(seed).standard_normal((M, K)) * 0.02).astype(np.float32)
    for rot in (False, True):
        src = w.copy()
        if rot:
            R.ref_apply_hadamard_rotation(oracle._ptr(src), src.size)
        n = R.ref_quantize(fmt, oracle._ptr(src), M, K, None, 0)
        ref = np.zeros(n, np.uint8)
        R.ref_quantize(fmt, oracle._ptr(src), M, K, oracle._ptr(ref), n)
        planes, scales, _ = L.quantize(fmt, w, 256, L.QUANT_ROTATE if rot else 0)
        assert np.array_equal(L.planes_to_blocks(fmt, planes, scales, M, K), ref), (name, rot)


@pytest.mark.parametrize("fmt,name", PLAIN_FORMATS)
def test_uniform_quantizers_match_reference_fixtures(fmt, name):
    g = load_golden("quantizers.npz")
    w = g["w"]
    M, K = w.shape
    planes, scales, _ = L.quantize(fmt, w, 256)
    assert np.array_equal(L.planes_to_blocks(fmt, planes, scales, M, K), g[name])


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref/libref.so not built")
@pytest.mark.parametrize("fmt,name", PLAIN_FORMATS)
@pytest.mark.parametrize("M,K,seed", [(300, 2048, 1), (64, 4096, 2), (8, 256, 3)])
def test_uniform_quantizers_match_reference_build(fmt, name, M, K, seed):
    R = oracle.ref()
    w = (np.random.default_rng(seed).standard_normal((M, K)) * 0.02).astype(np.float32)
    w[M // 2] = 0.0   # an all-zero row: scale 0, every code the format's zero
    n = R.ref_quantize(fmt, oracle._ptr(w), M, K, None, 0)
    ref = np.zeros(n, np.uint8)
    R.ref_quantize(fmt, oracle._ptr(w), M, K, oracle._ptr(ref), n)
    planes, scales, _ = L.quantize(fmt, w, 256)
    assert np.array_equal(L.planes_to_blocks(fmt, planes, scales, M, K), ref), name


@pytest.mark.parametrize("fmt,qmin,qmax,div", [(L.FMT_INT3, -4, 3, 4.0), (L.FMT_INT8, -127, 127, 127.0)])
@pytest.mark.parametrize("group", [128, 256])
def test_uniform_quantizers_closed_form(fmt, qmin, qmax, div, group):
    # per group: scale = absmax / div, and every weight's code is within half a
    # step of w / scale (clamped to the format's range); the planes hold the
    # code's bits, plane p = bit p (int3 code q + 4, int8 two's complement)
    w = (np.random.default_rng(7).standard_normal((12, 1024)) * 0.02).astype(np.float32)
    w[3, :group] = 0.0
    planes, scales, _ = L.quantize(fmt, w, group)
    P = planes.shape[0]
    bits = np.unpackbits(planes, axis=2)                       # [P][rows][cols], MSB-first per byte
    code = sum(bits[p].astype(np.int64) << p for p in range(P))
    q = code - 4 if fmt == L.FMT_INT3 else np.where(code >= 128, code - 256, code)
    absmax = np.abs(w).reshape(12, -1, group).max(axis=2)
    np.testing.assert_allclose(scales[0], absmax / div, rtol=2e-7, atol=0)
    s = np.repeat(scales[0], group, axis=1)
    want = np.clip(np.where(s > 0, w / np.where(s > 0, s, 1), 0), qmin, qmax)
    assert np.all(np.abs(q - want) <= 0.5 + 1e-4)
    assert np.all(q[3, :group] == 0)


@pytest.mark.parametrize("fmt", [L.FMT_TERNARY, L.FMT_BINARY, L.FMT_RRQ2, L.FMT_RRQ3])
@pytest.mark.parametrize("group", [128, 256])
def test_rotation_is_the_activation_fwht(fmt, group):
    # rotating inside the producer == quantizing weights rotated by the
    # oracle's FWHT-256 (the reference's scalar branch, bit-exact)
    w = (np.random.default_rng(4).standard_normal((16, 1024)) * 0.02).astype(np.float32)
    flags = L.QUANT_RESIDUAL if fmt == L.FMT_RRQ2 else 0
    a = L.quantize(fmt, w, group, flags | L.QUANT_ROTATE)
    b = L.quantize(fmt, oracle.fwht256(w.ravel()).reshape(w.shape), group, flags)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


@pytest.mark.parametrize("fmt,stages", [(L.FMT_RRQ2, 2), (L.FMT_RRQ3, 3)])
@pytest.mark.parametrize("group", [128, 256])
def test_residual_stages(fmt, stages, group):
    w = (np.random.default_rng(5).standard_normal((12, 768)) * 0.02).astype(np.float32)
    flags = L.QUANT_RESIDUAL if fmt == L.FMT_RRQ2 else 0
    planes, scales, _ = L.quantize(fmt, w, group, flags)
    # stage 1 is the binary producer
    bp, bs, _ = L.quantize(L.FMT_BINARY, w, group)
    assert np.array_equal(planes[0], bp[0]) and np.array_equal(scales[0], bs[0])
    res = w.astype(np.float32).copy()
    gidx = np.arange(w.shape[1]) // group
    errs = []
    for s in range(stages):
        bits = np.unpackbits(planes[s], axis=1, bitorder="big").astype(bool)
        assert np.array_equal(bits, res >= 0), s                     # sign of what is left
        want = np.abs(res.astype(np.float64)).reshape(12, -1, group).mean(axis=2)
        assert np.allclose(scales[s], want, rtol=1e-6, atol=0), s    # mean |residual| per group
        v = np.where(bits, scales[s][:, gidx], -scales[s][:, gidx]).astype(np.float32)
        res = (res - v).astype(np.float32)
        errs.append(float(np.sum(res.astype(np.float64) ** 2)))
    assert all(b < a for a, b in zip(errs, errs[1:]))
    # the dequantised sum of the stages (synth.dequant_f64) reconstructs w - residual
    W = synth.dequant_f64(fmt, planes, scales, 12, 768, group)
    assert np.allclose(W, w - res, atol=1e-7)


def test_ternary_groups_and_row_scale():
    # per-128 groups and one scale per row follow the same rule as 256
    w = (np.random.default_rng(6).standard_normal((10, 512)) * 0.02).astype(np.float32)
    thr = np.float32(np.abs(w.astype(np.float64)).sum() / w.size)
    for group in (128, 0):
        planes, scales, _ = L.quantize(L.FMT_TERNARY, w, group)
        t = synth.int_values(L.FMT_TERNARY, planes)
        assert np.array_equal(t == 0, np.abs(w) < np.float32(0.5) * thr)
        assert np.array_equal(t < 0, (np.abs(w) >= np.float32(0.5) * thr) & ~(w > 0))
        G = group or 512
        for r in range(10):
            for gi in range(512 // G):
                a = np.abs(w[r, gi * G:(gi + 1) * G])
                sel = a[a >= thr]
                want = sel.astype(np.float64).mean() if sel.size else 1.0
                assert abs(scales[0, r, gi] - want) <= 2e-7 * want


def test_quantize_rejects_bad_arguments():
    w = np.zeros((4, 256), np.float32)
    for fmt, group, flags in [(L.FMT_BINARY, 0, 0), (L.FMT_INT4, 128, L.QUANT_ROTATE),
                              (L.FMT_TERNARY, 256, L.QUANT_RESIDUAL), (L.FMT_INT8, 256, L.QUANT_ROTATE),
                              (L.FMT_INT3, 96, 0), (L.FMT_INT8, 0, 0),
                              (L.FMT_BINARY, 100, 0), (L.FMT_BINARY, 256, 8)]:
        with pytest.raises(L.LmxError):
            L.quantize(fmt, w, group, flags)
