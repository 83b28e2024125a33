"""Pins the CPU oracle (oracle/lutmac_oracle.c) before anything is checked
against it: the reference's own KATs (tests/test_lut_gemm.cpp,
tests/test_quantization.cpp in the LutMac tree), golden vectors produced by
the reference's compiled kernels (tests/golden/), closed forms and brute
force.  CPU only."""
import numpy as np
import pytest
import scipy.linalg

import oracle
from conftest import TOL, load_golden, rel_max_err

FORMAT_FILES = {1: "ternary", 2: "binary", 3: "int2", 5: "int3", 6: "int4", 7: "int8"}


# ---- tables -----------------------------------------------------------------

def test_precompute_lut_kat():
    # test_lut_gemm.cpp:17-55: x=[1,2,3,4], entry m sums a_j for bit (3-j).
    t = oracle.precompute_luts(np.array([1, 2, 3, 4], np.float32))
    expected = [0, 4, 3, 7, 2, 6, 5, 9, 1, 5, 4, 8, 3, 7, 6, 10]
    assert t.tolist() == expected


def test_precompute_luts_golden_bitexact():
    g = load_golden("tables_fwht.npz")
    assert np.array_equal(oracle.precompute_luts(g["x"]).view(np.uint32), g["luts"].view(np.uint32))
    assert np.array_equal(oracle.precompute_luts(g["x_rot"]).view(np.uint32), g["luts_rot"].view(np.uint32))


def test_precompute_luts_closed_form():
    # T_g[m] = sum_j bit(3-j, m) * x[4g+j], checked in fp64 on random inputs.
    x = np.random.default_rng(5).standard_normal(64).astype(np.float32)
    t = oracle.precompute_luts(x).reshape(16, 16).astype(np.float64)
    bits = np.array([[(m >> (3 - j)) & 1 for j in range(4)] for m in range(16)], np.float64)
    ref = x.reshape(16, 4).astype(np.float64) @ bits.T
    assert np.max(np.abs(t - ref)) < 1e-6


# ---- indices ----------------------------------------------------------------

def _indices(s, z, g):
    import ctypes
    a, b = ctypes.c_uint8(), ctypes.c_uint8()
    oracle.lib().orc_extract_indices(oracle._ptr(s), oracle._ptr(z), g, ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def test_extract_indices_kat():
    # test_lut_gemm.cpp:57-88: weights [+1,-1,0,+1] -> pos 0b1001, neg 0b0100.
    s = np.array([0b01000000, 0, 0, 0], np.uint8)
    z = np.array([0b00100000, 0, 0, 0], np.uint8)
    assert _indices(s, z, 0) == (0b1001, 0b0100)


def test_extract_indices_golden():
    g = load_golden("indices.npz")
    got = [_indices(g["sign"], g["zero"], i) for i in range(256)]
    assert [p for p, _ in got] == g["pos"].tolist()
    assert [n for _, n in got] == g["neg"].tolist()


# ---- FWHT-256 ---------------------------------------------------------------

def test_fwht256_golden_bitexact():
    g = load_golden("tables_fwht.npz")
    assert np.array_equal(oracle.fwht256(g["x"]).view(np.uint32), g["x_rot"].view(np.uint32))


def test_fwht256_is_sylvester_hadamard_over_16():
    x = np.random.default_rng(7).standard_normal(768).astype(np.float32)
    H = scipy.linalg.hadamard(256).astype(np.float64) / 16.0
    ref = (x.reshape(3, 256).astype(np.float64) @ H.T).ravel()
    assert np.max(np.abs(oracle.fwht256(x) - ref)) < 1e-5
    e0 = np.zeros(256, np.float32)
    e0[0] = 1.0
    assert np.all(oracle.fwht256(e0) == np.float32(1 / 16))     # H e0 = 1/16 * ones, exactly
    y = oracle.fwht256(oracle.fwht256(x))                        # involution
    assert np.max(np.abs(y - x)) < 1e-5
    assert abs(np.linalg.norm(oracle.fwht256(x)) - np.linalg.norm(x)) < 1e-3  # orthonormal


def test_fwht256_partial_chunk_untouched():
    # transform_simd.cpp:105-109 rotates whole 256-chunks only.
    x = np.arange(300, dtype=np.float32)
    y = oracle.fwht256(x)
    assert np.array_equal(y[256:], x[256:])


def test_fwht_full_closed_form():
    x = np.random.default_rng(8).standard_normal(1024).astype(np.float32)
    H = scipy.linalg.hadamard(1024).astype(np.float64) / 32.0
    assert np.max(np.abs(oracle.fwht_full(x) - H @ x.astype(np.float64))) < 1e-5


# ---- bit-plane packing ------------------------------------------------------

def test_pack_roundtrip_kat():
    # test_quantization.cpp:43-86: the 16-value +1,-1,0 pattern round-trips.
    t = np.array([1, -1, 0] * 5 + [1], np.int8)
    s = np.zeros(2, np.uint8)
    z = np.zeros(2, np.uint8)
    L = oracle.lib()
    L.orc_pack_to_bitplanes(oracle._ptr(t), 16, oracle._ptr(s), oracle._ptr(z))
    assert s.tolist() == [0b01001001, 0b00100100] and z.tolist() == [0b00100100, 0b10010010]
    back = np.zeros(16, np.int8)
    L.orc_unpack_from_bitplanes(oracle._ptr(s), oracle._ptr(z), 16, oracle._ptr(back))
    assert np.array_equal(back, t)


def test_pack_golden():
    g = load_golden("bitplanes.npz")
    s = np.zeros(125, np.uint8)
    z = np.zeros(125, np.uint8)
    oracle.lib().orc_pack_to_bitplanes(oracle._ptr(g["ternary"]), 1000, oracle._ptr(s), oracle._ptr(z))
    assert np.array_equal(s, g["sign"]) and np.array_equal(z, g["zero"])
    back = np.zeros(1000, np.int8)
    oracle.lib().orc_unpack_from_bitplanes(oracle._ptr(s), oracle._ptr(z), 1000, oracle._ptr(back))
    assert np.array_equal(back, g["unpacked"]) and np.array_equal(back, g["ternary"])


# ---- GEMVs over reference blocks --------------------------------------------

@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_lut_linear_golden(fmt):
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    y = oracle.lut_linear(fmt, g["blocks"], g["x"], M, K, bias=g["bias"], batch=2)
    assert rel_max_err(y[:M], g["y"][:M]) < TOL and rel_max_err(y[M:], g["y"][M:]) < TOL
    y0 = oracle.lut_linear(fmt, g["blocks"], g["x"], M, K, batch=2)
    assert rel_max_err(y0[:M], g["y_nobias"][:M]) < TOL


@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_blocks_to_planes_matches_reference_accessors(fmt):
    # Canonical planes + scales dequantize to exactly what the reference's
    # block.get() returns (types.hpp accessors), weight by weight.
    from lutmac_amd.synth import dequant_f64
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    Kp = (K + 255) // 256 * 256
    planes, scales = oracle.blocks_to_planes(fmt, g["blocks"], M, K)
    W = dequant_f64(fmt, planes.reshape(oracle.PLANES[fmt], M, Kp // 8), scales, M, Kp, 256)
    assert np.array_equal(W.astype(np.float32).ravel(), g["dequant"])


@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_block_gemv_vs_fp64_dequant(fmt):
    # The reference's own oracle style (test_tmac_correctness.cpp): dense
    # dequantized weights times x, here in fp64.
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    Kp = (K + 255) // 256 * 256
    W = g["dequant"].astype(np.float64).reshape(M, Kp)
    x = np.zeros(Kp, np.float32)
    x[:K] = g["x"][:K]
    if fmt in (1, 2, 3):
        x = oracle.fwht256(x)
    y = oracle.block_gemv(fmt, g["blocks"], x, M, K)
    assert rel_max_err(y, W @ x.astype(np.float64)) < TOL


def test_int4_ramp_kat():
    # test_lut_gemm.cpp:218-260: ramp (i%15)-7 times 0.5, x = 1 -> -6.5.
    blk = np.zeros(132, np.uint8)
    q = np.array([(i % 15) - 7 + 8 for i in range(32)] + [8] * 224, np.uint8)
    blk[:128] = (q[0::2] << 4) | q[1::2]
    blk[128:132] = np.array([0.5], np.float32).view(np.uint8)
    y = oracle.block_gemv(6, blk, np.r_[np.ones(32), np.zeros(224)].astype(np.float32), 1, 32)
    assert abs(y[0] - (-6.5)) < 0.01


def test_ternary_all_ones_kat():
    # test_lut_gemm.cpp:135-165: w = +1 (scale 1), x = [1,2,3,4] -> 10.
    blk = np.zeros(68, np.uint8)
    blk[32:64] = 0xFF
    blk[32] = 0x0F            # first 4 weights non-zero, sign 0 -> +1
    blk[64:68] = np.array([1.0], np.float32).view(np.uint8)
    x = np.zeros(256, np.float32)
    x[:4] = [1, 2, 3, 4]
    assert oracle.block_gemv(1, blk, x, 1, 4)[0] == 10.0


def test_binary_alternating_kat():
    # test_lut_gemm.cpp:262-307: w alternating +1/-1, x = 1 -> 0.
    blk = np.zeros(36, np.uint8)
    blk[:32] = 0b10101010
    blk[32:36] = np.array([1.0], np.float32).view(np.uint8)
    assert oracle.block_gemv(2, blk, np.ones(256, np.float32), 1, 256)[0] == 0.0


# ---- canonical-plane GEMV (BASELINE synthetic formats) ------------------------

@pytest.mark.parametrize("fmt", [1, 2, 3, 4, 5, 6, 7])
@pytest.mark.parametrize("group", [0, 128, 256])
def test_planes_gemv_vs_fp64(fmt, group):
    from lutmac_amd import synth
    M, K = 40, 512
    planes, scales, _ = synth.make_weights(fmt, M, K, seed=fmt * 10 + group // 128, group=group or 128)
    if group == 0:
        scales = np.ascontiguousarray(scales[:, :, :1])
    x = synth.make_activations(K, seed=3)
    y = oracle.planes_gemv(fmt, planes, scales, M, K, group or K, x)
    W = synth.dequant_f64(fmt, planes, scales, M, K, group)
    assert rel_max_err(y, W @ x.astype(np.float64)) < TOL


def test_rrq3_is_sum_of_binary_gemvs():
    # RRQ-3 = three binary (lut_gemv_binary) passes with their own scales.
    from lutmac_amd import synth
    M, K = 24, 512
    planes, scales, g = synth.make_weights(4, M, K, seed=11)
    x = synth.make_activations(K, seed=12)
    y3 = oracle.planes_gemv(4, planes, scales, M, K, g, x)
    ys = sum(oracle.planes_gemv(2, planes[i:i + 1], scales[i:i + 1], M, K, g, x).astype(np.float64)
             for i in range(3))
    assert rel_max_err(y3, ys) < TOL


def test_per128_embedding_into_reference_blocks():
    # A per-128-group 4-bit weight equals a reference Int4 GEMV whose every
    # 128-group is padded into its own 256-block (nibble 8, x = 0).
    from lutmac_amd import synth
    M, K = 16, 512
    planes, scales, g = synth.make_weights(6, M, K, seed=21)
    x = synth.make_activations(K, seed=22)
    y = oracle.planes_gemv(6, planes, scales, M, K, g, x)
    q = (synth.int_values(6, planes) + 8).astype(np.uint8)          # [M, K]
    ng = K // 128
    q2 = np.full((M, ng, 256), 8, np.uint8)
    q2[:, :, :128] = q.reshape(M, ng, 128)
    blocks = np.zeros((M, ng, 132), np.uint8)
    blocks[:, :, :128] = (q2[:, :, 0::2] << 4) | q2[:, :, 1::2]
    blocks[:, :, 128:] = scales[0].reshape(M, ng, 1).view(np.uint8).reshape(M, ng, 4)
    x2 = np.zeros((ng, 256), np.float32)
    x2[:, :128] = x.reshape(ng, 128)
    yb = oracle.block_gemv(6, blocks.ravel(), x2.ravel(), M, ng * 256)
    assert rel_max_err(y, yb) < TOL
    R = oracle.ref()
    if R is not None:  # and the reference's own int4_gemv agrees
        yr = np.zeros(M, np.float32)
        R.ref_gemv(6, oracle._ptr(blocks.ravel()), M * ng, oracle._ptr(x2.ravel()), oracle._ptr(yr), M, ng * 256)
        assert rel_max_err(y, yr) < TOL


@pytest.mark.skipif(oracle.ref() is None, reason="reference build (oracle/_ref) absent")
@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_oracle_vs_reference_build_random(fmt):
    # Fresh random blocks through both: the restatement and the real kernels.
    R = oracle.ref()
    rng = np.random.default_rng(100 + fmt)
    M = 37
    K = 1024 if fmt in (3, 5) else 1000   # flat 2/3-bit quantizers need K % 256 == 0
    w = (rng.standard_normal(M * K) * 0.05).astype(np.float32)
    nb = M * ((K + 255) // 256)
    blocks = np.zeros(nb * oracle.BLOCK_BYTES[fmt], np.uint8)
    R.ref_quantize(fmt, oracle._ptr(w), M, K, oracle._ptr(blocks), blocks.size)
    x = rng.standard_normal(K).astype(np.float32)
    yr = np.zeros(M, np.float32)
    R.ref_lut_linear(fmt, oracle._ptr(blocks), nb, None, oracle._ptr(x), oracle._ptr(yr), M, K, 1)
    assert rel_max_err(oracle.lut_linear(fmt, blocks, x, M, K), yr) < TOL
