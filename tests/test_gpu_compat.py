"""The reference's own kernel tests (tests/test_lut_gemm.cpp and
tests/test_tmac_correctness.cpp in the LutMac tree), restated against the
host-pointer drop-ins of include/lutmac_hip_compat.h, which run on the GPU
through the C ABI.  Inputs come from this build's seeded generators or the
golden fixtures (the reference's mt19937/uniform_real_distribution draws are
not portable)."""
import os
import subprocess

import numpy as np
import pytest

import lutmac_amd as L
import oracle
from conftest import ROOT, TOL, load_golden, rel_max_err

pytestmark = pytest.mark.gpu

FORMAT_FILES = {1: "ternary", 2: "binary", 3: "int2", 5: "int3", 6: "int4", 7: "int8"}


def test_lut_precomputation(cuda):
    # test_lut_gemm.cpp:17-55
    t = L.host_precompute_luts(np.array([1, 2, 3, 4], np.float32))
    assert t.tolist() == [0, 4, 3, 7, 2, 6, 5, 9, 1, 5, 4, 8, 3, 7, 6, 10]


def test_gemv_correctness_ternary_all_ones(cuda):
    # test_lut_gemm.cpp:135-165: +1 weights, x = [1,2,3,4] -> 10 (scale 1)
    blk = np.zeros(68, np.uint8)
    blk[32:64] = 0xFF
    blk[32] = 0x0F
    blk[64:68] = np.array([1.0], np.float32).view(np.uint8)
    x = np.zeros(256, np.float32)
    x[:4] = [1, 2, 3, 4]
    assert L.host_gemv(1, blk, x, 1, 4)[0] == 10.0


def test_int4_gemv_ramp(cuda):
    # test_lut_gemm.cpp:218-260: ramp (i%15)-7 at scale 0.5, x = 1 -> -6.5
    q = np.array([(i % 15) - 7 + 8 for i in range(32)] + [8] * 224, np.uint8)
    blk = np.zeros(132, np.uint8)
    blk[:128] = (q[0::2] << 4) | q[1::2]
    blk[128:] = np.array([0.5], np.float32).view(np.uint8)
    x = np.r_[np.ones(32), np.zeros(224)].astype(np.float32)
    assert abs(L.host_gemv(6, blk, x, 1, 32)[0] + 6.5) < 0.01
    assert abs(L.host_lut_linear(6, blk, np.ones(32, np.float32), 1, 32)[0] + 6.5) < 0.01


def test_binary_gemv_alternating(cuda):
    # test_lut_gemm.cpp:262-307: w = +1,-1,... , x = 1 -> 0
    blk = np.zeros(36, np.uint8)
    blk[:32] = 0b10101010
    blk[32:] = np.array([1.0], np.float32).view(np.uint8)
    assert abs(L.host_gemv(2, blk, np.ones(256, np.float32), 1, 256)[0]) < 1e-6


@pytest.mark.parametrize("fmt", [7, 1, 3, 5])
def test_gemv_vs_dequant(cuda, fmt):
    # test_lut_gemm.cpp:309-369 (int8, max diff < 1e-3) and
    # test_tmac_correctness.cpp:13-136 (ternary < 1e-4, int2/int3 < 1e-3):
    # the raw kernel against the dequantized weights (block.get()).
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    Kp = (K + 255) // 256 * 256
    W = g["dequant"].astype(np.float64).reshape(M, Kp)
    x = np.zeros(Kp, np.float32)
    x[:K] = g["x"][:K]
    y = L.host_gemv(fmt, g["blocks"], x, M, K)
    ref = W @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) < {7: 1e-3, 1: 1e-4, 3: 1e-3, 5: 1e-3}[fmt]
    assert rel_max_err(y, ref) < TOL


@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_lut_linear_host_golden(cuda, fmt):
    # lut_linear with bias at batch 2 against the reference build's outputs
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    y = L.host_lut_linear(fmt, g["blocks"], g["x"], M, K, bias=g["bias"], batch=2)
    for b in range(2):
        assert rel_max_err(y[b * M:(b + 1) * M], g["y"][b * M:(b + 1) * M]) < TOL


def test_apply_hadamard_rotation_host(cuda):
    g = load_golden("tables_fwht.npz")
    y = L.host_apply_hadamard_rotation(g["x"])
    assert np.array_equal(y.view(np.uint32), g["x_rot"].view(np.uint32))
    x = np.arange(300, dtype=np.float32)            # partial tail chunk untouched
    y = L.host_apply_hadamard_rotation(x)
    assert np.array_equal(y[256:], x[256:])
    assert np.array_equal(y[:256].view(np.uint32), oracle.fwht256(x[:256]).view(np.uint32))


def test_weight_cache_reuses_handle(cuda):
    # The same block array twice: second call hits the cached device handle.
    g = load_golden("blocks_int4.npz")
    M, K = int(g["M"]), int(g["K"])
    a = L.host_lut_linear(6, g["blocks"], g["x"][:K], M, K)
    b = L.host_lut_linear(6, g["blocks"], g["x"][:K], M, K)
    assert np.array_equal(a, b)


def test_cpp_dropins_compile_and_run(cuda):
    """tests/cpp/compat_smoke.cpp: the reference-named C++ wrappers against a
    PackedTensor-shaped struct (built by lutmac_amd.build)."""
    exe = os.path.join(ROOT, "tests", "cpp", "compat_smoke")
    assert os.path.exists(exe), "tests/cpp/compat_smoke not built (python -m lutmac_amd.build)"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
