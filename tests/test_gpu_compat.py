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


def test_precompute_lut_kat(cuda):
    # test_lut_gemm.cpp:17-55 through the single-group drop-in (lut_gemm.hpp:30-44)
    t = L.host_precompute_lut(np.array([1, 2, 3, 4], np.float32))
    assert t.tolist() == [0, 4, 3, 7, 2, 6, 5, 9, 1, 5, 4, 8, 3, 7, 6, 10]
    a = np.array([0.1, -2.5, 3e-3, 7.0], np.float32)
    assert np.array_equal(L.host_precompute_lut(a), oracle.precompute_luts(a))


def test_extract_indices_kat(cuda):
    # test_lut_gemm.cpp:57-88: weights [+1, -1, 0, +1] -> pos 0b1001, neg 0b0100
    sign = np.array([0b01000000, 0, 0, 0], np.uint8)
    zero = np.array([0b00100000, 0, 0, 0], np.uint8)
    assert L.host_extract_indices(sign, zero, 0) == (0b1001, 0b0100)
    # every nibble pair, even and odd groups, against the closed form
    rng = np.random.default_rng(5)
    s, z = rng.integers(0, 256, 8, dtype=np.uint8), rng.integers(0, 256, 8, dtype=np.uint8)
    for g in range(16):
        sh = 4 if g % 2 == 0 else 0
        sn, zn = (int(s[g // 2]) >> sh) & 0xF, (int(z[g // 2]) >> sh) & 0xF
        nz = ~zn & 0xF
        assert L.host_extract_indices(s, z, g) == (nz & ~sn & 0xF, nz & sn), g


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


def random_int4_blocks(M, K, seed):
    """M * ceil(K/256) Int4Blocks (types.hpp:174-202): random nibbles, scale |N(0,1)|*0.02."""
    rng = np.random.default_rng(seed)
    nb = M * ((K + 255) // 256)
    blk = rng.integers(0, 256, (nb, 132), dtype=np.uint8)
    blk[:, 128:] = (np.abs(rng.standard_normal(nb)) * 0.02).astype(np.float32).view(np.uint8).reshape(nb, 4)
    return blk.reshape(-1)


def test_weight_cache_sees_rewritten_blocks(cuda):
    # one host buffer, new contents in place (a freed PackedTensor's address
    # reused by another tensor of the same shape): the new weights are used
    M, K = 64, 512
    buf = random_int4_blocks(M, K, 1)
    x = np.random.default_rng(2).standard_normal(K).astype(np.float32)
    y1 = L.host_gemv(6, buf, x, M, K)
    assert rel_max_err(y1, oracle.block_gemv(6, buf, x, M, K)) < TOL
    buf[:] = random_int4_blocks(M, K, 3)
    y2 = L.host_gemv(6, buf, x, M, K)
    assert rel_max_err(y2, oracle.block_gemv(6, buf, x, M, K)) < TOL
    assert not np.array_equal(y1, y2)


def test_weight_cache_forget(cuda):
    # more blocks than the fingerprint samples: a change to one unsampled block
    # is the caller's to announce with lmx_host_forget
    M, K = 512, 1024
    buf = random_int4_blocks(M, K, 4)
    x = np.random.default_rng(5).standard_normal(K).astype(np.float32)
    L.host_gemv(6, buf, x, M, K)
    blk = buf.reshape(-1, 132)
    blk[777, :128] ^= 0x5A   # row 194
    L.host_forget(buf)
    y = L.host_gemv(6, buf, x, M, K)
    assert rel_max_err(y, oracle.block_gemv(6, buf, x, M, K)) < TOL
    L.host_cache_clear()
    assert rel_max_err(L.host_gemv(6, buf, x, M, K), y) == 0.0


def test_weight_cache_threads(cuda):
    # two threads on one cached weight (serialised on its scratch) and a third
    # on another weight: every result equals the single-threaded one
    import threading
    M, K = 1024, 2048   # split-K / full-K scratch in use
    bufs = [random_int4_blocks(M, K, 6), random_int4_blocks(M, K, 7)]
    xs = [np.random.default_rng(10 + i).standard_normal(K).astype(np.float32) for i in range(6)]
    want = {(b, i): L.host_gemv(6, bufs[b], xs[i], M, K) for b in range(2) for i in range(6)}
    bad = []

    def run(b, seed):
        order = np.random.default_rng(seed).integers(0, 6, 40)
        for i in order:
            y = L.host_gemv(6, bufs[b], xs[i], M, K)
            if not np.array_equal(y, want[(b, int(i))]):
                bad.append((b, int(i)))

    ts = [threading.Thread(target=run, args=(b, s)) for b, s in [(0, 1), (0, 2), (1, 3)]]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not bad, bad[:5]
