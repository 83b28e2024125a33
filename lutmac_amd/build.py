"""Build the in-tree HIP library (lutmac_amd/liblutmac_hip.so) for gfx950.

Run as ``python -m lutmac_amd.build``.  Object files go to lutmac_amd/_build/
(git-ignored); the shared library lands next to this file so it travels with
the tree.  Every HIP translation unit is compiled with packed-FP32 code
generation disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liblutmac_hip.so")
ARCH = os.environ.get("LMX_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
          "-I", os.path.join(ROOT, "include"), "-I", CSRC]
DEVICE = ["-x", "hip", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]

SOURCES = [
    ("lmx_kernels.hip", True),
    ("lmx_probe.hip", True),
    ("lmx_noalloc.hip", True),
    ("lmx_decode.hip", True),
    ("lmx_capi.cpp", False),
    ("lmx_repack.cpp", False),
    ("lut_gemm_compat.cpp", False),
    ("lmx_synth.cpp", False),
    ("lmx_quantize.cpp", False),
    ("lmx_model.cpp", False),
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose=True):
    """Compiles every translation unit (in parallel, one hipcc per file) and
    links the library."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OUT_DIR, exist_ok=True)
    jobs = []
    for src, device in SOURCES:
        path = os.path.join(CSRC, src)
        if not os.path.exists(path):
            continue
        obj = os.path.join(OUT_DIR, src + ".o")
        flags = COMMON + (DEVICE if device else ["-D__HIP_PLATFORM_AMD__"])
        jobs.append(([HIPCC] + flags + ["-c", path, "-o", obj], obj))
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "8"))))
    with ThreadPoolExecutor(workers) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd, _ in jobs]:
            f.result()
    objs = [obj for _, obj in jobs]
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs, verbose)
    os.replace(tmp, LIB)
    # C++ drop-in check program (run by tests/test_gpu_compat.py)
    smoke = os.path.join(ROOT, "tests", "cpp", "compat_smoke")
    _run([HIPCC, "-O2", "-std=c++17", "-I", os.path.join(ROOT, "include"),
          os.path.join(ROOT, "tests", "cpp", "compat_smoke.cpp"), "-L", HERE, "-llutmac_hip",
          "-Wl,-rpath,$ORIGIN/../../lutmac_amd", "-o", smoke], verbose)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
