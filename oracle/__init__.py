"""ctypes bindings for the CPU parity checker (test infrastructure only).

``lib()`` loads oracle/liboracle.so, the C restatement of LutMac's scalar
LUT-GEMV path; ``ref()`` loads oracle/_ref/libref.so, the reference's own
kernel sources compiled by oracle/Makefile, or returns None where it was not
built.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
use this package, and only as the checker or the timed CPU baseline.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

FMT_TERNARY, FMT_BINARY, FMT_RRQ2, FMT_RRQ3, FMT_INT3, FMT_INT4, FMT_INT8 = range(1, 8)
PLANES = {1: 2, 2: 1, 3: 2, 4: 3, 5: 3, 6: 4, 7: 8}
STAGES = {1: 1, 2: 1, 3: 2, 4: 3, 5: 1, 6: 1, 7: 1}
BLOCK_BYTES = {1: 68, 2: 36, 3: 72, 5: 100, 6: 132, 7: 260}

_p = ctypes.c_void_p
_sz = ctypes.c_size_t


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        for name, args, res in [
            ("orc_precompute_luts", [_p, _sz, _p], None),
            ("orc_extract_indices", [_p, _p, _sz, _p, _p], None),
            ("orc_fwht_256", [_p], None),
            ("orc_apply_hadamard_rotation", [_p, _sz], None),
            ("orc_fwht_full", [_p, _sz], None),
            ("orc_pack_to_bitplanes", [_p, _sz, _p, _p], None),
            ("orc_unpack_from_bitplanes", [_p, _p, _sz, _p], None),
            ("orc_lut_linear", [ctypes.c_int, _p, _p, _p, _p, _sz, _sz, _sz], ctypes.c_int),
            ("orc_blocks_to_planes", [ctypes.c_int, _p, _sz, _sz, _p, _p], ctypes.c_int),
            ("orc_planes_gemv", [ctypes.c_int, _p, _p, _sz, _sz, _sz, _p, _p], None),
        ]:
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        for name in ["orc_ternary_gemv", "orc_binary_gemv", "orc_int4_gemv",
                     "orc_int2_gemv", "orc_int3_gemv", "orc_int8_gemv"]:
            f = getattr(L, name)
            f.argtypes = [_p, _p, _p, _sz, _sz]
            f.restype = None
        _LIB = L
    return _LIB


def ref():
    """The reference's own kernels (oracle/_ref/libref.so) or None."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libref.so")
        if not os.path.exists(path):
            return None
        R = ctypes.CDLL(path)
        for name, args, res in [
            ("ref_sizeof_block", [ctypes.c_int], _sz),
            ("ref_precompute_luts", [_p, _sz, _p], None),
            ("ref_extract_indices", [_p, _p, _sz, _p, _p], None),
            ("ref_fwht_256", [_p], None),
            ("ref_apply_hadamard_rotation", [_p, _sz], None),
            ("ref_pack_to_bitplanes", [_p, _sz, _p, _p], None),
            ("ref_unpack_from_bitplanes", [_p, _p, _sz, _p], None),
            ("ref_gemv", [ctypes.c_int, _p, _sz, _p, _p, _sz, _sz], None),
            ("ref_lut_linear", [ctypes.c_int, _p, _sz, _p, _p, _p, _sz, _sz, _sz], ctypes.c_int),
            ("ref_quantize", [ctypes.c_int, _p, _sz, _sz, _p, _sz], _sz),
            ("ref_block_get", [ctypes.c_int, _p, _sz, _sz], ctypes.c_float),
        ]:
            f = getattr(R, name)
            f.argtypes = args
            f.restype = res
        _REF = R
    return _REF


# ---- numpy conveniences (oracle) ------------------------------------------

def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def precompute_luts(x):
    x = f32(x)
    out = np.zeros((x.size // 4) * 16, np.float32)
    lib().orc_precompute_luts(_ptr(x), x.size, _ptr(out))
    return out


def fwht256(x):
    x = f32(x).copy()
    lib().orc_apply_hadamard_rotation(_ptr(x), x.size)
    return x


def fwht_full(x):
    x = f32(x).copy()
    lib().orc_fwht_full(_ptr(x), x.size)
    return x


def block_gemv(fmt, blocks, x_padded, M, K):
    """Raw reference-style kernel: x must hold ceil(K/256)*256 floats."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    x = f32(x_padded)
    y = np.zeros(M, np.float32)
    name = {1: "orc_ternary_gemv", 2: "orc_binary_gemv", 3: "orc_int2_gemv",
            5: "orc_int3_gemv", 6: "orc_int4_gemv", 7: "orc_int8_gemv"}[fmt]
    getattr(lib(), name)(_ptr(blocks), _ptr(x), _ptr(y), M, K)
    return y


def lut_linear(fmt, blocks, x, M, K, bias=None, batch=1):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    x = f32(x)
    y = np.zeros(M * batch, np.float32)
    b = None if bias is None else f32(bias)
    rc = lib().orc_lut_linear(fmt, _ptr(blocks), _ptr(b), _ptr(x), _ptr(y), M, K, batch)
    if rc != 0:
        raise ValueError("unsupported format")
    return y


def blocks_to_planes(fmt, blocks, M, K):
    Kp = (K + 255) // 256 * 256
    P, S = PLANES[fmt], STAGES[fmt]
    planes = np.zeros(P * M * Kp // 8, np.uint8)
    scales = np.zeros(S * M * (Kp // 256), np.float32)
    blocks = np.ascontiguousarray(blocks, np.uint8)
    rc = lib().orc_blocks_to_planes(fmt, _ptr(blocks), M, K, _ptr(planes), _ptr(scales))
    if rc != 0:
        raise ValueError("unsupported format")
    return planes, scales


def planes_gemv(fmt, planes, scales, M, Kp, G, x):
    planes = np.ascontiguousarray(planes, np.uint8)
    scales = f32(scales)
    x = f32(x)
    y = np.zeros(M, np.float32)
    lib().orc_planes_gemv(fmt, _ptr(planes), _ptr(scales), M, Kp, G, _ptr(x), _ptr(y))
    return y
