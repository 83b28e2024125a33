"""CPU tests of the C-ABI library (lutmac_amd/liblutmac_hip.so): it loads,
exports every symbol include/lutmac_hip.h declares, its host-side repack is
bit-exact against the oracle and the reference's golden blocks, and argument
validation fails cleanly before any GPU work.  No compute calls."""
import ctypes
import os
import re

import numpy as np
import pytest

import lutmac_amd as L
import oracle
from conftest import ROOT, load_golden

FORMAT_FILES = {1: "ternary", 2: "binary", 3: "int2", 5: "int3", 6: "int4", 7: "int8"}


def _declared_symbols():
    """extern "C" entry points declared by every header under include/."""
    names = set()
    inc = os.path.join(ROOT, "include")
    for h in sorted(os.listdir(inc)):
        if not h.endswith(".h"):
            continue
        hdr = open(os.path.join(inc, h)).read()
        hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
        if '#ifdef __cplusplus\n}' in hdr:          # drop the C++-only wrapper section
            hdr = hdr.split('#ifdef __cplusplus\n}')[0]
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(lmx_[a-z0-9_]+)\s*\(", hdr, flags=re.M))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    declared = _declared_symbols()
    assert declared == sorted(L.EXPORTS)
    for name in declared:
        assert hasattr(lib, name), name


def test_format_enum_matches_oracle():
    for fmt in range(1, 8):
        p, s = ctypes.c_int(), ctypes.c_int()
        L.check(L.lib().lmx_format_info(fmt, ctypes.byref(p), ctypes.byref(s)))
        assert (p.value, s.value) == (oracle.PLANES[fmt], oracle.STAGES[fmt])
        if fmt in oracle.BLOCK_BYTES:
            n = ctypes.c_size_t()
            L.check(L.lib().lmx_block_bytes(fmt, ctypes.byref(n)))
            assert n.value == oracle.BLOCK_BYTES[fmt]
            R = oracle.ref()
            if R is not None:
                assert R.ref_sizeof_block(fmt) == n.value
    assert L.lib().lmx_format_info(99, None, None) == L.ERR_UNSUPPORTED_FORMAT
    assert L.lib().lmx_block_bytes(L.FMT_RRQ3, None) == L.ERR_UNSUPPORTED_FORMAT


@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_blocks_to_planes_bitexact(fmt):
    g = load_golden(f"blocks_{FORMAT_FILES[fmt]}.npz")
    M, K = int(g["M"]), int(g["K"])
    planes, scales = L.blocks_to_planes(fmt, g["blocks"], M, K)
    op, os_ = oracle.blocks_to_planes(fmt, g["blocks"], M, K)
    assert np.array_equal(planes, op)
    assert np.array_equal(scales.view(np.uint32), os_.view(np.uint32))
    back = L.planes_to_blocks(fmt, planes, scales, M, K)
    assert np.array_equal(back, g["blocks"])


@pytest.mark.parametrize("fmt", sorted(FORMAT_FILES))
def test_planes_to_blocks_roundtrip_random(fmt):
    rng = np.random.default_rng(fmt)
    M, K = 5, 512
    blocks = rng.integers(0, 256, M * 2 * oracle.BLOCK_BYTES[fmt], dtype=np.uint8)
    # keep the scale bytes finite floats
    bv = blocks.reshape(M * 2, oracle.BLOCK_BYTES[fmt])
    sc_off = {1: [64], 2: [32], 3: [64, 68], 5: [96], 6: [128], 7: [0]}[fmt]
    for off in sc_off:
        bv[:, off:off + 4] = rng.random(M * 2, dtype=np.float32).reshape(-1, 1).view(np.uint8)
    planes, scales = L.blocks_to_planes(fmt, blocks, M, K)
    assert np.array_equal(L.planes_to_blocks(fmt, planes, scales, M, K), blocks)
    op, _ = oracle.blocks_to_planes(fmt, blocks, M, K)
    assert np.array_equal(planes, op)


@pytest.mark.parametrize("fmt", [1, 2, 4, 5, 6, 7])
@pytest.mark.parametrize("rows,cols", [(64, 256), (100, 640), (3, 8), (130, 1024)])
def test_tile_layout(fmt, rows, cols):
    rng = np.random.default_rng(rows + cols)
    P = L.PLANES[fmt]
    planes = rng.integers(0, 256, P * rows * cols // 8, dtype=np.uint8)
    tiles = L.tile_planes(fmt, planes, rows, cols)
    Npad = -(-rows // 64) * 64
    Kp = -(-cols // 256) * 256
    assert tiles.size == (Kp // 128) * P * Npad * 16
    # restated index: tiles[c][p][r][j] = planes[p][r][16c + j], zero beyond
    t = tiles.reshape(Kp // 128, P, Npad, 16)
    pl = planes.reshape(P, rows, cols // 8)
    padded = np.zeros((P, Npad, Kp // 8), np.uint8)
    zero_code_plane = {1: 1, 5: 2, 6: 3}.get(fmt)      # plane set to 1 in padded columns
    if zero_code_plane is not None:
        padded[zero_code_plane, :rows, :] = 0xFF
    padded[:, :rows, :cols // 8] = pl
    assert np.array_equal(t, padded.reshape(P, Npad, Kp // 128, 16).transpose(2, 0, 1, 3))
    assert np.array_equal(L.untile_planes(fmt, tiles, rows, cols), planes)


def test_argument_validation_without_device():
    lib = L.lib()
    h = ctypes.c_void_p()
    assert lib.lmx_weight_create(None, ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    planes = np.zeros(64, np.uint8)
    scales = np.zeros(8, np.float32)
    d = L.PlanesDesc(99, 8, 64, 0, planes.ctypes.data, scales.ctypes.data)
    assert lib.lmx_weight_create(ctypes.byref(d), ctypes.byref(h)) == L.ERR_UNSUPPORTED_FORMAT
    d = L.PlanesDesc(L.FMT_BINARY, 8, 60, 0, planes.ctypes.data, scales.ctypes.data)
    assert lib.lmx_weight_create(ctypes.byref(d), ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    d = L.PlanesDesc(L.FMT_BINARY, 8, 64, 100, planes.ctypes.data, scales.ctypes.data)
    assert lib.lmx_weight_create(ctypes.byref(d), ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    assert b"multiple of 128" in lib.lmx_last_error()
    assert lib.lmx_weight_from_blocks(L.FMT_RRQ3, planes.ctypes.data, 8, 8, 256,
                                      ctypes.byref(h)) == L.ERR_UNSUPPORTED_FORMAT
    assert lib.lmx_weight_from_blocks(L.FMT_INT4, planes.ctypes.data, 7, 8, 256,
                                      ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    assert lib.lmx_gemv(None, None, None, 1, 0, None) == L.ERR_INVALID_ARGUMENT
    assert lib.lmx_linear(None, None, None, None, 1, None) == L.ERR_INVALID_ARGUMENT
    assert lib.lmx_fwht256(None, 256, None) == L.ERR_INVALID_ARGUMENT
    assert lib.lmx_precompute_luts(None, 16, 0, None, None) == L.ERR_INVALID_ARGUMENT
    assert lib.lmx_extract_indices(None, None, 4, None, None, None) == L.ERR_INVALID_ARGUMENT
    assert lib.lmx_weight_destroy(None) == L.OK
    assert lib.lmx_status_string(L.ERR_NO_DEVICE) == b"no device"


def test_no_device_is_reported():
    if L.device_count() > 0:
        pytest.skip("a GPU is visible")
    lib = L.lib()
    planes = np.zeros(8 * 8, np.uint8)
    scales = np.zeros(8, np.float32)
    d = L.PlanesDesc(L.FMT_BINARY, 8, 64, 0, planes.ctypes.data, scales.ctypes.data)
    h = ctypes.c_void_p()
    assert lib.lmx_weight_create(ctypes.byref(d), ctypes.byref(h)) == L.ERR_NO_DEVICE
    assert not h.value


@pytest.mark.parametrize("fmt,rows,cols,group", [(6, 70, 640, 128), (1, 65, 512, 0), (3, 3, 1000, 256),
                                                 (4, 64, 384, 128)])
def test_tile_scales_layout(fmt, rows, cols, group):
    # canonical [S][rows][groups] -> device [S][Kp/group][Npad], zero padded
    S = L.STAGES[fmt]
    ng = 1 if group == 0 else -(-cols // group)
    sc = np.random.default_rng(fmt).standard_normal((S, rows, ng)).astype(np.float32)
    out = L.tile_scales(fmt, sc, rows, cols, group)
    Npad, Kp = -(-rows // 64) * 64, -(-cols // 256) * 256
    ngd = 1 if group == 0 else Kp // group
    want = np.zeros((S, ngd, Npad), np.float32)
    want[:, :ng, :rows] = sc.transpose(0, 2, 1)
    assert np.array_equal(out, want.ravel())


def test_lutmac_v2_rejections_before_device_work(tmp_path):
    # plane records whose rotation flag contradicts lut_linear's rule, a
    # rotated embedding and a size mismatch are refused while parsing
    import ctypes
    from lutmac_amd import decode as D
    from lutmac_amd import lutmac_file as F
    cfg = D.small_config(n_layers=1, vocab=300)
    fmts = {n: (L.FMT_TERNARY, 128, 0) for n in D.QuantizedModel.NAMES}
    fmts["embed"] = (L.FMT_INT4, 128, 0)
    m = D.QuantizedModel(cfg, fmts, seed=1)
    good = tmp_path / "good.lutmac"
    m.save_v2(good)

    def load(path):
        h = ctypes.c_void_p()
        return L.lib().lmx_model_load(str(path).encode(), 64, ctypes.byref(h))

    m.rotated[(0, "q")] = False                     # ternary weights not rotated
    bad = tmp_path / "unrotated.lutmac"
    m.save_v2(bad)
    assert load(bad) == L.ERR_UNSUPPORTED_FORMAT
    assert b"rotated" in L.lib().lmx_last_error()
    m.rotated[(0, "q")] = True
    # version-1 files cannot hold plane records
    data = bytearray(open(good, "rb").read())
    data[8:12] = (1).to_bytes(4, "little")
    v1 = tmp_path / "v1.lutmac"
    v1.write_bytes(bytes(data))
    assert load(v1) == L.ERR_INVALID_ARGUMENT
