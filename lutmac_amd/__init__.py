"""lutmac_amd -- MI355X-native bit-serial LUT-GEMV path for LutMac.

Python host side over the C ABI in include/lutmac_hip.h (ctypes, no torch
types in the ABI).  torch is used only for device memory and streams.  The
shared library lutmac_amd/liblutmac_hip.so is built in-tree by
``python -m lutmac_amd.build``; importing this package without it raises, so
nothing can silently fall back to a CPU path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblutmac_hip.so")

# lmx_format (include/lutmac_hip.h)
FMT_TERNARY, FMT_BINARY, FMT_RRQ2, FMT_RRQ3, FMT_INT3, FMT_INT4, FMT_INT8 = range(1, 8)
FORMAT_NAMES = {1: "ternary", 2: "binary", 3: "rrq2", 4: "rrq3", 5: "int3", 6: "int4", 7: "int8"}
PLANES = {1: 2, 2: 1, 3: 2, 4: 3, 5: 3, 6: 4, 7: 8}
STAGES = {1: 1, 2: 1, 3: 2, 4: 3, 5: 1, 6: 1, 7: 1}
BLOCK_BYTES = {1: 68, 2: 36, 3: 72, 5: 100, 6: 132, 7: 260}

ROTATE_NONE, ROTATE_FWHT256, ROTATE_FWHT_FULL = 0, 1, 2

OK, ERR_INVALID_ARGUMENT, ERR_UNSUPPORTED_FORMAT, ERR_NO_DEVICE, ERR_OUT_OF_MEMORY, \
    ERR_LAUNCH_FAILED, ERR_HIP = range(7)

# Every symbol include/lutmac_hip.h declares (checked by the CPU tests).
EXPORTS = [
    "lmx_status_string", "lmx_last_error", "lmx_device_count", "lmx_version",
    "lmx_format_info", "lmx_block_bytes", "lmx_blocks_to_planes", "lmx_planes_to_blocks",
    "lmx_tile_bytes", "lmx_tile_planes", "lmx_untile_planes", "lmx_tile_scales", "lmx_gemv_tiles_noalloc",
    "lmx_weight_create", "lmx_weight_from_blocks", "lmx_weight_destroy", "lmx_weight_info",
    "lmx_weight_kernel_config", "lmx_weight_read_tiles", "lmx_gemv", "lmx_linear", "lmx_fwht256",
    "lmx_precompute_luts", "lmx_extract_indices", "lmx_hbm_read_probe", "lmx_hbm_read_probe_shape",
    "lmx_hbm_read_probe_tiles",
    # include/lutmac_hip_compat.h
    "lmx_host_gemv", "lmx_host_lut_linear", "lmx_host_apply_hadamard_rotation",
    "lmx_host_precompute_luts", "lmx_host_precompute_lut", "lmx_host_extract_indices", "lmx_host_forget",
    "lmx_host_cache_clear",
    # include/lutmac_decode.h
    "lmx_decoder_create", "lmx_decoder_create_batched", "lmx_decoder_destroy", "lmx_decoder_set_layer", "lmx_decoder_set_head",
    "lmx_decoder_reset", "lmx_decoder_step", "lmx_decoder_tokens", "lmx_decoder_generate",
    "lmx_decoder_set_repetition_penalty",
    # include/lutmac_synth.h
    "lmx_quantize_int4", "lmx_quantize", "lmx_synth_int4_normal", "lmx_synth_normal",
    # include/lutmac_model.h
    "lmx_model_load", "lmx_model_destroy", "lmx_model_config", "lmx_model_decoder", "lmx_model_weight_format",
]


class DecoderConfigC(ctypes.Structure):
    """lmx_decoder_config (include/lutmac_decode.h)."""
    _fields_ = [("hidden", ctypes.c_size_t), ("n_layers", ctypes.c_size_t), ("n_heads", ctypes.c_size_t),
                ("n_kv_heads", ctypes.c_size_t), ("head_dim", ctypes.c_size_t), ("ffn", ctypes.c_size_t),
                ("vocab", ctypes.c_size_t), ("max_seq", ctypes.c_size_t), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("rope_mode", ctypes.c_int), ("rope_factor", ctypes.c_float),
                ("rope_low_freq_factor", ctypes.c_float), ("rope_high_freq_factor", ctypes.c_float),
                ("rope_orig_max_pos", ctypes.c_size_t)]


class LmxError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"lmx status {status}: {msg}")
        self.status = status


class PlanesDesc(ctypes.Structure):
    _fields_ = [("format", ctypes.c_int), ("rows", ctypes.c_size_t), ("cols", ctypes.c_size_t),
                ("group", ctypes.c_size_t), ("planes", ctypes.c_void_p), ("scales", ctypes.c_void_p)]


_p, _sz, _i, _u = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint
_SIGS = {
    "lmx_status_string": ([_i], ctypes.c_char_p),
    "lmx_last_error": ([], ctypes.c_char_p),
    "lmx_device_count": ([ctypes.POINTER(_i)], _i),
    "lmx_version": ([], _i),
    "lmx_format_info": ([_i, ctypes.POINTER(_i), ctypes.POINTER(_i)], _i),
    "lmx_block_bytes": ([_i, ctypes.POINTER(_sz)], _i),
    "lmx_blocks_to_planes": ([_i, _p, _sz, _sz, _sz, _p, _p], _i),
    "lmx_planes_to_blocks": ([_i, _p, _p, _sz, _sz, _p, _sz], _i),
    "lmx_tile_bytes": ([_i, _sz, _sz, ctypes.POINTER(_sz)], _i),
    "lmx_tile_planes": ([_i, _p, _sz, _sz, _p], _i),
    "lmx_untile_planes": ([_i, _p, _sz, _sz, _p], _i),
    "lmx_weight_create": ([ctypes.POINTER(PlanesDesc), ctypes.POINTER(_p)], _i),
    "lmx_weight_from_blocks": ([_i, _p, _sz, _sz, _sz, ctypes.POINTER(_p)], _i),
    "lmx_weight_destroy": ([_p], _i),
    "lmx_weight_info": ([_p, ctypes.POINTER(_i), ctypes.POINTER(_sz), ctypes.POINTER(_sz),
                         ctypes.POINTER(_sz)], _i),
    "lmx_weight_kernel_config": ([_p, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)], _i),
    "lmx_weight_read_tiles": ([_p, _p, _sz], _i),
    "lmx_gemv": ([_p, _p, _p, _sz, _u, _p], _i),
    "lmx_linear": ([_p, _p, _p, _p, _sz, _p], _i),
    "lmx_fwht256": ([_p, _sz, _p], _i),
    "lmx_precompute_luts": ([_p, _sz, _u, _p, _p], _i),
    "lmx_extract_indices": ([_p, _p, _sz, _p, _p, _p], _i),
    "lmx_host_gemv": ([_i, _p, _sz, _p, _p, _sz, _sz], _i),
    "lmx_host_lut_linear": ([_i, _p, _sz, _p, _p, _p, _sz, _sz, _sz], _i),
    "lmx_host_apply_hadamard_rotation": ([_p, _sz], _i),
    "lmx_host_forget": ([_p], _i),
    "lmx_hbm_read_probe": ([_p, _sz, _p, _p], _i),
    "lmx_hbm_read_probe_shape": ([_p, _sz, _i, _i, _p, _p], _i),
    "lmx_hbm_read_probe_tiles": ([_p, _p, _i, _sz, _sz, _sz, _p, _p], _i),
    "lmx_tile_scales": ([_i, _p, _sz, _sz, _sz, _p, ctypes.POINTER(_sz)], _i),
    "lmx_gemv_tiles_noalloc": ([_i, _p, _p, _sz, _sz, _sz, _p, _p, _sz, _u, _p], _i),
    "lmx_host_cache_clear": ([], _i),
    "lmx_quantize_int4": ([_p, _sz, _sz, _sz, _p, _p], _i),
    "lmx_quantize": ([_i, _p, _sz, _sz, _sz, _u, _p, _p], _i),
    "lmx_synth_int4_normal": ([ctypes.c_uint64, ctypes.c_uint64, _sz, _sz, ctypes.c_float, _sz, _p, _p], _i),
    "lmx_synth_normal": ([ctypes.c_uint64, ctypes.c_uint64, _sz, _sz, ctypes.c_float, _p], _i),
    "lmx_model_load": ([ctypes.c_char_p, _sz, ctypes.POINTER(_p)], _i),
    "lmx_model_destroy": ([_p], _i),
    "lmx_model_config": ([_p, ctypes.POINTER(DecoderConfigC)], _i),
    "lmx_model_decoder": ([_p], _p),
    "lmx_model_weight_format": ([_p, _i, _i, ctypes.POINTER(_i)], _i),
    "lmx_decoder_create": ([ctypes.POINTER(DecoderConfigC), ctypes.POINTER(_p)], _i),
    "lmx_decoder_create_batched": ([ctypes.POINTER(DecoderConfigC), _sz, ctypes.POINTER(_p)], _i),
    "lmx_decoder_destroy": ([_p], _i),
    "lmx_decoder_set_layer": ([_p, _sz, _p, _p, _p, _p, _p, _p, _p], _i),
    "lmx_decoder_set_head": ([_p, _p, _p, _p], _i),
    "lmx_decoder_reset": ([_p, _p, _sz], _i),
    "lmx_decoder_step": ([_p, _p, _p], _i),
    "lmx_decoder_tokens": ([_p, _p, _sz, _p], _i),
    "lmx_decoder_generate": ([_p, _p, _sz, _sz, _p, ctypes.POINTER(ctypes.c_float),
                              ctypes.POINTER(ctypes.c_float), _p], _i),
    "lmx_host_precompute_luts": ([_p, _sz, _p], _i),
    "lmx_host_precompute_lut": ([_p, _p], _i),
    "lmx_decoder_set_repetition_penalty": ([_p, ctypes.c_float], _i),
    "lmx_host_extract_indices": ([_p, _p, _sz, _p, _p], _i),
}

_LIB = None


def lib():
    """The loaded C-ABI library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m lutmac_amd.build`")
        # torch's wheel carries its own HIP runtime; loading torch first makes
        # the library bind to that same runtime, so torch streams and device
        # pointers are valid in both (a library loaded first pulls in the
        # system runtime, and torch then finds no GPU).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _LIB = L
    return _LIB


def check(status):
    if status != OK:
        raise LmxError(status, lib().lmx_last_error().decode(errors="replace"))


def _np_ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dev_ptr(t):
    """Device pointer of a torch tensor (None passes NULL)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return ctypes.c_void_p(t.data_ptr())


def _stream_ptr(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


# ---- host-only helpers -----------------------------------------------------

def blocks_to_planes(fmt, blocks, rows, cols):
    Kp = (cols + 255) // 256 * 256
    planes = np.zeros(PLANES[fmt] * rows * Kp // 8, np.uint8)
    scales = np.zeros(STAGES[fmt] * rows * (Kp // 256), np.float32)
    blocks = np.ascontiguousarray(blocks, np.uint8)
    check(lib().lmx_blocks_to_planes(fmt, _np_ptr(blocks), rows * (Kp // 256), rows, cols,
                                     _np_ptr(planes), _np_ptr(scales)))
    return planes, scales


def planes_to_blocks(fmt, planes, scales, rows, cols):
    nb = rows * ((cols + 255) // 256)
    out = np.zeros(nb * BLOCK_BYTES[fmt], np.uint8)
    planes = np.ascontiguousarray(planes, np.uint8)
    scales = np.ascontiguousarray(scales, np.float32)
    check(lib().lmx_planes_to_blocks(fmt, _np_ptr(planes), _np_ptr(scales), rows, cols,
                                     _np_ptr(out), nb))
    return out


def tile_scales_bytes(fmt, rows, cols, group):
    """Bytes of the device scale layout (lmx_tile_scales with no buffers)."""
    n = ctypes.c_size_t()
    check(lib().lmx_tile_scales(fmt, None, rows, cols, group, None, ctypes.byref(n)))
    return n.value


def tile_scales(fmt, scales, rows, cols, group):
    """Canonical scales [S, rows, groups] -> the device scale layout (lmx_tile_scales)."""
    n = ctypes.c_size_t(tile_scales_bytes(fmt, rows, cols, group))
    out = np.zeros(n.value // 4, np.float32)
    sc = np.ascontiguousarray(scales, np.float32)
    check(lib().lmx_tile_scales(fmt, _np_ptr(sc), rows, cols, group, _np_ptr(out), ctypes.byref(n)))
    return out


def gemv_tiles_noalloc(fmt, tiles, scales, rows, cols, group, x, y, batch=1, flags=ROTATE_NONE, stream=None):
    """lmx_gemv_tiles_noalloc on device tensors (tiles uint8, scales fp32 in the
    device layouts, x [batch*cols], y [batch*rows]).  The C entry point takes no
    buffer sizes, so every buffer is checked against the shape here first: an
    undersized one raises LmxError instead of reaching the device."""
    need = {
        "tiles": (tiles.numel() * tiles.element_size(), tile_bytes(fmt, rows, cols)),
        "scales": (scales.numel() * scales.element_size(), tile_scales_bytes(fmt, rows, cols, group)),
        "x": (x.numel() * x.element_size(), 4 * batch * cols),
        "y": (y.numel() * y.element_size(), 4 * batch * rows),
    }
    for name, (have, want) in need.items():
        if have < want:
            raise LmxError(ERR_INVALID_ARGUMENT, f"{name} holds {have} bytes, {rows} x {cols} x batch {batch} "
                                                 f"needs {want}")
    check(lib().lmx_gemv_tiles_noalloc(fmt, _dev_ptr(tiles), _dev_ptr(scales), rows, cols, group, _dev_ptr(x),
                                       _dev_ptr(y), batch, flags, _stream_ptr(stream)))
    return y


def tile_bytes(fmt, rows, cols):
    n = ctypes.c_size_t()
    check(lib().lmx_tile_bytes(fmt, rows, cols, ctypes.byref(n)))
    return n.value


def tile_planes(fmt, planes, rows, cols):
    out = np.zeros(tile_bytes(fmt, rows, cols), np.uint8)
    planes = np.ascontiguousarray(planes, np.uint8)
    check(lib().lmx_tile_planes(fmt, _np_ptr(planes), rows, cols, _np_ptr(out)))
    return out


def untile_planes(fmt, tiles, rows, cols):
    out = np.zeros(PLANES[fmt] * rows * cols // 8, np.uint8)
    tiles = np.ascontiguousarray(tiles, np.uint8)
    check(lib().lmx_untile_planes(fmt, _np_ptr(tiles), rows, cols, _np_ptr(out)))
    return out


def quantize_int4(w, group):
    """fp32 [rows, cols] -> (planes [4, rows, cols/8], scales [1, rows, cols/group]) with the
    reference's 4-bit rule per group (lmx_quantize_int4)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    planes = np.zeros((4, rows, cols // 8), np.uint8)
    scales = np.zeros((1, rows, cols // group), np.float32)
    check(lib().lmx_quantize_int4(_np_ptr(w), rows, cols, group, _np_ptr(planes), _np_ptr(scales)))
    return planes, scales


QUANT_ROTATE = 1
QUANT_RESIDUAL = 2


def quantize(fmt, w, group, flags=0):
    """fp32 [rows, cols] -> (planes [P, rows, cols/8], scales [S, rows, groups], group) with
    the reference's rule for the format (lmx_quantize); group 0 = one scale per row."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    ng = 1 if group == 0 else -(-cols // group)
    planes = np.zeros((PLANES[fmt], rows, cols // 8), np.uint8)
    scales = np.zeros((STAGES[fmt], rows, ng), np.float32)
    check(lib().lmx_quantize(fmt, _np_ptr(w), rows, cols, group, flags, _np_ptr(planes), _np_ptr(scales)))
    return planes, scales, group


def synth_int4_normal(seed, stream, rows, cols, std, group):
    """Seeded N(0, std^2) weights quantized to 4-bit planes (lmx_synth_int4_normal)."""
    planes = np.zeros((4, rows, cols // 8), np.uint8)
    scales = np.zeros((1, rows, cols // group), np.float32)
    check(lib().lmx_synth_int4_normal(seed, stream, rows, cols, std, group, _np_ptr(planes), _np_ptr(scales)))
    return planes, scales


def synth_normal(seed, stream, rows, cols, std):
    w = np.zeros((rows, cols), np.float32)
    check(lib().lmx_synth_normal(seed, stream, rows, cols, std, _np_ptr(w)))
    return w


def device_count():
    n = ctypes.c_int()
    lib().lmx_device_count(ctypes.byref(n))
    return n.value


# ---- device weights and compute ---------------------------------------------

class Weight:
    """Device weight handle (lmx_weight); destroyed with the object."""

    def __init__(self, handle):
        self._h = handle
        fmt, rows, cols, nbytes = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().lmx_weight_info(handle, ctypes.byref(fmt), ctypes.byref(rows), ctypes.byref(cols),
                                    ctypes.byref(nbytes)))
        self.format, self.rows, self.cols, self.device_bytes = fmt.value, rows.value, cols.value, nbytes.value

    @classmethod
    def from_planes(cls, fmt, planes, scales, rows, cols, group):
        planes = np.ascontiguousarray(planes, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        d = PlanesDesc(fmt, rows, cols, group, planes.ctypes.data, scales.ctypes.data)
        h = ctypes.c_void_p()
        check(lib().lmx_weight_create(ctypes.byref(d), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_blocks(cls, fmt, blocks, rows, cols):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        nb = rows * ((cols + 255) // 256)
        h = ctypes.c_void_p()
        check(lib().lmx_weight_from_blocks(fmt, _np_ptr(blocks), nb, rows, cols, ctypes.byref(h)))
        return cls(h)

    @property
    def handle(self):
        return self._h

    def kernel_config(self):
        """(full-K configuration or 0 for split-K, split-K k-slice, staged loads)."""
        f, k, st = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        check(lib().lmx_weight_kernel_config(self._h, ctypes.byref(f), ctypes.byref(k), ctypes.byref(st)))
        return f.value, k.value, st.value

    def read_tiles(self):
        out = np.zeros(tile_bytes(self.format, self.rows, self.cols), np.uint8)
        check(lib().lmx_weight_read_tiles(self._h, _np_ptr(out), out.size))
        return out

    def gemv(self, x, y=None, flags=ROTATE_NONE, stream=None):
        import torch
        batch = x.numel() // self.cols
        if y is None:
            y = torch.empty(batch * self.rows, dtype=torch.float32, device=x.device)
        check(lib().lmx_gemv(self._h, _dev_ptr(x), _dev_ptr(y), batch, flags, _stream_ptr(stream)))
        return y

    def linear(self, x, bias=None, y=None, stream=None):
        import torch
        batch = x.numel() // self.cols
        if y is None:
            y = torch.empty(batch * self.rows, dtype=torch.float32, device=x.device)
        check(lib().lmx_linear(self._h, _dev_ptr(bias), _dev_ptr(x), _dev_ptr(y), batch,
                               _stream_ptr(stream)))
        return y

    def close(self):
        if self._h:
            lib().lmx_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def fwht256(x, stream=None):
    """In-place blockwise FWHT-256 of a device tensor."""
    check(lib().lmx_fwht256(_dev_ptr(x), x.numel(), _stream_ptr(stream)))
    return x


def hbm_read_probe(buf, sink, stream=None):
    """One plain streaming read of a device tensor (the achievable-bandwidth
    yardstick, lmx_hbm_read_probe); sink: a device int32 tensor."""
    check(lib().lmx_hbm_read_probe(_dev_ptr(buf), buf.numel() * buf.element_size(), _dev_ptr(sink),
                                   _stream_ptr(stream)))


def hbm_read_probe_shape(buf, sink, loads_in_flight, workgroups, stream=None):
    """The plain read with a chosen launch shape (lmx_hbm_read_probe_shape)."""
    check(lib().lmx_hbm_read_probe_shape(_dev_ptr(buf), buf.numel() * buf.element_size(), loads_in_flight,
                                         workgroups, _dev_ptr(sink), _stream_ptr(stream)))


def hbm_read_probe_tiles(tiles, scales, fmt, rows, cols, group, sink, stream=None):
    """A read of device tiles + scales with the interleaved GEMV's load schedule
    (lmx_hbm_read_probe_tiles); buffer sizes are checked against the shape."""
    if tiles.numel() * tiles.element_size() < tile_bytes(fmt, rows, cols) or \
            scales.numel() * scales.element_size() < tile_scales_bytes(fmt, rows, cols, group):
        raise LmxError(ERR_INVALID_ARGUMENT, "tiles or scales smaller than the shape's layouts")
    check(lib().lmx_hbm_read_probe_tiles(_dev_ptr(tiles), _dev_ptr(scales), fmt, rows, cols, group,
                                         _dev_ptr(sink), _stream_ptr(stream)))


def precompute_luts(x, rotate=False, stream=None):
    import torch
    n = x.numel()
    luts = torch.empty((n // 4) * 16, dtype=torch.float32, device=x.device)
    check(lib().lmx_precompute_luts(_dev_ptr(x), n, ROTATE_FWHT256 if rotate else ROTATE_NONE,
                                    _dev_ptr(luts), _stream_ptr(stream)))
    return luts


def extract_indices(sign_plane, zero_plane, n_groups, stream=None):
    import torch
    pos = torch.empty(n_groups, dtype=torch.uint8, device=sign_plane.device)
    neg = torch.empty(n_groups, dtype=torch.uint8, device=sign_plane.device)
    check(lib().lmx_extract_indices(_dev_ptr(sign_plane), _dev_ptr(zero_plane), n_groups,
                                    _dev_ptr(pos), _dev_ptr(neg), _stream_ptr(stream)))
    return pos, neg


# ---- host-pointer drop-ins (include/lutmac_hip_compat.h) ---------------------

def host_gemv(fmt, blocks, x_padded, M, K):
    """Raw per-format GEMV on host arrays (reference X_gemv semantics)."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    x = np.ascontiguousarray(x_padded, np.float32)
    y = np.zeros(M, np.float32)
    nb = M * ((K + 255) // 256)
    check(lib().lmx_host_gemv(fmt, _np_ptr(blocks), nb, _np_ptr(x), _np_ptr(y), M, K))
    return y


def host_lut_linear(fmt, blocks, x, M, K, bias=None, batch=1):
    """lut_linear on host arrays (reference semantics)."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    y = np.zeros(M * batch, np.float32)
    nb = M * ((K + 255) // 256)
    check(lib().lmx_host_lut_linear(fmt, _np_ptr(blocks), nb, _np_ptr(b), _np_ptr(x), _np_ptr(y), M, K, batch))
    return y


def host_forget(blocks):
    """Drop the cached device copy of a host block array (lmx_host_forget)."""
    check(lib().lmx_host_forget(_np_ptr(blocks)))


def host_cache_clear():
    check(lib().lmx_host_cache_clear())


def host_apply_hadamard_rotation(x):
    x = np.ascontiguousarray(x, np.float32).copy()
    check(lib().lmx_host_apply_hadamard_rotation(_np_ptr(x), x.size))
    return x


def host_precompute_luts(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros((x.size // 4) * 16, np.float32)
    check(lib().lmx_host_precompute_luts(_np_ptr(x), x.size, _np_ptr(out)))
    return out


def host_precompute_lut(a4):
    """precompute_lut on 4 host activations -> the 16-entry table."""
    a = np.ascontiguousarray(a4, np.float32)
    if a.size != 4:
        raise ValueError("precompute_lut takes 4 activations")
    out = np.zeros(16, np.float32)
    check(lib().lmx_host_precompute_lut(_np_ptr(a), _np_ptr(out)))
    return out


def host_extract_indices(sign_plane, zero_plane, group_idx):
    """extract_indices on host plane bytes -> (pos_idx, neg_idx)."""
    s = np.ascontiguousarray(sign_plane, np.uint8)
    z = np.ascontiguousarray(zero_plane, np.uint8)
    if group_idx // 2 >= min(s.size, z.size):
        raise ValueError("group_idx past the plane bytes")
    pos, neg = ctypes.c_uint8(), ctypes.c_uint8()
    check(lib().lmx_host_extract_indices(_np_ptr(s), _np_ptr(z), group_idx, ctypes.byref(pos), ctypes.byref(neg)))
    return pos.value, neg.value
