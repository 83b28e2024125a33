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


# ---- decoder forward (oracle restatement and the reference's Model) -------

class OrcMatrix(ctypes.Structure):
    _fields_ = [("fmt", ctypes.c_int), ("planes", _p), ("scales", _p), ("rows", _sz), ("cols", _sz),
                ("group", _sz)]


class OrcModel(ctypes.Structure):
    _fields_ = [("hidden", _sz), ("n_layers", _sz), ("n_heads", _sz), ("n_kv_heads", _sz),
                ("head_dim", _sz), ("ffn", _sz), ("vocab", _sz), ("max_seq", _sz),
                ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("rope_mode", ctypes.c_int),
                ("rope_factor", ctypes.c_float), ("rope_low_freq_factor", ctypes.c_float),
                ("rope_high_freq_factor", ctypes.c_float), ("rope_orig_max_pos", _sz),
                ("qkv", ctypes.POINTER(OrcMatrix)), ("o", ctypes.POINTER(OrcMatrix)),
                ("gate_up", ctypes.POINTER(OrcMatrix)), ("down", ctypes.POINTER(OrcMatrix)),
                ("in_norm", _p), ("post_norm", _p), ("qkv_bias", _p), ("head", OrcMatrix),
                ("final_norm", _p), ("kcache", _p), ("vcache", _p)]


class OracleDecoder:
    """orc_decode_step over a model in canonical planes (4-bit, fused q|k|v and
    gate|up rows): teacher-forced logits for the parity tests."""

    def __init__(self, model):
        L = lib()
        L.orc_decode_step.argtypes = [ctypes.POINTER(OrcModel), ctypes.c_int, _sz, _p]
        L.orc_decode_step.restype = ctypes.c_int
        c = model.cfg
        self.cfg, self._keep = c, []

        def mat(entry, rows, cols):
            # (planes, scales) of the model's 4-bit group, or (planes, scales, format, group)
            fmt, g = (entry[2], entry[3]) if len(entry) == 4 else (FMT_INT4, model.group)
            pl, sc = np.ascontiguousarray(entry[0], np.uint8), f32(entry[1])
            self._keep += [pl, sc]
            return OrcMatrix(fmt, _ptr(pl), _ptr(sc), rows, cols, g if g else cols)

        shapes = model.shapes()
        arrs = {}
        for n in ("qkv", "o", "gate_up", "down"):
            arrs[n] = (OrcMatrix * c.n_layers)(*[mat(Ly[n], *shapes[n]) for Ly in model.layers])
        self._keep.append(arrs)
        in_norm = f32(np.concatenate([Ly["in_norm"] for Ly in model.layers]))
        post_norm = f32(np.concatenate([Ly["post_norm"] for Ly in model.layers]))
        bias = None
        if model.layers[0]["qkv_bias"] is not None:
            bias = f32(np.concatenate([Ly["qkv_bias"] for Ly in model.layers]))
        self.kc = np.zeros(c.n_layers * c.max_seq * c.kv_dim, np.float32)
        self.vc = np.zeros_like(self.kc)
        fn = f32(model.final_norm)
        self._keep += [in_norm, post_norm, bias, fn]
        self.m = OrcModel(c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn, c.vocab, c.max_seq,
                          c.rms_eps, c.rope_theta, c.rope_mode, c.rope_factor, c.rope_low_freq_factor,
                          c.rope_high_freq_factor, c.rope_orig_max_pos, arrs["qkv"], arrs["o"], arrs["gate_up"],
                          arrs["down"], _ptr(in_norm), _ptr(post_norm), _ptr(bias),
                          mat(model.head, c.vocab, c.hidden), _ptr(fn), _ptr(self.kc), _ptr(self.vc))

    def step(self, token, pos):
        logits = np.zeros(self.cfg.vocab, np.float32)
        rc = lib().orc_decode_step(ctypes.byref(self.m), int(token), pos, _ptr(logits))
        if rc != 0:
            raise ValueError(f"orc_decode_step failed ({rc})")
        return logits


def greedy_pick(logits, history, penalty=1.0):
    """Greedy Model::sample (src/model.cpp:455-490 with temperature 0): the
    repetition penalty of :458-469 -- for every token of the history, once per
    occurrence, a positive logit is divided by the penalty and any other
    multiplied by it -- then the first maximum (:480-490).  Returns (token,
    penalised logits).  Pinned to the reference's own sample() by
    tests/test_decode_cpu.py."""
    v = f32(logits).copy()
    if penalty != 1.0:
        p = np.float32(penalty)
        for t in history:
            if 0 <= t < v.size:
                v[t] = v[t] / p if v[t] > 0 else v[t] * p
    return int(np.argmax(v)), v


def ref_greedy_pick(logits, history, penalty):
    """The reference's own Model::sample, greedy (oracle/_ref): (token, penalised logits)."""
    R = RefDecoder._bind()
    lg = f32(logits)
    h = np.ascontiguousarray(history, np.int32)
    out = np.zeros_like(lg)
    t = R.ref_greedy_sample(_ptr(lg), lg.size, _ptr(h), h.size, penalty, _ptr(out))
    return t, out


_SPREAD = None


def int4_blocks_from_planes(planes, scales):
    """Canonical 4-bit planes [4, rows, cols/8] + group-256 scales [1, rows, cols/256]
    -> the reference's Int4Block bytes (types.hpp:174-202: even index in the high nibble)."""
    global _SPREAD
    if _SPREAD is None:   # plane byte -> its 8 bits at nibble positions, weight j at nibble 7-j
        b = np.arange(256, dtype=np.uint32)
        _SPREAD = sum(((b >> (7 - j)) & 1) << (4 * (7 - j)) for j in range(8)).astype(np.uint32)
    rows, rb = planes.shape[1], planes.shape[2]
    codes = (_SPREAD[planes[0]] | (_SPREAD[planes[1]] << 1) | (_SPREAD[planes[2]] << 2)
             | (_SPREAD[planes[3]] << 3))                                  # [rows, cols/8] x 8 nibbles
    data = codes.astype(">u4").view(np.uint8).reshape(rows, rb * 4)      # byte i = q[2i] << 4 | q[2i+1]
    nb = rb * 8 // 256
    out = np.empty((rows, nb, 132), np.uint8)
    out[:, :, :128] = data.reshape(rows, nb, 128)
    out[:, :, 128:] = f32(scales[0].reshape(rows, nb)).view(np.uint8).reshape(rows, nb, 4)
    return out.reshape(-1)


class RefDecoder:
    """The reference's own Model::forward (oracle/_ref/libref.so) on a 4-bit model with
    group-256 scales and the reference's RoPE form: teacher-forced logits."""

    @staticmethod
    def _bind():
        R = ref()
        if R is None:
            raise RuntimeError("oracle/_ref/libref.so not built")
        for name, args, res in [
            ("ref_model_create", [_sz] * 8 + [ctypes.c_float] * 3, _p),
            ("ref_model_set_linear", [_p, _sz, ctypes.c_int, _p, _sz, _sz, _sz], None),
            ("ref_model_set_norms", [_p, _sz, _p, _p], None),
            ("ref_model_set_embed", [_p, _p, _sz, _p], None),
            ("ref_model_set_embed_fmt", [_p, ctypes.c_int, _p, _sz, _p], None),
            ("ref_model_set_biases", [_p, _sz, _p, _p, _p], None),
            ("ref_model_save", [_p, ctypes.c_char_p, ctypes.c_int], ctypes.c_int),
            ("ref_model_load", [ctypes.c_char_p], _p),
            ("ref_model_forward", [_p, ctypes.c_int, _sz, _p], None),
            ("ref_model_destroy", [_p], None),
            ("ref_greedy_sample", [_p, _sz, _p, _sz, ctypes.c_float, _p], ctypes.c_int),
        ]:
            f = getattr(R, name)
            f.argtypes, f.restype = args, res
        return R

    @classmethod
    def from_file(cls, path, vocab):
        """The reference's own load_model of a .lutmac file."""
        R = cls._bind()
        self = cls.__new__(cls)
        self.h = R.ref_model_load(str(path).encode())
        if not self.h:
            raise ValueError(f"reference load_model failed for {path}")
        self.vocab = vocab
        return self

    def save(self, path, with_biases=False):
        """Writes the model with the reference's own save_lutmac."""
        if ref().ref_model_save(self.h, str(path).encode(), int(with_biases)) != 1:
            raise ValueError("reference save_lutmac failed")

    def set_embedding(self, fmt, blocks, final_norm):
        """Replaces the (tied) embedding with reference blocks of format 6 or 7."""
        blocks = np.ascontiguousarray(blocks, np.uint8)
        fn = f32(final_norm)
        ref().ref_model_set_embed_fmt(self.h, fmt, _ptr(blocks), blocks.size // BLOCK_BYTES[fmt], _ptr(fn))

    def __init__(self, model, blocks=None):
        R = self._bind()
        c = model.cfg
        assert model.group == 256 and c.rope_mode == 0, "reference model: group-256 blocks, reference RoPE"
        self.cfg, self.vocab = c, c.vocab
        self.h = R.ref_model_create(c.hidden, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.ffn, c.vocab,
                                    c.max_seq, c.rms_eps, c.rope_theta, c.rope_factor)
        qd, kvd = c.q_dim, c.kv_dim
        for i, Ly in enumerate(model.layers):
            pl, sc = Ly["qkv"]
            parts = [(0, 0, qd), (1, qd, qd + kvd), (2, qd + kvd, qd + 2 * kvd)]
            for which, a, b in parts:
                self._set(i, which, pl[:, a:b], sc[:, a:b], b - a, c.hidden)
            pl, sc = Ly["gate_up"]
            self._set(i, 4, pl[:, :c.ffn], sc[:, :c.ffn], c.ffn, c.hidden)
            self._set(i, 5, pl[:, c.ffn:], sc[:, c.ffn:], c.ffn, c.hidden)
            self._set(i, 3, *Ly["o"], c.hidden, qd)
            self._set(i, 6, *Ly["down"], c.hidden, c.ffn)
            a, b = f32(Ly["in_norm"]), f32(Ly["post_norm"])
            R.ref_model_set_norms(self.h, i, _ptr(a), _ptr(b))
            if Ly["qkv_bias"] is not None:
                qb = f32(Ly["qkv_bias"])
                R.ref_model_set_biases(self.h, i, _ptr(qb[:qd].copy()), _ptr(qb[qd:qd + kvd].copy()),
                                       _ptr(qb[qd + kvd:].copy()))
        blk = int4_blocks_from_planes(*model.head)
        fn = f32(model.final_norm)
        R.ref_model_set_embed(self.h, _ptr(blk), blk.size // 132, _ptr(fn))

    def _set(self, layer, which, planes, scales, rows, cols):
        blk = int4_blocks_from_planes(np.ascontiguousarray(planes), np.ascontiguousarray(scales))
        ref().ref_model_set_linear(self.h, layer, which, _ptr(blk), blk.size // 132, rows, cols)

    def step(self, token, pos):
        logits = np.zeros(self.vocab, np.float32)
        ref().ref_model_forward(self.h, int(token), pos, _ptr(logits))
        return logits

    def close(self):
        if self.h:
            ref().ref_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
