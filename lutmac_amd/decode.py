"""Host side of the device-resident decoder (include/lutmac_decode.h).

Mirrors the reference engine's model path (src/model.cpp:47-490): a
Llama/Qwen-style config, a seeded random-init model whose linears are
quantized to 4-bit with the reference's rule (quantize.hpp:444-461: scale =
absmax/7 per group, q = round(w/scale) clamped to [-7, 7], stored q + 8),
and a ``Decoder`` that uploads it as LUT-GEMV weight handles and runs token
steps or whole greedy generations on the GPU.

Weights are kept in the canonical plane form (planes[p][row][cols/8],
scales[1][row][cols/group]) with the fused layouts the device decoder takes:
q|k|v rows in one matrix and gate|up rows in one matrix.
"""
import ctypes
from dataclasses import dataclass, replace

import numpy as np

from . import (FMT_INT4, DecoderConfigC, Weight, _np_ptr, _stream_ptr, check, lib, synth_int4_normal)

ROPE_REFERENCE = 0
ROPE_LLAMA3 = 1


@dataclass(frozen=True)
class DecoderConfig:
    hidden: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_seq: int
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_mode: int = ROPE_LLAMA3
    rope_factor: float = 32.0
    rope_low_freq_factor: float = 1.0
    rope_high_freq_factor: float = 4.0
    rope_orig_max_pos: int = 8192
    qkv_bias: bool = False

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def c_struct(self):
        return DecoderConfigC(self.hidden, self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim,
                              self.ffn, self.vocab, self.max_seq, self.rms_eps, self.rope_theta,
                              self.rope_mode, self.rope_factor, self.rope_low_freq_factor,
                              self.rope_high_freq_factor, self.rope_orig_max_pos)


# Llama-3.2-1B architecture, 64 prompt + 256 new tokens.
LLAMA_3_2_1B = DecoderConfig(hidden=2048, n_layers=16, n_heads=32, n_kv_heads=8, head_dim=64, ffn=8192,
                             vocab=128256, max_seq=320)
# Qwen-2.5-1.5B architecture (QKV bias, theta 1e6, no scaling).
QWEN_2_5_1_5B = DecoderConfig(hidden=1536, n_layers=28, n_heads=12, n_kv_heads=2, head_dim=128, ffn=8960,
                              vocab=151936, max_seq=2048, rms_eps=1e-6, rope_theta=1000000.0,
                              rope_mode=ROPE_REFERENCE, rope_factor=1.0, qkv_bias=True)


def round_half_away(v):
    """std::round on float32 values (halves away from zero)."""
    r = np.round(v)
    frac = np.abs(v - np.trunc(v))
    half = frac == np.float32(0.5)
    if half.any():
        r[half] = np.trunc(v[half]) + np.sign(v[half])
    return r


def quantize_int4_np(w, group):
    """numpy restatement of lmx_quantize_int4 (checks the C++ producer): fp32 [rows, cols]
    -> (planes [4, rows, cols/8], scales [1, rows, cols/group]) with the reference's
    4-bit rule (quantize.hpp:437-461) applied per `group` weights, in the arithmetic
    of its -ffast-math build (scale = absmax * (1/7), q = round(w / scale))."""
    rows, cols = w.shape
    g = w.reshape(rows, cols // group, group)
    scale = (np.abs(g).max(axis=2) * np.float32(1.0 / 7.0)).astype(np.float32)
    live = scale > np.float32(1e-10)
    safe = np.where(live, scale, np.float32(1.0))
    q = round_half_away((g / safe[:, :, None]).astype(np.float32)) * live[:, :, None]
    q = (np.clip(q, -7, 7).astype(np.int16) + 8).astype(np.uint8).reshape(rows, cols)
    planes = np.stack([np.packbits((q >> p) & 1, axis=1, bitorder="big") for p in range(4)])
    return planes, scale[None]


class SyntheticModel:
    """Seeded random-init decoder: linears N(0, 0.02) quantized to 4-bit per `group`;
    norm weights 1 (or 1 + 0.1 N(0,1) with ``random_norms``); tied embedding/head."""

    def __init__(self, cfg, seed=0, group=128, random_norms=False):
        self.cfg, self.group = cfg, group
        rng = np.random.default_rng(seed)
        stream = iter(range(1 << 30))

        def lin(rows, cols):   # matrix i of the model draws from generator stream i
            return synth_int4_normal(seed, next(stream), rows, cols, 0.02, group)

        def norm():
            if random_norms:
                return (1.0 + 0.1 * rng.standard_normal(cfg.hidden)).astype(np.float32)
            return np.ones(cfg.hidden, np.float32)

        h = cfg.hidden
        self.layers = []
        for _ in range(cfg.n_layers):
            L = {"qkv": lin(cfg.q_dim + 2 * cfg.kv_dim, h), "o": lin(h, cfg.q_dim),
                 "gate_up": lin(2 * cfg.ffn, h), "down": lin(h, cfg.ffn),
                 "in_norm": norm(), "post_norm": norm(), "qkv_bias": None}
            if cfg.qkv_bias:
                L["qkv_bias"] = (0.02 * rng.standard_normal(cfg.q_dim + 2 * cfg.kv_dim)).astype(np.float32)
            self.layers.append(L)
        self.head = lin(cfg.vocab, h)
        self.final_norm = norm()

    def shapes(self):
        c = self.cfg
        return {"qkv": (c.q_dim + 2 * c.kv_dim, c.hidden), "o": (c.hidden, c.q_dim),
                "gate_up": (2 * c.ffn, c.hidden), "down": (c.hidden, c.ffn)}


def _fuse(parts):
    """Row-wise concatenation of plane-form matrices (planes [P, rows, cols/8],
    scales [S, rows, groups], same format and group)."""
    return (np.concatenate([p[0] for p in parts], axis=1), np.concatenate([p[1] for p in parts], axis=1),
            parts[0][2], parts[0][3])


class QuantizedModel:
    """A decoder whose linears are quantized from fp32 weights with lmx_quantize
    in any format (the reference quantize tool's role, tools/lutmac-quantize.cpp):
    ``formats`` maps q, k, v, o, gate, up, down, embed to (format, group, flags);
    ternary, binary and RRQ weights get the tool's FWHT (LMX_QUANT_ROTATE).  The
    fp32 weights are seeded N(0, 0.02) (lmx_synth_normal, one generator stream
    per matrix); norms 1 + 0.1 N(0,1).  layers[i] holds the fused q|k|v and
    gate|up matrices as (planes, scales, format, group), the form Decoder and
    the oracle take; ``save_v2`` writes the unfused tensors as a .lutmac
    version-2 file."""

    NAMES = ("q", "k", "v", "o", "gate", "up", "down")

    def __init__(self, cfg, formats, seed=0):
        from . import quantize, synth_normal, QUANT_ROTATE
        from .lutmac_file import ROTATED
        self.cfg, self.formats, self.group = cfg, formats, 0
        rng = np.random.default_rng(seed)
        stream = iter(range(1 << 30))
        h = cfg.hidden
        shapes = {"q": (cfg.q_dim, h), "k": (cfg.kv_dim, h), "v": (cfg.kv_dim, h), "o": (h, cfg.q_dim),
                  "gate": (cfg.ffn, h), "up": (cfg.ffn, h), "down": (h, cfg.ffn), "embed": (cfg.vocab, h)}

        def quant(name):
            fmt, group, flags = formats[name]
            w = synth_normal(seed, next(stream), *shapes[name], 0.02)
            rot = fmt in ROTATED
            pl, sc, g = quantize(fmt, w, group, flags | (QUANT_ROTATE if rot else 0))
            return (pl, sc, fmt, g), rot

        self.raw, self.rotated, self.layers = [], {}, []
        for i in range(cfg.n_layers):
            mats = {}
            for n in self.NAMES:
                mats[n], self.rotated[(i, n)] = quant(n)
            L = {"qkv": _fuse([mats["q"], mats["k"], mats["v"]]), "o": mats["o"],
                 "gate_up": _fuse([mats["gate"], mats["up"]]), "down": mats["down"],
                 "in_norm": (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32),
                 "post_norm": (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32), "qkv_bias": None}
            self.raw.append(mats)
            self.layers.append(L)
        self.head, rot = quant("embed")
        if rot:
            raise ValueError("the embedding is read row by row: use int3, int4 or int8")
        self.final_norm = (1.0 + 0.1 * rng.standard_normal(h)).astype(np.float32)

    def shapes(self):
        return SyntheticModel.shapes(self)

    def save_v2(self, path):
        """The model as a .lutmac version-2 file (plane records, HF tensor names)."""
        from .lutmac_file import Planes, write
        c = self.cfg
        config = {"model_type": "llama", "vocab_size": c.vocab, "hidden_size": c.hidden,
                  "intermediate_size": c.ffn, "num_hidden_layers": c.n_layers,
                  "num_attention_heads": c.n_heads, "num_key_value_heads": c.n_kv_heads, "head_dim": c.head_dim,
                  "rms_norm_eps": c.rms_eps, "rope_theta": c.rope_theta, "rope_scaling_factor": c.rope_factor}
        names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
                 "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
        tensors = [("model.embed_tokens.weight", Planes(self.head[2], self.head[0], self.head[1], self.head[3],
                                                        False))]
        for i, (mats, L) in enumerate(zip(self.raw, self.layers)):
            for n in self.NAMES:
                m = mats[n]
                tensors.append((f"model.layers.{i}.{names[n]}.weight",
                                Planes(m[2], m[0], m[1], m[3], self.rotated[(i, n)])))
            tensors.append((f"model.layers.{i}.input_layernorm.weight", L["in_norm"]))
            tensors.append((f"model.layers.{i}.post_attention_layernorm.weight", L["post_norm"]))
        tensors.append(("model.norm.weight", self.final_norm))
        write(path, config, tensors)


class _DecoderOps:
    """Token-step operations over an lmx_decoder handle (self._h)."""

    cfg = None
    _h = None

    batch = 1

    def reset(self, tokens):
        """tokens: [n], or [batch, n] for a batched decoder."""
        t = np.ascontiguousarray(tokens, np.int32)
        check(lib().lmx_decoder_reset(self._h, _np_ptr(t), t.size // self.batch))

    def set_repetition_penalty(self, penalty):
        """The reference's repetition penalty in the greedy pick (1 = off), from the
        next reset or generate on (lmx_decoder_set_repetition_penalty)."""
        check(lib().lmx_decoder_set_repetition_penalty(self._h, penalty))

    def step(self, logits=None, stream=None):
        """One forward step at the current position; logits (device float32 tensor of
        vocab entries, batch x vocab for a batched decoder) receives the step's logits
        when given."""
        from . import _dev_ptr
        check(lib().lmx_decoder_step(self._h, _dev_ptr(logits), _stream_ptr(stream)))
        return logits

    def tokens(self, n, stream=None):
        out = np.zeros((self.batch, n), np.int32)
        check(lib().lmx_decoder_tokens(self._h, _np_ptr(out), n, _stream_ptr(stream)))
        return out[0] if self.batch == 1 else out

    def generate(self, prompt, n_new, stream=None):
        """Greedy generation; prompt [n_prompt] (or [batch, n_prompt]); returns
        (tokens[n_prompt + n_new] (or [batch, ...]), prefill_ms, decode_ms)."""
        p = np.ascontiguousarray(prompt, np.int32)
        n_prompt = p.size // self.batch
        out = np.zeros((self.batch, n_prompt + n_new), np.int32)
        t0, t1 = ctypes.c_float(), ctypes.c_float()
        check(lib().lmx_decoder_generate(self._h, _np_ptr(p), n_prompt, n_new, _np_ptr(out),
                                         ctypes.byref(t0), ctypes.byref(t1), _stream_ptr(stream)))
        return (out[0] if self.batch == 1 else out), t0.value, t1.value

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Decoder(_DecoderOps):
    """Device decoder over LUT-GEMV weight handles built from a SyntheticModel;
    batch > 1 decodes that many sequences in lockstep."""

    def __init__(self, model, batch=1):
        self.model, self.cfg = model, model.cfg
        self.batch = batch
        self._h = None
        self.weights = []
        self.head = None
        shapes = model.shapes()
        c = self.cfg
        h = ctypes.c_void_p()
        cs = c.c_struct()
        check(lib().lmx_decoder_create_batched(ctypes.byref(cs), batch, ctypes.byref(h)))
        self._h = h
        def weight(entry, rows, cols):
            # (planes, scales) of the model's 4-bit group, or (planes, scales, format, group)
            fmt, g = (entry[2], entry[3]) if len(entry) == 4 else (FMT_INT4, model.group)
            return Weight.from_planes(fmt, entry[0], entry[1], rows, cols, g)

        for i, L in enumerate(model.layers):
            ws = [weight(L[n], *shapes[n]) for n in ("qkv", "o", "gate_up", "down")]
            self.weights += ws
            bias = None if L["qkv_bias"] is None else L["qkv_bias"]
            check(lib().lmx_decoder_set_layer(self._h, i, *[w.handle for w in ws], _np_ptr(L["in_norm"]),
                                              _np_ptr(L["post_norm"]),
                                              None if bias is None else _np_ptr(bias)))
        self.head = weight(model.head, c.vocab, c.hidden)
        check(lib().lmx_decoder_set_head(self._h, self.head.handle, self.head.handle, _np_ptr(model.final_norm)))

    def close(self):
        if self._h:
            lib().lmx_decoder_destroy(self._h)
            self._h = None
        for w in self.weights:
            w.close()
        self.weights = []
        if self.head is not None:
            self.head.close()
            self.head = None


class LutmacModel(_DecoderOps):
    """A .lutmac v1 file loaded onto the device decoder (lutmac_model.h): the
    counterpart of load_model (src/model.cpp:576-701)."""

    def __init__(self, path, max_seq=0):
        m = ctypes.c_void_p()
        check(lib().lmx_model_load(str(path).encode(), max_seq, ctypes.byref(m)))
        self._m = m
        cs = DecoderConfigC()
        check(lib().lmx_model_config(self._m, ctypes.byref(cs)))
        self.config_c = cs
        self.cfg = DecoderConfig(cs.hidden, cs.n_layers, cs.n_heads, cs.n_kv_heads, cs.head_dim, cs.ffn, cs.vocab,
                                 cs.max_seq, cs.rms_eps, cs.rope_theta, cs.rope_mode, cs.rope_factor,
                                 cs.rope_low_freq_factor, cs.rope_high_freq_factor, cs.rope_orig_max_pos)
        self._h = ctypes.c_void_p(lib().lmx_model_decoder(self._m))

    def weight_format(self, layer, which=0):
        f = ctypes.c_int()
        check(lib().lmx_model_weight_format(self._m, layer, which, ctypes.byref(f)))
        return f.value

    def close(self):
        if getattr(self, "_m", None):
            lib().lmx_model_destroy(self._m)
            self._m = None
            self._h = None


def small_config(**kw):
    """A small model of the same architecture for parity tests (cols multiples of 256)."""
    base = DecoderConfig(hidden=256, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000,
                         max_seq=64)
    return replace(base, **kw)
