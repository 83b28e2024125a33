"""Seeded synthetic weights and activations for the BASELINE configurations.

Weights are produced directly in the canonical bit-plane form the C ABI takes
(``lmx_planes_desc``): planes[p][row][cols/8], MSB-first within each byte,
plus fp32 scales[stage][row][groups].  All randomness comes from
numpy.random.default_rng(seed), so the same seed gives the same bytes on the
host and in the tests.

Configs:
  1  4-bit N=K=2048, q ~ U{0..15}, zero point 8, scales |N(0,1)|*0.02 per
     128-group, x ~ N(0,1), no rotation.
  2  ternary Llama-3.2-1B projection shapes, t ~ U{-1,0,+1}, per-row absmean
     scale of a latent N(0,0.02) row, x ~ N(0,1) with 0.5% of channels x20,
     rotated before the table build.
  3  N=K=8192 sweep: binary, RRQ-2, RRQ-3 (stage scales decay x0.5), 4-bit,
     8-bit (q ~ U{-127..127}), per-128-group scales, x ~ N(0,1) rotated.
"""
import numpy as np

from . import (FMT_BINARY, FMT_INT3, FMT_INT4, FMT_INT8, FMT_RRQ2, FMT_RRQ3,
               FMT_TERNARY, PLANES, STAGES)

LLAMA_TERNARY_SHAPES = {  # (rows N, cols K)
    "q_proj": (2048, 2048), "o_proj": (2048, 2048),
    "k_proj": (512, 2048), "v_proj": (512, 2048),
    "gate_proj": (8192, 2048), "up_proj": (8192, 2048),
    "down_proj": (2048, 8192),
}


def pack_bits(bits):
    """bool/uint8 array [rows, cols] -> bytes [rows, cols/8], MSB-first."""
    return np.packbits(bits.astype(np.uint8), axis=-1, bitorder="big")


def planes_from_ints(fmt, q):
    """Integer weight codes [rows, cols] -> canonical planes [P, rows, cols/8].

    ternary: q in {-1,0,1} -> (sign, zero); binary/RRQ: q is [S, rows, cols]
    of {0,1} stage bits; int3/int4: unsigned codes; int8: signed int8.
    """
    if fmt == FMT_TERNARY:
        return np.stack([pack_bits(q < 0), pack_bits(q == 0)])
    if fmt in (FMT_BINARY, FMT_RRQ2, FMT_RRQ3):
        q = q.reshape((-1,) + q.shape[-2:])
        return np.stack([pack_bits(q[i]) for i in range(q.shape[0])])
    u = q.astype(np.uint8)
    return np.stack([pack_bits((u >> p) & 1) for p in range(PLANES[fmt])])


def int_values(fmt, planes, stage=0):
    """Canonical planes -> integer weight values [rows, cols] (per stage)."""
    bits = np.unpackbits(planes, axis=-1, bitorder="big").astype(np.int64)
    if fmt == FMT_TERNARY:
        return np.where(bits[1] == 1, 0, np.where(bits[0] == 1, -1, 1))
    if fmt in (FMT_BINARY, FMT_RRQ2, FMT_RRQ3):
        return 2 * bits[stage] - 1
    q = sum(bits[p] << p for p in range(PLANES[fmt]))
    if fmt == FMT_INT3:
        return q - 4
    if fmt == FMT_INT4:
        return q - 8
    return np.where(q >= 128, q - 256, q)


def dequant_f64(fmt, planes, scales, rows, cols, group):
    """fp64 dense weights W[rows, cols] from canonical planes and scales."""
    ng = 1 if group == 0 else -(-cols // group)
    sc = np.asarray(scales, np.float64).reshape(STAGES[fmt], rows, ng)
    g = np.arange(cols) // (cols if group == 0 else group)
    W = np.zeros((rows, cols))
    for s in range(STAGES[fmt]):
        W += int_values(fmt, planes, s)[:, :cols] * sc[s][:, g]
    return W


def group_scales(rng, rows, cols, group=128, stages=1, decay=0.5):
    ng = -(-cols // group)
    s1 = (np.abs(rng.standard_normal((rows, ng))) * 0.02).astype(np.float32)
    return np.stack([(s1 * decay ** i).astype(np.float32) for i in range(stages)])


def make_weights(fmt, rows, cols, seed, group=128):
    """Synthetic weights of `fmt` as in BASELINE configs 1-3.

    group is the scale group along K (multiple of 128), or 0 for one scale
    per row (ternary only: config 2's absmean row scale).
    Returns (planes [P, rows, cols/8] uint8, scales [S, rows, ng] fp32, group).
    """
    rng = np.random.default_rng(seed)
    if fmt == FMT_TERNARY:
        t = rng.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        if group:
            return planes_from_ints(fmt, t), group_scales(rng, rows, cols, group, 1), group
        # config 2: one absmean scale per row of a latent N(0, 0.02) row
        latent = rng.standard_normal((rows, cols), dtype=np.float32) * 0.02
        s = np.abs(latent).mean(axis=1, dtype=np.float64).astype(np.float32)
        return planes_from_ints(fmt, t), s.reshape(1, rows, 1), 0
    if fmt in (FMT_BINARY, FMT_RRQ2, FMT_RRQ3):
        S = STAGES[fmt]
        bits = rng.integers(0, 2, size=(S, rows, cols), dtype=np.uint8)
        return planes_from_ints(fmt, bits), group_scales(rng, rows, cols, group, S), group
    if fmt == FMT_INT4:
        q = rng.integers(0, 16, size=(rows, cols), dtype=np.uint8)
    elif fmt == FMT_INT3:
        q = rng.integers(0, 8, size=(rows, cols), dtype=np.uint8)
    elif fmt == FMT_INT8:
        q = rng.integers(-127, 128, size=(rows, cols), dtype=np.int16).astype(np.int8)
    else:
        raise ValueError(f"unknown format {fmt}")
    return planes_from_ints(fmt, q), group_scales(rng, rows, cols, group, 1), group


def make_activations(cols, seed, outliers=False):
    """x ~ N(0,1); with outliers, ceil(0.005*cols) seeded channels x20."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(cols).astype(np.float32)
    if outliers:
        idx = rng.choice(cols, size=int(np.ceil(0.005 * cols)), replace=False)
        x[idx] *= 20.0
    return x


def algorithmic_bytes(fmt, rows, cols, group=128, batch=1):
    """B = N*K*P/8 + 4*S_count + 4*K*batch + 4*N*batch (planes, scales, x, y)."""
    P = PLANES[fmt]
    n_scales = rows if group == 0 else rows * (-(-cols // group)) * STAGES[fmt]
    return rows * cols * P // 8 + 4 * n_scales + 4 * cols * batch + 4 * rows * batch
