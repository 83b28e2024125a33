"""Write the golden fixtures under tests/golden/ from the reference's own code.

Runs only where oracle/_ref/libref.so was built from the LutMac sources
(oracle/Makefile; this container).  Inputs are seeded numpy draws; every
expected output comes from the reference kernels, quantizers and accessors
(through oracle/ref_shim.cpp).  The fixtures are data only: inputs and the
reference's outputs.

    python tests/golden/gen_golden.py
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

P = oracle._ptr


def main():
    R = oracle.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libref.so not built (make -C oracle)")
    rng = np.random.default_rng(20260101)

    # Tables and FWHT-256 (scalar branch) on 512 activations.
    x = rng.standard_normal(512).astype(np.float32)
    luts = np.zeros(128 * 16, np.float32)
    R.ref_precompute_luts(P(x), 512, P(luts))
    xr = x.copy()
    R.ref_apply_hadamard_rotation(P(xr), 512)
    luts_rot = np.zeros(128 * 16, np.float32)
    R.ref_precompute_luts(P(xr), 512, P(luts_rot))
    np.savez(os.path.join(HERE, "tables_fwht.npz"), x=x, luts=luts, x_rot=xr, luts_rot=luts_rot)

    # Ternary index extraction over 256 groups of random sign/zero bytes.
    s = rng.integers(0, 256, 128, dtype=np.uint8)
    z = rng.integers(0, 256, 128, dtype=np.uint8)
    pos = np.zeros(256, np.uint8)
    neg = np.zeros(256, np.uint8)
    for g in range(256):
        a, b = ctypes.c_uint8(), ctypes.c_uint8()
        R.ref_extract_indices(P(s), P(z), g, ctypes.byref(a), ctypes.byref(b))
        pos[g], neg[g] = a.value, b.value
    np.savez(os.path.join(HERE, "indices.npz"), sign=s, zero=z, pos=pos, neg=neg)

    # Ternary bit-plane packing of 1000 values (ragged last byte).
    t = rng.integers(-1, 2, 1000, dtype=np.int8)
    sp = np.zeros(125, np.uint8)
    zp = np.zeros(125, np.uint8)
    R.ref_pack_to_bitplanes(P(t), 1000, P(sp), P(zp))
    back = np.zeros(1000, np.int8)
    R.ref_unpack_from_bitplanes(P(sp), P(zp), 1000, P(back))
    np.savez(os.path.join(HERE, "bitplanes.npz"), ternary=t, sign=sp, zero=zp, unpacked=back)

    # Per format: reference-quantized blocks, their dequantized weights
    # (block.get), and lut_linear outputs with bias at batch 2.
    # K=640 gives 3 blocks per row with the last one padded.  The reference's
    # 2-bit and 3-bit quantizers index the tensor flat (quantize.hpp:949-972,
    # 1013-1036), so with a ragged K their rows misalign and trailing blocks
    # get scale 0, which the reference kernels turn into NaN (x/0); those two
    # formats use K=768.
    M, batch = 32, 2
    for fmt, name in [(1, "ternary"), (2, "binary"), (3, "int2"), (5, "int3"), (6, "int4"), (7, "int8")]:
        K = 768 if fmt in (3, 5) else 640
        bpr = (K + 255) // 256
        w = (rng.standard_normal(M * K) * 0.05).astype(np.float32)
        nb = M * bpr
        cap = nb * R.ref_sizeof_block(fmt)
        blocks = np.zeros(cap, np.uint8)
        n = R.ref_quantize(fmt, P(w), M, K, P(blocks), cap)
        assert n == cap
        if fmt == 3:
            # The reference 2-bit quantizer never sets scale2 (quantize.hpp:951);
            # give the residual stage a scale of half the primary one.
            bv = blocks.reshape(nb, 72)
            s1 = bv[:, 64:68].copy().view(np.float32)
            bv[:, 68:72] = (s1 * 0.5).astype(np.float32).view(np.uint8)
        deq = np.array([R.ref_block_get(fmt, P(blocks), b, i) for b in range(nb) for i in range(256)],
                       np.float32)
        xs = rng.standard_normal(batch * K).astype(np.float32)
        bias = rng.standard_normal(M).astype(np.float32)
        y = np.zeros(batch * M, np.float32)
        assert R.ref_lut_linear(fmt, P(blocks), nb, P(bias), P(xs), P(y), M, K, batch) == 0
        y_nobias = np.zeros(batch * M, np.float32)
        assert R.ref_lut_linear(fmt, P(blocks), nb, None, P(xs), P(y_nobias), M, K, batch) == 0
        np.savez_compressed(os.path.join(HERE, f"blocks_{name}.npz"), fmt=fmt, M=M, K=K, blocks=blocks,
                 dequant=deq, x=xs, bias=bias, y=y, y_nobias=y_nobias)
    quantizer_fixtures(R)
    print("golden fixtures written to", HERE)


def quantizer_fixtures(R):
    """The reference quantizers (quantize_tensor, _binary, _int2) on seeded
    N(0, 0.02) weights, plain and after the tool's weight rotation
    (apply_hadamard_rotation over the tensor, tools/lutmac-quantize.cpp:426-447),
    and _int3 / _int8 on the plain weights (the tool never rotates them):
    inputs and the reference's block bytes (own generator, so the fixtures
    above are unchanged)."""
    rng = np.random.default_rng(20260202)
    M, K = 24, 768
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    w[5] = 0.0   # an all-zero row (ternary scale 1, binary scale 0)
    out = {"w": w}
    for fmt, name in [(1, "ternary"), (2, "binary"), (3, "int2")]:
        for rot in (False, True):
            src = w.copy()
            if rot:
                R.ref_apply_hadamard_rotation(P(src), src.size)
            n = R.ref_quantize(fmt, P(src), M, K, None, 0)
            blocks = np.zeros(n, np.uint8)
            R.ref_quantize(fmt, P(src), M, K, P(blocks), n)
            out[f"{name}{'_rot' if rot else ''}"] = blocks
    for fmt, name in [(5, "int3"), (7, "int8")]:
        n = R.ref_quantize(fmt, P(w), M, K, None, 0)
        blocks = np.zeros(n, np.uint8)
        R.ref_quantize(fmt, P(w), M, K, P(blocks), n)
        out[name] = blocks
    np.savez_compressed(os.path.join(HERE, "quantizers.npz"), **out)


if __name__ == "__main__":
    main()
