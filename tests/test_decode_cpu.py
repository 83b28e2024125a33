"""CPU checks of the decoder path's oracle and producer (no GPU).

* The oracle's decode step (oracle/lutmac_oracle.c orc_decode_step) against
  the reference's own Model::forward (src/model.cpp:47-453, built into
  oracle/_ref/libref.so) on small 4-bit models with group-256 blocks.
* The Llama-3 RoPE frequency scaling through properties the published rule
  fixes (unchanged high frequencies, low frequencies / factor, continuity).
* The 4-bit producer (lmx_quantize_int4) against the reference's own
  quantize_tensor_int4 (quantize.hpp:437-461) and a numpy restatement.
* The greedy pick with the repetition penalty (oracle.greedy_pick) against
  the reference's own Model::sample (src/model.cpp:455-490).
"""
import ctypes

import numpy as np
import pytest

import lutmac_amd as L
import oracle
from conftest import TOL, rel_max_err
from lutmac_amd import decode as D

needs_ref = pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref/libref.so not built")


def teacher_forced(dec_a, dec_b, tokens):
    errs = []
    for pos, t in enumerate(tokens):
        a, b = dec_a.step(t, pos), dec_b.step(t, pos)
        errs.append(rel_max_err(a, b))
    return max(errs)


@needs_ref
@pytest.mark.parametrize("rope_factor", [1.0, 32.0])
def test_oracle_decode_matches_reference_model(rope_factor):
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=rope_factor, rope_theta=10000.0)
    m = D.SyntheticModel(cfg, seed=3, group=256, random_norms=True)
    toks = np.random.default_rng(4).integers(0, cfg.vocab, 12)
    assert teacher_forced(oracle.OracleDecoder(m), oracle.RefDecoder(m), toks) < TOL


@needs_ref
def test_oracle_decode_matches_reference_model_hd128():
    cfg = D.small_config(hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=768, rope_mode=D.ROPE_REFERENCE,
                         rope_factor=1.0, rope_theta=1e6, rms_eps=1e-6)
    m = D.SyntheticModel(cfg, seed=5, group=256, random_norms=True)
    toks = np.random.default_rng(6).integers(0, cfg.vocab, 8)
    assert teacher_forced(oracle.OracleDecoder(m), oracle.RefDecoder(m), toks) < TOL


def llama3_freqs(theta, hd, factor, low, high, orig):
    """Frequencies through a one-layer oracle model: recover them from RoPE of a
    unit query (angle = pos * freq for rope_mode LLAMA3)."""
    L_ = oracle.lib()
    L_.orc_rope_freqs.argtypes = [ctypes.POINTER(oracle.OrcModel), ctypes.c_void_p]
    m = oracle.OrcModel()
    m.head_dim, m.rope_theta, m.rope_mode = hd, theta, 1
    m.rope_factor, m.rope_low_freq_factor, m.rope_high_freq_factor, m.rope_orig_max_pos = factor, low, high, orig
    out = np.zeros(hd // 2, np.float32)
    L_.orc_rope_freqs(ctypes.byref(m), oracle._ptr(out))
    return out.astype(np.float64)


def test_llama3_rope_frequency_properties():
    theta, hd, factor, low, high, orig = 500000.0, 64, 32.0, 1.0, 4.0, 8192
    f = llama3_freqs(theta, hd, factor, low, high, orig)
    base = 1.0 / theta ** (np.arange(hd // 2) * 2.0 / hd)
    wl = 2 * np.pi / base
    hi = wl < orig / high            # short wavelengths: untouched
    lo = wl > orig / low             # long wavelengths: divided by the factor
    mid = ~hi & ~lo
    assert hi.any() and lo.any() and mid.any()
    np.testing.assert_allclose(f[hi], base[hi], rtol=1e-6)
    np.testing.assert_allclose(f[lo], base[lo] / factor, rtol=1e-6)
    # in between: strictly between the two limits, and monotone in d
    assert np.all(f[mid] < base[mid]) and np.all(f[mid] > base[mid] / factor)
    assert np.all(np.diff(f) < 0)
    # scaling off (factor 1) leaves every frequency at theta^(-2d/hd)
    np.testing.assert_allclose(llama3_freqs(theta, hd, 1.0, low, high, orig), base, rtol=1e-6)


@needs_ref
@pytest.mark.parametrize("seed", [0, 1])
def test_quantize_int4_matches_reference_quantizer(seed):
    rng = np.random.default_rng(seed)
    M, K = 33, 1024
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    w[3, :256] = 0.0                      # an all-zero block: scale 0, codes 8
    w[5, 7] = 0.5 * (w[5, :256].max())    # exact halves are rare; cover a large spread instead
    nb = M * (K // 256)
    blocks = np.zeros(nb * 132, np.uint8)
    oracle.ref().ref_quantize(6, oracle._ptr(w), M, K, oracle._ptr(blocks), blocks.size)
    planes_ref, scales_ref = oracle.blocks_to_planes(6, blocks, M, K)
    planes, scales = L.quantize_int4(w, 256)
    assert np.array_equal(planes.ravel(), planes_ref)
    assert np.array_equal(scales.ravel(), scales_ref)


def test_quantize_int4_matches_numpy_restatement():
    w = L.synth_normal(9, 2, 70, 1024, 0.02)
    w[0, :128] = 0.0
    w[1, 5] = 1.0
    for group in (128, 256):
        a, b = L.quantize_int4(w, group), D.quantize_int4_np(w, group)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    c = L.synth_int4_normal(9, 2, 70, 1024, 0.02, 128)
    d = L.quantize_int4(L.synth_normal(9, 2, 70, 1024, 0.02), 128)
    assert np.array_equal(c[0], d[0]) and np.array_equal(c[1], d[1])


def test_synth_normal_statistics_and_streams():
    a = L.synth_normal(1, 0, 512, 2048, 0.02).astype(np.float64)
    assert abs(a.mean()) < 1e-4 and abs(a.std() - 0.02) < 2e-4
    assert abs(np.mean(a ** 4) / np.mean(a ** 2) ** 2 - 3.0) < 0.05        # Gaussian kurtosis
    assert np.array_equal(a, L.synth_normal(1, 0, 512, 2048, 0.02))        # seeded
    b = L.synth_normal(1, 1, 512, 2048, 0.02)
    assert abs(np.corrcoef(a.ravel(), b.ravel())[0, 1]) < 0.01               # streams independent
    # rows are independent of the matrix height (keyed by element index)
    assert np.array_equal(L.synth_normal(1, 0, 3, 2048, 0.02), a[:3].astype(np.float32))


def test_synthetic_model_shapes_and_determinism():
    cfg = D.small_config(qkv_bias=True)
    m1, m2 = D.SyntheticModel(cfg, seed=7), D.SyntheticModel(cfg, seed=7)
    s = m1.shapes()
    for n, (r, c) in s.items():
        assert m1.layers[0][n][0].shape == (4, r, c // 8)
        assert m1.layers[0][n][1].shape == (1, r, c // 128)
        assert np.array_equal(m1.layers[1][n][0], m2.layers[1][n][0])
    assert m1.head[0].shape == (4, cfg.vocab, cfg.hidden // 8)
    assert m1.layers[0]["qkv_bias"].shape == (cfg.q_dim + 2 * cfg.kv_dim,)


@needs_ref
def test_oracle_decode_matches_reference_model_bias_and_rope_factor():
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=2.0, rope_theta=10000.0, qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=21, group=256, random_norms=True)
    toks = np.random.default_rng(22).integers(0, cfg.vocab, 10)
    assert teacher_forced(oracle.OracleDecoder(m), oracle.RefDecoder(m), toks) < TOL


@needs_ref
def test_reference_lutmac_round_trip(tmp_path):
    # the reference's own save_lutmac + load_model reproduce the in-memory model exactly
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=10000.0, qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=23, group=256, random_norms=True)
    r = oracle.RefDecoder(m)
    path = tmp_path / "m.lutmac"
    r.save(path, with_biases=True)
    r2 = oracle.RefDecoder.from_file(path, cfg.vocab)
    for pos, t in enumerate(np.random.default_rng(24).integers(0, cfg.vocab, 4)):
        assert np.array_equal(r.step(t, pos), r2.step(t, pos))


def _lutmac_bytes(meta, data=b""):
    import json
    import struct
    js = json.dumps(meta).encode()
    head = b"LUTMAC01" + struct.pack("<II", 1, len(js)) + js
    return head + b"\0" * ((-len(head)) % 256) + data


def test_lutmac_loader_rejects_bad_files(tmp_path):
    import ctypes
    h = ctypes.c_void_p()
    L.lib().lmx_model_load(b"/nonexistent/x.lutmac", 0, ctypes.byref(h))
    assert L.lib().lmx_model_load(b"/nonexistent/x.lutmac", 0, ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    p = tmp_path / "bad.lutmac"
    p.write_bytes(b"NOTLUTMAC" * 4)
    assert L.lib().lmx_model_load(str(p).encode(), 0, ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    cfg = {"model_type": "llama", "vocab_size": 512, "hidden_size": 256, "intermediate_size": 512,
           "num_hidden_layers": 1, "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 64,
           "rms_norm_eps": 1e-5, "rope_theta": 10000.0, "activation": 2, "norm_type": 1}
    def t(name, shape, typ, nb):
        return {"name": name, "shape": shape, "offset": 0, "type": typ, "num_blocks": nb}
    lin = lambda n, r, c, typ="int4": t(f"model.layers.0.{n}", [r, c], typ, r * (c // 256))
    tensors = [t("model.embed_tokens.weight", [512, 256], "int4", 512),
               lin("self_attn.q_proj.weight", 256, 256), lin("self_attn.k_proj.weight", 128, 256),
               lin("self_attn.v_proj.weight", 128, 256), lin("self_attn.o_proj.weight", 256, 256),
               lin("mlp.gate_proj.weight", 512, 256, "int5"), lin("mlp.up_proj.weight", 512, 256),
               lin("mlp.down_proj.weight", 256, 512)]
    p.write_bytes(_lutmac_bytes({"config": cfg, "tensors": tensors}))
    st = L.lib().lmx_model_load(str(p).encode(), 0, ctypes.byref(h))
    assert st == L.ERR_UNSUPPORTED_FORMAT and b"int5" in L.lib().lmx_last_error()
    bad = dict(cfg, activation=1)   # GELU
    p.write_bytes(_lutmac_bytes({"config": bad, "tensors": tensors}))
    assert L.lib().lmx_model_load(str(p).encode(), 0, ctypes.byref(h)) == L.ERR_UNSUPPORTED_FORMAT
    p.write_bytes(_lutmac_bytes({"config": cfg, "tensors": tensors[1:]}))   # no embedding
    assert L.lib().lmx_model_load(str(p).encode(), 0, ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    raw = b"LUTMAC01" + (3).to_bytes(4, "little") + (2).to_bytes(4, "little") + b"{}"
    p.write_bytes(raw)                                                        # version 3
    assert L.lib().lmx_model_load(str(p).encode(), 0, ctypes.byref(h)) == L.ERR_UNSUPPORTED_FORMAT


@needs_ref
@pytest.mark.parametrize("penalty", [1.0, 1.1, 1.7])
def test_greedy_pick_matches_reference_sample(penalty):
    # The reference's sample() penalises the history's tokens (once per
    # occurrence, sign-dependent) before its first-maximum scan; the oracle's
    # restatement must rank the same values and pick the same token.  The
    # reference is built with -ffast-math, which may turn the division into a
    # multiplication by 1/penalty: 1 ulp per application is allowed.
    rng = np.random.default_rng(int(penalty * 10))
    for trial in range(40):
        vocab = 300
        lg = rng.standard_normal(vocab).astype(np.float32) * 3
        lg[rng.integers(0, vocab, 5)] = 0.0
        hist = rng.integers(0, vocab, rng.integers(0, 60))
        top = int(np.argmax(lg))
        hist = np.r_[hist, [top] * int(rng.integers(0, 4))].astype(np.int32)   # the raw maximum repeats
        t_ref, v_ref = oracle.ref_greedy_pick(lg, hist, penalty)
        t_orc, v_orc = oracle.greedy_pick(lg, hist, penalty)
        counts = np.bincount(hist, minlength=vocab)
        assert np.allclose(v_orc, v_ref, rtol=2e-7 * (1 + counts), atol=0)
        assert t_orc == t_ref or abs(v_orc[t_orc] - v_orc[t_ref]) <= 1e-6 * abs(v_orc[t_orc])
    # the closed form on one token: 3 occurrences of a positive and a negative logit
    lg = np.array([2.0, -2.0, 1.0], np.float32)
    _, v = oracle.greedy_pick(lg, [0, 0, 0, 1, 1, 1], 2.0)
    assert v.tolist() == [0.25, -16.0, 1.0]
    assert oracle.greedy_pick(lg, [0, 0, 0, 1, 1, 1], 2.0)[0] == 2


def test_greedy_pick_penalty_one_is_argmax():
    rng = np.random.default_rng(3)
    lg = rng.standard_normal(500).astype(np.float32)
    lg[10] = lg[20] = lg.max() + 1   # tie: the first maximum
    assert oracle.greedy_pick(lg, rng.integers(0, 500, 30), 1.0)[0] == 10
