"""GPU parity of the device-resident decoder (include/lutmac_decode.h).

Teacher-forced logits of every step against the oracle's decode restatement
(orc_decode_step, itself pinned to the reference's Model::forward by
tests/test_decode_cpu.py) and, in the reference's own configuration
(group-256 4-bit blocks, its RoPE form), against the reference's Model::forward
directly.  Bar: max |logit - ref| <= DECODE_TOL * ||ref||_2 at every step
(fp32 accumulation-order differences compounded over the layers).
Greedy generation: the captured-graph replay must reproduce eager steps
token for token, and every generated token must be the oracle's argmax up
to the same tolerance.
"""
import numpy as np
import pytest
import torch

import lutmac_amd as L
import oracle
from conftest import rel_max_err
from lutmac_amd import decode as D

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-5


def device_logits(dec, tokens):
    dec.reset(tokens)
    out = []
    lg = torch.empty(dec.cfg.vocab, dtype=torch.float32, device="cuda")
    for _ in range(len(tokens)):
        dec.step(lg)
        out.append(lg.cpu().numpy().copy())
    return out


def check_against(dec, ref, tokens, tol=DECODE_TOL):
    got = device_logits(dec, tokens)
    for pos, t in enumerate(tokens):
        want = ref.step(t, pos)
        err = rel_max_err(got[pos], want)
        assert err < tol, f"step {pos}: rel err {err:.3e}"


@pytest.mark.parametrize("ps", ["0", "1"])
@pytest.mark.parametrize("rope_mode", [D.ROPE_LLAMA3, D.ROPE_REFERENCE])
def test_decoder_matches_oracle_small(cuda, monkeypatch, rope_mode, ps):
    # LMX_PS: the 4 x 4 x 1 linears (RMSNorm fused) with and without the
    # plane split
    monkeypatch.setenv("LMX_PS", ps)
    cfg = D.small_config(rope_mode=rope_mode, rope_factor=32.0 if rope_mode == D.ROPE_LLAMA3 else 4.0,
                         rope_orig_max_pos=64, rope_theta=10000.0)
    m = D.SyntheticModel(cfg, seed=11, group=128, random_norms=True)
    toks = np.random.default_rng(12).integers(0, cfg.vocab, 24)
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)


def test_decoder_matches_oracle_qwen_style(cuda):
    # head_dim 128, 6 query heads per KV head, QKV bias, theta 1e6
    cfg = D.small_config(hidden=512, n_heads=12, n_kv_heads=2, head_dim=128, ffn=768, vocab=1500,
                         rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6, rms_eps=1e-6,
                         qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=13, group=128, random_norms=True)
    toks = np.random.default_rng(14).integers(0, cfg.vocab, 20)
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)


def test_decoder_long_ffn(cuda, monkeypatch):
    # FFN 8960 (Qwen-2.5-1.5B's width): the down projection's K = 8960 takes
    # the layered 8 x 8 x 2 plan (70 chunks on 64 slices), gate|up (17920
    # rows) the 8 x 32 small-K configuration; with LMX_SILU_PAIR=0 the down
    # projection forms SiLU*up in its own table build
    cfg = D.small_config(hidden=256, ffn=8960, vocab=1000, rope_mode=D.ROPE_REFERENCE, rope_factor=1.0,
                         rope_theta=1e6)
    m = D.SyntheticModel(cfg, seed=31, group=128, random_norms=True)
    dec = D.Decoder(m)
    assert [w.kernel_config()[0] for w in dec.weights[:4]] == [6, 6, 3, 8]   # qkv, o, gate|up, down
    toks = np.random.default_rng(32).integers(0, cfg.vocab, 12)
    check_against(dec, oracle.OracleDecoder(m), toks)
    monkeypatch.setenv("LMX_SILU_PAIR", "0")
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)


def test_decoder_layered_head_takes_split_k(cuda):
    # hidden 8960: the tied 1000 x 8960 head gets the layered 8 x 8 x 2 plan,
    # which has no argmax form, so the head GEMV (RMSNorm in, argmax keys out)
    # runs the split-K kernel; the down projection (8960 x 256) is full-K
    cfg = D.small_config(hidden=8960, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=64, ffn=256, vocab=1000,
                         max_seq=32, rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6)
    m = D.SyntheticModel(cfg, seed=45, group=128, random_norms=True)
    dec = D.Decoder(m)
    assert dec.head.kernel_config()[0] == 8
    toks = np.random.default_rng(46).integers(0, cfg.vocab, 6)
    check_against(dec, oracle.OracleDecoder(m), toks)
    out, _, _ = dec.generate(toks[:3], 6)                  # greedy: the argmax epilogue
    o = oracle.OracleDecoder(m)
    for pos in range(len(out) - 1):
        lg = o.step(out[pos], pos)
        if pos + 1 >= 3:
            assert lg[out[pos + 1]] >= lg.max() - DECODE_TOL * np.linalg.norm(lg)


@pytest.mark.parametrize("ffn,ps", [(768, "1"), (4096, "1"), (4096, "2")])
def test_decoder_silu_pair_epilogue(cuda, monkeypatch, ffn, ps):
    # gate|up writing SiLU(gate)*up itself (the 4-bit batch-1 step) against
    # the down projection forming it (LMX_SILU_PAIR=0): the same values, and
    # both within the bar of the oracle.  ffn 4096 gives down (512 x 4096)
    # 8 rows per workgroup: the 16 x 4 x 1 plan with its planes split over
    # two lanes (the default), or the 8-row x 64-slice plan (LMX_PS=2: only
    # the 4 x 4 x 1 plan splits)
    monkeypatch.setenv("LMX_PS", ps)
    cfg = D.small_config(hidden=512, ffn=ffn, vocab=900, rope_mode=D.ROPE_REFERENCE, rope_factor=1.0,
                         rope_theta=1e6)
    m = D.SyntheticModel(cfg, seed=41 + ffn, group=128, random_norms=True)
    toks = np.random.default_rng(42).integers(0, cfg.vocab, 10)
    dec = D.Decoder(m)
    if ffn == 4096:
        assert dec.weights[3].kernel_config()[0] == (5 if ps == "1" else 7)
    paired = device_logits(dec, toks)
    monkeypatch.setenv("LMX_SILU_PAIR", "0")
    unpaired = device_logits(D.Decoder(m), toks)
    ref = oracle.OracleDecoder(m)
    for pos, t in enumerate(toks):
        want = ref.step(t, pos)
        assert rel_max_err(paired[pos], unpaired[pos]) < 1e-6, pos
        assert rel_max_err(paired[pos], want) < DECODE_TOL, pos


@pytest.mark.parametrize("hs", [None, "1", "group"])
@pytest.mark.parametrize("cpw", ["1", "2"])
@pytest.mark.parametrize("head_dim,n_heads,n_kv", [(64, 8, 2), (128, 12, 2)])
def test_decoder_multi_chunk_context(cuda, monkeypatch, head_dim, n_heads, n_kv, cpw, hs):
    # 150 positions span three 64-position attention chunks (a fourth, empty,
    # chunk takes no ticket): the chunk merge of the attention kernel at every
    # step, against the oracle's single-pass softmax; one chunk per workgroup,
    # or two (LMX_ATTN_CPW=2: the second chunk of the second unit is empty);
    # a KV head's query heads in the automatic number of workgroups, in one,
    # or one head per workgroup (LMX_ATTN_HS)
    monkeypatch.setenv("LMX_ATTN_CPW", cpw)
    if hs is not None:
        monkeypatch.setenv("LMX_ATTN_HS", str(n_heads // n_kv) if hs == "group" else hs)
    cfg = D.small_config(hidden=512 if head_dim == 128 else 256, n_heads=n_heads, n_kv_heads=n_kv,
                         head_dim=head_dim, ffn=768, vocab=1200, max_seq=256, rope_mode=D.ROPE_REFERENCE,
                         rope_factor=1.0, rope_theta=1e6, qkv_bias=head_dim == 128)
    m = D.SyntheticModel(cfg, seed=21 + head_dim, group=128, random_norms=True)
    toks = np.random.default_rng(22).integers(0, cfg.vocab, 150)
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)


@pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref/libref.so not built")
def test_decoder_matches_reference_model(cuda):
    # the reference's own configuration: group-256 blocks, (pos/factor) RoPE
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=10000.0)
    m = D.SyntheticModel(cfg, seed=15, group=256, random_norms=True)
    toks = np.random.default_rng(16).integers(0, cfg.vocab, 16)
    check_against(D.Decoder(m), oracle.RefDecoder(m), toks)


# short, and long: 600 positions = 10 attention chunks, past the 8-chunk
# speculative window, replayed from one captured step
@pytest.mark.parametrize("n_prompt,n_new,max_seq", [(8, 24, 48), (560, 40, 640)], ids=["short", "long"])
def test_generate_graph_equals_eager_and_oracle(cuda, n_prompt, n_new, max_seq):
    cfg = D.small_config(max_seq=max_seq)
    m = D.SyntheticModel(cfg, seed=17, group=128, random_norms=True)
    dec = D.Decoder(m)
    prompt = np.random.default_rng(18).integers(0, cfg.vocab, n_prompt)
    out, t_pre, t_dec = dec.generate(prompt, n_new)
    assert np.array_equal(out[:n_prompt], prompt) and t_pre > 0 and t_dec > 0
    # eager steps from the same prompt
    dec.reset(prompt)
    for _ in range(len(prompt) + n_new - 1):
        dec.step()
    assert np.array_equal(dec.tokens(len(prompt) + n_new), out)
    # every generated token is the oracle's argmax (teacher-forced on the device's sequence)
    o = oracle.OracleDecoder(m)
    for pos in range(len(out) - 1):
        lg = o.step(out[pos], pos)
        if pos + 1 >= len(prompt):
            assert lg[out[pos + 1]] >= lg.max() - DECODE_TOL * np.linalg.norm(lg)
    # a second generation on the same decoder repeats the first
    out2, _, _ = dec.generate(prompt, n_new)
    assert np.array_equal(out, out2)


def test_llama_1b_architecture_steps(cuda):
    cfg = D.LLAMA_3_2_1B
    m = D.SyntheticModel(cfg, seed=19, group=128)
    toks = np.random.default_rng(20).integers(0, cfg.vocab, 2)
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)


def test_decoder_rejects_bad_arguments(cuda):
    import ctypes
    bad = D.small_config(head_dim=96)
    h = ctypes.c_void_p()
    cs = bad.c_struct()
    assert L.lib().lmx_decoder_create(ctypes.byref(cs), ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    cfg = D.small_config()
    cs = cfg.c_struct()
    assert L.lib().lmx_decoder_create(ctypes.byref(cs), ctypes.byref(h)) == L.OK
    try:
        # not ready: no layers or head set
        assert L.lib().lmx_decoder_step(h, None, None) == L.ERR_INVALID_ARGUMENT
        # wrong shape for the qkv weight
        from lutmac_amd import synth
        planes, scales, g = synth.make_weights(L.FMT_INT4, 64, 256, seed=1)
        w = L.Weight.from_planes(L.FMT_INT4, planes, scales, 64, 256, g)
        ones = np.ones(cfg.hidden, np.float32)
        st = L.lib().lmx_decoder_set_layer(h, 0, w.handle, w.handle, w.handle, w.handle,
                                           L._np_ptr(ones), L._np_ptr(ones), None)
        assert st == L.ERR_INVALID_ARGUMENT
    finally:
        L.lib().lmx_decoder_destroy(h)


# ---- .lutmac v1 files (lutmac_model.h) ---------------------------------------
needs_ref = pytest.mark.skipif(oracle.ref() is None, reason="oracle/_ref/libref.so not built")


@needs_ref
def test_lutmac_file_matches_reference_load_model(cuda, tmp_path):
    # written by the reference's own save_lutmac; read by its load_model and by ours
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=2.0, rope_theta=10000.0, qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=31, group=256, random_norms=True)
    path = tmp_path / "model.lutmac"
    oracle.RefDecoder(m).save(path, with_biases=True)
    ours = D.LutmacModel(path, max_seq=64)
    assert ours.cfg.vocab == cfg.vocab and ours.cfg.n_kv_heads == cfg.n_kv_heads
    assert ours.cfg.rope_factor == 2.0 and ours.weight_format(-1) == L.FMT_INT4
    toks = np.random.default_rng(32).integers(0, cfg.vocab, 16)
    check_against(ours, oracle.RefDecoder.from_file(path, cfg.vocab), toks)
    out, _, _ = ours.generate(toks[:4], 8)
    assert np.array_equal(out[:4], toks[:4])


@needs_ref
def test_lutmac_file_int8_embedding(cuda, tmp_path):
    # real reference files carry int8 tied embeddings (tools/lutmac-quantize.cpp:385)
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=10000.0)
    m = D.SyntheticModel(cfg, seed=33, group=256, random_norms=True)
    ref = oracle.RefDecoder(m)
    w = L.synth_normal(33, 999, cfg.vocab, cfg.hidden, 0.02)
    nb = cfg.vocab * (cfg.hidden // 256)
    blocks = np.zeros(nb * 260, np.uint8)
    oracle.ref().ref_quantize(7, oracle._ptr(w), cfg.vocab, cfg.hidden, oracle._ptr(blocks), blocks.size)
    ref.set_embedding(7, blocks, m.final_norm)
    path = tmp_path / "int8emb.lutmac"
    ref.save(path)
    ours = D.LutmacModel(path, max_seq=64)
    assert ours.weight_format(-1) == L.FMT_INT8 and ours.weight_format(-2) == L.FMT_INT8
    toks = np.random.default_rng(34).integers(0, cfg.vocab, 10)
    check_against(ours, oracle.RefDecoder.from_file(path, cfg.vocab), toks)


# ---- batched decoder: several sequences in lockstep --------------------------
def batched_check(dec, m, toks, tol=DECODE_TOL):
    """Teacher-forced logits of every sequence at every step against one oracle
    decoder per sequence."""
    B, n = toks.shape
    dec.reset(toks)
    lg = torch.empty(B * m.cfg.vocab, dtype=torch.float32, device="cuda")
    refs = [oracle.OracleDecoder(m) for _ in range(B)]
    for pos in range(n):
        dec.step(lg)
        got = lg.cpu().numpy().reshape(B, m.cfg.vocab)
        for b in range(B):
            want = refs[b].step(toks[b, pos], pos)
            err = rel_max_err(got[b], want)
            assert err < tol, f"sequence {b} step {pos}: rel err {err:.3e}"


# B = 4: one group of the batched GEMV; B = 6: a group of 4 and two rows by the
# single-vector GEMV; 70 positions cross a 64-position attention chunk.
@pytest.mark.parametrize("batch", [4, 6])
def test_batched_decoder_matches_oracle(cuda, batch):
    cfg = D.small_config(max_seq=128, rope_mode=D.ROPE_LLAMA3, rope_factor=32.0, rope_orig_max_pos=64,
                         rope_theta=10000.0)
    m = D.SyntheticModel(cfg, seed=31, group=128, random_norms=True)
    toks = np.random.default_rng(32).integers(0, cfg.vocab, (batch, 70))
    batched_check(D.Decoder(m, batch=batch), m, toks)


@pytest.mark.parametrize("batch", [8, 16])
def test_batched_decoder_fused_epilogues(cuda, monkeypatch, batch):
    # o/down reductions writing the normed rows and the gate|up reduction
    # writing SiLU(gate)*up (every row in a batched group) against the row
    # kernels (LMX_FUSED_ROWS=0): the same bits, and the oracle's logits.
    # The qkv split partials summed inside attention (the default for one
    # group) against the batched reduction writing the rows first
    # (LMX_QKV_PARTS=0): the same bits as well.
    cfg = D.small_config(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=700, max_seq=64,
                         rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6, qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=35 + batch, group=128, random_norms=True)
    toks = np.random.default_rng(36).integers(0, cfg.vocab, (batch, 12))

    def logits(dec):
        dec.reset(toks)
        lg = torch.empty(batch * cfg.vocab, dtype=torch.float32, device="cuda")
        out = []
        for _ in range(toks.shape[1]):
            dec.step(lg)
            out.append(lg.cpu().numpy().reshape(batch, cfg.vocab).copy())
        return out

    fused = logits(D.Decoder(m, batch=batch))
    monkeypatch.setenv("LMX_QKV_PARTS", "0")
    reduced = logits(D.Decoder(m, batch=batch))
    monkeypatch.setenv("LMX_FUSED_ROWS", "0")
    rows = logits(D.Decoder(m, batch=batch))
    refs = [oracle.OracleDecoder(m) for _ in range(batch)]
    for pos in range(toks.shape[1]):
        assert np.array_equal(fused[pos].view(np.uint32), reduced[pos].view(np.uint32)), pos
        assert np.array_equal(fused[pos].view(np.uint32), rows[pos].view(np.uint32)), pos
        for b in range(batch):
            assert rel_max_err(fused[pos][b], refs[b].step(toks[b, pos], pos)) < DECODE_TOL, (b, pos)


@pytest.mark.parametrize("plan", [3, 6])
def test_batched_decoder_four_vector_kernel(cuda, monkeypatch, plan):
    # batch 4 on K <= 2048 plans: qkv and gate|up (SiLU(gate)*up written by
    # the workgroup) take the four-vector full-K kernel; against the batched
    # kernel with its reductions (LMX_NO_QUAD=1) and the oracle's logits
    monkeypatch.setenv("LMX_FULLK", str(plan))
    cfg = D.small_config(hidden=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn=1024, vocab=700, max_seq=64,
                         rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6, qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=51 + plan, group=128, random_norms=True)
    toks = np.random.default_rng(52).integers(0, cfg.vocab, (4, 12))
    dec = D.Decoder(m, batch=4)
    assert all(w.kernel_config()[0] == plan for w in dec.weights[:4])

    def logits(dec):
        dec.reset(toks)
        lg = torch.empty(4 * cfg.vocab, dtype=torch.float32, device="cuda")
        out = []
        for _ in range(toks.shape[1]):
            dec.step(lg)
            out.append(lg.cpu().numpy().reshape(4, cfg.vocab).copy())
        return out

    quad = logits(dec)
    monkeypatch.setenv("LMX_NO_QUAD", "1")
    batched = logits(dec)
    refs = [oracle.OracleDecoder(m) for _ in range(4)]
    for pos in range(toks.shape[1]):
        for b in range(4):
            assert rel_max_err(quad[pos][b], batched[pos][b]) < 1e-5, (b, pos)
            assert rel_max_err(quad[pos][b], refs[b].step(toks[b, pos], pos)) < DECODE_TOL, (b, pos)


def test_batched_decoder_qwen_style(cuda):
    cfg = D.small_config(hidden=512, n_heads=12, n_kv_heads=2, head_dim=128, ffn=768, vocab=1500, max_seq=128,
                         rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6, rms_eps=1e-6,
                         qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=33, group=128, random_norms=True)
    toks = np.random.default_rng(34).integers(0, cfg.vocab, (4, 70))
    batched_check(D.Decoder(m, batch=4), m, toks)


# B = 4: the four-vector step; B = 16: one group of the batched kernel with
# the qkv partials summed inside attention, captured and replayed
@pytest.mark.parametrize("B", [4, 16])
def test_batched_generate_graph_equals_eager_and_oracle(cuda, B):
    cfg = D.small_config(max_seq=96)
    m = D.SyntheticModel(cfg, seed=35, group=128, random_norms=True)
    n_prompt, n_new = 8, 72
    dec = D.Decoder(m, batch=B)
    prompt = np.random.default_rng(36).integers(0, cfg.vocab, (B, n_prompt))
    out, t_pre, t_dec = dec.generate(prompt, n_new)
    assert out.shape == (B, n_prompt + n_new) and np.array_equal(out[:, :n_prompt], prompt)
    assert t_pre > 0 and t_dec > 0
    dec.reset(prompt)
    for _ in range(n_prompt + n_new - 1):
        dec.step()
    assert np.array_equal(dec.tokens(n_prompt + n_new), out)
    for b in range(B):   # every generated token is the oracle's argmax for its sequence
        o = oracle.OracleDecoder(m)
        for pos in range(n_prompt + n_new - 1):
            lg = o.step(out[b, pos], pos)
            if pos + 1 >= n_prompt:
                assert lg[out[b, pos + 1]] >= lg.max() - DECODE_TOL * np.linalg.norm(lg)


@pytest.mark.parametrize("parts", [None, "1", "3"])
@pytest.mark.parametrize("vocab", [1000, 1001])
def test_batched_greedy_token_is_first_maximum(cuda, monkeypatch, vocab, parts):
    # argmax_rows_kernel: 16-byte loads when vocab % 4 == 0 (1000), the scalar
    # loop otherwise (1001); each row split over the default number of
    # workgroups, over one, or over three; every chosen token is numpy's first
    # maximum of the step's own logits row.  Head rows repeat with period 97,
    # so every maximum recurs in other workgroups' slices of the row.
    if parts is not None:
        monkeypatch.setenv("LMX_ARGMAX_PARTS", parts)
    cfg = D.small_config(vocab=vocab, max_seq=32)
    m = D.SyntheticModel(cfg, seed=61, group=128, random_norms=True)
    per = np.arange(vocab) % 97
    m.head = (m.head[0][:, per].copy(), m.head[1][:, per].copy())
    B, n = 4, 12
    dec = D.Decoder(m, batch=B)
    dec.reset(np.random.default_rng(62).integers(0, vocab, (B, 1)))
    lg = torch.empty(B * vocab, dtype=torch.float32, device="cuda")
    rows = []
    for _ in range(n):
        dec.step(lg)
        rows.append(lg.cpu().numpy().reshape(B, vocab).copy())
    toks = dec.tokens(n + 1)
    for pos in range(n):
        assert np.array_equal(toks[:, pos + 1], rows[pos].argmax(axis=1)), pos


# ---- BASELINE config 5 code paths: long KV context, batch 16, full Qwen ------
def check_positions(dec, ref, tokens, check_from, tol=DECODE_TOL):
    """Teacher-forced run over all of `tokens`; logits compared from position
    `check_from` on (earlier steps only fill both KV caches)."""
    dec.reset(tokens)
    lg = torch.empty(dec.cfg.vocab, dtype=torch.float32, device="cuda")
    for pos, t in enumerate(tokens):
        want = ref.step(t, pos)
        if pos < check_from:
            dec.step()
            continue
        dec.step(lg)
        err = rel_max_err(lg.cpu().numpy(), want)
        assert err < tol, f"step {pos}: rel err {err:.3e}"


def qwen_small(**kw):
    # Qwen-2.5 attention geometry (head_dim 128, 12 query / 2 KV heads, QKV bias)
    base = dict(hidden=256, n_layers=1, n_heads=12, n_kv_heads=2, head_dim=128, ffn=512, vocab=512,
                rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6, rms_eps=1e-6, qkv_bias=True)
    base.update(kw)
    return D.small_config(**base)


@pytest.mark.parametrize("spec", [8, 1])
def test_decoder_past_512_positions(cuda, monkeypatch, spec):
    # 600 positions = 10 attention chunks: the merge takes its 32-chunk batch
    # (merge_pass<128, 32>), and chunks past the speculative window (LMX_ATTN_SPEC)
    # wait for the position and skip their loads while they lie past it.
    monkeypatch.setenv("LMX_ATTN_SPEC", str(spec))
    cfg = qwen_small(max_seq=640)
    m = D.SyntheticModel(cfg, seed=51, group=128, random_norms=True)
    toks = np.random.default_rng(52).integers(0, cfg.vocab, 600)
    check_positions(D.Decoder(m), oracle.OracleDecoder(m), toks, check_from=0)


@pytest.mark.parametrize("head_dim,n_heads,n_kv", [(64, 8, 2), (128, 12, 2)])
def test_attention_two_chunk_units_odd_cache(cuda, monkeypatch, head_dim, n_heads, n_kv):
    # two chunks per workgroup over a 3-chunk cache: the second unit's second
    # chunk lies past the cache (its loads are clamped to the last chunk, it
    # holds no position), speculatively loaded from the first step on
    monkeypatch.setenv("LMX_ATTN_CPW", "2")
    cfg = D.small_config(hidden=512 if head_dim == 128 else 256, n_heads=n_heads, n_kv_heads=n_kv,
                         head_dim=head_dim, ffn=768, vocab=700, max_seq=192, rope_mode=D.ROPE_REFERENCE,
                         rope_factor=1.0, rope_theta=1e6, qkv_bias=head_dim == 128)
    m = D.SyntheticModel(cfg, seed=63 + head_dim, group=128, random_norms=True)
    toks = np.random.default_rng(64).integers(0, cfg.vocab, 190)
    check_positions(D.Decoder(m), oracle.OracleDecoder(m), toks, check_from=0)


def test_decoder_past_4096_positions(cuda):
    # 4112 positions = 65 chunks: two passes of the merge (64 chunks, then 1)
    cfg = qwen_small(n_heads=4, n_kv_heads=2, vocab=256, max_seq=4160)
    m = D.SyntheticModel(cfg, seed=53, group=128, random_norms=True)
    toks = np.random.default_rng(54).integers(0, cfg.vocab, 4112)
    check_positions(D.Decoder(m), oracle.OracleDecoder(m), toks, check_from=4030)


@pytest.mark.parametrize("batch,hs", [(8, None), (8, "3"), (4, None)])
def test_batched_qkv_partials_head_dim_128(cuda, monkeypatch, batch, hs):
    # Qwen attention geometry (head_dim 128, 6 query heads per KV head, QKV
    # bias) with the qkv split partials summed inside attention: the KV
    # head's query heads over 2 workgroups (the default for this small
    # grid) or 3 (LMX_ATTN_HS), batch 8 and 4 (the fused-reduction step,
    # LMX_QUAD_STEP=0); the same bits as the reduced rows (LMX_QKV_PARTS=0)
    # and the oracle's logits, across two attention chunks.  At batch 4 the
    # reduced path's qkv takes the four-vector kernel, unsplit here
    # (LMX_QPS=0): its chunk sums are then the batched reduction's bits.
    monkeypatch.setenv("LMX_QUAD_STEP", "0")
    monkeypatch.setenv("LMX_QPS", "0")
    if hs:
        monkeypatch.setenv("LMX_ATTN_HS", hs)
    cfg = qwen_small(max_seq=128)
    m = D.SyntheticModel(cfg, seed=57 + batch, group=128, random_norms=True)
    toks = np.random.default_rng(58).integers(0, cfg.vocab, (batch, 70))

    def logits(dec):
        dec.reset(toks)
        lg = torch.empty(batch * cfg.vocab, dtype=torch.float32, device="cuda")
        out = []
        for _ in range(toks.shape[1]):
            dec.step(lg)
            out.append(lg.cpu().numpy().reshape(batch, cfg.vocab).copy())
        return out

    parts = logits(D.Decoder(m, batch=batch))
    monkeypatch.setenv("LMX_QKV_PARTS", "0")
    reduced = logits(D.Decoder(m, batch=batch))
    refs = [oracle.OracleDecoder(m) for _ in range(batch)]
    for pos in range(toks.shape[1]):
        assert np.array_equal(parts[pos].view(np.uint32), reduced[pos].view(np.uint32)), pos
        for b in range(batch):
            assert rel_max_err(parts[pos][b], refs[b].step(toks[b, pos], pos)) < DECODE_TOL, (b, pos)


@pytest.mark.parametrize("cpw", [None, "2"])
def test_batched_decoder_batch16_past_512(cuda, monkeypatch, cpw):
    # batch 16 = one full group of the batched GEMV, with the attention of every
    # sequence past 512 positions (32-chunk merge); one chunk per workgroup
    # (the automatic choice at this cache size) or two (5 units over 9 chunks)
    if cpw is not None:
        monkeypatch.setenv("LMX_ATTN_CPW", cpw)
    cfg = qwen_small(max_seq=576)
    m = D.SyntheticModel(cfg, seed=55, group=128, random_norms=True)
    B, n = 16, 530
    toks = np.random.default_rng(56).integers(0, cfg.vocab, (B, n))
    dec = D.Decoder(m, batch=B)
    dec.reset(toks)
    lg = torch.empty(B * cfg.vocab, dtype=torch.float32, device="cuda")
    refs = [oracle.OracleDecoder(m) for _ in range(B)]
    for pos in range(n):
        dec.step(lg)
        if pos % 8 and pos < n - 4:   # every sequence's KV cache is filled; logits checked on a subset
            for b in range(B):
                refs[b].step(toks[b, pos], pos)
            continue
        got = lg.cpu().numpy().reshape(B, cfg.vocab)
        for b in range(B):
            err = rel_max_err(got[b], refs[b].step(toks[b, pos], pos))
            assert err < DECODE_TOL, f"sequence {b} step {pos}: rel err {err:.3e}"


def test_qwen_1_5b_architecture_steps(cuda):
    # BASELINE config 5's model at full size: 28 layers, hidden 1536, QKV bias,
    # GQA 12/2 with head_dim 128, FFN 8960 (down projection split-K at K = 8960),
    # tied 151936 x 1536 head (split-K at K = 1536)
    cfg = D.QWEN_2_5_1_5B
    m = D.SyntheticModel(cfg, seed=57, group=128)
    toks = np.random.default_rng(58).integers(0, cfg.vocab, 2)
    print("qwen model built", flush=True)
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)


# ---- the producer side: mixed formats, per-128 groups, RRQ-3, .lutmac v2 -----
MIXED = {"q": (L.FMT_TERNARY, 128, 0), "k": (L.FMT_TERNARY, 128, 0), "v": (L.FMT_TERNARY, 128, 0),
         "o": (L.FMT_BINARY, 128, 0), "gate": (L.FMT_RRQ3, 128, 0), "up": (L.FMT_RRQ3, 128, 0),
         "down": (L.FMT_RRQ2, 128, L.QUANT_RESIDUAL), "embed": (L.FMT_INT4, 128, 0)}


# 3- and 8-bit linears and an 8-bit embedding from the producer's uniform rules
UNIFORM = {"q": (L.FMT_INT8, 128, 0), "k": (L.FMT_INT8, 128, 0), "v": (L.FMT_INT8, 128, 0),
           "o": (L.FMT_INT3, 256, 0), "gate": (L.FMT_INT3, 128, 0), "up": (L.FMT_INT3, 128, 0),
           "down": (L.FMT_INT8, 256, 0), "embed": (L.FMT_INT8, 128, 0)}


@pytest.mark.parametrize("formats", [MIXED, UNIFORM], ids=["mixed", "uniform"])
def test_mixed_format_model_and_lutmac_v2_round_trip(cuda, tmp_path, formats):
    # linears quantized by lmx_quantize (mixed: ternary / binary / RRQ-3 /
    # residual RRQ-2 at group 128, weights FWHT-rotated as the quantize tool
    # does; uniform: 8- and 3-bit at groups 128 and 256), decoded on the
    # device from memory and from a version-2 file, against the oracle's
    # decode step (which rotates the 1-2 bit formats' activations as
    # lut_linear does)
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=10000.0, max_seq=64)
    m = D.QuantizedModel(cfg, formats, seed=61)
    toks = np.random.default_rng(62).integers(0, cfg.vocab, 16)
    check_against(D.Decoder(m), oracle.OracleDecoder(m), toks)
    path = tmp_path / "mixed.lutmac"
    m.save_v2(path)
    ours = D.LutmacModel(path, max_seq=64)
    want = [formats[n][0] for n in ("q", "o", "gate", "down")]
    assert [ours.weight_format(0, w) for w in range(4)] == want
    assert ours.weight_format(-1) == formats["embed"][0] and ours.weight_format(-2) == formats["embed"][0]
    check_against(ours, oracle.OracleDecoder(m), toks)


@pytest.mark.parametrize("batch,max_blocks", [(4, None), (4, "50"), (8, None)])
def test_batched_mixed_format_decoder(cuda, monkeypatch, batch, max_blocks):
    # the batched decoder on ternary / binary / RRQ-3 / RRQ-2 linears, whose
    # activations the kernels rotate, against one oracle decoder per
    # sequence: batch 8 with the fused norm / SiLU epilogues, batch 4 with
    # the four-vector kernels (LMX_QUAD_MAX_BLOCKS = 50: gate|up (64
    # workgroups) and the head (63) on the batched kernel with its RMSNorm
    # prologue and the rotation after it)
    if max_blocks:
        monkeypatch.setenv("LMX_QUAD_MAX_BLOCKS", max_blocks)
    cfg = D.small_config(rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=10000.0, max_seq=64)
    m = D.QuantizedModel(cfg, MIXED, seed=63)
    toks = np.random.default_rng(64).integers(0, cfg.vocab, (batch, 12))
    batched_check(D.Decoder(m, batch=batch), m, toks)


@pytest.mark.parametrize("max_blocks", [None, "100"])
def test_batched_decoder_quad_step(cuda, monkeypatch, max_blocks):
    # Batch 4 with qkv and o on the four-vector kernel (RMSNorm in its table
    # build, the residual in its epilogue, no reduction).  LMX_QUAD_MAX_BLOCKS
    # = 100 keeps gate|up and the head (256 workgroups each) on the batched
    # kernel with the RMSNorm in its own prologue.  Against the step with
    # the fused reductions (LMX_QUAD_STEP=0) and the oracle's logits.
    if max_blocks:
        monkeypatch.setenv("LMX_QUAD_MAX_BLOCKS", max_blocks)
    cfg = D.small_config(hidden=256, n_heads=8, n_kv_heads=2, head_dim=64, ffn=2048, vocab=4096, max_seq=64,
                         rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, rope_theta=1e6, qkv_bias=True)
    m = D.SyntheticModel(cfg, seed=71, group=128, random_norms=True)
    toks = np.random.default_rng(72).integers(0, cfg.vocab, (4, 10))

    def logits(dec):
        dec.reset(toks)
        lg = torch.empty(4 * cfg.vocab, dtype=torch.float32, device="cuda")
        out = []
        for _ in range(toks.shape[1]):
            dec.step(lg)
            out.append(lg.cpu().numpy().reshape(4, cfg.vocab).copy())
        return out

    dec = D.Decoder(m, batch=4)
    assert [w.kernel_config()[0] for w in dec.weights[:3]] == [6, 6, 6]   # qkv, o, gate|up: 4 x 4 x 1
    quad = logits(dec)
    monkeypatch.setenv("LMX_QUAD_STEP", "0")
    fused = logits(dec)
    refs = [oracle.OracleDecoder(m) for _ in range(4)]
    for pos in range(toks.shape[1]):
        for b in range(4):
            want = refs[b].step(toks[b, pos], pos)
            assert rel_max_err(quad[pos][b], fused[pos][b]) < 1e-5, (b, pos)
            assert rel_max_err(quad[pos][b], want) < DECODE_TOL, (b, pos)
