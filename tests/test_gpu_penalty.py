"""Repetition penalty of the device greedy pick
(lmx_decoder_set_repetition_penalty, include/lutmac_decode.h) against the
reference's rule (src/model.cpp:458-469, then the first maximum of :480-490),
restated by oracle.greedy_pick (pinned to the reference's own Model::sample in
tests/test_decode_cpu.py).  At every picked position the device token must be
the oracle's pick over the oracle's logits with the history so far (the
prompt, then every picked token), up to the decode tolerance for near-ties;
the logits themselves stay unpenalised and within the decode bar; the
captured-graph generation must equal the eager steps.  Both the batch-1 path
(penalty in the head GEMV's argmax epilogue, counts advanced by the greedy
finish) and the batched one (argmax_rows_kernel) are covered."""
import numpy as np
import pytest
import torch

import oracle
from conftest import rel_max_err
from lutmac_amd import decode as D

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-5


def eager(dec, prompt, n_new):
    """Eager steps over a prompt ([batch, n]) and n_new picks: (tokens [batch, n + n_new],
    logits per step [batch, vocab])."""
    dec.reset(prompt)
    n = prompt.shape[1]
    lg = torch.empty(dec.batch * dec.cfg.vocab, dtype=torch.float32, device="cuda")
    out = []
    for _ in range(n + n_new - 1):
        dec.step(lg)
        out.append(lg.cpu().numpy().reshape(dec.batch, dec.cfg.vocab).copy())
    toks = np.asarray(dec.tokens(n + n_new)).reshape(dec.batch, n + n_new)
    return toks, out


def check_picks(m, prompt, toks, logits, penalty):
    """Every sequence's logits against the oracle and every pick against the
    oracle's penalised pick; returns how many picks the penalty changed."""
    n = prompt.shape[1]
    changed = 0
    for b in range(toks.shape[0]):
        ref = oracle.OracleDecoder(m)
        for pos in range(toks.shape[1] - 1):
            want = ref.step(toks[b, pos], pos)
            assert rel_max_err(logits[pos][b], want) < DECODE_TOL, (b, pos)
            if pos + 1 < n:
                assert toks[b, pos + 1] == prompt[b, pos + 1]
                continue
            t, v = oracle.greedy_pick(want, toks[b, :pos + 1], penalty)
            got = int(toks[b, pos + 1])
            assert got == t or v[got] >= v[t] - DECODE_TOL * np.linalg.norm(want), (b, pos, got, t)
            changed += int(t != int(np.argmax(want)))
    return changed


@pytest.mark.parametrize("batch,penalty", [(1, 1.1), (1, 2.0), (4, 1.1), (4, 2.0)])
def test_repetition_penalty_against_oracle(cuda, batch, penalty):
    cfg = D.small_config(vocab=600, max_seq=48)
    m = D.SyntheticModel(cfg, seed=71, group=128, random_norms=True)
    rng = np.random.default_rng(72)
    prompt = rng.integers(0, cfg.vocab, (batch, 6)).astype(np.int32)
    dec = D.Decoder(m, batch=batch)
    dec.set_repetition_penalty(penalty)
    toks, logits = eager(dec, prompt, 24)
    changed = check_picks(m, prompt, toks, logits, penalty)
    if penalty == 2.0:
        assert changed > 0, "the penalty never changed a pick: the test does not exercise it"
    out, _, _ = dec.generate(prompt if batch > 1 else prompt[0], 24)   # captured graph, replayed
    assert np.array_equal(np.asarray(out).reshape(batch, -1), toks)
    # back to plain greedy: the picks are the raw argmax again
    dec.set_repetition_penalty(1.0)
    toks1, logits1 = eager(dec, prompt, 8)
    check_picks(m, prompt, toks1, logits1, 1.0)
    dec.close()


def test_repetition_penalty_rejects_bad_values(cuda):
    cfg = D.small_config()
    dec = D.Decoder(D.SyntheticModel(cfg, seed=73, group=128))
    for bad in (0.0, -1.1, float("inf"), float("nan")):
        with pytest.raises(Exception):
            dec.set_repetition_penalty(bad)
    dec.close()
