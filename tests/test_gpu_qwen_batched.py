"""BASELINE config 5 on its real shapes at batch 4 and 16: the batched GEMVs
the Qwen-2.5-1.5B decode step runs, against the oracle per vector (the
reference's lut_linear batch loop, lut_gemm_scalar.cpp:76-79), and a
Qwen-2.5-1.5B-width decoder of 2 layers (hidden 1536, GQA 12/2 at head_dim
128, QKV bias, FFN 8960, tied 151936 x 1536 head, KV capacity 2048) at batch
4 and 16 against one oracle decode step per sequence (Model::forward,
src/model.cpp:47-453) and the oracle's greedy pick.

The kernel plans are those of the bench's config-5 rows (same matrices, same
batch, same cache capacity; only the layer count differs):
  * down 1536 x 8960: 35 k-slices of 256, so the batched reduction keeps 48
    split loads in flight (batched_reduce_kernel<48>, batch 4 in the
    four-vector step) or the fused norm reduction sums 35 splits
    (batched_reduce_norm_kernel, batch 16);
  * gate|up 17920 x 1536 with SiLU(gate)*up written by its reduction
    (batched_reduce_pair_kernel, batch 16) or by the four-vector plan;
  * the 151936 x 1536 head on the batched kernel (3564 workgroups at batch 16)
    with the batched greedy pick over 151936 columns (argmax_rows_kernel).
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

import lutmac_amd as L
import oracle
from conftest import TOL, rel_max_err
from lutmac_amd import decode as D

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-5

QWEN_SHAPES = {"qkv": (2048, 1536), "o": (1536, 1536), "gate_up": (17920, 1536), "down": (1536, 8960),
               "head": (151936, 1536)}


@pytest.mark.parametrize("batch", [4, 16])
@pytest.mark.parametrize("name", list(QWEN_SHAPES))
def test_qwen_batched_linears(cuda, name, batch):
    rows, cols = QWEN_SHAPES[name]
    planes, scales = L.synth_int4_normal(91, list(QWEN_SHAPES).index(name), rows, cols, 0.02, 128)
    w = L.Weight.from_planes(L.FMT_INT4, planes, scales, rows, cols, 128)
    rng = np.random.default_rng(92 + batch)
    xs = rng.standard_normal((batch, cols)).astype(np.float32)
    bias = (0.02 * rng.standard_normal(rows)).astype(np.float32) if name == "qkv" else None
    xd = torch.from_numpy(xs.ravel()).cuda()
    y = (w.linear(xd, bias=torch.from_numpy(bias).cuda()) if bias is not None else w.gemv(xd))
    y = y.cpu().numpy().reshape(batch, rows)
    for b in range(batch):
        ref = oracle.planes_gemv(L.FMT_INT4, planes, scales, rows, cols, 128, xs[b])
        if bias is not None:
            ref = ref + bias
        assert rel_max_err(y[b], ref) < TOL, f"{name} vector {b}"
    w.close()


def qwen_2layer():
    return replace(D.QWEN_2_5_1_5B, n_layers=2)


@pytest.mark.parametrize("batch", [4, 16])
def test_qwen_width_batched_decoder(cuda, batch):
    cfg = qwen_2layer()
    m = D.SyntheticModel(cfg, seed=93, group=128, random_norms=True)
    print(f"qwen-width model built, batch {batch}", flush=True)
    dec = D.Decoder(m, batch=batch)
    rng = np.random.default_rng(94 + batch)
    toks = rng.integers(0, cfg.vocab, (batch, 3)).astype(np.int32)
    # teacher-forced logits of 3 steps
    dec.reset(toks)
    lg = torch.empty(batch * cfg.vocab, dtype=torch.float32, device="cuda")
    got = []
    for _ in range(3):
        dec.step(lg)
        got.append(lg.cpu().numpy().reshape(batch, cfg.vocab).copy())
    # greedy generation from the same prompt (captured graph): 2 new tokens
    out, _, _ = dec.generate(toks, 2)
    out = np.asarray(out).reshape(batch, 5)
    assert np.array_equal(out[:, :3], toks)
    for b in range(batch):
        ref = oracle.OracleDecoder(m)
        for pos in range(4):
            want = ref.step(out[b, pos], pos)
            if pos < 3:
                err = rel_max_err(got[pos][b], want)
                assert err < DECODE_TOL, f"sequence {b} step {pos}: rel err {err:.3e}"
            if pos >= 2:   # positions 3 and 4 were picked by the device
                pick = int(out[b, pos + 1])
                assert want[pick] >= want.max() - DECODE_TOL * np.linalg.norm(want), (b, pos)
    dec.close()
