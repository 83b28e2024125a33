"""lmx_gemv_tiles_noalloc (include/lutmac_hip.h): the GEMV of lmx_gemv over
caller-held device tiles and scales, with its scratch (split-K partials,
ticket counters, x staging) in the library's static per-GPU array.  Its
output must equal lmx_gemv's on a handle built from the same planes (same
kernels and plan; bit-identical below batch 4, where lmx_gemv runs one
vector at a time too; within TOL at batch 5, where lmx_gemv batches), call
after call, the second call smaller than the first."""
import numpy as np
import pytest
import torch

import lutmac_amd as L
from conftest import TOL, rel_max_err
from lutmac_amd import synth

pytestmark = pytest.mark.gpu


def layouts(fmt, rows, cols, group, seed):
    planes, scales, g = synth.make_weights(fmt, rows, cols, seed=seed, group=group)
    tiles = torch.from_numpy(L.tile_planes(fmt, planes, rows, cols)).cuda()
    sc = torch.from_numpy(L.tile_scales(fmt, scales, rows, cols, g)).cuda()
    return tiles, sc, g, L.Weight.from_planes(fmt, planes, scales, rows, cols, g)


# (format, rows, cols, group, flags, batch): a split-K shape (K = 8960 fits no
# full-K configuration) first, then smaller full-K shapes, then batch 5
CASES = [
    (L.FMT_INT4, 1536, 8960, 128, L.ROTATE_NONE, 2),
    (L.FMT_TERNARY, 300, 640, 0, L.ROTATE_FWHT256, 1),
    (L.FMT_RRQ2, 64, 2048, 128, L.ROTATE_FWHT_FULL, 1),
    (L.FMT_INT8, 513, 1536, 256, L.ROTATE_NONE, 3),
]


def test_noalloc_equals_gemv_call_after_call(cuda):
    for i, (fmt, rows, cols, group, flags, batch) in enumerate(CASES):
        tiles, sc, g, w = layouts(fmt, rows, cols, group, seed=40 + i)
        x = torch.randn(batch * cols, device="cuda")
        want = w.gemv(x, flags=flags)
        for _ in range(2):   # a repeat on the same shape reuses the scratch left by the first
            y = torch.full((batch * rows,), float("nan"), device="cuda")
            L.gemv_tiles_noalloc(fmt, tiles, sc, rows, cols, g, x, y, batch, flags)
            torch.cuda.synchronize()
            assert torch.equal(y, want), (L.FORMAT_NAMES[fmt], rows, cols)
        w.close()


def test_noalloc_batch5_against_batched_gemv(cuda):
    fmt, rows, cols = L.FMT_INT4, 1000, 2048
    tiles, sc, g, w = layouts(fmt, rows, cols, 128, seed=50)
    x = torch.randn(5 * cols, device="cuda")
    want = w.gemv(x).cpu().numpy().reshape(5, rows)
    y = torch.empty(5 * rows, device="cuda")
    L.gemv_tiles_noalloc(fmt, tiles, sc, rows, cols, g, x, y, 5)
    got = y.cpu().numpy().reshape(5, rows)
    for b in range(5):
        assert rel_max_err(got[b], want[b]) < TOL
    w.close()


def test_noalloc_unaligned_x_uses_staging(cuda):
    fmt, rows, cols = L.FMT_INT4, 256, 1000
    tiles, sc, g, w = layouts(fmt, rows, cols, 128, seed=51)
    buf = torch.randn(cols + 1, device="cuda")
    x = buf[1:]   # 4 bytes off a 16-byte boundary: staged into the scratch
    want = w.gemv(x)
    y = torch.empty(rows, device="cuda")
    L.gemv_tiles_noalloc(fmt, tiles, sc, rows, cols, g, x, y)
    assert torch.equal(y, want)
    w.close()


def test_noalloc_rejects_shapes_beyond_its_scratch(cuda):
    # split-K partials of 400000 rows x 35 slices exceed the 8 MiB array
    rows, cols = 400000, 8960
    tiles = torch.zeros(16, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(4, dtype=torch.float32, device="cuda")
    x = torch.zeros(cols, device="cuda")
    y = torch.zeros(rows, device="cuda")
    with pytest.raises(L.LmxError) as e:
        L.gemv_tiles_noalloc(L.FMT_INT4, tiles, sc, rows, cols, 128, x, y)
    assert "scratch" in str(e.value)
