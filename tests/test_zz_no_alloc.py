"""lmx_gemv_tiles_noalloc (include/lutmac_hip.h): the GEMV of lmx_gemv over
caller-held device tiles and scales, with its scratch (split-K partials,
ticket counters, x staging) in the library's static per-GPU array.  Its
output must equal lmx_gemv's on a handle built from the same planes (same
kernels and plan; bit-identical below batch 4, where lmx_gemv runs one
vector at a time too; within TOL at batch 5, where lmx_gemv batches), call
after call, the second call smaller than the first.

The first test of this file makes the process's first call (the one that
zeroes the array) on one stream and the next call on another stream."""
import ctypes

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


# (format, rows, cols, group, flags, batch): a split-K shape (10240 rows at
# K = 4096 leave no full-K plan within one workgroup per CU) first, then the
# layered full-K plan at K = 8960, then smaller full-K shapes, then batch 5
CASES = [
    (L.FMT_INT4, 10240, 4096, 128, L.ROTATE_NONE, 1),
    (L.FMT_INT4, 1536, 8960, 128, L.ROTATE_NONE, 2),
    (L.FMT_TERNARY, 300, 640, 0, L.ROTATE_FWHT256, 1),
    (L.FMT_RRQ2, 64, 2048, 128, L.ROTATE_FWHT_FULL, 1),
    (L.FMT_INT8, 513, 1536, 256, L.ROTATE_NONE, 3),
]


def test_noalloc_first_call_then_other_stream(cuda):
    # Call 1 (a full-K plan, aligned x: its kernel touches no scratch) is the
    # first on the device, so it zeroes the array on stream s1; call 2, a
    # split-K plan that needs zeroed ticket counters, goes out at once on s2.
    # The first call returns only after its zero fill has finished, so call 2
    # cannot run on counters that are not zeroed yet.
    a = layouts(L.FMT_INT4, 2048, 2048, 128, seed=60)
    b = layouts(L.FMT_INT4, 10240, 4096, 128, seed=61)
    assert a[3].kernel_config()[0] != 0 and b[3].kernel_config()[0] == 0
    xa = torch.randn(2048, device="cuda")
    xb = torch.randn(4096, device="cuda")
    want_a, want_b = a[3].gemv(xa), b[3].gemv(xb)
    ya = torch.full((2048,), float("nan"), device="cuda")
    yb = torch.full((10240,), float("nan"), device="cuda")
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    L.gemv_tiles_noalloc(L.FMT_INT4, a[0], a[1], 2048, 2048, a[2], xa, ya, stream=s1)
    L.gemv_tiles_noalloc(L.FMT_INT4, b[0], b[1], 10240, 4096, b[2], xb, yb, stream=s2)
    torch.cuda.synchronize()
    assert torch.equal(ya, want_a)
    assert torch.equal(yb, want_b)
    a[3].close()
    b[3].close()


def test_noalloc_staged_small_then_split_k_over_4096_rows(cuda):
    # A staged call (unaligned x) on a small shape, then split-K calls with
    # more than 4096 rows: the ticket counters of the large plan must not sit
    # where the small call staged its x (the counters have a fixed region).
    small = layouts(L.FMT_INT4, 256, 1000, 128, seed=62)
    big = layouts(L.FMT_INT4, 14336, 4096, 128, seed=63)
    assert big[3].kernel_config()[0] == 0, "14336 x 4096 must run split-K"
    buf = torch.randn(1001, device="cuda")
    xs = buf[1:]
    ys = torch.empty(256, device="cuda")
    L.gemv_tiles_noalloc(L.FMT_INT4, small[0], small[1], 256, 1000, small[2], xs, ys)
    assert torch.equal(ys, small[3].gemv(xs))
    xb = torch.randn(4096, device="cuda")
    want = big[3].gemv(xb)
    for _ in range(2):
        yb = torch.full((14336,), float("nan"), device="cuda")
        L.gemv_tiles_noalloc(L.FMT_INT4, big[0], big[1], 14336, 4096, big[2], xb, yb)
        torch.cuda.synchronize()
        assert torch.equal(yb, want)
    small[3].close()
    big[3].close()


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
    # split-K partials of 400000 rows x 35 slices exceed the 8 MiB array; the
    # C entry point rejects the shape before it touches any buffer, so it is
    # called directly here with placeholder buffers (the Python wrapper would
    # refuse them for their size first)
    rows, cols = 400000, 8960
    tiles = torch.zeros(16, dtype=torch.uint8, device="cuda")
    sc = torch.zeros(4, dtype=torch.float32, device="cuda")
    x = torch.zeros(cols, device="cuda")
    y = torch.zeros(16, device="cuda")
    st = L.lib().lmx_gemv_tiles_noalloc(L.FMT_INT4, ctypes.c_void_p(tiles.data_ptr()),
                                        ctypes.c_void_p(sc.data_ptr()), rows, cols, 128,
                                        ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), 1, 0,
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == L.ERR_INVALID_ARGUMENT
    assert "scratch" in L.lib().lmx_last_error().decode()


def test_noalloc_wrapper_checks_buffer_sizes(cuda):
    fmt, rows, cols = L.FMT_INT4, 256, 1024
    tiles, sc, g, w = layouts(fmt, rows, cols, 128, seed=64)
    x = torch.randn(cols, device="cuda")
    y = torch.empty(rows, device="cuda")
    cases = [("tiles", dict(tiles=tiles[:-16])), ("scales", dict(scales=sc[:-1])),
             ("x", dict(x=x[:-4])), ("y", dict(y=y[:-1]))]
    for name, repl in cases:
        args = dict(tiles=tiles, scales=sc, x=x, y=y)
        args.update(repl)
        with pytest.raises(L.LmxError) as e:
            L.gemv_tiles_noalloc(fmt, args["tiles"], args["scales"], rows, cols, g, args["x"], args["y"])
        assert name in str(e.value)
    w.close()
