"""LUT-GEMV benchmark on one MI355X (BASELINE metric: LUT-GEMV HBM GB/s at
8192x8192, % of the 8 TB/s HBM peak).

A step is one GEMV y = W x over an 8192x8192 weight with batch 1.  The
headline workload is the 4-bit format with per-128-group scales (BASELINE
config 3) on FWHT-rotated activations, run like the reference's int4 operator
(which never rotates inside the op: the input is rotated once, untimed); the
other formats of the sweep are reported beside it, ternary and the 1-2 bit
formats with the FWHT fused into the kernel as lut_linear applies it, and
int4 with the rotation fused in as "int4_rot".  Weights
rotate over >= 512 MiB of distinct device copies so neither the 256 MB MALL
nor the L2 holds them between launches.  The K timed GEMVs are captured in
one HIP graph (the launch path of a captured decode step), replayed once
untimed and then --replays times, each replay after a 1 GiB HBM flush and
bracketed by torch.cuda.synchronize() and HIP events recorded on the stream
the graph is launched on; value = algorithmic bytes per GEMV / (median
replay time / K).  The per-launch stream time is reported beside it
(--no-graph times only that).  BASELINE configs 1 and 2 are timed the same
way at their own shapes ("configs"), and a 1 GiB device copy and read give
the achievable-bandwidth yardstick ("achievable_bandwidth").

The reference's own lut_linear (built from its sources, oracle/_ref) is
timed on the host for int4, ternary (1 thread each) and binary (its
ThreadPool), with the CPU model and core counts ("cpu_baselines").

Beside it, the metric's second half: batch-1 greedy decode tokens/s of a
random-init Llama-3.2-1B architecture in "decode", and
the Qwen-2.5-1.5B architecture at batch 1/4/16 (config 5) in "qwen_decode".

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--formats int4,ternary,...]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "LUT-GEMV HBM GB/s (% of peak) at 8192x8192; 1B-arch decode tokens/s bs=1"
HBM_PEAK_GBPS = 8000.0
ROTATE_BYTES = 512 * 2**20

FORMATS = {"int4": 6, "ternary": 1, "binary": 2, "rrq2": 3, "rrq3": 4, "int8": 7, "int4_rot": 6}
# Config 3's activations are FWHT-rotated.  Where the reference's operator
# rotates inside lut_linear (ternary and the 1-2 bit formats,
# lut_gemm_scalar.cpp:92-93) the kernel rotates them (fused into its table
# build, inside the timed region).  The 4- and 8-bit paths never rotate inside
# the operator, so their input is rotated once on the device before timing
# (lmx_fwht256) and the kernel runs unrotated, as the reference's int4_gemv /
# int8_gemv do; "int4_rot" times int4 with the rotation fused in anyway.
ROTATE_IN_KERNEL = {"ternary", "binary", "rrq2", "rrq3", "int4_rot"}


class Flush:
    """Streams 1 GiB through HBM (read + write) between timed replays, so the
    first GEMVs of a replay find none of their weights in the 256 MB MALL."""

    def __init__(self, torch):
        self.buf = torch.empty(2**28, dtype=torch.float32, device="cuda")

    def __call__(self):
        self.buf.add_(1.0)


def gemv_bench(L, synth, torch, fmt, n, steps, warmup, graph=True, rotate_in_kernel=True, cols=None,
               group=None, outliers=False, seed=None, flush=None, replays=7):
    """Time `steps` GEMVs of an n x cols weight of format fmt; returns a dict.
    rotate_in_kernel: FWHT-256 of x fused into the kernel (flags), else x is
    rotated once on the device before the timed region and the kernel runs
    without rotation.  The `steps` GEMVs are captured in one HIP graph over
    >= 512 MiB of weight copies; the graph is replayed once untimed and then
    `replays` times, each after a 1 GiB HBM flush, each timed with HIP events
    on the launch stream; us_per_gemv is the median replay / steps."""
    cols = n if cols is None else cols
    if group is None:
        group = 0 if fmt == L.FMT_TERNARY else 128
    planes, scales, g = synth.make_weights(fmt, n, cols, seed=(1000 + fmt) if seed is None else seed, group=group)
    B = synth.algorithmic_bytes(fmt, n, cols, group=g)
    copies = max(2, -(-ROTATE_BYTES // B))
    ws = [L.Weight.from_planes(fmt, planes, scales, n, cols, g) for _ in range(copies)]
    del planes
    x = torch.from_numpy(synth.make_activations(cols, seed=5, outliers=outliers)).cuda()
    if rotate_in_kernel:
        flags = L.ROTATE_FWHT256
    else:
        flags = L.ROTATE_NONE
        L.fwht256(x)                # the input is FWHT-rotated data; rotated once, untimed
        torch.cuda.synchronize()
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    flush = flush or Flush(torch)
    for i in range(warmup):
        ws[i % copies].gemv(x, y, flags=flags, stream=stream)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # (a) one launch per GEMV on the stream
    flush()
    start.record(stream)
    for i in range(steps):
        ws[i % copies].gemv(x, y, flags=flags, stream=stream)
    end.record(stream)
    torch.cuda.synchronize()
    ms_stream = start.elapsed_time(end) / steps
    ms_graph, reps = None, []
    if graph:
        # (b) the same `steps` launches captured once in a HIP graph and
        # replayed: what a decode loop captured per token sees.
        cg = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.graph(cg, stream=side):
            for i in range(steps):
                ws[i % copies].gemv(x, y, flags=flags)
        stream.wait_stream(side)
        cg.replay()                     # untimed: uploads the graph
        torch.cuda.synchronize()
        for _ in range(replays):
            flush()
            torch.cuda.synchronize()
            start.record(stream)
            cg.replay()
            end.record(stream)
            torch.cuda.synchronize()
            reps.append(start.elapsed_time(end) / steps)
        ms_graph = float(np.median(reps))
        del cg
    ms = ms_graph if ms_graph is not None else ms_stream
    gbps = B / (ms * 1e-3) / 1e9
    out = {"format": L.FORMAT_NAMES[fmt], "rows": n, "cols": cols, "group": g,
           "rotation": "FWHT-256 in the kernel" if rotate_in_kernel else "input pre-rotated (FWHT-256), kernel unrotated",
           "kernel_plan": dict(zip(("fullk", "kslice", "staged"), ws[0].kernel_config())),
           "algorithmic_bytes": B, "us_per_gemv": round(ms * 1e3, 3), "GB_per_s": round(gbps, 1),
           "launch": "hip_graph" if ms_graph is not None else "stream",
           "replays_us_per_gemv": [round(r * 1e3, 3) for r in reps],
           "us_per_gemv_stream_launch": round(ms_stream * 1e3, 3),
           "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4), "weight_copies": copies,
           "rotated_MiB": round(copies * B / 2**20, 1)}
    if outliers:
        out["activations"] = "N(0,1), ceil(0.5% of K) channels x20"
    for w in ws:
        w.close()
    return out


def config_rows(L, synth, torch, steps, warmup, flush):
    """BASELINE configs 1 and 2 at their own shapes: 4-bit 2048 x 2048 with
    per-128 scales, unrotated (config 1), and the ternary Llama-3.2-1B
    projections with a per-row absmean scale and FWHT-256-rotated outlier
    activations (config 2), each timed like the 8192^2 sweep."""
    rows = {"config1_int4_2048x2048": gemv_bench(L, synth, torch, L.FMT_INT4, 2048, steps, warmup,
                                                 rotate_in_kernel=False, group=128, seed=1, flush=flush)}
    rows["config1_int4_2048x2048"]["rotation"] = "none (the reference's int4 operator does not rotate)"
    for name, (n, k) in synth.LLAMA_TERNARY_SHAPES.items():
        if name in ("o_proj", "v_proj", "up_proj"):
            continue            # same shapes as q/k/gate
        key = "config2_ternary_" + {"q_proj": "q_o", "k_proj": "k_v", "gate_proj": "gate_up",
                                    "down_proj": "down"}[name] + f"_{n}x{k}"
        rows[key] = gemv_bench(L, synth, torch, L.FMT_TERNARY, n, steps, warmup, cols=k, group=0,
                               outliers=True, seed=2, flush=flush)
    return rows


PROBE_SHAPES = [(2, 512), (4, 256), (8, 256), (16, 256), (4, 512), (8, 512), (4, 1024)]


def time_graph(torch, launch, n, flush, replays):
    """Median per-launch time (ms) of n launches captured in one HIP graph,
    each replay after a cache flush, HIP events on the launch stream."""
    stream = torch.cuda.current_stream()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cg = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.graph(cg, stream=side):
        for i in range(n):
            launch(i)
    stream.wait_stream(side)
    cg.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        flush()
        torch.cuda.synchronize()
        s.record(stream)
        cg.replay()
        e.record(stream)
        torch.cuda.synchronize()
        ts.append(s.elapsed_time(e) / n)
    del cg
    return float(np.median(ts))


def achievable_bandwidth(torch, L, sizes, steps, flush, replays=7):
    """The achievable-bandwidth yardstick at each GEMV size, every read timed
    exactly like the GEMVs (steps launches over >= 512 MiB of distinct buffers
    in one HIP graph, replayed after a flush, median):
      * us_per_read: lmx_hbm_read_probe (2 loads in flight per lane, 512
        workgroups of 1024 lanes), the figure earlier runs reported;
      * shapes: the same linear read at other loads-in-flight x workgroups
        (lmx_hbm_read_probe_shape), best_us the fastest of them;
      * tile_schedule_us (sizes given with a weight shape): the weight's own
        tiles and scales read with the interleaved GEMV's load schedule, the
        CU's whole share requested at once (lmx_hbm_read_probe_tiles);
      * achievable_us: the fastest of all these reads, the yardstick of
        frac_of_achievable.
    Plus a 1 GiB read and torch's 1 GiB device copy for scale."""
    out = {}
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for name, spec in sizes.items():
        spec = spec if isinstance(spec, dict) else {"bytes": spec}
        nbytes = spec["bytes"] // 16 * 16
        copies = max(2, -(-ROTATE_BYTES // nbytes))
        bufs = [torch.ones(nbytes // 4, dtype=torch.float32, device="cuda") for _ in range(copies)]
        n = steps if nbytes < 2**28 else 3
        ms = time_graph(torch, lambda i: L.hbm_read_probe(bufs[i % copies], sink), n, flush, replays)
        r = {"bytes": nbytes, "us_per_read": round(ms * 1e3, 3),
             "GB_per_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
             "frac_of_peak": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        shapes = {}
        for inf, wg in PROBE_SHAPES:
            t = time_graph(torch, lambda i: L.hbm_read_probe_shape(bufs[i % copies], sink, inf, wg), n, flush,
                           replays)
            shapes[f"{inf}x{wg}"] = round(t * 1e3, 3)
        r["shapes_us"] = shapes
        best = min(shapes, key=shapes.get)
        r["best_us"], r["best_shape"] = shapes[best], best
        del bufs
        if "fmt" in spec:
            fmt, rows, cols, g = spec["fmt"], spec["rows"], spec["cols"], spec["group"]
            tb, sb = L.tile_bytes(fmt, rows, cols), L.tile_scales_bytes(fmt, rows, cols, g)
            wcopies = max(2, -(-ROTATE_BYTES // (tb + sb)))
            tiles = [torch.ones(tb // 4, dtype=torch.float32, device="cuda") for _ in range(wcopies)]
            scl = [torch.ones(sb // 4, dtype=torch.float32, device="cuda") for _ in range(wcopies)]
            t = time_graph(torch, lambda i: L.hbm_read_probe_tiles(tiles[i % wcopies], scl[i % wcopies], fmt, rows,
                                                                   cols, g, sink), n, flush, replays)
            r["tile_schedule_us"] = round(t * 1e3, 3)
            r["tile_schedule_bytes"] = tb + sb
            del tiles, scl
        r["achievable_us"] = min([r["us_per_read"], r["best_us"]] + ([r["tile_schedule_us"]] if "fmt" in spec
                                                                        else []))
        r["achievable_GB_per_s"] = round(nbytes / (r["achievable_us"] * 1e-6) / 1e9, 1)
        out[name] = r
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a = torch.empty(2**28, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        s.record()
        b.copy_(a)
        e.record()
        torch.cuda.synchronize()
        ts.append(s.elapsed_time(e))
    ms = float(np.median(ts))
    out["torch_copy_1GiB"] = {"bytes_moved": 2 * 2**30, "GB_per_s": round(2 * 2**30 / (ms * 1e-3) / 1e9, 1)}
    out["note"] = ("plain streaming reads of the same bytes (no arithmetic), timed like the GEMVs: what the "
                   "memory system delivers per launch at that size; us_per_read the default probe shape, "
                   "shapes_us other loads-in-flight x workgroups, tile_schedule_us the weight's tiles read with "
                   "the GEMV's own load schedule; frac_of_achievable in the sweep = GEMV GB/s / the fastest "
                   "(achievable_GB_per_s)")
    del a, b
    return out


def host_cpu():
    """CPU model and core counts of the host the CPU baselines run on."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"model": model, "nproc": affinity, "hardware_concurrency": os.cpu_count()}


# Reference CPU operators timed beside the GPU: (format, block bytes, threads).
# The reference's x86 lut_linear runs int4 and ternary single-threaded and
# binary on its ThreadPool of hardware_concurrency threads
# (lut_gemm_scalar.cpp:186-222, 7-61, 228-259; thread_pool.hpp:15-16).
CPU_FORMATS = {"int4": (6, "1"), "ternary": (1, "1"), "binary": (2, "pool")}


def cpu_baselines(n, budget_s=8.0):
    """The reference's own lut_linear (oracle/_ref/libref.so, built from its
    sources with its flags) on the n x n GEMV of each format in CPU_FORMATS, in
    its native 256-weight blocks (ternary with the row scale in every block,
    binary and int4 with per-256 scales), repeated for ~budget_s each; the
    C restatement (oracle, 1 thread) where the reference build is absent."""
    import oracle
    import lutmac_amd as L
    from lutmac_amd import synth
    R = oracle.ref()
    cpu = host_cpu()
    out = {}
    x = synth.make_activations(n, seed=5)
    for name, (fmt, threads) in CPU_FORMATS.items():
        planes, scales, _ = synth.make_weights(fmt, n, n, seed=3000 + fmt, group=256 if fmt != 1 else 0)
        if fmt == 1:   # one row scale, replicated into every block
            scales = np.repeat(scales.reshape(1, n, 1), n // 256, axis=2)
        blocks = L.planes_to_blocks(fmt, planes, scales, n, n)
        del planes
        nb = n * (n // 256)
        y = np.zeros(n, np.float32)
        reps, t0 = 0, time.perf_counter()
        while True:
            if R is not None:
                R.ref_lut_linear(fmt, oracle._ptr(blocks), nb, None, oracle._ptr(x), oracle._ptr(y), n, n, 1)
            else:
                oracle.lut_linear(fmt, blocks, x, n, n)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        t = el / reps
        B = synth.algorithmic_bytes(fmt, n, n, group=256)
        cores = (cpu["hardware_concurrency"] if threads == "pool" else 1) if R is not None else 1
        out[name] = {"value": round(B / t / 1e9, 4), "unit": "GB/s", "cores": cores,
                     "kind": "reference" if R is not None else "port",
                     "ms_per_gemv": round(t * 1e3, 2),
                     "sample": (f"{'oracle/_ref lut_linear (reference lut_gemm_scalar.cpp:68-180)' if R else 'oracle port'}"
                                f" {L.FORMAT_NAMES[fmt]} {n}x{n} batch 1, native 256-weight blocks, {reps} GEMVs in "
                                f"{el:.1f} s ({t * 1e3:.1f} ms each), "
                                + ("1 thread" if cores == 1 else
                                   f"the reference ThreadPool of {cores} threads on {cpu['nproc']} usable CPUs"))}
    for v in out.values():
        v["cpu"] = cpu["model"]
        v["nproc"] = cpu["nproc"]
    return out


def decode_weight_bytes(cfg, group):
    """HBM bytes of the weights one token step reads: every linear and the tied
    head (4-bit codes + fp32 group scales), plus the norm weights."""
    rows_cols = [(cfg.q_dim + 2 * cfg.kv_dim, cfg.hidden), (cfg.hidden, cfg.q_dim),
                 (2 * cfg.ffn, cfg.hidden), (cfg.hidden, cfg.ffn)]
    per_layer = sum(r * c // 2 + r * (c // group) * 4 for r, c in rows_cols) + 2 * cfg.hidden * 4
    head = cfg.vocab * cfg.hidden // 2 + cfg.vocab * (cfg.hidden // group) * 4
    return cfg.n_layers * per_layer + head + cfg.hidden * 4


def decode_bench(n_prompt, n_new, seed=2024):
    """greedy batch-1 decode of a random-init Llama-3.2-1B
    architecture, all linears and the tied head 4-bit with per-128 scales;
    64 seeded prompt tokens, then n_new generated tokens (one captured HIP
    graph per token step, replayed)."""
    from lutmac_amd import decode as D
    from dataclasses import replace
    cfg = replace(D.LLAMA_3_2_1B, max_seq=max(D.LLAMA_3_2_1B.max_seq, n_prompt + n_new))
    t0 = time.perf_counter()
    model = D.SyntheticModel(cfg, seed=seed, group=128)
    dec = D.Decoder(model)
    setup_s = time.perf_counter() - t0
    prompt = np.random.default_rng(seed + 1).integers(0, cfg.vocab, n_prompt)
    dec.generate(prompt, n_new)                         # untimed: first launches, graph set-up
    out, pre_ms, dec_ms = dec.generate(prompt, n_new)
    tok_s = (n_new - 1) / (dec_ms / 1e3)
    B = decode_weight_bytes(cfg, 128)
    kv_avg = 2 * cfg.n_layers * cfg.kv_dim * 4 * (n_prompt + n_new / 2)   # K and V read per step, mean length
    dec.close()
    return {"metric": "1B-arch decode tokens/s bs=1", "tokens_per_s": round(tok_s, 1),
            "ms_per_token": round(dec_ms / (n_new - 1), 4),
            "prefill_tokens_per_s": round(n_prompt / (pre_ms / 1e3), 1),
            "n_prompt": n_prompt, "n_new": n_new,
            "timing": "HIP events around the graph replays; decode = the n_new-1 steps after the prompt",
            "config": {"workload": "Llama-3.2-1B architecture, random-init N(0,0.02) weights, 4-bit per-128-group "
                                   "linears and tied 4-bit embedding/head, greedy (BASELINE config 4)",
                       "layers": cfg.n_layers, "hidden": cfg.hidden, "heads": cfg.n_heads,
                       "kv_heads": cfg.n_kv_heads, "ffn": cfg.ffn, "vocab": cfg.vocab,
                       "rope": "theta 500000, llama3 scaling factor 32"},
            "weight_bytes_per_token": B, "kv_bytes_per_token_mean": int(kv_avg),
            "achieved_GB_s": round((B + kv_avg) * tok_s / 1e9, 1),
            "frac_of_peak": round((B + kv_avg) * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
            "first_tokens": [int(t) for t in out[n_prompt:n_prompt + 8]],
            "setup_s": round(setup_s, 1)}


def qwen_decode_bench(context, n_new, batches=(1, 4, 16), seed=2025):
    """greedy decode of a random-init Qwen-2.5-1.5B
    architecture (QKV bias, GQA 12/2, head_dim 128, tied 151936 x 1536 4-bit
    head) with a KV context of `context` positions, at each batch size: B
    seeded prompts of context - n_new tokens prefilled in lockstep, then n_new
    generated tokens per sequence, each step attending over ~context
    positions.  Per batch: step time, tokens/s per sequence and in aggregate,
    and the HBM bytes a step reads (weights once, every sequence's KV)."""
    from lutmac_amd import decode as D
    from dataclasses import replace
    cfg = replace(D.QWEN_2_5_1_5B, max_seq=context)
    t0 = time.perf_counter()
    model = D.SyntheticModel(cfg, seed=seed, group=128)
    setup_s = time.perf_counter() - t0
    W = decode_weight_bytes(cfg, 128)
    kv_seq = 2 * cfg.n_layers * cfg.kv_dim * 4 * (context - n_new / 2)
    per_batch = {}
    for B in batches:
        dec = D.Decoder(model, batch=B)
        prompt = np.random.default_rng(seed + 1).integers(0, cfg.vocab, (B, context - n_new))
        out, pre_ms, dec_ms = dec.generate(prompt if B > 1 else prompt[0], n_new)
        dec.close()
        step_ms = dec_ms / (n_new - 1)
        per_batch[str(B)] = {"ms_per_step": round(step_ms, 4),
                             "tokens_per_s_per_sequence": round(1e3 / step_ms, 1),
                             "tokens_per_s_aggregate": round(B * 1e3 / step_ms, 1),
                             "prefill_ms": round(pre_ms, 1),
                             "step_bytes": int(W + B * kv_seq),
                             "achieved_GB_s": round((W + B * kv_seq) / step_ms / 1e6, 1)}
    return {"metric": "Qwen-2.5-1.5B-arch decode tokens/s bs=1/4/16, KV context " + str(context),
            "tokens_per_s": per_batch[str(batches[0])]["tokens_per_s_per_sequence"],
            "ms_per_token": per_batch[str(batches[0])]["ms_per_step"], "kv_context": context,
            "prefill_tokens": context - n_new, "n_new": n_new,
            "weight_bytes_per_step": W, "kv_bytes_per_sequence_step_mean": int(kv_seq),
            "per_batch": per_batch,
            "config": {"workload": "Qwen-2.5-1.5B architecture, random-init N(0,0.02) weights, 4-bit per-128-group "
                                   "linears, QKV bias, tied 4-bit embedding/head, greedy, sequences in lockstep "
                                   "(BASELINE config 5)",
                       "layers": cfg.n_layers, "hidden": cfg.hidden, "heads": cfg.n_heads,
                       "kv_heads": cfg.n_kv_heads, "head_dim": cfg.head_dim, "ffn": cfg.ffn, "vocab": cfg.vocab},
            "setup_s": round(setup_s, 1)}


def attention_position_check(caps=(128, 2048), n_prompt=64, n_new=8, seed=2024):
    """Attention cost follows the position, not the KV capacity: the
    Llama-3.2-1B decode step at positions 64..71 with the cache sized for
    `caps` positions (the attention kernel launches one workgroup per KV head
    and 64-position chunk of the capacity; chunks past the position load
    nothing).  Returns the decode ms per step for each capacity; a kernel
    trace separates the attention kernels by their grid size."""
    from dataclasses import replace
    from lutmac_amd import decode as D
    model = D.SyntheticModel(replace(D.LLAMA_3_2_1B, max_seq=max(caps)), seed=seed, group=128)
    prompt = np.random.default_rng(seed + 1).integers(0, model.cfg.vocab, n_prompt)
    out = {}
    for cap in caps:
        model.cfg = replace(model.cfg, max_seq=cap)
        dec = D.Decoder(model)
        dec.generate(prompt, n_new)
        _, _, dec_ms = dec.generate(prompt, n_new)
        dec.close()
        out[str(cap)] = {"ms_per_step": round(dec_ms / (n_new - 1), 4), "attention_grid": 8 * (-(-cap // 64))}
    return {"positions": f"{n_prompt}..{n_prompt + n_new - 1}", "per_capacity": out}


def cpu_decode_baseline(budget_s, seed=2024):
    """The reference's own Model::forward (oracle/_ref/libref.so, 1 thread:
    lut_linear -> int4_gemv scalar) on the same architecture in its native
    form (group-256 Int4Blocks, its RoPE), token steps until ~budget_s."""
    import oracle
    from lutmac_amd import decode as D
    from dataclasses import replace
    if oracle.ref() is None:
        return None
    cfg = replace(D.LLAMA_3_2_1B, rope_mode=D.ROPE_REFERENCE, rope_factor=1.0, max_seq=64)
    ref = oracle.RefDecoder(D.SyntheticModel(cfg, seed=seed, group=256))
    toks = np.random.default_rng(seed + 1).integers(0, cfg.vocab, 64)
    n, t0 = 0, time.perf_counter()
    while True:
        ref.step(toks[n], n)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 64:
            break
    ref.close()
    return {"value": round(n / el, 3), "unit": "tokens/s", "cores": 1, "kind": "reference",
            "sample": f"reference Model::forward (src/model.cpp:47-453) via oracle/_ref, Llama-3.2-1B "
                      f"architecture in group-256 Int4Blocks, {n} token steps at positions 0..{n - 1} "
                      f"in {el:.1f} s, 1 thread"}


QWEN_SHAPES = {   # BASELINE config 5 linears (rows, cols): q|k|v fused, o, gate|up fused, down, tied head
    "qkv": (2048, 1536), "o": (1536, 1536), "gate_up": (17920, 1536), "down": (1536, 8960),
    "head": (151936, 1536)}


def batched_bench(torch, L, batches=(1, 4, 16), steps=100):
    """BASELINE config 5's question: the 4-bit LUT-GEMVs of a Qwen-2.5-1.5B
    architecture at batch 1/4/16, weights streamed once per group of vectors
    (batched kernel from batch 4).  Per shape: us per call; per batch: the
    time of one decode step's linears (28 layers + head) and the implied
    linear-layer tokens/s (attention and the rest of the step excluded)."""
    out = {"shapes": {}, "per_batch": {}}
    rng = np.random.default_rng(11)
    for name, (n, k) in QWEN_SHAPES.items():
        planes = rng.integers(0, 256, (4, n, k // 8), dtype=np.uint8)
        scales = (np.abs(rng.standard_normal((1, n, k // 128))) * 0.02).astype(np.float32)
        wbytes = n * k // 2 + n * (k // 128) * 4
        copies = max(2, -(-ROTATE_BYTES // wbytes))
        ws = [L.Weight.from_planes(L.FMT_INT4, planes, scales, n, k, 128) for _ in range(copies)]
        res = {}
        for B in batches:
            x = torch.randn(B * k, device="cuda")
            y = torch.empty(B * n, device="cuda")
            stream = torch.cuda.current_stream()
            for w in ws:                      # first batched call per handle grows its scratch
                w.gemv(x, y, stream=stream)
            torch.cuda.synchronize()
            cg = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(stream)
            with torch.cuda.graph(cg, stream=side):
                for i in range(steps):
                    ws[i % copies].gemv(x, y)
            stream.wait_stream(side)
            cg.replay()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            cg.replay()
            b.record(stream)
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / steps
            res[str(B)] = {"us": round(us, 3), "weight_GB_per_s": round(wbytes / us / 1e3, 1),
                           "us_per_vector": round(us / B, 3)}
            del cg
        out["shapes"][name] = {"rows": n, "cols": k, **res}
        for w in ws:
            w.close()
    for B in batches:
        per_layer = sum(out["shapes"][s][str(B)]["us"] for s in ("qkv", "o", "gate_up", "down"))
        step_us = 28 * per_layer + out["shapes"]["head"][str(B)]["us"]
        out["per_batch"][str(B)] = {"linears_us_per_step": round(step_us, 1),
                                    "linear_tokens_per_s": round(B / (step_us * 1e-6), 1)}
    return out


def calibrate_copy(nbytes=35717120, steps=200):
    """Plain device copy of a known size (torch's copy kernel), the yardstick
    that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch
    a = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(steps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": nbytes, "steps": steps}), flush=True)


def load_traffic(workload_key):
    """HBM bytes per GEMV measured with rocprofv3 --pmc (profiles/traffic.json)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(workload_key, {}).get("bytes_per_gemv")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--size", type=int, default=8192)
    ap.add_argument("--formats", default="int4,ternary,binary,rrq2,rrq3,int8,int4_rot")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU baseline budget per format")
    ap.add_argument("--replays", type=int, default=7, help="timed graph replays (median reported)")
    ap.add_argument("--no-configs", action="store_true", help="skip the BASELINE config 1/2 shape rows")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the 1B-architecture decode")
    ap.add_argument("--no-batched", action="store_true", help="skip the Qwen-shape batch 1/4/16 sweep")
    ap.add_argument("--batched-steps", type=int, default=100, help="launches per timed graph in that sweep")
    ap.add_argument("--no-qwen-decode", action="store_true", help="skip the Qwen-2.5-1.5B batch-1 decode")
    ap.add_argument("--qwen-context", type=int, default=2048)
    ap.add_argument("--qwen-tokens", type=int, default=64)
    ap.add_argument("--decode-prompt", type=int, default=64)
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--cpu-decode-seconds", type=float, default=10.0)
    ap.add_argument("--no-graph", action="store_true",
                    help="time one stream launch per GEMV only (no HIP-graph replay)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain device copy of 35717120 bytes (counter calibration)")
    ap.add_argument("--attn-check", action="store_true",
                    help="only run the attention-vs-KV-capacity check (Llama-1B decode at positions 64..71)")
    args = ap.parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.attn_check:
        print(json.dumps({"attention_position_check": attention_position_check()}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(a sharded GEMV would run this path on each GPU's row block)", file=sys.stderr)
        sys.exit(2)

    import torch
    import lutmac_amd as L
    from lutmac_amd import synth
    assert torch.cuda.is_available(), "bench.py needs a GPU"

    names = [f for f in args.formats.split(",") if f]
    flush = Flush(torch)
    sweep = {}
    for name in names:
        r = gemv_bench(L, synth, torch, FORMATS[name], args.size, args.steps, args.warmup,
                       graph=not args.no_graph, rotate_in_kernel=name in ROTATE_IN_KERNEL, flush=flush,
                       replays=args.replays)
        sweep[name] = r
        print(f"# {name}: {r['us_per_gemv']} us/GEMV, {r['GB_per_s']} GB/s "
              f"({100 * r['frac_of_peak']:.1f}% of peak)", file=sys.stderr, flush=True)
    head = sweep.get("int4") or sweep[names[0]]
    configs = None
    if not args.no_configs:
        configs = config_rows(L, synth, torch, args.steps, args.warmup, flush)
        for k, r in configs.items():
            print(f"# {k}: {r['us_per_gemv']} us/GEMV, {r['GB_per_s']} GB/s "
                  f"({100 * r['frac_of_peak']:.1f}% of peak)", file=sys.stderr, flush=True)
    def read_spec(v):
        return {"bytes": v["algorithmic_bytes"], "fmt": FORMATS[v["format"]], "rows": v["rows"], "cols": v["cols"],
                "group": v["group"]}
    read_sizes = {f"{k}_{args.size}": read_spec(v) for k, v in sweep.items()}
    if configs:
        read_sizes.update({k: read_spec(v) for k, v in configs.items()})
    read_sizes["1GiB"] = 2**30
    achievable = achievable_bandwidth(torch, L, read_sizes, args.steps, flush, replays=args.replays)
    for k, r in list(sweep.items()) + list((configs or {}).items()):
        key = f"{k}_{args.size}" if k in sweep else k
        a = achievable[key]
        r["read_probe_us"] = a["us_per_read"]
        r["read_probe_best_us"] = a["best_us"]
        r["read_probe_tiles_us"] = a.get("tile_schedule_us")
        r["achievable_us"] = a["achievable_us"]
        r["frac_of_achievable"] = round(r["GB_per_s"] / a["achievable_GB_per_s"], 4)
    print("# achievable (plain reads of the same bytes): " + ", ".join(
        f"{k} {v['us_per_read']} us (best shape {v['best_shape']} {v['best_us']} us, tile schedule "
        f"{v.get('tile_schedule_us')} us)" for k, v in achievable.items() if isinstance(v, dict) and "us_per_read" in v),
        file=sys.stderr, flush=True)
    del flush
    decode = None
    if not args.no_decode:
        decode = decode_bench(args.decode_prompt, args.decode_tokens)
        print(f"# decode: {decode['tokens_per_s']} tokens/s ({decode['ms_per_token']} ms/token)",
              file=sys.stderr, flush=True)
    qwen = None
    if not args.no_decode and not args.no_qwen_decode:
        qwen = qwen_decode_bench(args.qwen_context, args.qwen_tokens)
        print(f"# qwen decode (KV {qwen['kv_context']}): " + ", ".join(
            f"bs {b}: {v['tokens_per_s_aggregate']} tokens/s ({v['ms_per_step']} ms/step)"
            for b, v in qwen["per_batch"].items()), file=sys.stderr, flush=True)
    batched = None if args.no_batched else batched_bench(torch, L, steps=args.batched_steps)
    if batched is not None:
        print("# batched linears per step: " + ", ".join(
            f"bs {b}: {v['linears_us_per_step']} us" for b, v in batched["per_batch"].items()),
            file=sys.stderr, flush=True)
    cpus = None if args.no_cpu else cpu_baselines(args.size, args.cpu_seconds)
    cpu = None if cpus is None else cpus["int4" if head["format"] == "int4" else head["format"]]
    if cpus is not None:
        print("# cpu: " + ", ".join(f"{k} {v['ms_per_gemv']} ms/GEMV ({v['cores']} threads)"
                                    for k, v in cpus.items()), file=sys.stderr, flush=True)
    if decode is not None and not args.no_cpu:
        decode["cpu_baseline"] = cpu_decode_baseline(args.cpu_decode_seconds)
    line = {
        "metric": METRIC,
        "value": head["GB_per_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_gemv"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded uniform codes, |N(0,1)|*0.02 group scales, N(0,1) activations)",
        "config": {"workload": f"LUT-GEMV {head['format']} {args.size}x{args.size} batch 1, "
                               f"group {head['group']}, {head['rotation']} (BASELINE config 3)",
                   "rows": args.size, "cols": args.size, "format": head["format"],
                   "group": head["group"], "batch": 1, "weight_copies": head["weight_copies"],
                   "rotated_MiB": head["rotated_MiB"]},
        "roofline": {"bound": "hbm", "achieved": head["GB_per_s"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": head["frac_of_peak"],
                     "traffic": load_traffic(f"{head['format']}_{args.size}"),
                     "achievable_read_GB_s": round(head["GB_per_s"] / head["frac_of_achievable"], 1),
                     "frac_of_achievable": head["frac_of_achievable"]},
        "cpu_baseline": cpu,
        "cpu_baselines": cpus,
        "achievable_bandwidth": achievable,
        "configs": configs,
        "decode": decode,
        "qwen_decode": qwen,
        "batched_qwen_linears": batched,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
