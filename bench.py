"""Benchmark of the quantized-weight matmul path on one MI355X.

A step is one fp8-weight DiT MLP at the 1024x1024-image shape: H = gelu_tanh(X . W_up^T * s_up) (GELU fused
in the GEMM epilogue) then Y = H . W_down^T * s_down, with M = 4096 tokens, hidden 3072, MLP 12288,
bf16 activations, fp8 e4m3fn weights with per-tensor f32 scales, fp32 accumulation. `value` is the
step's TFLOP/s (2 GEMMs x 2*M*N*K). Inputs are synthetic, generated with numpy and uploaded before the
timed region.

The same run reports, measured with HIP events on the context's compute stream (the stream every kernel
is launched on):
  * roofline: the up-projection GEMM (the dominant kernel): 2*M*N*K FLOP per launch over its average launch
    time in the timed steps (timestamps between the launches), against the bf16 / f16 dense MFMA peak;
  * roofline_int4: the int4 decode GEMV (M = 1, K = 3584, N = 18944, group 64): algorithmic bytes per
    launch (every tensor read or written once) over its average launch time, against HBM peak; 10
    weight copies rotate (> 256 MB) so no launch reads its weights from the Infinity Cache; M = 8 and 16
    are reported beside it. These launches (~10 us) are shorter than the host's launch path, so they are
    timed as replays of a HIP graph of 20 launches (HIP events around the replays, no host gaps). A plain
    streaming read of one weight copy (we_read_peak, same rotation and timing) is the same-size probe the
    GEMV's rate is also reported against;
  * the dense bf16 GEMM at the DiT QKV shape and the small fp8 GEMM (M = 64);
  * c5_double_block: the double-stream DiT block (512 text + 4096 image tokens, hidden 3072, 24 heads,
    fp8 weights, bf16 activations) with its weights resident, the per-block weight copy from pinned host
    memory alone (H2D GB/s), and 4 blocks streamed through two device slots (overlap efficiency);
  * traffic: HBM bytes per launch from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this script, scaled by
    what the same counters read for the elementwise add kernel of known traffic that this script also
    launches (calibration); the measured values live in profiles/traffic.json;
  * cpu_baseline: the same workload on the host's cores: an f32 AVX-512 GEMM on every CPU of the process's
    affinity (oracle/cpu_gemm.c; the headline CPU number) and the float64 triple loop of the reference's tests
    on one core, over C1-C4, with the CPU model and core counts; sampled rows are extrapolated and say so.
"""
import argparse
import json
import os
import pathlib
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "web-engine_amd"))
import block as B  # noqa: E402
import we  # noqa: E402

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 / f16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
METRIC = "dequant-GEMM TFLOP/s @M=4096 (%MFMA peak); int4 GEMV GB/s (%HBM peak)"
TRAFFIC = ROOT / "profiles" / "traffic.json"


def bf16_bits(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def fp8_finite_codes(rng, n):
    v = rng.integers(0, 254, n, dtype=np.int32)  # the 254 finite e4m3fn codes: skip 0x7f and 0xff
    return (v + (v >= 0x7F)).astype(np.uint8)


def time_launches(g, fn, iters):
    g.sync()
    g.timer_start()
    for i in range(iters):
        fn(i)
    return g.timer_stop() / iters  # ms per launch, HIP events on the compute stream


def time_graph(g, fn, per_graph, replays):
    """Kernels too short for the host to keep the GPU fed (~12 us) are timed as replays of a HIP graph that
    holds per_graph calls: ms per call, HIP events on the compute stream, no host gaps between kernels."""
    g.sync()
    g.graph_begin()
    for i in range(per_graph):
        fn(i)
    graph = g.graph_end()
    g.graph_launch(graph)  # warm
    g.sync()
    g.timer_start()
    for _ in range(replays):
        g.graph_launch(graph)
    ms = g.timer_stop() / (replays * per_graph)
    g.graph_destroy(graph)
    return ms


def settle_steps(g, step, group=10, min_ms=40.0, max_ms=400.0, tol=0.01):
    """Runs untimed steps in groups until the time per step stops drifting (a group within tol of the previous one,
    after at least min_ms; at most max_ms). Returns the count, the time and the first and last groups' us per step."""
    total, n, prev, first, last = 0.0, 0, None, None, None
    while True:
        ms = time_launches(g, lambda i: step(n + i), group) * group
        total += ms
        n += group
        per = ms / group * 1e3
        first = per if first is None else first
        done = prev is not None and abs(per - prev) <= tol * per and total >= min_ms
        prev = last = per
        if done or total >= max_ms:
            break
    return {"steps": n, "ms": round(total, 2), "first_group_us_per_step": round(first, 1),
            "last_group_us_per_step": round(last, 1)}


def bench_mlp(g, steps, warmup, rng):
    m, h, f = 4096, 3072, 12288
    x = g.buffer(bf16_bits(rng.standard_normal(m * h, dtype=np.float32)))
    w_up = g.buffer(fp8_finite_codes(rng, f * h))
    w_dn = g.buffer(fp8_finite_codes(rng, h * f))
    hid = g.buffer(m * f * 2)
    y = g.buffer(m * h * 2)
    p_up = we.matmul_params(m, f, h, 0.02, graph=g)
    p_dn = we.matmul_params(m, h, f, 0.02, graph=g)

    def up(_=0):
        g.matmul(p_up, we.BF16, x, we.FP8, w_up, we.BF16, hid, flags=we.EPI_GELU)

    def down(_=0):
        g.matmul(p_dn, we.BF16, hid, we.FP8, w_dn, we.BF16, y)

    def step(_=0):
        up()
        down()

    # The chip's power management answers the first milliseconds of sustained MFMA load from idle with a transient:
    # measured on MI355X from a cold start, steps 1-3 take 512-528 us, step 7 651 us, and the time decays back to
    # 490 us by about step 50 (28 ms), where it stays (381 further steps at 487-499 us). So untimed steps run first
    # until the step time has settled (groups of 10 steps within 1% of the previous group, at least 40 ms, at most
    # 400 ms); the line reports what that took. Then `warmup` untimed steps, then `steps` timed ones with a timestamp
    # before each GEMM and after the last (events on the compute stream, no host round trip): the line's value is the
    # whole run (first to last timestamp), and each GEMM's duration inside it is what the roofline reports, from the
    # same launches.
    settle = settle_steps(g, step)
    for _ in range(warmup):
        step()
    n = steps
    assert 2 * n + 1 <= we.TIMER_MARKS, "at most 127 timed steps"
    g.sync()
    for i in range(n):
        g.timer_mark(2 * i)
        up()
        g.timer_mark(2 * i + 1)
        down()
    g.timer_mark(2 * n)
    ms_step = g.timer_between(0, 2 * n) / n
    ups = [g.timer_between(2 * i, 2 * i + 1) for i in range(n)]
    dns = [g.timer_between(2 * i + 1, 2 * i + 2) for i in range(n)]
    ms_up, ms_dn = float(np.mean(ups)), float(np.mean(dns))
    flop = 2.0 * m * f * h
    res = {
        "settle": settle,
        "ms_per_step": ms_step,
        "step_tflops": 2 * flop / ms_step / 1e9,
        "up": {"ms": ms_up, "tflops": flop / ms_up / 1e9, "flop": flop, "median_ms": float(np.median(ups)),
               "launches": n, "timed": "the timed steps' up-projections (timestamps between the launches)"},
        "down": {"ms": ms_dn, "tflops": flop / ms_dn / 1e9, "median_ms": float(np.median(dns))},
    }
    for b in (x, w_up, w_dn, hid, y):
        g.free(b)
    return res


def bench_int4(g, rng, iters=200, copies=10):
    n, k, group = 18944, 3584, 64
    ws = [g.buffer(rng.integers(0, 2 ** 32, n * k // 8, dtype=np.uint32)) for _ in range(copies)]
    ss = [g.buffer(np.abs(rng.normal(0, 0.01, n * k // group)).astype(np.float16)) for _ in range(copies)]
    out = {}
    for m in (1, 8, 16):
        x = g.buffer(rng.standard_normal(m * k).astype(np.float16))
        y = g.buffer(m * n * 2)
        p = we.matmul_params(m, n, k, 1.0, graph=g)

        def run(i):
            g.matmul(p, we.F16, x, we.INT4, ws[i % copies], we.F16, y, scales=ss[i % copies], group=group)

        for i in range(copies):
            run(i)
        ms = time_graph(g, run, 2 * copies, iters // (2 * copies))
        nbytes = n * k // 2 + n * (k // group) * 2 + m * k * 2 + m * n * 2
        out[f"M{m}"] = {"us": ms * 1e3, "gbs": nbytes / ms / 1e6, "bytes": nbytes,
                        "frac_hbm": nbytes / ms / 1e6 / PEAK_HBM_GBS}
        g.free(x)
        g.free(y)
    # the same-size read probe: one streaming read of a weight copy (we_read_peak), the same rotation and graph
    # timing, i.e. what one launch that only reads these bytes achieves on this box
    wbytes = n * k // 2
    pout = g.buffer(we.read_peak_out_words(wbytes) * 4)

    def probe(i):
        g.read_peak(ws[i % copies], wbytes, pout)

    for i in range(copies):
        probe(i)
    ms = time_graph(g, probe, 2 * copies, iters // (2 * copies))
    out["read_probe_same_size"] = {"bytes": wbytes, "us": ms * 1e3, "gbs": wbytes / ms / 1e6}
    g.free(pout)
    for b in ws + ss:
        g.free(b)
    return out


def bench_gemm(g, rng, m, n, k, x_dt, w_dt, y_dt, iters=20, rotate=0):
    """One GEMM timed over repeated calls on the same operands. rotate > 0 (small M only): also the time per call
    when the calls cycle through `rotate` copies of the weights, so that they stream from HBM rather than from
    the caches (`us_rotating_weights`)."""
    xs = rng.standard_normal(m * k, dtype=np.float32)
    x = g.buffer(bf16_bits(xs) if x_dt == we.BF16 else xs.astype(np.float16) if x_dt == we.F16 else xs)

    def weights():
        if w_dt == we.FP8:
            return g.buffer(fp8_finite_codes(rng, n * k))
        return g.buffer(bf16_bits(rng.normal(0, 0.02, n * k).astype(np.float32)))

    ws = [weights() for _ in range(max(1, rotate))]
    y = g.buffer(m * n * we.ELEM_BYTES[y_dt])
    p = we.matmul_params(m, n, k, 0.02 if w_dt == we.FP8 else 1.0, graph=g)

    def run(i, w=ws[0]):
        g.matmul(p, x_dt, x, w_dt, w, y_dt, y)

    settle = None
    if m <= 64:
        for i in range(3):
            run(i)
    else:  # large GEMMs: past the power management's start transient (as the MLP steps)
        settle = settle_steps(g, run)
    ms = time_graph(g, run, 10, max(1, iters // 10)) if m <= 64 else time_launches(g, run, iters)
    flop = 2.0 * m * n * k
    res = {"us": ms * 1e3, "tflops": flop / ms / 1e9}
    if settle:
        res["settle_launches"] = settle["steps"]
    if rotate and m <= 64:
        def run_rot(i):
            g.matmul(p, x_dt, x, w_dt, ws[i % rotate], y_dt, y)

        for i in range(rotate):
            run_rot(i)
        ms_rot = time_graph(g, run_rot, rotate, 3)
        res["us_rotating_weights"] = ms_rot * 1e3
        res["rotating_copies"] = rotate
    for b in [x, y] + ws:
        g.free(b)
    return res


# Tile configurations of the fast GEMM (gemm_cfg tuning values) and the shapes the sweep times them on: the
# benchmarked DiT shapes (M = 4096 image tokens, the M = 512 text stream) and the reference tuner's own shapes
# (src/bench/tune.ts:5-9, 1928x1088 at 8740 tokens), all with fp8 weights unless named.
SWEEP_CFGS = {0: "256x256", 1: "256x128", 2: "128x128", 3: "64x64", 4: "32x64", 5: "256x192"}
SWEEP_SHAPES = [
    ("C3 up + GELU", 4096, 12288, 3072, we.FP8, we.EPI_GELU),
    ("C3 down", 4096, 3072, 12288, we.FP8, 0),
    ("C2 QKV, bf16 weights", 4096, 9216, 3072, we.BF16, 0),
    ("text QKV (M = 512)", 512, 9216, 3072, we.FP8, 0),
    ("text down (M = 512)", 512, 3072, 12288, we.FP8, 0),
    ("C1 (M = 64)", 64, 3072, 3072, we.FP8, 0),
    ("tune: q / gate / out", 8740, 6144, 6144, we.FP8, 0),
    ("tune: mlp gate / up", 8740, 16384, 6144, we.FP8, 0),
    ("tune: mlp down", 8740, 6144, 16384, we.FP8, 0),
]


def sweep_tiles(g, rng, iters=10):
    """The tile sweep behind the fast GEMM's tile pick (the role of tuneMatmul, src/bench/tune.ts:14-30): every
    tile configuration on every sweep shape, bf16 activations and output, TFLOP/s from HIP events. Each shape is
    warmed up first and the configurations are timed twice, in opposite orders, keeping the faster run, so no
    configuration is measured on cold clocks. "auto" is the library's own pick (gemm_cfg -1)."""
    rows = []
    for name, m, n, k, w_dt, flags in SWEEP_SHAPES:
        x = g.buffer(bf16_bits(rng.standard_normal(m * k, dtype=np.float32)))
        w = g.buffer(fp8_finite_codes(rng, n * k) if w_dt == we.FP8 else
                     bf16_bits(rng.normal(0, 0.02, n * k).astype(np.float32)))
        y = g.buffer(m * n * 2)
        p = we.matmul_params(m, n, k, 0.02, graph=g)
        flop = 2.0 * m * n * k

        def run(_=0):
            g.matmul(p, we.BF16, x, w_dt, w, we.BF16, y, flags=flags)

        best = {}
        order = ["auto"] + list(SWEEP_CFGS)
        for _ in range(3):
            run()
        for sweep_pass in (order, order[::-1]):
            for cfg in sweep_pass:
                g.set_tuning("gemm_cfg", -1 if cfg == "auto" else cfg)
                run()
                reps = iters if m <= 512 or cfg not in (3, 4) else 2
                ms = time_graph(g, run, 10, 1) if m <= 64 else time_launches(g, run, reps)
                best[cfg] = min(best.get(cfg, float("inf")), ms)
        g.set_tuning("gemm_cfg", -1)
        tflops = {("auto" if c == "auto" else SWEEP_CFGS[c]): flop / ms / 1e9 for c, ms in best.items()}
        top = max(v for c, v in tflops.items() if c != "auto")
        rows.append({"shape": name, "m": m, "n": n, "k": k, "weights": "fp8" if w_dt == we.FP8 else "bf16",
                     "gelu": bool(flags), "tflops": tflops,
                     "best": max((c for c in tflops if c != "auto"), key=tflops.get),
                     "auto_frac_of_best": tflops["auto"] / top})
        print(f"[sweep] {name}: " + ", ".join(f"{c} {v:.0f}" for c, v in tflops.items()), file=sys.stderr, flush=True)
        for b in (x, w, y):
            g.free(b)
    return rows


def bench_block(g, rng, layers=16, pinned_sets=4, iters=10):
    """The double-stream DiT block (512 text + 4096 image tokens, hidden 3072, 24 heads of 128, MLP 12288, fp8
    weights, bf16 activations): resident (weights already in HBM), the weight copies alone, and `layers`
    blocks whose weights stream from pinned host memory (block i from buffer i % pinned_sets, every block a
    full copy) through two device slots while the block before computes. Overlap efficiency =
    (t_copy + t_compute - t_streamed) / min(t_copy, t_compute), per block."""
    cfg, tt, rows, cols = B.DIT_DOUBLE_BLOCK, 512, 64, 64
    ti, H = rows * cols, cfg.hidden
    blk = B.DoubleBlock(g, cfg, tt, ti, we.BF16)
    layout = B.StreamLayout(cfg)
    host = np.empty(layout.nbytes, np.uint8)
    layout.fill(host, rng)
    scales = {s: {n: 0.02 / np.sqrt(cfg.mlp if n == "down" else H) for n in ("qkv", "proj", "up", "down")}
              for s in ("txt", "img")}
    rope = B.rope_for_image(g, rows, cols)
    tvec = g.buffer((rng.uniform(-0.2, 0.2, 6 * H)).astype(np.float32))
    xs = [(g.buffer(bf16_bits(rng.standard_normal(tt * H))), g.buffer(bf16_bits(rng.standard_normal(ti * H))))
          for _ in range(2)]
    resident = g.buffer(host)
    w_res = layout.weights(resident, scales)

    def forward(i, weights):
        a, b = xs[i % 2], xs[(i + 1) % 2]
        blk.forward(weights[0], weights[1], a[0], a[1], tvec, rope, b[0], b[1])

    settle = settle_steps(g, lambda i: forward(i, w_res), group=5)  # past the power management's start transient
    t_comp = time_launches(g, lambda i: forward(i, w_res), iters)
    # the joint attention alone, settled, right after the whole-block timing (after the long profile pass below
    # the chip runs it slower for a while: 286 against 251 us settled on one box)

    def attention(_=0):
        g.attention(tt + ti, 24, 24, 128, False, we.BF16, blk.qkv, we.Graph.slice(blk.qkv, H * 2, 0),
                    we.Graph.slice(blk.qkv, 2 * H * 2, 0), blk.o, q_stride=3 * H, k_stride=3 * H, v_stride=3 * H,
                    out_stride=H)

    attn_settle = settle_steps(g, attention)
    attn_ms = time_launches(g, attention, iters)
    # profileBlock (src/bench/block.ts:17-95): every step on its own, serial, each settled first: after the host-side gaps between steps the power management runs the
    # first milliseconds of a step at other clocks (attention: ~250 us settled, 300-320 unsettled, same box)
    ops = blk.profile(w_res[0], w_res[1], xs[0][0], xs[0][1], tvec, rope, xs[1][0], xs[1][1],
                      warm=lambda fn: settle_steps(g, lambda i: fn(), min_ms=20.0, max_ms=200.0))
    op_sum = {kind: sum(o["us"] for o in ops if o["kind"] == kind) for kind in ("linear", "attention", "other")}
    g.free(resident)

    pinned = [g.host_alloc(layout.nbytes) for _ in range(pinned_sets)]
    for p in pinned:
        g.host_view(p, layout.nbytes)[:] = host
    streamer = B.BlockStreamer(g, layout)
    # copies alone: the copy stream, ordered after a compute-stream event taken at the timer start
    g.sync()
    g.timer_start()
    start = g.record_compute()
    last = 0
    for i in range(layers):
        last = g.stream_copy(streamer.slots[i % 2], pinned[i % pinned_sets], layout.nbytes, start if i == 0 else last)
    g.wait_ticket(last)
    t_copy = g.timer_stop() / layers
    # streamed blocks
    g.sync()
    g.timer_start()
    streamer.run(pinned, lambda i, slot: forward(i, layout.weights(slot, scales)), start=g.record_compute(),
                 blocks=layers)
    t_stream = g.timer_stop() / layers
    g.sync()
    streamer.free()
    file_read = file_read_rate(layout, host, scales, pinned[0])
    for p in pinned:
        g.host_free(p)
    blk.free()
    flop = 2.0 * (tt + ti) * H * (3 * H + H + 2 * cfg.mlp) + 4.0 * (tt + ti) ** 2 * H
    attn_flop = 4.0 * (tt + ti) ** 2 * H
    return {"tokens": f"{tt} text + {ti} image", "layers_streamed": layers, "flop_per_block": flop,
            "resident_ms": t_comp, "resident_tflops": flop / t_comp / 1e9, "settle_forwards": settle["steps"],
            "attention_us": attn_ms * 1e3, "attention_tflops": attn_flop / attn_ms / 1e9,
            "attention_settle_launches": attn_settle["steps"],
            "weight_bytes_per_block": layout.nbytes, "copy_ms_per_block": t_copy,
            "h2d_gbs": layout.nbytes / t_copy / 1e6, "streamed_ms_per_block": t_stream,
            "overlap_efficiency": (t_copy + t_comp - t_stream) / min(t_copy, t_comp), "file_read": file_read,
            "profile": {"ops": ops, "linear_us": op_sum["linear"], "attention_us": op_sum["attention"],
                        "other_us": op_sum["other"], "sum_of_ops_us": sum(op_sum.values()),
                        "whole_block_us": t_comp * 1e3,
                        "note": "each step alone on one stream (profileBlock); the whole block overlaps the text "
                                "stream with the image stream and groups their projections"}}


def file_read_rate(layout, host, scales, pinned, threads=8, reps=3):
    """One block image written as a .safetensors file, then read by the native reader into pinned host memory
    (fill_from_file): the rate a streamed model is fed at when the file is in the page cache."""
    import tempfile
    import weights as W
    with tempfile.TemporaryDirectory() as d:
        path = pathlib.Path(d) / "block.safetensors"
        W.save(path, layout.file_tensors(host, scales, "double_blocks.0."))
        best = float("inf")
        with W.read_header(path) as st:
            for _ in range(reps):
                t0 = time.perf_counter()
                layout.fill_from_file(st, "double_blocks.0.", pinned, threads)
                best = min(best, time.perf_counter() - t0)
    return {"ms_per_block": best * 1e3, "gbs": layout.nbytes / best / 1e9, "threads": threads,
            "source": "page cache (file just written)"}


def measured_peaks(g, warmup_ms=500, rounds=3, runs=5, read_bytes=2 << 30):
    """The build's own ceilings, timePeak style (src/bench/peak.ts:69-109: warm up, then the fastest of `rounds`
    rounds of `runs` dispatches): dense bf16 MFMA on constant operands and on operands with the fp8-weight GEMM's
    bit statistics (the chip is power-bound under the GEMM, and toggling operand bits cost power), scalar f32 FMA,
    packed f16 FMA, int8 dot4, and a streaming read of `read_bytes` (beyond the 256 MB Infinity Cache)."""
    out = g.buffer(max(16384 * 256, we.read_peak_out_words(read_bytes)) * 4)
    kinds = {"mfma_bf16_tflops": (we.PEAK_MFMA_BF16, 2048, 2048),
             "mfma_bf16_data_tflops": (we.PEAK_MFMA_BF16_DATA, 2048, 2048), "f32_fma_tflops": (we.PEAK_F32, 16384, 4096),
             "f16_fma_tflops": (we.PEAK_F16, 16384, 4096), "i8_dot4_tops": (we.PEAK_I8, 16384, 4096)}
    res = {}
    for name, (kind, wg, iters) in kinds.items():
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < warmup_ms:
            g.peak(kind, wg, iters, out)
            g.sync()
        best = float("inf")
        for _ in range(rounds):
            g.timer_start()
            for _ in range(runs):
                ops = g.peak(kind, wg, iters, out)
            best = min(best, g.timer_stop() / runs)
        res[name] = ops / best / 1e9
    buf = g.buffer(read_bytes)
    for _ in range(3):
        g.read_peak(buf, read_bytes, out)
    best = float("inf")
    for _ in range(rounds):
        g.timer_start()
        for _ in range(runs):
            g.read_peak(buf, read_bytes, out)
        best = min(best, g.timer_stop() / runs)
    res["hbm_read_gbs"] = read_bytes / best / 1e6
    res["hbm_read_bytes"] = read_bytes
    g.free(buf)
    g.free(out)
    return res


def calibration_copy(g, nbytes=256 << 20):
    """A plain streaming kernel of known traffic (out = a + b over f32): reads 2 * nbytes, writes nbytes.
    Its FETCH_SIZE / WRITE_SIZE under rocprofv3 scale the counters of the kernels above."""
    n = nbytes // 4
    a, b, o = g.buffer(n * 4), g.buffer(n * 4), g.buffer(n * 4)
    for _ in range(3):
        g.elementwise(we.OP_ADD, n, 1, we.F32, a, b, None, o)
    g.sync()
    for buf in (a, b, o):
        g.free(buf)
    return {"kernel": "elementwise_kernel<F32> (add)", "read_bytes": 2 * nbytes, "write_bytes": nbytes}


def host_info():
    """The host the CPU numbers come from: CPU model, online CPUs, this process's affinity, vector ISA."""
    model, flags = "unknown", set()
    try:
        for line in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    affinity = sorted(os.sched_getaffinity(0))
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": len(affinity),
            "isa": [f for f in ("avx2", "fma", "avx512f", "avx512_bf16", "amx_bf16") if f in flags]}


def _timed(fn, min_s=0.0):
    """Seconds per call of fn: one call, repeated until min_s has passed (best of the repeats)."""
    best, total = float("inf"), 0.0
    while True:
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        best, total = min(best, dt), total + dt
        if total >= min_s:
            return best


def cpu_baseline(budget_s):
    """The reference's CPU path for this op is the float64 triple loop of tests/gpu/matmul.test.ts:26-35.

    Two legs, both on the same inputs' shapes as the GPU run:
      * faithful: that loop through the oracle's C restatement (or_matmul_f64), one core, float64 accumulation;
        C1 (64 x 3072 x 3072) in full, and whole rows of C2 / the C3 up-projection / C4 (M = 1) until about
        `budget_s` is used, extrapolated to the full M;
      * strong: oracle/cpu_gemm.c on every CPU of this process's affinity (at most 16), f32 accumulation, AVX-512
        when present: C1 in full, the C3 MLP step (up + GELU-tanh + down) and C2 on 192 sampled rows
        extrapolated to M = 4096 (the cost is linear in M at these sizes), C4 in full at M = 1, 8, 16.
    The headline value is the strong leg on the benchmarked workload (the C3 MLP step)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O
    rng = np.random.default_rng(7)
    threads = max(1, min(len(os.sched_getaffinity(0)), 16))
    hidden, mlp_n, mt = 3072, 12288, 4096
    w_up, w_down = fp8_finite_codes(rng, mlp_n * hidden), fp8_finite_codes(rng, hidden * mlp_n)
    w_qkv = bf16_bits(rng.normal(0, 0.02, 9216 * hidden).astype(np.float32))
    w_c1 = fp8_finite_codes(rng, 3072 * 3072)
    x_c1 = rng.standard_normal(64 * 3072).astype(np.float16).view(np.uint16)
    n4, k4, g4 = 18944, 3584, 64
    w4 = rng.integers(0, 2 ** 32, n4 * k4 // 8, dtype=np.uint64).astype(np.uint32)
    s4 = np.abs(rng.normal(0, 0.01, n4 * k4 // g4)).astype(np.float16).view(np.uint16)
    int4_bytes = lambda m: n4 * k4 // 2 + n4 * (k4 // g4) * 2 + m * k4 * 2 + m * n4 * 2

    # ---- strong leg
    rows = 192
    xs = bf16_bits(rng.standard_normal(rows * hidden, dtype=np.float32))

    def mlp_step():  # as on the GPU: GELU in the up GEMM's epilogue, bf16 hidden activations
        h = O.cpu_matmul(rows, mlp_n, hidden, 0.02, O.BF16, xs, O.FP8, w_up, y_dtype=O.BF16, threads=threads,
                         gelu=True)
        O.cpu_matmul(rows, hidden, mlp_n, 0.02, O.BF16, h, O.FP8, w_down, y_dtype=O.BF16, threads=threads)

    t_mlp = _timed(mlp_step, 1.0)
    mlp_flop = 2 * 2 * mt * hidden * mlp_n
    strong = {"c3_mlp_step": {"tflops": 2 * 2 * rows * hidden * mlp_n / t_mlp / 1e12,
                              "ms_extrapolated": t_mlp * mt / rows * 1e3,
                              "sample": f"{rows} of {mt} rows (up + GELU + down), extrapolated"}}
    t = _timed(lambda: O.cpu_matmul(rows, 9216, hidden, 1.0, O.BF16, xs, O.BF16, w_qkv, y_dtype=O.BF16,
                                    threads=threads), 0.5)
    strong["c2_bf16_qkv_4096x9216x3072"] = {"tflops": 2 * rows * 9216 * hidden / t / 1e12,
                                           "sample": f"{rows} of {mt} rows, extrapolated"}
    t = _timed(lambda: O.cpu_matmul(64, 3072, 3072, 0.02, O.F16, x_c1, O.FP8, w_c1, y_dtype=O.F16,
                                    threads=threads), 0.5)
    strong["c1_fp8_64x3072x3072"] = {"us": t * 1e6, "tflops": 2 * 64 * 3072 * 3072 / t / 1e12, "sample": "full"}
    for m in (1, 8, 16):
        x4 = rng.standard_normal(m * k4).astype(np.float16).view(np.uint16)
        t = _timed(lambda: O.cpu_matmul(m, n4, k4, 1.0, O.F16, x4, O.INT4, w4, s4, g4, y_dtype=O.F16,
                                        threads=threads), 0.5)
        strong[f"c4_int4_M{m}"] = {"us": t * 1e6, "gbs": int4_bytes(m) / t / 1e9, "sample": "full"}

    # ---- faithful leg: float64 loop, one core
    faithful = {}
    share = max(0.5, (budget_s - 2.5) / 3)  # the C4 row below takes about 2.5 s
    xf = bf16_bits(rng.standard_normal(64 * hidden, dtype=np.float32))
    for name, m_full, n, x_dt, x, w, w_dt in (
            ("c1_fp8_64x3072x3072", 64, 3072, O.F16, x_c1, w_c1, O.FP8),
            ("c3_up_4096x12288x3072", mt, mlp_n, O.BF16, xf, w_up, O.FP8),
            ("c2_bf16_qkv_4096x9216x3072", mt, 9216, O.BF16, xf, w_qkv, O.BF16)):
        p = O.matmul_params(64, n, hidden, 0.02)
        done, t0 = 0, time.perf_counter()
        while done < 64 and (done == 0 or time.perf_counter() - t0 < share):
            O.matmul_rows(p, x_dt, x, w_dt, w, done, done + 1)
            done += 1
        t = time.perf_counter() - t0
        faithful[name] = {"tflops": 2 * done * n * hidden / t / 1e12,
                          "sample": f"{done} of {m_full} rows, {t:.1f} s, extrapolated"}
    x4 = rng.standard_normal(k4).astype(np.float16).view(np.uint16)
    t0 = time.perf_counter()
    O.matmul(O.matmul_params(1, n4, k4, 1.0), O.F16, x4, O.INT4, w4, scales=s4, group=g4)
    t = time.perf_counter() - t0
    faithful["c4_int4_M1"] = {"us": t * 1e6, "gbs": int4_bytes(1) / t / 1e9, "sample": "full"}

    head = strong["c3_mlp_step"]
    return {"value": head["tflops"], "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"the benchmarked MLP step (up GEMM + GELU-tanh + down GEMM) on {rows} of {mt} token rows, "
                      f"oracle/cpu_gemm.c, f32 accumulation, {threads} threads, AVX-512: "
                      f"{'yes' if O.lib.cb_has_avx512() else 'no'}; extrapolated to M = {mt} "
                      f"({head['ms_extrapolated']:.0f} ms per step)",
            "host": host_info(), "strong": strong,
            "faithful": dict(faithful, cores=1,
                             note="float64 triple loop of tests/gpu/matmul.test.ts:26-35 (or_matmul_f64)"),
            "mlp_flop_per_step": mlp_flop}


def measured_traffic(name):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter runs, or None; with where they were
    measured (the commit and box recorded in profiles/traffic.json)."""
    try:
        data = json.loads(TRAFFIC.read_text())
        entry = data["kernels"][name]
        source = {k: data[k] for k in ("commit", "box", "command") if k in data}
        source["measured"] = "an earlier rocprofv3 --pmc run of this script (not this run)"
        return float(entry["fetch_bytes"]) + float(entry["write_bytes"]), source
    except (OSError, KeyError, ValueError):
        return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["mlp", "int4", "block", "gemm", "all"], default="all")
    ap.add_argument("--sweep", action="store_true",
                    help="time every GEMM tile configuration on the sweep shapes and print that table instead")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported: the library has no multi-GPU "
              f"path (sharding across GPUs is designed, not built)", file=sys.stderr)
        sys.exit(2)

    rng = np.random.default_rng(0)
    g = we.Graph(0)
    info = g.device_info()
    print(f"[bench] device {info}", file=sys.stderr, flush=True)
    if args.sweep:
        print(json.dumps({"sweep": sweep_tiles(g, rng), "device": info}), flush=True)
        g.destroy()
        return
    mlp = bench_mlp(g, args.steps, args.warmup, rng) if args.only in ("mlp", "all") else None
    print("[bench] mlp done", file=sys.stderr, flush=True)
    int4 = bench_int4(g, rng) if args.only in ("int4", "all") else None
    print("[bench] int4 done", file=sys.stderr, flush=True)
    extra = {}
    if args.only in ("block", "all"):
        extra["c5_double_block"] = bench_block(g, rng)
        print("[bench] block done", file=sys.stderr, flush=True)
    if args.only in ("gemm", "all"):
        extra["c2_bf16_qkv_4096x9216x3072"] = bench_gemm(g, rng, 4096, 9216, 3072, we.BF16, we.BF16, we.BF16)
        extra["c1_fp8_64x3072x3072"] = bench_gemm(g, rng, 64, 3072, 3072, we.F16, we.FP8, we.F16, rotate=32)
        # the drop-in caller's own dtypes: an unchanged src/model/ops.ts reaches we_matmul through
        # Graph.run(matmulFp8Wgsl, ...) with f32 x and f32 y (src/kernels/matmul.ts:129-131)
        extra["c3_up_f32_activations"] = dict(
            bench_gemm(g, rng, 4096, 12288, 3072, we.F32, we.FP8, we.F32, iters=10),
            note="up-projection shape with f32 x and f32 y, as Graph.run(matmulFp8Wgsl) issues it")
    extra["calibration"] = calibration_copy(g)
    peaks = measured_peaks(g) if args.only == "all" else None
    if peaks:
        extra["measured_peaks"] = peaks
    g.destroy()
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    line = {"metric": METRIC, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (numpy): X ~ N(0,1) as bf16, fp8 e4m3fn weights uniform over the 254 finite codes, "
                    "per-tensor scale 0.02",
            "config": {"workload": "fp8-weight DiT MLP, M=4096 tokens, hidden 3072, MLP 12288: up GEMM + fused "
                                   "GELU-tanh, then down GEMM (bf16 activations, fp32 accumulation)",
                       "m": 4096, "hidden": 3072, "mlp": 12288, "weights": "fp8_e4m3fn", "activations": "bf16"}}
    if mlp:
        line.update({"value": mlp["step_tflops"], "ms_per_step": mlp["ms_per_step"]})
        line["settle"] = dict(mlp["settle"], note="untimed steps before the warmup, run until the step time stopped "
                                                  "drifting (the power management's start transient)")
        up = mlp["up"]
        traffic, source = measured_traffic("gemm_fp8_up")
        line["roofline"] = {"bound": "mfma", "achieved": up["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                            "frac": up["tflops"] / PEAK_BF16_TFLOPS, "traffic": traffic, "traffic_source": source,
                            "kernel": "gemm_lds_kernel<256,256,2,4,bf16,fp8, ping-pong> up-projection "
                                      "4096x12288x3072 (+ fused GELU)",
                            "algorithmic": f"{up['flop']:.0f} FLOP per launch / {up['ms'] * 1e3:.1f} us"}
        if peaks:
            line["roofline"]["frac_of_measured_peak"] = up["tflops"] / peaks["mfma_bf16_tflops"]
            line["roofline"]["frac_of_data_peak"] = up["tflops"] / peaks["mfma_bf16_data_tflops"]
        line["up_proj_tflops"] = up["tflops"]
        line["down_proj_tflops"] = mlp["down"]["tflops"]
    if int4:
        line["int4_gemv"] = int4
        m1 = int4["M1"]
        traffic, source = measured_traffic("int4_decode_m1")
        line["roofline_int4"] = {"bound": "hbm", "achieved": m1["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                 "frac": m1["gbs"] / PEAK_HBM_GBS, "traffic": traffic, "traffic_source": source,
                                 "kernel": "int4_gemv_direct_kernel<7> M=1 K=3584 N=18944 group 64 (f16 x)",
                                 "algorithmic": f"{m1['bytes']} B per launch / {m1['us']:.2f} us",
                                 "frac_of_same_size_read_probe": m1["gbs"] / int4["read_probe_same_size"]["gbs"]}
        if peaks:
            line["roofline_int4"]["frac_of_measured_peak"] = m1["gbs"] / peaks["hbm_read_gbs"]
    line.update(extra)
    if cpu:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
