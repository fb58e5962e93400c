#!/usr/bin/env python3
"""Benchmark of the MI355X quantized matrix-product path.

Headline (BASELINE.json metric, configuration 2): the bandwidth-bound Q4 GEMV,
W4A16, M = 1 row of f16 activations, K = N = 4096, g32/f16 weights.
A step is one pass of the activations through WEIGHT_COPIES distinct Q4
[4096 x 4096] weights (one GEMV launch each, replayed as one HIP graph), so
the 256 MB Infinity Cache cannot serve repeated weights and the number is an
HBM number. `value` is whole-job GB/s of algorithmic bytes over the timed
region; `roofline` prices the GEMV kernel's average launch duration (the
timed region, HIP events on the library stream, over the launch count)
against 8 TB/s. `roofline.traffic` is the HBM bytes per launch measured with
rocprofv3 counters (profiles/q4_gemv_m1_k4096_n4096_traffic.json), when that
file is present.

Secondary configurations (GEMV at M = 4 and 8, the bit-exact W4A8 GEMV, the
int8 GEMM, the Q4 prefill GEMM and the encoder forward) are reported under
"secondary" in the same JSON line, each timed over back-to-back launches.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]
                    [--no-graph] [--calibrate-copy] [--tune MS]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
HBM_PEAK_GBS = 8000.0
F16_PEAK_TFLOPS = 2500.0
I8_PEAK_TOPS = 5000.0
WEIGHT_COPIES = 96
M_ROWS, K_DIM, N_DIM = 1, 4096, 4096
METRIC = "Q4 GEMM GB/s & TFLOP/s (% roofline); Pplx embeddings/sec @seq1024, 1 GPU"
TRAFFIC_FILE = ROOT / "profiles" / "q4_gemv_m1_k4096_n4096_traffic.json"
COPY_BYTES = 256 << 20


def gemv_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one W4A16 GEMV launch: packed codes (4 bits) and
    f16 scales per 32-run, f16 activations in, f32 outputs."""
    return n * k // 2 + n * (k // 32) * 2 + m * k * 2 + m * n * 4


def w4a8_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one W4A8 (g64/f32) product launch: codes, f32
    scales per 64-run, int8 activation codes with f32 scales per 64-run, f32
    outputs."""
    return n * k // 2 + n * (k // 64) * 4 + m * k + m * (k // 64) * 4 + m * n * 4


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def timed_ms(torch, stream, fn, reps: int) -> float:
    """Average duration of fn() over `reps` back-to-back calls: HIP events at
    both ends of the region, on the stream the kernels are launched on."""
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for r in range(reps):
        fn(r)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def graph_ms(torch, stream, step, launches: int, reps: int = 20) -> float:
    """Average launch duration of `step` (which enqueues `launches` launches)
    captured once as a HIP graph and replayed `reps` times back to back."""
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    ms = timed_ms(torch, stream, lambda r: graph.replay(), reps)
    return ms / launches


def cpu_baseline(seconds: float = 10.0) -> dict:
    """The reference's CPU W4A8 algorithm (C restatement of int8.rs:229-585,
    AVX2 rows<4,Q4>, threaded over 32-column tiles) on the same GEMV shape."""
    from oracle import oracle as o
    threads = max(1, min(16, os.cpu_count() or 1))
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((N_DIM, K_DIM)) * 0.02).astype(np.float32)
    codes, scales = o.weight_quantize(o.f32_to_bf16(w), N_DIM, K_DIM, 4)
    data, ps = o.panel_pack(codes, scales, N_DIM, K_DIM, 4)
    x = np.random.default_rng(0).standard_normal((M_ROWS, K_DIM)).astype(np.float32)
    if not o.has_avx2():
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", "sample": "AVX2 unavailable"}
    reps, start = 0, time.perf_counter()
    while time.perf_counter() - start < seconds:
        qx, sx = o.act_quantize(x, M_ROWS, K_DIM, 8)
        o.panel_apply_avx2(data, ps, N_DIM, K_DIM, 4, qx, sx, M_ROWS, threads)
        reps += 1
    elapsed = time.perf_counter() - start
    gbs = reps * gemv_bytes(M_ROWS, K_DIM, N_DIM) / elapsed / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} W4A8 GEMVs M={M_ROWS} K=N={K_DIM} (reference CPU algorithm, C restatement, "
                      f"AVX2, {threads} threads) in {elapsed:.1f} s, priced at the W4A16 launch's bytes; "
                      f"Rust toolchain unavailable"}


def gemv_lines(torch, ctx, rocm, weights, stream) -> dict:
    """Config 2 at M = 4 and 8 (W4A16) and the bit-exact W4A8 GEMV at M = 1."""
    out = {}
    for m in (4, 8):
        x = torch.randn((m, K_DIM), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda").half()
        y = torch.empty((m, N_DIM), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        def step():
            for w in weights:
                ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)
        ms = graph_ms(torch, stream, step, len(weights))
        gbs = gemv_bytes(m, K_DIM, N_DIM) / (ms * 1e-3) / 1e9
        out[f"q4_gemv_w4a16_m{m}_k4096_n4096"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                                  "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def w4a8_line(torch, ctx, rocm, stream) -> dict:
    """The reference's numeric mode (W4A8, g64/f32, bit-exact with the CPU
    path) on the config-2 shape, M = 1, over rotating weight copies."""
    copies = 48
    tmp = torch.empty((N_DIM, K_DIM), dtype=torch.float32, device="cuda")
    ws = []
    for c in range(copies):
        tmp.normal_(0.0, 0.02, generator=torch.Generator(device="cuda").manual_seed(1 + c))
        torch.cuda.synchronize()
        ws.append(ctx.quantize(tmp, rocm.F32, N_DIM, K_DIM, 4, 64))
    del tmp
    x = torch.randn((1, K_DIM), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda")
    y = torch.empty((1, N_DIM), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    def step():
        for w in ws:
            ctx.linear(w, x, rocm.F32, 1, y, rocm.W4A8)
    ms = graph_ms(torch, stream, step, copies)
    gbs = w4a8_bytes(1, K_DIM, N_DIM) / (ms * 1e-3) / 1e9
    for w in ws:
        w.free()
    return {"us_per_product": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
            "note": "one launch per product: activation quantization inside the grouped kernel (hip graph)"}


def secondary(torch, ctx, rocm, stream) -> dict:
    out = {}
    # config 4: int8 GEMM M=8192 K=N=4096
    m, n, k = 8192, 4096, 4096
    a = torch.randn((m, k), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda")
    b = torch.randn((n, k), generator=torch.Generator(device="cuda").manual_seed(1), device="cuda") * 0.02
    qa = torch.empty((m, k), dtype=torch.int8, device="cuda")
    qb = torch.empty((n, k), dtype=torch.int8, device="cuda")
    sa = torch.empty(m, device="cuda")
    sb = torch.empty(n, device="cuda")
    torch.cuda.synchronize()
    ctx.i8_quantize_rows(a, m, k, qa, sa)
    ctx.i8_quantize_rows(b, n, k, qb, sb)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ctx.sync()
    fn = lambda r: ctx.i8_gemm(qa, sa, m, qb, sb, n, k, y, raw=False)  # noqa: E731
    for r in range(3):
        fn(r)
    ms = timed_ms(torch, stream, fn, 20)
    tops = 2 * m * n * k / (ms * 1e-3) / 1e12
    out["int8_gemm_m8192_k4096_n4096"] = {"ms": round(ms, 4), "TOP/s": round(tops, 1),
                                          "frac_of_i8_peak": round(tops / I8_PEAK_TOPS, 4),
                                          "variant": ctx.info()["variants"]["i8_gemm"]}
    del a, b, qa, qb, y
    # config 5: Q4 prefill M=16384 K=4096 N=14336
    m, k, n = 16384, 4096, 14336
    wf = torch.randn((n, k), generator=torch.Generator(device="cuda").manual_seed(1), device="cuda") * 0.02
    torch.cuda.synchronize()
    w = ctx.quantize(wf, rocm.F32, n, k, 4, 32)
    del wf
    x = torch.randn((m, k), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda").half()
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    fn = lambda r: ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)  # noqa: E731
    for r in range(2):
        fn(r)
    ms = timed_ms(torch, stream, fn, 10)
    tf = 2 * m * n * k / (ms * 1e-3) / 1e12
    out["q4_prefill_w4a16_m16384_k4096_n14336"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                                   "frac_of_f16_peak": round(tf / F16_PEAK_TFLOPS, 4),
                                                   "variant": ctx.info()["variants"]["gemm_w4a16"],
                                                   "out": "f32"}
    del y
    # the same product in prefill form: f16 out (what the next layer reads), one rounding
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    fn = lambda r: ctx.linear_f16(w, x, m, y)  # noqa: E731
    for r in range(2):
        fn(r)
    ms = timed_ms(torch, stream, fn, 10)
    tf = 2 * m * n * k / (ms * 1e-3) / 1e12
    out["q4_prefill_w4a16_f16out_m16384_k4096_n14336"] = {
        "ms": round(ms, 4), "TFLOP/s": round(tf, 1), "frac_of_f16_peak": round(tf / F16_PEAK_TFLOPS, 4),
        "variant": ctx.info()["variants"]["gemm_w4a16"], "out": "f16",
        "note": "dz_linear_f16: f32 accumulation, each output rounded once to f16"}
    w.free()
    del x, y
    # the reference's own numerics (bit-exact W4A8, int8.rs fold order) at the config 5 shape:
    # f32 activations quantized to A8 on device, then the grouped product
    wf = torch.randn((n, k), generator=torch.Generator(device="cuda").manual_seed(1), device="cuda") * 0.02
    torch.cuda.synchronize()
    w = ctx.quantize(wf, rocm.F32, n, k, 4, 64)
    del wf
    x = torch.randn((m, k), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    fn = lambda r: ctx.linear(w, x, rocm.F32, m, y, rocm.W4A8)  # noqa: E731
    fn(0)
    ms = timed_ms(torch, stream, fn, 5)
    tops = 2 * m * n * k / (ms * 1e-3) / 1e12
    out["q4_prefill_w4a8_bitexact_m16384_k4096_n14336"] = {
        "ms": round(ms, 4), "TOP/s": round(tops, 1), "frac_of_i8_peak": round(tops / I8_PEAK_TOPS, 4),
        "variant": ctx.info()["variants"].get("grouped"),
        "note": "includes the A8 quantization of the f32 activations; VALU-bound fold (3 ops per output per group)"}
    w.free()
    del x, y
    # config 3: encoder forward, 24 x (1024, 16x64, 4096), batch 8 x 1024 tokens
    cfg = rocm.EncoderConfig(layers=24, hidden=1024, heads=16, head_dim=64, ffn=4096, vocab=32000, ln_eps=1e-5)
    enc = ctx.encoder_random(cfg, 1)
    ids = torch.from_numpy(np.random.default_rng(1).integers(0, 32000, 8 * 1024).astype(np.int32)).cuda()
    emb = torch.empty((8, 1024), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    enc.forward(ids, 8, 1024, emb)
    ctx.sync()
    ms = timed_ms(torch, stream, lambda r: enc.forward(ids, 8, 1024, emb), 5)
    flops = 2 * 8192 * (4 * 1024 * 1024 + 2 * 1024 * 4096) * 24 + 4 * 8 * 16 * 1024 * 1024 * 64 * 24
    out["encoder_forward_b8_s1024"] = {"ms": round(ms, 3), "embeddings/s": round(8 / (ms * 1e-3), 1),
                                       "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
                                       "frac_of_f16_peak": round(flops / (ms * 1e-3) / 1e12 / F16_PEAK_TFLOPS, 4)}
    enc.close()
    return out


def traffic_per_launch():
    """HBM bytes per GEMV launch from the committed rocprofv3 counter summary."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
        return int(data["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="plain launches (for counter collection)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help=f"also run a {COPY_BYTES >> 20} MiB device copy (counter calibration)")
    ap.add_argument("--tune", type=int, default=0, help="tuner budget in ms (0 keeps reference variants)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the hot path shards along N with one all-gather; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch
    from decisive_amd import rocm

    ctx = rocm.Context(0)
    if args.tune:
        ctx.tune(args.tune)
    log(f"[bench] device {ctx.info()}")

    if args.calibrate_copy:
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {COPY_BYTES} bytes done")
        del src, dst

    # inputs resident in HBM before the timed region
    x = torch.randn((M_ROWS, K_DIM), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda").half()
    weights = []
    tmp = torch.empty((N_DIM, K_DIM), dtype=torch.float32, device="cuda")
    for c in range(WEIGHT_COPIES):
        tmp.normal_(0.0, 0.02, generator=torch.Generator(device="cuda").manual_seed(1 + c))
        torch.cuda.synchronize()
        weights.append(ctx.quantize(tmp, rocm.F32, N_DIM, K_DIM, 4, 32))
    del tmp
    y = torch.empty((WEIGHT_COPIES, M_ROWS, N_DIM), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    log(f"[bench] {WEIGHT_COPIES} weight copies resident ({weights[0].device_bytes * WEIGHT_COPIES / 1e6:.0f} MB)")

    side = torch.cuda.Stream()
    ctx.set_stream(side.cuda_stream)

    def step():
        for c in range(WEIGHT_COPIES):
            ctx.linear(weights[c], x, rocm.F16, M_ROWS, y[c], rocm.W4A16)

    with torch.cuda.stream(side):
        step()
        torch.cuda.synchronize()
        if args.no_graph:
            run = step
        else:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=side):
                step()
            torch.cuda.synchronize()
            run = graph.replay
        for _ in range(args.warmup):
            run()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        wall0 = time.perf_counter()
        t0.record(side)
        for _ in range(args.steps):
            run()
        t1.record(side)
        torch.cuda.synchronize()
        wall = time.perf_counter() - wall0
        total_ms = t0.elapsed_time(t1)

    per_launch = gemv_bytes(M_ROWS, K_DIM, N_DIM)
    launches = args.steps * WEIGHT_COPIES
    # The launches run back to back on one stream, so the timed region divided
    # by the launch count is the kernel's average launch duration (what
    # rocprofv3's kernel trace reports per dispatch).
    kernel_ms = total_ms / launches
    value = launches * per_launch / (total_ms * 1e-3) / 1e9
    achieved = per_launch / (kernel_ms * 1e-3) / 1e9
    y_host = y[0].float().cpu().numpy()
    assert np.isfinite(y_host).all()
    log(f"[bench] timed {args.steps} steps: {total_ms:.3f} ms GPU, {wall * 1e3:.3f} ms wall; "
        f"kernel avg {kernel_ms * 1e3:.3f} us")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(total_ms / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (x N(0,1) seed 0; W N(0,0.02) seeds 1..96, Q4 g32/f16 quantized on device)",
        "config": {"workload": "q4_gemv_w4a16_m1_k4096_n4096_g32f16", "m": M_ROWS, "k": K_DIM, "n": N_DIM,
                   "weight_copies": WEIGHT_COPIES,
                   "launch": "plain launches" if args.no_graph else "hip graph of one GEMV per weight copy",
                   "variant": ctx.info()["variants"]["gemv"]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_per_launch(),
                     "kernel_us": round(kernel_ms * 1e3, 3), "bytes_per_launch": per_launch},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline()
    if not args.no_secondary:
        stream = torch.cuda.Stream()  # library kernels and timing events share this stream
        ctx.set_stream(stream.cuda_stream)
        with torch.cuda.stream(stream):
            sec = gemv_lines(torch, ctx, rocm, weights, stream)
            for wgt in weights:
                wgt.free()
            weights.clear()
            sec["q4_gemv_w4a8_m1_k4096_n4096_g64f32"] = w4a8_line(torch, ctx, rocm, stream)
            sec.update(secondary(torch, ctx, rocm, stream))
        result["secondary"] = sec
    ctx.set_stream(None)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
