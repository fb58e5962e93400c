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
    python bench.py --only pplx                      (the decider line alone)
    python bench.py --only encoder / floors / gemv (the encoder line; launch floors
                     at the GEMV's size; the GEMV at N = 16384 to 131072)
    python bench.py --only tune [--tune MS] [--tune-cache F] [--tune-out F]
                    (the tuner's selection, then each family's reference and
                     selected variants at the tuning shape, for rocprofv3)
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


def warm(torch, fn, ms: float = 60.0, least: int = 2):
    """Untimed calls of fn until about `ms` of wall time has passed (at least
    `least` calls): the clocks reach their steady state before timing."""
    start, r = time.perf_counter(), 0
    while r < least or (time.perf_counter() - start) * 1e3 < ms:
        fn(r)
        torch.cuda.synchronize()
        r += 1


def graph_ms(torch, stream, step, launches: int, reps: int = 20) -> float:
    """Average launch duration of `step` (which enqueues `launches` launches)
    captured once as a HIP graph and replayed `reps` times back to back."""
    from decisive_amd import rocm

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with rocm.capture(graph, stream):
        step()
    torch.cuda.synchronize()
    for _ in range(3):
        graph.replay()
    ms = timed_ms(torch, stream, lambda r: graph.replay(), reps)
    return ms / launches


def host_cpu() -> dict:
    """The host the CPU baselines run on: model, the vector extensions the
    reference's kernels could use, and the CPUs this process may run on (its
    affinity set, capped by a cgroup CPU quota when one is set)."""
    model, flags = None, []
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model is None:
                model = line.split(":", 1)[1].strip()
            if line.startswith("flags") and not flags:
                flags = line.split(":", 1)[1].split()
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if q != "max":
            quota = int(q) / int(period)
            usable = max(1, min(usable, int(quota)))
    except (OSError, ValueError):
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "usable_threads": usable, "cgroup_cpu_quota": quota,
            "avx2": "avx2" in flags and "fma" in flags, "avx512f": "avx512f" in flags}


def _timed_loop(body, seconds: float, least: int = 1):
    reps, start = 0, time.perf_counter()
    while reps < least or time.perf_counter() - start < seconds:
        body()
        reps += 1
    return reps, time.perf_counter() - start


def cpu_baseline(seconds: float = 8.0) -> dict:
    """The reference's CPU W4A8 algorithm (C restatement of int8.rs:229-585,
    AVX2 rows<4,Q4>, threaded over 32-column tiles like int8.rs:235-256) on
    the same GEMV shape, on one thread and on every usable thread of the host.
    `value` and `cores` are the all-threads figure."""
    from oracle import oracle as o
    host = host_cpu()
    threads = host["usable_threads"]
    if not o.has_avx2():
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "port", "sample": "AVX2 unavailable", "host": host}
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((N_DIM, K_DIM)) * 0.02).astype(np.float32)
    codes, scales = o.weight_quantize(o.f32_to_bf16(w), N_DIM, K_DIM, 4)
    data, ps = o.panel_pack(codes, scales, N_DIM, K_DIM, 4)
    x = np.random.default_rng(0).standard_normal((M_ROWS, K_DIM)).astype(np.float32)

    def leg(t):
        def body():
            qx, sx = o.act_quantize(x, M_ROWS, K_DIM, 8)
            o.panel_apply_avx2(data, ps, N_DIM, K_DIM, 4, qx, sx, M_ROWS, t)
        reps, elapsed = _timed_loop(body, seconds)
        return reps, elapsed, reps * gemv_bytes(M_ROWS, K_DIM, N_DIM) / elapsed / 1e9

    r1, e1, g1 = leg(1)
    rn, en, gn = leg(threads)
    return {"value": round(gn, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "single_thread": {"value": round(g1, 3), "cores": 1},
            "host": host,
            "sample": f"W4A8 GEMVs M={M_ROWS} K=N={K_DIM} by the reference CPU algorithm (C restatement of "
                      f"int8.rs rows<4,Q4>, AVX2 as the reference; the host also has AVX-512: "
                      f"{host['avx512f']}), priced at the W4A16 launch's bytes: {rn} in {en:.1f} s on {threads} "
                      f"threads (every usable CPU of the host, {host['model']}), {r1} in {e1:.1f} s on 1 thread; "
                      f"Rust toolchain unavailable"}


def encoder_cpu_baseline(seconds: float = 8.0) -> dict:
    """Config 3's encoder layer on the host cores, for one 1024-token sequence:
    the four projections by the reference's CPU W4A8 algorithm (C restatement
    of int8.rs:229-585, AVX2 rows<4,Q4>, threaded), attention by numpy float32
    matrix products (the reference's CPU attention is an sgemm), LayerNorm and
    GELU vectorized in numpy. Layers run until `seconds` have passed, on one
    thread (numpy's BLAS limited to one thread too) and on every usable
    thread; the per-layer time is scaled to the 24-layer forward."""
    from oracle import oracle as o
    from scipy.special import erf
    host = host_cpu()
    if not o.has_avx2():
        return {"value": None, "unit": "embeddings/s", "cores": 0, "kind": "port", "sample": "AVX2 unavailable",
                "host": host}
    threads = host["usable_threads"]
    d, heads, hd, ff, seq, layers = 1024, 16, 64, 4096, 1024, 24
    rng = np.random.default_rng(1)
    panels = []
    for rows, cols in ((3 * d, d), (d, d), (ff, d), (d, ff)):
        w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        codes, scales = o.weight_quantize(o.f32_to_bf16(w), rows, cols, 4)
        panels.append((o.panel_pack(codes, scales, rows, cols, 4), rows, cols))
    del w

    def layernorm(x):
        mu = x.mean(1, keepdims=True)
        c = x - mu
        return (c / np.sqrt((c * c).mean(1, keepdims=True) + 1e-5)).astype(np.float32)

    def run(t):
        def apply(i, x):
            (data, ps), rows, cols = panels[i]
            qx, sx = o.act_quantize(x, x.shape[0], cols, 8)
            return o.panel_apply_avx2(data, ps, rows, cols, 4, qx, sx, x.shape[0], t)

        def layer(h):
            qkv = apply(0, h)
            att = np.empty((seq, d), np.float32)
            for a in range(heads):
                q, k, v = (qkv[:, j * d + a * hd:j * d + (a + 1) * hd] for j in range(3))
                sc = (q @ k.T) * np.float32(1 / 8)
                p = np.exp(sc - sc.max(1, keepdims=True))
                att[:, a * hd:(a + 1) * hd] = (p @ v) / p.sum(1, keepdims=True)
            h = layernorm(apply(1, att) + h)
            f = apply(2, h)
            f = (0.5 * f * (1.0 + erf(f * np.float32(0.70710678)))).astype(np.float32)
            return layernorm(apply(3, f) + h)

        state = [layernorm(np.random.default_rng(1).standard_normal((seq, d)).astype(np.float32))]

        def body():
            state[0] = layer(state[0])
        try:
            from threadpoolctl import threadpool_limits
            with threadpool_limits(limits=t):
                done, elapsed = _timed_loop(body, seconds, least=2)
        except ImportError:
            done, elapsed = _timed_loop(body, seconds, least=2)
        assert np.isfinite(state[0]).all()
        return done, elapsed, 1.0 / (elapsed / done * layers)

    d1, e1, v1 = run(1)
    dn, en, vn = run(threads)
    return {"value": float(f"{vn:.4g}"), "unit": "embeddings/s", "cores": threads, "kind": "port",
            "single_thread": {"value": float(f"{v1:.4g}"), "cores": 1},
            "host": host,
            "sample": f"encoder layers of one 1024-token sequence scaled to 24 layers: {dn} in {en:.1f} s on "
                      f"{threads} threads ({host['model']}), {d1} in {e1:.1f} s on 1 thread (W4A8 AVX2 products "
                      f"by the reference CPU algorithm, numpy f32 attention/LayerNorm/GELU; one layer's weights "
                      f"reused); Rust toolchain unavailable"}


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


def wide_gemv_lines(torch, ctx, rocm, stream) -> dict:
    """The W4A16 GEMV's streaming rate where a launch's fixed cost is small:
    K = 4096 at N = 16384, 65536 and 131072 (37.7, 151 and 302 MB per launch),
    M = 1, 4 and 8, over rotating copies of about 906 MB (24, 6 and 3 copies),
    each a HIP graph of one launch per copy; the library's default variant
    ("auto")."""
    out = {}
    for n, copies in ((16384, 24), (65536, 6), (131072, 3)):
        tmp = torch.empty((n, K_DIM), dtype=torch.float32, device="cuda")
        ws = []
        for c in range(copies):
            tmp.normal_(0.0, 0.02, generator=torch.Generator(device="cuda").manual_seed(1 + c))
            torch.cuda.synchronize()
            ws.append(ctx.quantize(tmp, rocm.F32, n, K_DIM, 4, 32))
        del tmp
        for m in (1, 4, 8):
            x = torch.randn((m, K_DIM), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda").half()
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()

            def step():
                for w in ws:
                    ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)
            ms = graph_ms(torch, stream, step, len(ws))
            gbs = gemv_bytes(m, K_DIM, n) / (ms * 1e-3) / 1e9
            out[f"q4_gemv_w4a16_m{m}_k4096_n{n}"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                                     "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                                     "weight_copies": copies}
        for w in ws:
            w.free()
        del ws
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


def encoder_line(torch, ctx, rocm, stream) -> dict:
    """Config 3: the encoder forward, 24 x (1024, 16x64, 4096), batch 8 x 1024
    tokens, random Q4 g32 weights."""
    cfg = rocm.EncoderConfig(layers=24, hidden=1024, heads=16, head_dim=64, ffn=4096, vocab=32000, ln_eps=1e-5)
    enc = ctx.encoder_random(cfg, 1)
    ids = torch.from_numpy(np.random.default_rng(1).integers(0, 32000, 8 * 1024).astype(np.int32)).cuda()
    emb = torch.empty((8, 1024), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    warm(torch, lambda r: enc.forward(ids, 8, 1024, emb))
    ms = timed_ms(torch, stream, lambda r: enc.forward(ids, 8, 1024, emb), 5)
    flops = 2 * 8192 * (4 * 1024 * 1024 + 2 * 1024 * 4096) * 24 + 4 * 8 * 16 * 1024 * 1024 * 64 * 24
    enc.close()
    return {"ms": round(ms, 3), "embeddings/s": round(8 / (ms * 1e-3), 1),
            "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac_of_f16_peak": round(flops / (ms * 1e-3) / 1e12 / F16_PEAK_TFLOPS, 4)}


def int8_line(torch, ctx, stream) -> dict:
    """Config 4: the per-row int8 GEMM at M=8192, K=N=4096 (f32 out), the
    vendor library on the same codes, and the same launch on all-zero codes."""
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
    warm(torch, fn)
    ms = timed_ms(torch, stream, fn, 20)
    tops = 2 * m * n * k / (ms * 1e-3) / 1e12
    # the vendor library on the same codes (torch._int_mm: int8 x int8 -> int32,
    # the raw product without the f32 rescale), operands made contiguous first
    try:
        qbt = qb.t().contiguous()
        ri = torch.empty((m, n), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        lib = lambda r: torch._int_mm(qa, qbt, out=ri)  # noqa: E731
        warm(torch, lib)
        vendor = {"ms": round(timed_ms(torch, torch.cuda.current_stream(), lib, 20), 4),
                  "what": "torch._int_mm (hipBLASLt), raw int32 output"}
        del qbt, ri
    except Exception as e:  # the library may not take this shape on every build
        vendor = {"error": str(e)[:200]}
    # the same launch on all-zero codes: the difference is the power the operand
    # bits draw (the clock drops under toggling data), not work
    qa.zero_()
    qb.zero_()
    torch.cuda.synchronize()
    warm(torch, fn)
    ms_zero = timed_ms(torch, stream, fn, 20)
    line = {"ms": round(ms, 4), "TOP/s": round(tops, 1), "frac_of_i8_peak": round(tops / I8_PEAK_TOPS, 4),
            "ms_on_zero_codes": round(ms_zero, 4), "vendor_library": vendor,
            "variant": ctx.info()["variants"]["i8_gemm"]}
    del a, b, qa, qb, y
    return line


def secondary(torch, ctx, rocm, stream, cpu=True) -> dict:
    out = {"int8_gemm_m8192_k4096_n4096": int8_line(torch, ctx, stream)}
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
    warm(torch, fn)
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
    warm(torch, fn)
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
    warm(torch, fn)
    ms = timed_ms(torch, stream, fn, 5)
    tops = 2 * m * n * k / (ms * 1e-3) / 1e12
    out["q4_prefill_w4a8_bitexact_m16384_k4096_n14336"] = {
        "ms": round(ms, 4), "TOP/s": round(tops, 1), "frac_of_i8_peak": round(tops / I8_PEAK_TOPS, 4),
        "variant": ctx.info()["variants"].get("grouped"),
        "note": "includes the A8 quantization of the f32 activations; VALU-bound fold (3 ops per output per group)"}
    w.free()
    del x, y
    out["encoder_forward_b8_s1024"] = encoder_line(torch, ctx, rocm, stream)
    if cpu:
        out["encoder_forward_b8_s1024"]["cpu_baseline"] = encoder_cpu_baseline()
    # the Pplx decider at real size, one 1024-token chunk
    out["pplx_decider_forward_s1024"] = pplx_line(torch, ctx, rocm, stream)
    return out


def random_wire(rng, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    """A random Q4 g64/f32 wire matrix (packed.rs:3-56): codes uniform in
    [-7, 7] (nibbles code + 8), each group's f32 scale near std / 4.3 so the
    weights have about the standard deviation `std`."""
    groups = cols // 64
    wire = np.empty((rows, groups, 36), np.uint8)
    nib = rng.integers(1, 16, (rows, groups, 32, 2), dtype=np.uint8)
    wire[..., :32] = nib[..., 0] | (nib[..., 1] << 4)
    scale = (std / 4.3) * rng.uniform(0.8, 1.2, (rows, groups)).astype(np.float32)
    wire[..., 32:] = scale.astype(np.float32)[..., None].view(np.uint8)
    return wire.reshape(-1)


def pplx_line(torch, ctx, rocm, stream, n: int = 1024, layers: int = 32) -> dict:
    """The Pplx decider (backbone.rs:11-22 shape: 32 layers, hidden 2560, three
    gated-delta layers then one gated-attention layer, FFN 9216) on one chunk
    of `n` tokens with 4 answer markers, through dz_pplx_forward_rows: packed
    embedding rows in, logits out (both host buffers, so the 3.7 MB row copy is
    inside the timed region). Random wire weights: one delta layer's and one
    attention layer's tensors, uploaded to every layer of that kind (each
    layer holds its own device copy)."""
    cfg = rocm.PplxConfig(layers=layers, hidden=2560, ff=9216, delta_heads=32, delta_key_heads=16,
                          delta_head_dim=128, attn_heads=16, attn_kv_heads=4, attn_head_dim=256)
    d, ff, ld, ad = 2560, 9216, 128, 256
    cw = 2 * 16 * ld + 32 * ld
    rng = np.random.default_rng(5)
    delta = {"linear_attn.in_proj_qkv.weight": (cw, d), "linear_attn.in_proj_z.weight": (32 * ld, d),
             "linear_attn.in_proj_a.weight": (32, d), "linear_attn.in_proj_b.weight": (32, d),
             "linear_attn.out_proj.weight": (d, 32 * ld)}
    attn = {"self_attn.q_proj.weight": (2 * 16 * ad, d), "self_attn.k_proj.weight": (4 * ad, d),
            "self_attn.v_proj.weight": (4 * ad, d), "self_attn.o_proj.weight": (d, 16 * ad)}
    mlp = {"mlp.gate_proj.weight": (ff, d), "mlp.up_proj.weight": (ff, d), "mlp.down_proj.weight": (d, ff)}
    wires = {name: (random_wire(rng, r, c), r, c) for name, (r, c) in {**delta, **attn, **mlp}.items()}
    vec = lambda size, scale, base=0.0: (base + rng.standard_normal(size) * scale).astype(np.float32)
    vectors = {"linear_attn.conv1d.weight": vec(cw * 4, 0.4), "linear_attn.A_log": np.log(
        rng.uniform(1.0, 16.0, 32)).astype(np.float32), "linear_attn.dt_bias": vec(32, 0.5),
        "linear_attn.norm.weight": vec(ld, 0.1, 1.0), "self_attn.q_norm.weight": vec(ad, 0.1),
        "self_attn.k_norm.weight": vec(ad, 0.1)}
    norms = {"input_layernorm.weight": vec(d, 0.1), "post_attention_layernorm.weight": vec(d, 0.1)}
    p = ctx.pplx_create(cfg)
    for i in range(layers):
        names = attn if i % 4 == 3 else delta
        for name in list(names) + list(mlp):
            wire, r, c = wires[name]
            p.set_weight(f"language_model.layers.{i}.{name}", wire, rocm.Q4_G64_F32, r, c)
        mixer = "self_attn." if i % 4 == 3 else "linear_attn."
        for name, values in {**vectors, **norms}.items():
            if name in norms or name.startswith(mixer):
                p.set_vector(f"language_model.layers.{i}.{name}", values)
    p.set_vector("language_model.norm.weight", vec(d, 0.1))
    p.set_weight("readout", random_wire(rng, 255, d, 0.05), rocm.Q4_G64_F32, 255, d)
    del wires
    rows = random_wire(rng, n, d, 1.0).reshape(n, -1)
    markers = [n - 1, n // 2, n // 3, 0]
    logits = p.forward_rows(rows, n, markers)
    assert np.isfinite(logits).all()
    warm(torch, lambda r: p.forward_rows(rows, n, markers))
    # three rounds of five forwards; the median round is reported (one round on a
    # box that has just run other work can read several percent slow)
    reps, rounds = 5, 3
    wall = time.perf_counter()
    round_ms = [timed_ms(torch, stream, lambda r: p.forward_rows(rows, n, markers), reps) for _ in range(rounds)]
    wall = (time.perf_counter() - wall) * 1e3 / (reps * rounds)
    ms = sorted(round_ms)[rounds // 2]
    # the same model with its layer projections streamed from pinned host memory
    # through two device banks (webgpu/streaming.rs): same kernels, same bits
    p.set_residency(rocm.PPLX_STREAMED)
    info = p.residency_info()
    if not np.array_equal(p.forward_rows(rows, n, markers).view(np.uint32), logits.view(np.uint32)):
        raise AssertionError("streamed decider logits differ from the resident ones")
    warm(torch, lambda r: p.forward_rows(rows, n, markers))
    s_ms = timed_ms(torch, stream, lambda r: p.forward_rows(rows, n, markers), 3)
    streamed = {"ms": round(s_ms, 3), "sequences/s": round(1e3 / s_ms, 2),
                "device_layer_weight_bytes": info["device_layer_weight_bytes"],
                "resident_layer_weight_bytes": info["layer_weight_bytes"],
                "host_to_device_GB/s": round(info["host_layer_weight_bytes"] / (s_ms * 1e-3) / 1e9, 1),
                "note": "every layer's projections copied host-to-device once per forward, one layer ahead of "
                        "the compute; logits bitwise equal to the resident forward"}
    p.close()
    prods = 24 * 2 * n * (d * (cw + 32 * ld + 64) + 32 * ld * d) + 8 * 2 * n * (d * (2 * 16 * ad + 8 * ad) + 16 * ad * d)
    prods += layers * 2 * n * 3 * d * ff
    return {"ms": round(ms, 3), "ms_rounds": [round(x, 3) for x in round_ms], "wall_ms": round(wall, 3),
            "sequences/s": round(1e3 / ms, 2),
            "tokens/s": round(n * 1e3 / ms, 1), "product_TOP/s": round(prods / (ms * 1e-3) / 1e12, 1),
            "streamed_weights": streamed,
            "note": f"{layers} layers (24 gated-delta, 8 gated-attention), hidden 2560, one chunk of {n} tokens, "
                    "4 markers; W4A8 products bit-exact with the CPU path; random Q4 g64 wire weights; "
                    "host rows in and logits out inside the timed region"}


TUNE_SHAPES = {"grouped": (256, 8192, 2560), "mlp": (128, 9216, 2560), "gemv": (1, 8192, 2560),
               "gemm_w4a16": (256, 8192, 2560), "i8_gemm": (256, 8192, 2560)}
TUNE_REFERENCE = {"grouped": "pipe-auto", "mlp": "pipe-auto", "gemv": "auto", "gemm_w4a16": "pipe-auto",
                  "i8_gemm": "256x256p2w8"}


def tune_line(torch, ctx, rocm, stream, budget_ms: int, cache_in: str | None, cache_out: str | None,
              reps: int = 30) -> dict:
    """dz_tune (or a cached selection re-checked for equality), then each
    family's reference variant and its selected variant at the tuning shape
    on real-valued inputs, `reps` launches each, timed by HIP events: the
    dispatches a rocprofv3 run attributes to each variant's kernel."""
    cache = Path(cache_in).read_text() if cache_in else None
    sel = ctx.tune(budget_ms, cache)
    if cache_out:
        Path(cache_out).write_text(json.dumps(sel))
    gen = lambda seed: torch.Generator(device="cuda").manual_seed(seed)  # noqa: E731
    out = {}
    for fam, (m, n, k) in TUNE_SHAPES.items():
        wf = torch.randn((n, k), generator=gen(1), device="cuda") * 0.02
        torch.cuda.synchronize()
        if fam in ("grouped", "mlp"):
            w = ctx.quantize(wf, rocm.F32, n, k, 4, 64)
            w2 = ctx.quantize(wf.flip(0).contiguous(), rocm.F32, n, k, 4, 64)
            x = torch.randn((m, k), generator=gen(0), device="cuda")
            q = torch.empty((m, k), dtype=torch.int8, device="cuda")
            sx = torch.empty((m, k // 64), device="cuda")
            ctx.act_quantize(x, m, k, 8, q, sx)
            if fam == "grouped":
                y = torch.empty((m, n), device="cuda")
                fn = lambda r: ctx.linear_q8(w, q, sx, m, y)  # noqa: E731
            else:
                qo = torch.empty((m, n), dtype=torch.int8, device="cuda")
                so = torch.empty((m, n // 64), device="cuda")
                fn = lambda r: ctx.mlp_requant(w, w2, x, m, qo, so)  # noqa: E731
        elif fam in ("gemv", "gemm_w4a16"):
            w = ctx.quantize(wf, rocm.F32, n, k, 4, 32)
            w2 = None
            x = torch.randn((m, k), generator=gen(0), device="cuda").half()
            y = torch.empty((m, n), device="cuda")
            fn = lambda r: ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)  # noqa: E731
        else:
            w = w2 = None
            a = torch.empty((m, k), dtype=torch.int8, device="cuda")
            b = torch.empty((n, k), dtype=torch.int8, device="cuda")
            sa, sb = torch.empty(m, device="cuda"), torch.empty(n, device="cuda")
            ctx.i8_quantize_rows(torch.randn((m, k), generator=gen(0), device="cuda"), m, k, a, sa)
            ctx.i8_quantize_rows(wf, n, k, b, sb)
            y = torch.empty((m, n), device="cuda")
            fn = lambda r: ctx.i8_gemm(a, sa, m, b, sb, n, k, y, raw=False)  # noqa: E731
        line = {"shape": [m, n, k]}
        for role, name in (("reference", TUNE_REFERENCE[fam]), ("selected", sel["selected"][fam])):
            ctx.select_variant(fam, name)
            warm(torch, fn, ms=20.0)
            line[role] = {"variant": name, "us": round(timed_ms(torch, stream, fn, reps) * 1e3, 3)}
        ctx.select_variant(fam, sel["selected"][fam])
        out[fam] = line
        for t in (w, w2):
            if t is not None:
                t.free()
    return {"tuning": sel, "variants": out}


def traffic_per_launch():
    """HBM bytes per GEMV launch from the committed rocprofv3 counter summary."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
        return int(data["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def floors_line(torch, ctx, rocm, stream) -> dict:
    """What a launch of the headline GEMV's size costs with no product in it,
    over the same rotation of 96 copies as the headline, each a HIP graph of
    one launch per copy: a one-element fill (the launch floor in a graph), a
    device copy moving the GEMV's byte count (half read, half written), the
    vendor library's f16 GEMV over an f16 matrix of the GEMV's byte count
    (1155 x 4096, torch.mv) and the GEMV itself."""
    per_launch = gemv_bytes(M_ROWS, K_DIM, N_DIM)
    bufs = [torch.empty(per_launch // 4, dtype=torch.float32, device="cuda").uniform_() for _ in range(WEIGHT_COPIES)]
    halves = [torch.empty(per_launch // 8, dtype=torch.float32, device="cuda") for _ in range(WEIGHT_COPIES)]
    tiny = torch.zeros(1, dtype=torch.float32, device="cuda")
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

    def fills():
        for c in range(WEIGHT_COPIES):
            tiny.fill_(float(c + 1))

    def copies():
        for c in range(WEIGHT_COPIES):
            halves[c].copy_(bufs[c][:per_launch // 8])

    def gemvs():
        for c in range(WEIGHT_COPIES):
            ctx.linear(weights[c], x, rocm.F16, M_ROWS, y[c], rocm.W4A16)

    # f16 matrices of the same byte count for the vendor GEMV
    vrows = per_launch // (2 * K_DIM)
    assert vrows * 2 * K_DIM == per_launch
    mats = [torch.randn((vrows, K_DIM), generator=torch.Generator(device="cuda").manual_seed(200 + c), device="cuda",
                        dtype=torch.float16) * 0.02 for c in range(WEIGHT_COPIES)]
    xv = x[0].contiguous()
    yv = torch.empty((WEIGHT_COPIES, vrows), dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()

    def vendor():
        for c in range(WEIGHT_COPIES):
            torch.mv(mats[c], xv, out=yv[c])

    out = {}
    for name, fn in (("fill_1_element", fills), ("copy_same_bytes", copies), ("vendor_f16_gemv_same_bytes", vendor),
                     ("gemv_w4a16", gemvs)):
        us = graph_ms(torch, stream, fn, WEIGHT_COPIES, reps=200) * 1e3
        out[name] = {"us_per_launch": round(us, 3), "launch": "hip graph"}
        if name != "fill_1_element":
            out[name]["GB/s"] = round(per_launch / (us * 1e-6) / 1e9, 1)
    assert torch.isfinite(y).all()
    for wgt in weights:
        wgt.free()
    del mats
    out["vendor_f16_gemv_same_bytes"]["what"] = f"torch.mv, f16 [{vrows} x {K_DIM}] matrix times an f16 vector"
    out["bytes_per_launch"] = per_launch
    del bufs, halves, y
    torch.cuda.empty_cache()
    # the HBM rates plain framework kernels reach where a launch's fixed cost is
    # negligible: a 1 GiB device copy (read + write) and a 1 GiB f32 sum (read)
    big = torch.empty(1 << 28, dtype=torch.float32, device="cuda").normal_()
    dst = torch.empty_like(big)
    torch.cuda.synchronize()
    warm(torch, lambda r: dst.copy_(big))
    ms = timed_ms(torch, torch.cuda.current_stream(), lambda r: dst.copy_(big), 10)
    out["copy_1GiB"] = {"TB/s_read_plus_write": round((2 << 30) / (ms * 1e-3) / 1e12, 3), "what": "torch copy_"}
    warm(torch, lambda r: big.sum())
    ms = timed_ms(torch, torch.cuda.current_stream(), lambda r: big.sum(), 10)
    out["sum_1GiB"] = {"TB/s_read": round((1 << 30) / (ms * 1e-3) / 1e12, 3), "what": "torch sum over f32"}
    del big, dst
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=150)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true", help="plain launches (for counter collection)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help=f"also run a {COPY_BYTES >> 20} MiB device copy (counter calibration)")
    ap.add_argument("--tune", type=int, default=0, help="tuner budget in ms (0 keeps reference variants)")
    ap.add_argument("--only", choices=["pplx", "tune", "floors", "encoder", "gemv", "int8"],
                    help="run one secondary line alone and print it (for profiling)")
    ap.add_argument("--tune-cache", help="with --only tune: a selection JSON from an earlier run to reuse")
    ap.add_argument("--tune-out", help="with --only tune: write the selection JSON here")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the hot path would shard along N, with one all-gather of the outputs)", file=sys.stderr)
        sys.exit(2)

    import torch
    from decisive_amd import rocm

    ctx = rocm.Context(0)
    if args.only == "tune":
        stream = torch.cuda.Stream()
        ctx.set_stream(stream.cuda_stream)
        with torch.cuda.stream(stream):
            line = tune_line(torch, ctx, rocm, stream, args.tune or 2000, args.tune_cache, args.tune_out)
        ctx.set_stream(None)
        print(json.dumps(line), flush=True)
        return
    if args.tune:
        ctx.tune(args.tune)
    log(f"[bench] device {ctx.info()}")
    if args.only == "gemv":
        stream = torch.cuda.Stream()
        ctx.set_stream(stream.cuda_stream)
        with torch.cuda.stream(stream):
            line = wide_gemv_lines(torch, ctx, rocm, stream)
        ctx.set_stream(None)
        print(json.dumps({"wide_gemv": line}), flush=True)
        return
    if args.only == "floors":
        stream = torch.cuda.Stream()
        ctx.set_stream(stream.cuda_stream)
        with torch.cuda.stream(stream):
            line = floors_line(torch, ctx, rocm, stream)
        ctx.set_stream(None)
        print(json.dumps({"launch_floors_q4_gemv_size": line}), flush=True)
        return
    if args.only == "int8":
        stream = torch.cuda.Stream()
        ctx.set_stream(stream.cuda_stream)
        with torch.cuda.stream(stream):
            line = int8_line(torch, ctx, stream)
        ctx.set_stream(None)
        print(json.dumps({"int8_gemm_m8192_k4096_n4096": line}), flush=True)
        return
    if args.only in ("pplx", "encoder"):
        stream = torch.cuda.Stream()
        ctx.set_stream(stream.cuda_stream)
        with torch.cuda.stream(stream):
            if args.only == "pplx":
                line = {"pplx_decider_forward_s1024": pplx_line(torch, ctx, rocm, stream)}
            else:
                line = {"encoder_forward_b8_s1024": encoder_line(torch, ctx, rocm, stream)}
        ctx.set_stream(None)
        print(json.dumps(line), flush=True)
        return

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
            with rocm.capture(graph, side):
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
            sec.update(wide_gemv_lines(torch, ctx, rocm, stream))
            sec["q4_gemv_w4a8_m1_k4096_n4096_g64f32"] = w4a8_line(torch, ctx, rocm, stream)
            sec.update(secondary(torch, ctx, rocm, stream, cpu=not args.no_cpu))
        result["secondary"] = sec
    ctx.set_stream(None)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
