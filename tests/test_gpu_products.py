"""GPU parity of the quantized products.

W4A8/W8A8/W4A4 and the per-row int8 GEMM are integer work folded in a fixed
float order: bit-exact against the oracle. W4A16 has no reference kernel: it is
checked against the float64 closed form with the north-star tolerance
(max-abs <= 1e-2, cosine >= 0.9999)."""
import json
from pathlib import Path

import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, cosine, dev, empty, host

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
MAX_ABS = 1e-2  # north_star tolerance for f16/f32 GEMM outputs
MIN_COS = 0.9999


# ---- grouped W{4,8}A{8,4} ------------------------------------------------------------

@pytest.mark.parametrize("wb,ab", GOLDEN["grouped_dot_shapes"]["bits"])
def test_grouped_matches_avx2_order_bit_exact(ctx, oracle, wb, ab):
    """int8.rs:678-772 shapes and generators: GPU == oracle fused (AVX2) order."""
    torch = pytest.importorskip("torch")
    for m, k, n in GOLDEN["grouped_dot_shapes"]["mkn"]:
        i = np.arange(k * n)
        raw = oracle.f32_to_bf16(((i * 37 % 257) - 128.0) / 31.0)
        x = (((np.arange(m * k) * 13 % 255) - 127.0) / 17.0).astype(np.float32)
        w = ctx.quantize(dev(raw), rocm.BF16, n, k, wb, 64)
        y = empty((max(m, 1), n), torch.float32)
        ctx.linear(w, dev(x) if m else 0, rocm.F32, m, y if m else 0, rocm.W4A4 if ab == 4 else rocm.W4A8)
        if m == 0:
            continue
        codes, scales = oracle.weight_quantize(raw, n, k, wb)
        want = oracle.matrix_apply(x, m, codes, scales, n, k, ab, fused=True)
        got = host(ctx, y)[:m]
        assert bits_equal(got, want), (m, k, n, float(np.abs(got - want).max()))


@pytest.mark.parametrize("wb,ab", [(4, 8), (8, 8), (4, 4), (8, 4)])
@pytest.mark.parametrize("m,k,n", [(300, 4096, 520), (257, 1088, 200), (513, 64, 129), (40, 640, 1040)])
def test_grouped_large_m_pipeline_bit_exact(ctx, oracle, wb, ab, m, k, n):
    """M > 16 runs the pipelined grouped kernel: bit for bit the AVX2 fold
    order of int8.rs:524-585 and the one-wave-per-tile kernel (ragged rows and
    columns, an odd group count, a single group)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(m + k + n + wb + ab)
    raw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    x = (rng.standard_normal((m, k)) * 1.5).astype(np.float32)
    w = ctx.quantize(dev(raw), rocm.BF16, n, k, wb, 64)
    mode = rocm.W4A4 if ab == 4 else rocm.W4A8
    outs = []
    names = ("pipe256x128w8", "wave16x16", "pipe128x128w4", "pipe64x128w2", "pipe128x128m8", "pipe128x128n8",
             "pipe32x128w8", "pipe64x128w8", "pipe32x128w8g4", "pipe64x128w8g4", "fewrow16", "pipe32x64w4", "pipe64x64w8", "pipe-auto")
    for name in names:
        ctx.select_variant("grouped", name)
        y = empty((m, n), torch.float32)
        ctx.linear(w, dev(x), rocm.F32, m, y, mode)
        outs.append(host(ctx, y))
    ctx.select_variant("grouped", "pipe-auto")
    codes, scales = oracle.weight_quantize(raw, n, k, wb)
    want = oracle.matrix_apply(x, m, codes, scales, n, k, ab, fused=True)
    assert bits_equal(outs[0], want), float(np.abs(outs[0] - want).max())
    for name, o in zip(names[1:], outs[1:]):
        assert bits_equal(o, outs[0]), name


def test_grouped_large_m_nonfinite_activation_makes_every_output_nan(ctx, oracle):
    """int8.rs:170-173 at M > 16: one non-finite activation -> every output NaN."""
    torch = pytest.importorskip("torch")
    raw = oracle.f32_to_bf16(np.full((48, 256), 0.01, np.float32))
    w = ctx.quantize(dev(raw), rocm.BF16, 48, 256, 4, 64)
    x = np.ones((40, 256), np.float32)
    x[33, 5] = np.inf
    y = empty((40, 48), torch.float32)
    ctx.linear(w, dev(x), rocm.F32, 40, y, rocm.W4A8)
    assert np.isnan(host(ctx, y)).all()


@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("bits", [4, 8])
def test_kernel_check_cases_vs_project(ctx, oracle, case, bits):
    """webgpu/grouped_q4.rs:215-311 cases through the wire layout: bit-exact with
    the AVX2 order and within 1e-4 + 2e-6*|a||b| of packed::project."""
    torch = pytest.importorskip("torch")
    m, n, k = GOLDEN["kernel_check_shapes"]["mnk"][case]
    i = np.arange(m * k)
    if case == 4:
        a = np.where((i // k) % 2 == 0, 127.0, -127.0)
    elif case == 3:
        a = ((i * 73 % 1021) - 510.0) / 113.0
    else:
        a = ((i * 17 % 255) - 127.0) * np.where(i % k < 64, 0.125, 4.0)
    a = a.astype(np.float32)
    j = np.arange(n * k)
    if case == 4:
        b = np.where(((j // k) + (j % k) // 64) % 3 == 0, -7.0, 7.0)
    elif case == 3:
        b = ((j * 47 % 257) - 128.0) / 193.0
    else:
        b = ((j * 11 % 15) - 7.0) * np.where(j % k < 64, 0.25, 8.0)
    b = b.astype(np.float32)
    raw = (b.view(np.uint32) >> 16).astype(np.uint16)  # truncating BF16, grouped_q4.rs:247-250
    packed = oracle.pack_g64(raw, n, k, bits)
    w = ctx.upload(packed, rocm.Q4_G64_F32 if bits == 4 else rocm.Q8_G64_F32, n, k)
    y = empty((m, n), torch.float32)
    ctx.linear(w, dev(a), rocm.F32, m, y, rocm.W4A8)
    got = host(ctx, y)
    codes, scales = oracle.weight_quantize(raw, n, k, bits)
    assert bits_equal(got, oracle.matrix_apply(a, m, codes, scales, n, k, 8, fused=True))
    packed_abs = oracle.pack_g64((np.abs(b).view(np.uint32) >> 16).astype(np.uint16), n, k, bits)
    for r in range(m):
        want = oracle.project(packed, bits, k, a[r * k:(r + 1) * k], n)
        mag = oracle.project(packed_abs, bits, k, np.abs(a[r * k:(r + 1) * k]), n)
        assert np.all(np.abs(got[r] - want) <= 1e-4 + mag * 2e-6)


def test_config1_q4_linear_bit_exact(ctx, oracle):
    """x N(0,1) [128 x 1024] seed 0, W N(0,0.02) [1024 x 1024]
    seed 1, through the reference's g64 quantizer (BF16 input)."""
    torch = pytest.importorskip("torch")
    m = k = n = 1024
    m = 128
    x = np.random.default_rng(0).standard_normal((m, k)).astype(np.float32)
    wf = (np.random.default_rng(1).standard_normal((n, k)) * 0.02).astype(np.float32)
    raw = oracle.f32_to_bf16(wf)
    packed = oracle.pack_g64(raw, n, k, 4)
    w = ctx.upload(packed, rocm.Q4_G64_F32, n, k)
    y = empty((m, n), torch.float32)
    ctx.linear(w, dev(x), rocm.F32, m, y, rocm.W4A8)
    codes, scales = oracle.weight_quantize(raw, n, k, 4)
    want = oracle.matrix_apply(x, m, codes, scales, n, k, 8, fused=True)
    assert bits_equal(host(ctx, y), want)
    # the g32/f16 twin in W4A16 against the float64 closed form
    packed32 = oracle.pack_g32_f16(wf, n, k)
    w32 = ctx.upload(packed32, rocm.Q4_G32_F16, n, k)
    xh = oracle.f32_to_f16_bits(x)
    ctx.linear(w32, dev(xh.view(np.float16)), rocm.F16, m, y, rocm.W4A16)
    closed = oracle.w4a16(xh, m, k, oracle.unpack_g32_f16(packed32).reshape(n, k), n)
    got = host(ctx, y)
    assert np.abs(got - closed).max() <= MAX_ABS and cosine(got, closed) >= MIN_COS


def test_nonfinite_activation_makes_every_output_nan(ctx, oracle):
    """int8.rs:170-173 and :952-962."""
    torch = pytest.importorskip("torch")
    raw = oracle.f32_to_bf16(np.ones((9, 70), np.float32))
    w = ctx.quantize(dev(raw), rocm.BF16, 9, 70, 4, 64)
    x = np.zeros((3, 70), np.float32)
    x[2, 69] = np.inf
    y = empty((3, 9), torch.float32)
    ctx.linear(w, dev(x), rocm.F32, 3, y, rocm.W4A8)
    assert np.isnan(host(ctx, y)).all()
    x[2, 69] = 0.0
    ctx.linear(w, dev(x), rocm.F32, 3, y, rocm.W4A8)
    assert (host(ctx, y) == 0).all()


def test_pair_shares_one_quantization(ctx, oracle):
    """int8.rs:204-227 apply_pair == two applies (and thread-count invariance
    becomes launch invariance: repeated calls are bitwise identical)."""
    torch = pytest.importorskip("torch")
    m, k, n = 33, 320, 96
    rng = np.random.default_rng(11)
    a = ctx.quantize(dev(rng.standard_normal((n, k)).astype(np.float32)), rocm.F32, n, k, 4, 64)
    b = ctx.quantize(dev(rng.standard_normal((n, k)).astype(np.float32)), rocm.F32, n, k, 4, 64)
    x = dev(rng.standard_normal((m, k)).astype(np.float32))
    ya, yb, y1, y2 = (empty((m, n), torch.float32) for _ in range(4))
    ctx.linear_pair(a, b, x, m, ya, yb)
    ctx.linear(a, x, rocm.F32, m, y1, rocm.W4A8)
    ctx.linear(b, x, rocm.F32, m, y2, rocm.W4A8)
    assert bits_equal(host(ctx, ya), host(ctx, y1)) and bits_equal(host(ctx, yb), host(ctx, y2))


def test_fused_mlp_large_m_pipeline_equals_unfused(ctx, oracle):
    """Every fused MLP variant (256- and 128-row pipelined blocks, one-wave
    blocks; ragged m, an odd group count) is word-exact with the unfused
    composition."""
    torch = pytest.importorskip("torch")
    m, n, k = 600, 2752, 1088
    rng = np.random.default_rng(11)
    graw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.03).astype(np.float32))
    uraw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.03).astype(np.float32))
    gate = ctx.quantize(dev(graw), rocm.BF16, n, k, 4, 64)
    up = ctx.quantize(dev(uraw), rocm.BF16, n, k, 4, 64)
    x = (rng.standard_normal((m, k)) * 1.3).astype(np.float32)
    xd = dev(x)
    g = empty((m, n), torch.float32)
    u = empty((m, n), torch.float32)
    ctx.linear_pair(gate, up, xd, m, g, u)
    ctx.silu_mul(g, u, m * n)
    q2 = empty((m, n), torch.int8)
    s2 = empty((m, n // 64), torch.float32)
    ctx.act_quantize(g, m, n, 8, q2, s2)
    q = empty((m, n), torch.int8)
    s = empty((m, n // 64), torch.float32)
    for name in ("pipe256x64w8", "pipe128x64w4", "wave16x64", "pipe256x64n2", "pipe128x64n2", "pipe-auto"):
        ctx.select_variant("mlp", name)
        q.zero_()
        torch.cuda.synchronize()  # the fill runs on torch's stream, the product on the context's
        ctx.mlp_requant(gate, up, xd, m, q, s)
        assert np.array_equal(host(ctx, q), host(ctx, q2)), name
        assert bits_equal(host(ctx, s), host(ctx, s2)), name
    # a non-finite activation: every scale NaN, every code 0 (int8.rs:170-173)
    x[599, 7] = np.nan
    ctx.mlp_requant(gate, up, dev(x), m, q, s)
    assert np.isnan(host(ctx, s)).all() and not host(ctx, q).any()


def test_product_flags_do_not_leak_across_calls(ctx, oracle):
    """Each asynchronous W4A8 product has its own non-finite flag: over 140
    calls (past two wraps of the flag ring) only the calls given a NaN
    activation produce NaN, every other call equals a clean call bit for bit."""
    torch = pytest.importorskip("torch")
    m, n, k = 40, 128, 256
    rng = np.random.default_rng(21)
    w = ctx.quantize(dev((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), rocm.F32, n, k, 4, 64)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bad = x.copy()
    bad[3, 7] = np.nan
    xd, bd = dev(x), dev(bad)
    want = empty((m, n), torch.float32)
    ctx.linear(w, xd, rocm.F32, m, want, rocm.W4A8)
    want = host(ctx, want)
    ys = [empty((m, n), torch.float32) for _ in range(140)]
    nan_calls = {5, 100}
    for i, y in enumerate(ys):
        ctx.linear(w, bd if i in nan_calls else xd, rocm.F32, m, y, rocm.W4A8)
    for i, y in enumerate(ys):
        got = host(ctx, y)
        if i in nan_calls:
            assert np.isnan(got).any(), i
        else:
            assert bits_equal(got, want), i
    w.free()


def test_fused_mlp_requant_equals_unfused(ctx, oracle):
    """grouped_q4.rs:313-354: fused gate/up/SiLU/requant == unfused, word-exact;
    both against the oracle composition within one code."""
    torch = pytest.importorskip("torch")
    m, n, k = GOLDEN["fused_mlp_check"]["mnk"]

    def weight(seed):
        v = (((np.arange(n * k) * seed % 251) - 125.0) / 400.0).astype(np.float32)
        return (v.view(np.uint32) >> 16).astype(np.uint16)

    graw, uraw = weight(37), weight(53)
    gate = ctx.upload(oracle.pack_g64(graw, n, k, 4), rocm.Q4_G64_F32, n, k)
    up = ctx.upload(oracle.pack_g64(uraw, n, k, 4), rocm.Q4_G64_F32, n, k)
    x = (((np.arange(m * k) * 29 % 509) - 254.0) / 97.0).astype(np.float32)
    xd = dev(x)
    g = empty((m, n), torch.float32)
    u = empty((m, n), torch.float32)
    ctx.linear_pair(gate, up, xd, m, g, u)
    ctx.silu_mul(g, u, m * n)
    q2 = empty((m, n), torch.int8)
    s2 = empty((m, n // 64), torch.float32)
    ctx.act_quantize(g, m, n, 8, q2, s2)
    q = empty((m, n), torch.int8)
    s = empty((m, n // 64), torch.float32)
    for name in ("pipe256x64w8", "pipe128x64w4", "wave16x64", "pipe256x64n2", "pipe128x64n2", "pipe-auto"):
        ctx.select_variant("mlp", name)
        q.zero_()
        torch.cuda.synchronize()  # the fill runs on torch's stream, the product on the context's
        ctx.mlp_requant(gate, up, xd, m, q, s)
        assert np.array_equal(host(ctx, q), host(ctx, q2)), name
        assert bits_equal(host(ctx, s), host(ctx, s2)), name
    # oracle composition (its expf may differ from the GPU's by an ulp)
    gc, gs = oracle.weight_quantize(graw, n, k, 4)
    uc, us = oracle.weight_quantize(uraw, n, k, 4)
    go = oracle.matrix_apply(x, m, gc, gs, n, k, 8, fused=True)
    uo = oracle.matrix_apply(x, m, uc, us, n, k, 8, fused=True)
    oq, os_ = oracle.silu_requant(go, uo)
    assert np.abs(host(ctx, q).astype(np.int32) - oq.astype(np.int32)).max() <= 1
    assert np.allclose(host(ctx, s), os_, rtol=1e-5)
    # down_proj consumer of the A8 records equals the oracle's grouped product
    draw = oracle.f32_to_bf16(np.random.default_rng(3).standard_normal((64, n)).astype(np.float32))
    down = ctx.quantize(dev(draw), rocm.BF16, 64, n, 4, 64)
    yd = empty((m, 64), torch.float32)
    ctx.linear_q8(down, q, s, m, yd)
    dq, dsc = oracle.weight_quantize(draw, 64, n, 4)
    want = oracle.grouped_gemm(host(ctx, q), host(ctx, s), m, dq, dsc, 64, n, fused=True)
    assert bits_equal(host(ctx, yd), want)


# ---- W4A16 ---------------------------------------------------------------------------

@pytest.mark.parametrize("m", [1, 4, 8])
def test_config2_gemv_vs_closed_form(ctx, oracle, m):
    """f16 x N(0,1) seed 0, K = N = 4096, W N(0,0.02) seed 1, g32/f16."""
    torch = pytest.importorskip("torch")
    k = n = 4096
    x = np.random.default_rng(0).standard_normal((m, k)).astype(np.float32)
    wf = (np.random.default_rng(1).standard_normal((n, k)) * 0.02).astype(np.float32)
    packed = oracle.pack_g32_f16(wf, n, k)
    w = ctx.upload(packed, rocm.Q4_G32_F16, n, k)
    xh = oracle.f32_to_f16_bits(x)
    y = empty((m, n), torch.float32)
    ctx.linear(w, dev(xh.view(np.float16)), rocm.F16, m, y, rocm.W4A16)
    got = host(ctx, y)
    want = oracle.w4a16(xh, m, k, oracle.unpack_g32_f16(packed).reshape(n, k), n)
    assert np.abs(got - want).max() <= MAX_ABS
    assert cosine(got, want) >= MIN_COS
    # every GEMV variant keeps the reduction order: bitwise equal outputs
    for name in ("auto", "w16", "w8", "stream8", "stream4", "persist"):
        ctx.select_variant("gemv", name)
        y2 = empty((m, n), torch.float32)
        ctx.linear(w, dev(xh.view(np.float16)), rocm.F16, m, y2, rocm.W4A16)
        assert bits_equal(host(ctx, y2), got), name
    ctx.select_variant("gemv", "auto")


@pytest.mark.parametrize("k,n", [(96, 17), (2560, 300), (4160, 33), (8, 1)])
def test_gemv_ragged_rows_are_independent_of_m(ctx, oracle, k, n):
    """Skinny path for every row count 1..16: closed form within tolerance, and
    each output row bitwise equal to the same row computed alone (a row's
    arithmetic does not depend on how many rows share the launch)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(k * 31 + n)
    x = rng.standard_normal((16, k)).astype(np.float32)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w = ctx.quantize(dev(wf), rocm.F32, n, k, 4, 32)
    deq = empty((n, k), torch.float32)
    ctx.dequant(w, deq)
    deq = host(ctx, deq)
    xh = oracle.f32_to_f16_bits(x)
    xd = dev(xh.view(np.float16))
    want = oracle.w4a16(xh, 16, k, deq, n)
    alone = []
    for r in range(16):
        y1 = empty((1, n), torch.float32)
        ctx.linear(w, xd[r:r + 1], rocm.F16, 1, y1, rocm.W4A16)
        alone.append(host(ctx, y1)[0])
    alone = np.stack(alone)
    assert np.abs(alone - want).max() <= MAX_ABS
    for m in (2, 3, 5, 8, 9, 16):
        y = empty((m, n), torch.float32)
        ctx.linear(w, xd, rocm.F16, m, y, rocm.W4A16)
        got = host(ctx, y)
        assert bits_equal(got, alone[:m]), m


@pytest.mark.parametrize("k,n", [(2048, 1000), (6144, 4099), (4160, 300)])
def test_gemv_stream_variants_equal_the_split_kernel(ctx, oracle, k, n):
    """The streaming GEMV (one wave per 16-row tile, K a multiple of 2048) keeps
    the split kernel's chunk order: for every row count 1..8 and ragged N its
    outputs equal the default kernel's bit for bit and the closed form within
    tolerance. At K = 4160 it does not apply and the split kernel runs."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(k + n)
    x = rng.standard_normal((8, k)).astype(np.float32)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w = ctx.quantize(dev(wf), rocm.F32, n, k, 4, 32)
    deq = empty((n, k), torch.float32)
    ctx.dequant(w, deq)
    deq = host(ctx, deq)
    xh = oracle.f32_to_f16_bits(x)
    xd = dev(xh.view(np.float16))
    want = oracle.w4a16(xh, 8, k, deq, n)
    try:
        for m in range(1, 9):
            ctx.select_variant("gemv", "w16")
            y = empty((m, n), torch.float32)
            ctx.linear(w, xd, rocm.F16, m, y, rocm.W4A16)
            base = host(ctx, y).copy()
            assert np.abs(base - want[:m]).max() <= MAX_ABS
            for name in ("stream8", "stream4", "auto"):
                ctx.select_variant("gemv", name)
                y.fill_(7.0)
                torch.cuda.synchronize()  # the fill runs on torch's stream, the product on the context's
                ctx.linear(w, xd, rocm.F16, m, y, rocm.W4A16)
                assert bits_equal(host(ctx, y), base), (name, m)
    finally:
        ctx.select_variant("gemv", "auto")
    w.free()


@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("k,n", [(4096, 8197), (2560, 8200), (1024, 300), (96, 33), (4160, 700)])
def test_gemv_persistent_equals_the_split_kernel(ctx, oracle, group, k, n):
    """The persistent GEMV (K <= 4096: a block walks tiles b, b + grid, ...,
    the next tile's loads in flight through the chunk reduction) keeps the split
    kernel's chunk order: for every row count 1..8, ragged N, chunks past K
    (K = 1024 and 96) and both scale layouts its outputs equal the split
    kernel's bit for bit and the closed form within tolerance. N = 8197 and 8200
    give most blocks several tiles; at K = 4160 it does not apply and the split
    kernel runs."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(k + n + group)
    x = rng.standard_normal((8, k)).astype(np.float32)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w = ctx.quantize(dev(wf), rocm.F32, n, k, 4, group)
    deq = empty((n, k), torch.float32)
    ctx.dequant(w, deq)
    deq = host(ctx, deq)
    xh = oracle.f32_to_f16_bits(x)
    xd = dev(xh.view(np.float16))
    want = oracle.w4a16(xh, 8, k, deq, n)
    try:
        for m in range(1, 9):
            ctx.select_variant("gemv", "w16")
            y = empty((m, n), torch.float32)
            ctx.linear(w, xd, rocm.F16, m, y, rocm.W4A16)
            base = host(ctx, y).copy()
            assert np.abs(base - want[:m]).max() <= MAX_ABS
            assert cosine(base, want[:m]) >= MIN_COS
            for name in ("persist", "auto"):
                ctx.select_variant("gemv", name)
                y.fill_(7.0)
                torch.cuda.synchronize()  # the fill runs on torch's stream, the product on the context's
                ctx.linear(w, xd, rocm.F16, m, y, rocm.W4A16)
                assert bits_equal(host(ctx, y), base), (name, m)
    finally:
        ctx.select_variant("gemv", "auto")
    w.free()


def test_w4a16_rejects_misaligned_activations(ctx, oracle):
    torch = pytest.importorskip("torch")
    k = n = 64
    w = ctx.quantize(dev(np.ones((n, k), np.float32) * 0.01), rocm.F32, n, k, 4, 32)
    buf = empty((2 * k + 8,), torch.float16)
    y = empty((1, n), torch.float32)
    with pytest.raises(rocm.DzError) as e:
        ctx.linear(w, buf.data_ptr() + 2, rocm.F16, 1, y, rocm.W4A16)
    assert e.value.code == "INVALID_PARAMETERS"


W4A16_VARIANTS = ("pipe-auto", "256x256p2w8", "128x128p2w4", "128x256p2w8", "256x128w2x2", "128x128w2x2",
                  "128x64w2x2", "256x256p2w8-persist", "256x192p2w8-persist", "256x128p2w8")


@pytest.mark.parametrize("layout", [rocm.Q4_G32_F16, rocm.Q4_G64_F32])
@pytest.mark.parametrize("m,k,n", [(3, 512, 80), (17, 256, 48), (256, 1024, 1024), (1000, 512, 1536), (33, 4096, 272),
                                   (300, 576, 200), (513, 192, 1040), (257, 4096, 257)])
def test_large_m_gemm_vs_closed_form(ctx, oracle, layout, m, k, n):
    """Every W4A16 GEMM variant against the float64 closed form, and all of
    them bitwise equal (ragged m and n, k tails inside a 128-k block)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(m + k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    if layout == rocm.Q4_G32_F16:
        packed = oracle.pack_g32_f16(wf, n, k)
        deq = oracle.unpack_g32_f16(packed).reshape(n, k)
    else:
        packed = oracle.pack_g64(oracle.f32_to_bf16(wf), n, k, 4)
        deq = oracle.unpack_g64(packed, 4).reshape(n, k)
    w = ctx.upload(packed, layout, n, k)
    xh = oracle.f32_to_f16_bits(x)
    want = oracle.w4a16(xh, m, k, deq, n)
    outs = []
    for name in W4A16_VARIANTS:
        ctx.select_variant("gemm_w4a16", name)
        y = empty((m, n), torch.float32)
        ctx.linear(w, dev(xh.view(np.float16)), rocm.F16, m, y, rocm.W4A16)
        got = host(ctx, y)
        assert np.abs(got - want).max() <= MAX_ABS, name
        assert cosine(got, want) >= MIN_COS, name
        outs.append(got)
    ctx.select_variant("gemm_w4a16", W4A16_VARIANTS[0])
    for name, o in zip(W4A16_VARIANTS[1:], outs[1:]):
        assert bits_equal(o, outs[0]), name


@pytest.mark.parametrize("epilogue", [rocm.EPI_NONE, rocm.EPI_GELU, rocm.EPI_RESIDUAL])
@pytest.mark.parametrize("m,k,n", [(3, 512, 80), (300, 576, 200), (1000, 1024, 1536), (257, 4096, 257)])
def test_w4a16_f16_output_is_the_f32_product_rounded_once(ctx, oracle, epilogue, m, k, n):
    """dz_linear_f16: the f32 product of dz_linear, then the epilogue in f32
    (GELU by dz_gelu, residual added in f32), rounded once to f16 -- bit for
    bit, on every GEMM variant."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(m + 3 * k + n + epilogue)
    xh = oracle.f32_to_f16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w = ctx.upload(oracle.pack_g32_f16(wf, n, k), rocm.Q4_G32_F16, n, k)
    res = rng.standard_normal((m, n)).astype(np.float16)
    x = dev(xh.view(np.float16))
    ctx.select_variant("gemm_w4a16", W4A16_VARIANTS[0])
    y32 = empty((m, n), torch.float32)
    ctx.linear(w, x, rocm.F16, m, y32, rocm.W4A16)
    if epilogue == rocm.EPI_GELU:
        ctx.gelu(y32, rocm.F32, m * n)
    want = host(ctx, y32)
    if epilogue == rocm.EPI_RESIDUAL:
        want = (want + res.astype(np.float32)).astype(np.float32)
    want = want.astype(np.float16)
    rd = dev(res)
    for name in W4A16_VARIANTS:
        ctx.select_variant("gemm_w4a16", name)
        y = empty((m, n), torch.float16)
        ctx.linear_f16(w, x, m, y, epilogue, rd if epilogue == rocm.EPI_RESIDUAL else None)
        got = host(ctx, y)
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), name
    ctx.select_variant("gemm_w4a16", W4A16_VARIANTS[0])


@pytest.mark.parametrize("epilogue", [None, rocm.EPI_NONE, rocm.EPI_GELU, rocm.EPI_RESIDUAL])
def test_persistent_gemm_walks_several_tiles_per_block(ctx, oracle, epilogue):
    """The persistent W4A16 kernel (one block per compute unit) on 18 x 16 =
    288 tiles of 256 x 256, so blocks take two tiles, with ragged last row and
    column tiles: bitwise equal to one block per tile, for the f32 output and
    every f16 epilogue; sampled rows against the float64 closed form."""
    torch = pytest.importorskip("torch")
    m, k, n = 4400, 256, 4000
    rng = np.random.default_rng(77 + (epilogue if epilogue is not None else 9))
    xh = oracle.f32_to_f16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed = oracle.pack_g32_f16(wf, n, k)
    w = ctx.upload(packed, rocm.Q4_G32_F16, n, k)
    x = dev(xh.view(np.float16))
    rd = dev(rng.standard_normal((m, n)).astype(np.float16))
    outs = []
    for name in ("256x256p2w8", "256x256p2w8-persist"):
        ctx.select_variant("gemm_w4a16", name)
        if epilogue is None:
            y = empty((m, n), torch.float32)
            ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)
        else:
            y = empty((m, n), torch.float16)
            ctx.linear_f16(w, x, m, y, epilogue, rd if epilogue == rocm.EPI_RESIDUAL else None)
        outs.append(host(ctx, y))
    ctx.select_variant("gemm_w4a16", W4A16_VARIANTS[0])
    assert bits_equal(outs[1], outs[0])
    if epilogue is None:
        rows = np.array([0, 255, 256, 2047, 4351, 4399])
        deq = oracle.unpack_g32_f16(packed).reshape(n, k)
        want = oracle.w4a16(xh[rows], len(rows), k, deq, n)
        assert np.abs(outs[1][rows] - want).max() <= MAX_ABS and cosine(outs[1][rows], want) >= MIN_COS


def test_w4a16_f16_output_rejects_bad_arguments(ctx, oracle):
    torch = pytest.importorskip("torch")
    w = ctx.quantize(dev(np.ones((64, 64), np.float32) * 0.01), rocm.F32, 64, 64, 4, 32)
    x = empty((2, 64), torch.float16)
    y = empty((2, 64), torch.float16)
    for epilogue, res, code in [(3, None, "INVALID_PARAMETERS"), (rocm.EPI_RESIDUAL, None, "INVALID_REQUEST")]:
        with pytest.raises(rocm.DzError) as e:
            ctx.linear_f16(w, x, 2, y, epilogue, res)
        assert e.value.code == code
    w8 = ctx.quantize(dev(np.ones((64, 64), np.float32) * 0.01), rocm.F32, 64, 64, 8, 64)
    with pytest.raises(rocm.DzError) as e:
        ctx.linear_f16(w8, x, 2, y)
    assert e.value.code == "INVALID_PARAMETERS"


@pytest.mark.parametrize("n", [3072, 3120])
def test_w4a16_column_split_matches_register_kernel(ctx, oracle, n):
    """M=8192, K=1024: n = 3072 runs on persistent 256x192 tiles (two whole
    waves of compute units, the encoder's QKV shape); at n = 3120 256x256
    tiles fill whole waves over the leading columns and 128x256 tiles take the
    rest (two launches). The bits equal the register-staged kernel's, and
    sampled rows the float64 product of the dequantized weights."""
    torch = pytest.importorskip("torch")
    m, k = 8192, 1024
    g = torch.Generator(device="cuda").manual_seed(n)
    wdev = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    torch.cuda.synchronize()  # the context's stream is not ordered after torch's
    w = ctx.quantize(wdev, rocm.F32, n, k, 4, 32)
    del wdev
    x = torch.randn((m, k), generator=torch.Generator(device="cuda").manual_seed(3), device="cuda").half()
    torch.cuda.synchronize()
    ys = []
    for name in ("pipe-auto", "256x128w2x2"):
        ctx.select_variant("gemm_w4a16", name)
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)
        ctx.sync()
        ys.append(y)
    ctx.select_variant("gemm_w4a16", W4A16_VARIANTS[0])
    assert torch.equal(ys[0], ys[1])
    deq = torch.empty((n, k), dtype=torch.float32, device="cuda")
    ctx.dequant(w, deq)
    ctx.sync()
    rows = torch.arange(0, m, 509, device="cuda")
    ref = (x[rows].double() @ deq.double().T).float()
    assert (ys[0][rows] - ref).abs().max().item() <= MAX_ABS
    w.free()


def test_config5_prefill_rows_vs_fp32(ctx, oracle):
    """BASELINE config 5 at full size (M=16384, K=4096, N=14336); a row sample is
    checked against an fp32 product of the dequantized weights."""
    torch = pytest.importorskip("torch")
    m, k, n = 16384, 4096, 14336
    g = torch.Generator(device="cuda").manual_seed(1)
    wdev = torch.randn((n, k), generator=g, device="cuda", dtype=torch.float32) * 0.02
    torch.cuda.synchronize()  # the context's stream is not ordered after torch's
    w = ctx.quantize(wdev, rocm.F32, n, k, 4, 32)
    del wdev
    x = torch.randn((m, k), generator=torch.Generator(device="cuda").manual_seed(0), device="cuda").half()
    torch.cuda.synchronize()
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ctx.linear(w, x, rocm.F16, m, y, rocm.W4A16)
    deq = torch.empty((n, k), dtype=torch.float32, device="cuda")
    ctx.dequant(w, deq)
    ctx.sync()
    rows = torch.arange(0, m, 61, device="cuda")
    ref = (x[rows].double() @ deq.double().T).float()
    got = y[rows]
    err = (got - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.double().reshape(1, -1), ref.double().reshape(1, -1)).item()
    assert err <= MAX_ABS and cos >= MIN_COS, (err, cos)
    assert torch.isfinite(y).all().item()


# ---- per-row int8 ----------------------------------------------------------------------

I8_VARIANTS = ("256x256p2w8", "256x256p4k64w8", "256x128p3w8", "256x128p3", "128x128w2x2", "256x128w2x2",
               "64x64w2x2", "256x256p2w8-stream", "256x256p2w8-stream-mid", "256x128k64p2-stream2")


@pytest.mark.parametrize("m,n,k", GOLDEN["q4_raw_check_shapes"]["mnk"] + [[77, 45, 100], [1, 1, 4], [130, 260, 4100],
                                                                          [300, 520, 4112], [256, 256, 256], [513, 257, 80]])
def test_i8_gemm_exact(ctx, oracle, m, n, k):
    """webgpu/q4.rs:476-501 known answers plus ragged shapes: raw int32 and the
    f32 epilogue are bit-exact; every variant agrees."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(m * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    qa, sa, _ = oracle.i8_quantize_rows(a, m, k)
    qb, sb, _ = oracle.i8_quantize_rows(b, n, k)
    raw, yf = oracle.i8_gemm(qa, sa, m, qb, sb, n, k, threads=8)
    for name in I8_VARIANTS:
        ctx.select_variant("i8_gemm", name)
        r = empty((m, n), torch.int32)
        y = empty((m, n), torch.float32)
        da, db, dsa, dsb = dev(qa), dev(qb), dev(sa), dev(sb)
        ctx.i8_gemm(da, dsa, m, db, dsb, n, k, r, raw=True)
        ctx.i8_gemm(da, dsa, m, db, dsb, n, k, y, raw=False)
        assert np.array_equal(host(ctx, r), raw), name
        assert bits_equal(host(ctx, y), yf), name
    ctx.select_variant("i8_gemm", I8_VARIANTS[0])


@pytest.mark.parametrize("m,n,k", [[1, 1, 4], [77, 45, 100], [130, 260, 4100], [256, 512, 4096], [513, 257, 80]])
def test_i8_gemm_fused_silu(ctx, oracle, m, n, k):
    """webgpu/int8.rs:226-230 fused mode against the oracle: bit for bit but
    for the rare value where the device and host f64 exponentials round to
    different f32 exp (then one ulp); and equal to silu applied to the two
    plain products of the same codes."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(m + 7 * n + k)
    qa, sa, _ = oracle.i8_quantize_rows(rng.standard_normal((m, k)).astype(np.float32), m, k)
    qg, sg, _ = oracle.i8_quantize_rows(rng.standard_normal((n, k)).astype(np.float32), n, k)
    qu, su, _ = oracle.i8_quantize_rows(rng.standard_normal((n, k)).astype(np.float32), n, k)
    sa = (sa * np.float32(4.0 / np.sqrt(k))).astype(np.float32)  # gates of a few units
    want = oracle.i8_gemm_fused(qa, sa, m, qg, sg, qu, su, n, k)
    y = empty((m, n), torch.float32)
    ctx.i8_gemm_fused(dev(qa), dev(sa), m, dev(qg), dev(sg), dev(qu), dev(su), n, k, y)
    got = host(ctx, y)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert np.count_nonzero(ulps) <= max(1, got.size // 10000)
    gate = empty((m, n), torch.float32)
    up = empty((m, n), torch.float32)
    ctx.i8_gemm(dev(qa), dev(sa), m, dev(qg), dev(sg), n, k, gate, raw=False)
    ctx.i8_gemm(dev(qa), dev(sa), m, dev(qu), dev(su), n, k, up, raw=False)
    g, u = host(ctx, gate), host(ctx, up)
    composed = ((g / (np.float32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32))) * u).astype(np.float32)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - composed.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1


def test_config4_int8_full_size(ctx, oracle):
    """W f32 [4096 x 4096] N(0,0.02) per-channel, A f32
    [8192 x 4096] N(0,1) per-token; quantized on the GPU (bit-exact with the
    oracle) and the i32 accumulators bit-exact on a row sample."""
    torch = pytest.importorskip("torch")
    m, n, k = 8192, 4096, 4096
    a = np.random.default_rng(0).standard_normal((m, k)).astype(np.float32)
    b = (np.random.default_rng(1).standard_normal((n, k)) * 0.02).astype(np.float32)
    qa = empty((m, k), torch.int8)
    sa = empty(m, torch.float32)
    qb = empty((n, k), torch.int8)
    sb = empty(n, torch.float32)
    ctx.i8_quantize_rows(dev(a), m, k, qa, sa)
    ctx.i8_quantize_rows(dev(b), n, k, qb, sb)
    oqa, osa, _ = oracle.i8_quantize_rows(a, m, k)
    oqb, osb, _ = oracle.i8_quantize_rows(b, n, k)
    assert np.array_equal(host(ctx, qa), oqa) and np.array_equal(host(ctx, qb), oqb)
    assert bits_equal(host(ctx, sa), osa) and bits_equal(host(ctx, sb), osb)
    r = empty((m, n), torch.int32)
    ctx.i8_gemm(qa, sa, m, qb, sb, n, k, r, raw=True)
    got = host(ctx, r)
    rows = np.arange(0, m, 97)
    want, _ = oracle.i8_gemm(oqa[rows], osa[rows], rows.size, oqb, osb, n, k, threads=16, scaled=False)
    assert np.array_equal(got[rows], want)
    # every row: sum_j C[i, j] == A[i] . (sum_j B[j]) exactly (integer checksum)
    colsum = oqb.astype(np.int64).sum(axis=0)
    assert np.array_equal(got.astype(np.int64).sum(axis=1), oqa.astype(np.int64) @ colsum)
    # every variant (the persistent ones walk several tiles per block) gives the same bits
    yf = empty((m, n), torch.float32)
    ctx.i8_gemm(qa, sa, m, qb, sb, n, k, yf, raw=False)
    for name in I8_VARIANTS:
        ctx.select_variant("i8_gemm", name)
        rv = torch.full((m, n), -7, dtype=torch.int32, device="cuda")
        yv = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()  # the fills run on torch's stream, the products on the context's
        ctx.i8_gemm(qa, sa, m, qb, sb, n, k, rv, raw=True)
        ctx.i8_gemm(qa, sa, m, qb, sb, n, k, yv, raw=False)
        ctx.sync()
        assert torch.equal(rv, r), name
        assert torch.equal(yv.view(torch.int32), yf.view(torch.int32)), name
    ctx.select_variant("i8_gemm", I8_VARIANTS[0])


# ---- per-row Q4 product (webgpu/q4.rs:99-105) ----------------------------------------

@pytest.mark.parametrize("m,n,k", GOLDEN["q4_raw_check_shapes"]["mnk"] + [[77, 45, 104], [130, 260, 4104], [256, 512, 4096]])
def test_q4_rows_gemm_exact(ctx, oracle, m, n, k):
    """Exact int32 dots of int8 activations with per-row Q4 codes (brute
    force), and the (f32(dot)*sa)*sw epilogue bit for bit; the first two
    shapes use the known-answer inputs of q4.rs:107-142."""
    torch = pytest.importorskip("torch")
    if [m, n, k] in GOLDEN["q4_raw_check_shapes"]["mnk"]:
        i = np.arange(m * k)
        a = np.where(i % k == 0, 127.0, ((i * 17 % 255) - 127.0)).astype(np.float32)
        j = np.arange(n * k)
        b = np.where(j % k == 0, 7.0, ((j * 11 % 15) - 7.0)).astype(np.float32)
    else:
        rng = np.random.default_rng(m + n + k)
        a = rng.standard_normal(m * k).astype(np.float32)
        b = (rng.standard_normal(n * k) * 0.02).astype(np.float32)
    bits16 = oracle.f32_to_f16_bits(b)
    words = empty((n * (k // 8) + 2 * n,), torch.int32)
    ctx.q4_quantize_rows(dev(bits16.view(np.float16)), rocm.F16, n, k, words)
    qa, sa, _ = oracle.i8_quantize_rows(a, m, k)
    raw = empty((m, n), torch.int32)
    y = empty((m, n), torch.float32)
    ctx.q4_rows_gemm(dev(qa), dev(sa), m, words, n, k, raw, raw=True)
    ctx.q4_rows_gemm(dev(qa), dev(sa), m, words, n, k, y, raw=False)
    codes, scales, _ = oracle.q4_rows_split(oracle.q4_quantize_rows(bits16, n, k), n, k)
    expected = qa.astype(np.int64) @ codes.astype(np.int64).T
    assert np.array_equal(host(ctx, raw).astype(np.int64), expected)
    _, want = oracle.i8_gemm(qa, sa, m, codes, scales, n, k, raw=False)
    assert bits_equal(host(ctx, y), want)
