"""GPU parity of the fitted Q4 forms (quantization.rs mse / affine / nf4).

The fitting runs on the CPU in the oracle, as the reference fits at load; the
GPU takes the fitted codes, scales and offsets through
dz_weight_upload_fitted. The grouped products fold each group as
int8.rs:524-571 does, the affine offset term included: bit-exact against the
oracle's fused order (itself pinned bit for bit to an AVX2 restatement of
int8.rs rows<R,Q4>). Row decoding follows quantized_rows.rs:89-110 bit for
bit."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, cosine, dev, empty, host

pytestmark = pytest.mark.gpu
MAX_ABS = 1e-2  # north_star tolerance for f16/f32 GEMM outputs
MIN_COS = 0.9999
GROUPED_VARIANTS = ("pipe256x128w8", "wave16x16", "pipe128x128w4", "pipe64x128w2", "pipe128x128m8",
                    "pipe128x128n8", "pipe32x128w8", "pipe64x128w8", "pipe32x128w8g4", "pipe64x128w8g4", "fewrow16", "pipe32x64w4", "pipe64x64w8", "pipe-auto")


def fitted(oracle, n, k, mode, seed, spread=0.05, shift=0.0):
    """BF16 weights N(shift, spread) fitted by the oracle -> (bf16, codes, scales, offsets)."""
    rng = np.random.default_rng(seed)
    raw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * spread + shift).astype(np.float32))
    codes, scales, offsets = oracle.weight_quantize_fitted(raw, n, k, mode)
    return raw, codes, scales, offsets


def upload(ctx, oracle, codes, scales, offsets, n, k, form):
    wire = oracle.pack_wire_codes(codes, scales, n, k)
    return ctx.upload_fitted(wire, n, k, form, offsets if form == rocm.FIT_AFFINE else None)


def grouped(ctx, w, x, m, n, mode=rocm.W4A8):
    torch = pytest.importorskip("torch")
    y = empty((m, n), torch.float32)
    ctx.linear(w, dev(x), rocm.F32, m, y, mode)
    return host(ctx, y)


@pytest.mark.parametrize("m,k,n", [(1, 128, 40), (5, 640, 33), (16, 1024, 130), (17, 256, 64), (40, 640, 1040),
                                   (300, 1088, 200), (257, 64, 129)])
@pytest.mark.parametrize("ab", [8, 4])
def test_affine_grouped_products_bit_exact(ctx, oracle, m, k, n, ab):
    """Affine weights (offsets centred away from zero) through dz_linear: the
    few-row kernel (m <= 16), the pipelined kernels and the one-wave-per-tile
    kernel all equal the oracle's fused fold bit for bit."""
    _, codes, scales, offsets = fitted(oracle, n, k, "affine", m + k + n, shift=0.03)
    assert np.abs(offsets).max() > 0
    w = upload(ctx, oracle, codes, scales, offsets, n, k, rocm.FIT_AFFINE)
    x = (np.random.default_rng(m * 7 + ab).standard_normal((m, k)) * 1.5 + 0.4).astype(np.float32)
    q, sx = oracle.act_quantize(x, m, k, ab)
    want = oracle.grouped_gemm_affine(q, sx, m, codes, scales, offsets, n, k, fused=True)
    mode = rocm.W4A4 if ab == 4 else rocm.W4A8
    got = grouped(ctx, w, x, m, n, mode)
    assert bits_equal(got, want), (m, k, n, float(np.abs(got - want).max()))
    if m > 16:
        for name in GROUPED_VARIANTS:
            ctx.select_variant("grouped", name)
            assert bits_equal(grouped(ctx, w, x, m, n, mode), want), name
        ctx.select_variant("grouped", "pipe-auto")


@pytest.mark.parametrize("m,k,n", [(1, 128, 40), (9, 640, 33), (40, 640, 1040), (300, 1088, 200)])
def test_scaled_fit_grouped_products_bit_exact(ctx, oracle, m, k, n):
    """MSE-fitted weights (negative scales, -8 codes) fold as symmetric ones."""
    _, codes, scales, offsets = fitted(oracle, n, k, "mse", m + n)
    assert (scales < 0).any() and (codes == -8).any()
    w = upload(ctx, oracle, codes, scales, None, n, k, rocm.FIT_SCALED)
    x = (np.random.default_rng(m).standard_normal((m, k)) * 1.5).astype(np.float32)
    q, sx = oracle.act_quantize(x, m, k, 8)
    want = oracle.grouped_gemm(q, sx, m, codes, scales, n, k, fused=True)
    assert bits_equal(grouped(ctx, w, x, m, n), want), (m, k, n)


@pytest.mark.parametrize("m,k,n", [(1, 4096, 512), (8, 1024, 300), (64, 512, 256)])
def test_scaled_fit_w4a16_vs_closed_form(ctx, oracle, m, k, n):
    """W4A16 takes MSE-fitted weights: the f64 closed form within north_star."""
    torch = pytest.importorskip("torch")
    _, codes, scales, _ = fitted(oracle, n, k, "mse", n + k)
    w = upload(ctx, oracle, codes, scales, None, n, k, rocm.FIT_SCALED)
    x = np.random.default_rng(k).standard_normal((m, k)).astype(np.float32)
    xh = oracle.f32_to_f16_bits(x)
    y = empty((m, n), torch.float32)
    ctx.linear(w, dev(xh.view(np.float16)), rocm.F16, m, y, rocm.W4A16)
    got = host(ctx, y)
    wd = oracle.rows_decode(codes, scales, None, False, n, k)
    want = oracle.w4a16(xh, m, k, wd, n)
    assert np.abs(got - want).max() <= MAX_ABS
    assert cosine(got, want) >= MIN_COS


@pytest.mark.parametrize("m", [5, 40])
def test_affine_pair_and_noalloc_equal_the_single_product(ctx, oracle, m):
    """dz_linear_pair (an affine and an MSE weight on one quantization) and
    dz_linear_noalloc give the single products' bits, twice in a row."""
    torch = pytest.importorskip("torch")
    k, n1, n2 = 640, 200, 72
    _, c1, s1, o1 = fitted(oracle, n1, k, "affine", 1, shift=-0.02)
    _, c2, s2, _ = fitted(oracle, n2, k, "mse", 2)
    a = upload(ctx, oracle, c1, s1, o1, n1, k, rocm.FIT_AFFINE)
    b = upload(ctx, oracle, c2, s2, None, n2, k, rocm.FIT_SCALED)
    x = (np.random.default_rng(m).standard_normal((m, k)) + 0.3).astype(np.float32)
    ya, yb = empty((m, n1), torch.float32), empty((m, n2), torch.float32)
    xd = dev(x)
    ctx.linear_pair(a, b, xd, m, ya, yb)
    q, sx = oracle.act_quantize(x, m, k, 8)
    want_a = oracle.grouped_gemm_affine(q, sx, m, c1, s1, o1, n1, k, fused=True)
    want_b = oracle.grouped_gemm(q, sx, m, c2, s2, n2, k, fused=True)
    assert bits_equal(host(ctx, ya), want_a)
    assert bits_equal(host(ctx, yb), want_b)
    for rows in (m, max(m // 2, 1)):
        y = empty((rows, n1), torch.float32)
        ctx.linear_noalloc(a, xd, rocm.F32, rows, y, rocm.W4A8)
        assert bits_equal(host(ctx, y), want_a[:rows]), rows


@pytest.mark.parametrize("mode,form", [("mse", rocm.FIT_SCALED), ("affine", rocm.FIT_AFFINE), ("nf4", rocm.FIT_NF4)])
def test_fitted_rows_decode_bit_exact(ctx, oracle, mode, form):
    """dz_dequant and dz_dequant_rows decode every form as
    quantized_rows.rs:89-110 append: f32 bit for bit, f16 the f32 rounded once."""
    torch = pytest.importorskip("torch")
    n, k = 50, 384
    _, codes, scales, offsets = fitted(oracle, n, k, mode, 11, shift=0.01)
    w = upload(ctx, oracle, codes, scales, offsets, n, k, form)
    want = oracle.rows_decode(codes, scales, offsets if form == rocm.FIT_AFFINE else None, form == rocm.FIT_NF4, n, k)
    y = empty((n, k), torch.float32)
    ctx.dequant(w, y)
    assert bits_equal(host(ctx, y), want)
    ids = np.array([7, 0, 49, 7, 13], np.int32)
    for dtype, tdt in ((rocm.F32, torch.float32), (rocm.F16, torch.float16)):
        y = empty((ids.size, k), tdt)
        ctx.dequant_rows(w, dev(ids), ids.size, y, dtype)
        got = host(ctx, y)
        ref = want[ids] if dtype == rocm.F32 else want[ids].astype(np.float16)
        assert bits_equal(got, ref), dtype


def test_fitted_upload_and_product_refusals(ctx, oracle):
    """Forms a product does not take are refused, as are bad fitted uploads."""
    torch = pytest.importorskip("torch")
    n, k = 64, 128
    _, codes, scales, offsets = fitted(oracle, n, k, "affine", 3, shift=0.02)
    wire = oracle.pack_wire_codes(codes, scales, n, k)

    def refused(code, fn):
        with pytest.raises(rocm.DzError) as e:
            fn()
        assert e.value.code == code

    refused("INVALID_REQUEST", lambda: ctx.upload_fitted(wire, n, k, rocm.FIT_AFFINE, None))
    refused("INVALID_REQUEST", lambda: ctx.upload_fitted(wire, n, k, rocm.FIT_SCALED, offsets))
    refused("INVALID_PARAMETERS", lambda: ctx.upload_fitted(wire, n, k, 7, None))
    bad = offsets.copy()
    bad[3, 1] = np.nan
    refused("INVALID_CHECKPOINT", lambda: ctx.upload_fitted(wire, n, k, rocm.FIT_AFFINE, bad))
    zero = scales.copy()
    zero[5, 0] = 0.0
    refused("INVALID_CHECKPOINT",
            lambda: ctx.upload_fitted(oracle.pack_wire_codes(codes, zero, n, k), n, k, rocm.FIT_SCALED))
    negative = oracle.pack_wire_codes(codes, -np.abs(scales), n, k)
    refused("INVALID_CHECKPOINT", lambda: ctx.upload(negative, rocm.Q4_G64_F32, n, k))  # packed.rs: positive only
    affine = ctx.upload_fitted(wire, n, k, rocm.FIT_AFFINE, offsets)
    nf4 = ctx.upload_fitted(wire, n, k, rocm.FIT_NF4, None)
    scaled = ctx.upload_fitted(negative, n, k, rocm.FIT_SCALED, None)
    x = dev(np.ones((40, k), np.float32))  # sized for every call below, refused or not
    xh = dev(np.ones((4, k), np.float16))
    y = empty((40, n), torch.float32)
    refused("INVALID_PARAMETERS", lambda: ctx.linear(nf4, x, rocm.F32, 4, y, rocm.W4A8))
    refused("INVALID_PARAMETERS", lambda: ctx.linear_noalloc(nf4, x, rocm.F32, 40, y, rocm.W4A8))
    refused("INVALID_PARAMETERS", lambda: ctx.linear_pair(affine, nf4, x, 4, y, y))
    refused("INVALID_PARAMETERS", lambda: ctx.linear(affine, xh, rocm.F16, 4, y, rocm.W4A16))
    refused("INVALID_PARAMETERS", lambda: ctx.linear(nf4, xh, rocm.F16, 4, y, rocm.W4A16))
    q = dev(np.zeros((4, k), np.int8))
    s = dev(np.ones((4, k // 64), np.float32))
    refused("INVALID_PARAMETERS", lambda: ctx.linear_q8(affine, q, s, 4, y))
    refused("INVALID_PARAMETERS", lambda: ctx.mlp_requant(affine, affine, x, 4, dev(np.zeros((4, n), np.int8)), s))
    # the weights refused above still run where they belong
    ctx.linear(scaled, xh, rocm.F16, 4, y, rocm.W4A16)
    ctx.linear(affine, x, rocm.F32, 4, y, rocm.W4A8)
    assert np.isfinite(host(ctx, y)).all()


@pytest.mark.parametrize("m", [5, 300])
def test_scaled_fit_mlp_and_code_products_equal_their_compositions(ctx, oracle, m):
    """MSE-fitted gate/up through the fused MLP (every variant) give the codes
    and scales of the grouped pair, SiLU * up and the A8 quantizer word for
    word (grouped_q4.rs:313-354), and dz_linear_q8 on codes gives dz_linear's
    bits for the same rows."""
    torch = pytest.importorskip("torch")
    k, n = 640, 192
    _, gc, gs, _ = fitted(oracle, n, k, "mse", 21)
    _, uc, us, _ = fitted(oracle, n, k, "mse", 22)
    gate = upload(ctx, oracle, gc, gs, None, n, k, rocm.FIT_SCALED)
    up = upload(ctx, oracle, uc, us, None, n, k, rocm.FIT_SCALED)
    x = (np.random.default_rng(m).standard_normal((m, k)) * 1.3).astype(np.float32)
    xd = dev(x)
    g, u = empty((m, n), torch.float32), empty((m, n), torch.float32)
    ctx.linear_pair(gate, up, xd, m, g, u)
    ctx.silu_mul(g, u, m * n)
    q2, s2 = empty((m, n), torch.int8), empty((m, n // 64), torch.float32)
    ctx.act_quantize(g, m, n, 8, q2, s2)
    q2h, s2h = host(ctx, q2).copy(), host(ctx, s2).copy()
    q, s = empty((m, n), torch.int8), empty((m, n // 64), torch.float32)
    try:
        for name in ("pipe256x64w8", "pipe128x64w4", "wave16x64", "pipe256x64n2", "pipe128x64n2", "pipe-auto"):
            ctx.select_variant("mlp", name)
            q.zero_()
            torch.cuda.synchronize()  # the fill runs on torch's stream, the product on the context's
            ctx.mlp_requant(gate, up, xd, m, q, s)
            assert np.array_equal(host(ctx, q), q2h), name
            assert bits_equal(host(ctx, s), s2h), name
    finally:
        ctx.select_variant("mlp", "pipe-auto")
    qx, sx = empty((m, k), torch.int8), empty((m, k // 64), torch.float32)
    ctx.act_quantize(xd, m, k, 8, qx, sx)
    y1, y2 = empty((m, n), torch.float32), empty((m, n), torch.float32)
    ctx.linear_q8(gate, qx, sx, m, y1)
    ctx.linear(gate, xd, rocm.F32, m, y2, rocm.W4A8)
    assert bits_equal(host(ctx, y1), host(ctx, y2))
    want = oracle.grouped_gemm(host(ctx, qx), host(ctx, sx), m, gc, gs, n, k, fused=True)
    assert bits_equal(host(ctx, y1), want)
