"""Few-row grouped products (grouped_gemv_kernel): the reference numeric mode at
M <= 16, the portable readout product packed::project, and the 17-word A8
records of the WebGPU quantizer. Everything here is bit-exact against the
oracle (integer dots, fixed fold order)."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, dev, empty, host

pytestmark = pytest.mark.gpu


def _weight(ctx, oracle, n, k, bits, seed):
    rng = np.random.default_rng(seed)
    raw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed = oracle.pack_g64(raw, n, k, bits)
    w = ctx.upload(packed, rocm.Q4_G64_F32 if bits == 4 else rocm.Q8_G64_F32, n, k)
    return raw, packed, w


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m,k,n", [(1, 2560, 255), (3, 64, 7), (5, 128, 67), (16, 192, 33), (17, 256, 40),
                                   (1, 4096, 4096)])
def test_project_is_packed_project_bit_for_bit(ctx, oracle, bits, m, k, n):
    """packed.rs:75-119: sum += f32(dot) * (sx*sw), groups in order; the
    readout shape (255 outputs over 2560) is mod.rs:149-185's."""
    torch = pytest.importorskip("torch")
    _, packed, w = _weight(ctx, oracle, n, k, bits, m + k + n)
    x = np.random.default_rng(1).standard_normal((m, k)).astype(np.float32) * 3
    y = empty((m, n), torch.float32)
    ctx.project(w, dev(x), m, y)
    got = host(ctx, y)
    for r in range(m):
        want = oracle.project(packed, bits, k, x[r], n)
        assert bits_equal(got[r], want), (r, float(np.abs(got[r] - want).max()))


@pytest.mark.parametrize("m", [1, 20])
def test_project_rejects_nonfinite_activations(ctx, oracle, m):
    torch = pytest.importorskip("torch")
    _, _, w = _weight(ctx, oracle, 32, 128, 4, 3)
    x = np.ones((m, 128), np.float32)
    x[m - 1, 77] = np.inf
    y = empty((m, 32), torch.float32)
    with pytest.raises(rocm.DzError) as e:
        ctx.project(w, dev(x), m, y)
    assert e.value.code == "INFERENCE_FAILED"
    assert "nonfinite readout activation" in str(e.value)


def test_project_rejects_group32_and_ragged_cols(ctx, oracle):
    torch = pytest.importorskip("torch")
    w32 = ctx.quantize(dev(np.ones((16, 64), np.float32)), rocm.F32, 16, 64, 4, 32)
    y = empty((1, 16), torch.float32)
    with pytest.raises(rocm.DzError) as e:
        ctx.project(w32, dev(np.ones((1, 64), np.float32)), 1, y)
    assert e.value.code == "INVALID_PARAMETERS"
    w = ctx.quantize(dev(np.ones((16, 65), np.float32)), rocm.F32, 16, 65, 4, 64)
    with pytest.raises(rocm.DzError):
        ctx.project(w, dev(np.ones((1, 65), np.float32)), 1, y)


@pytest.mark.parametrize("m,k", [(1, 64), (5, 256), (16, 2560), (40, 1024)])
def test_records_hold_the_act_quantizer_codes_and_feed_the_product(ctx, oracle, m, k):
    """grouped_q4.rs:3-25: 16 code words + the f32 scale per (row, group); the
    product from records equals the product from the activations."""
    torch = pytest.importorskip("torch")
    x = (np.random.default_rng(m * k).standard_normal((m, k)) * 2).astype(np.float32)
    g = k // 64
    recs = empty((m, g, 17), torch.int32)
    ctx.act_quantize_records(dev(x), m, k, recs)
    recs_h = host(ctx, recs).view(np.uint32)
    q, s = oracle.act_quantize(x, m, k, 8)
    codes = recs_h[:, :, :16].copy().view(np.int8).reshape(m, g * 64)
    assert bits_equal(codes, q)
    assert bits_equal(recs_h[:, :, 16].copy().view(np.float32), s)
    for bits in (4, 8):
        _, _, w = _weight(ctx, oracle, 48, k, bits, k + bits)
        y1 = empty((m, 48), torch.float32)
        y2 = empty((m, 48), torch.float32)
        ctx.linear(w, dev(x), rocm.F32, m, y1, rocm.W4A8)
        ctx.linear_records(w, recs, m, y2)
        assert bits_equal(host(ctx, y2), host(ctx, y1)), bits


def test_records_need_whole_groups(ctx):
    torch = pytest.importorskip("torch")
    recs = empty((1, 2, 17), torch.int32)
    with pytest.raises(rocm.DzError) as e:
        ctx.act_quantize_records(dev(np.ones((1, 100), np.float32)), 1, 100, recs)
    assert e.value.code == "INVALID_PARAMETERS"


@pytest.mark.parametrize("wb,ab", [(4, 8), (8, 8), (4, 4), (8, 4)])
@pytest.mark.parametrize("k,n", [(100, 17), (1000, 50), (4096, 64)])
def test_every_row_count_up_to_16_matches_the_avx2_order(ctx, oracle, wb, ab, k, n):
    """M = 1..16 runs the few-row kernel: up to 4 rows it quantizes x in
    every block, from 5 rows over codes quantized once (tails zero padded as
    int8.rs:178-202 does either way); the codes + scales entry (dz_linear_q8)
    gives the same bits."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(k + n + wb + ab)
    raw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    w = ctx.quantize(dev(raw), rocm.BF16, n, k, wb, 64)
    codes, scales = oracle.weight_quantize(raw, n, k, wb)
    x = (rng.standard_normal((16, k)) * 1.5).astype(np.float32)
    for m in (1, 2, 3, 4, 5, 8, 9, 16):
        want = oracle.matrix_apply(x[:m], m, codes, scales, n, k, ab, fused=True)
        y = empty((m, n), torch.float32)
        ctx.linear(w, dev(x[:m]), rocm.F32, m, y, rocm.W4A4 if ab == 4 else rocm.W4A8)
        assert bits_equal(host(ctx, y), want), (m, float(np.abs(host(ctx, y) - want).max()))
        if ab == 8:
            q, s = oracle.act_quantize(x[:m], m, k, 8)
            y2 = empty((m, n), torch.float32)
            ctx.linear_q8(w, dev(q), dev(s), m, y2)
            assert bits_equal(host(ctx, y2), want), m


def test_few_rows_nonfinite_activation_makes_every_output_nan(ctx, oracle):
    """int8.rs:170-173: one non-finite activation anywhere -> every output NaN,
    whether the kernel quantizes (3 rows) or takes codes quantized once (12)."""
    torch = pytest.importorskip("torch")
    _, _, w = _weight(ctx, oracle, 40, 256, 4, 9)
    for m in (3, 12):
        x = np.ones((m, 256), np.float32)
        x[m - 1, 200] = np.nan
        y = empty((m, 40), torch.float32)
        ctx.linear(w, dev(x), rocm.F32, m, y, rocm.W4A8)
        assert np.isnan(host(ctx, y)).all(), m
        x[m - 1, 200] = 1.0  # the flag is the call's own: a clean call after it is finite
        ctx.linear(w, dev(x), rocm.F32, m, y, rocm.W4A8)
        assert not np.isnan(host(ctx, y)).any(), m
