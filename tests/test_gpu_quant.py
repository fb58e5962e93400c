"""GPU parity: weight re-tiling, device quantizers, dequantization and the
activation quantizers, all bit-exact against the oracle."""
import json
from pathlib import Path

import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, dev, empty, host

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _bf16_weights(oracle, n, k, seed):
    rng = np.random.default_rng(seed)
    return oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k", [(1, 64), (7, 128), (33, 192), (100, 1024), (16, 4096)])
def test_upload_g64_dequant_is_unpack(ctx, oracle, bits, n, k):
    torch = pytest.importorskip("torch")
    raw = _bf16_weights(oracle, n, k, n * 31 + k)
    packed = oracle.pack_g64(raw, n, k, bits)
    w = ctx.upload(packed, rocm.Q4_G64_F32 if bits == 4 else rocm.Q8_G64_F32, n, k)
    y = empty((n, k), torch.float32)
    ctx.dequant(w, y)
    assert bits_equal(host(ctx, y).reshape(-1), oracle.unpack_g64(packed, bits))


@pytest.mark.parametrize("n,k", [(1, 32), (5, 96), (64, 4096), (17, 1024)])
def test_upload_g32_dequant_is_unpack(ctx, oracle, n, k):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(n + k)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed = oracle.pack_g32_f16(wf, n, k)
    w = ctx.upload(packed, rocm.Q4_G32_F16, n, k)
    y = empty((n, k), torch.float32)
    ctx.dequant(w, y)
    assert bits_equal(host(ctx, y).reshape(-1), oracle.unpack_g32_f16(packed))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k", [(1, 1), (7, 65), (9, 129), (32, 127), (65, 1025), (3, 63)])
def test_device_quantizer_matches_matrix_quantizer(ctx, oracle, bits, n, k):
    """int8.rs:51-152 on device: codes and scales equal the oracle's."""
    torch = pytest.importorskip("torch")
    i = np.arange(n * k)
    raw = oracle.f32_to_bf16(((i * 37 % 257) - 128.0) / 31.0)
    w = ctx.quantize(dev(raw), rocm.BF16, n, k, bits, 64)
    y = empty((n, k), torch.float32)
    ctx.dequant(w, y)
    codes, scales = oracle.weight_quantize(raw, n, k, bits)
    want = (codes[:, :k].astype(np.float32) * np.repeat(scales, 64, 1)[:, :k]).astype(np.float32)
    assert bits_equal(host(ctx, y), want)


@pytest.mark.parametrize("n,k", [(4, 32), (33, 160), (128, 4096)])
def test_device_g32_quantizer_matches_pack(ctx, oracle, n, k):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(k)
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wf[0, :32] = 0.0
    w = ctx.quantize(dev(wf), rocm.F32, n, k, 4, 32)
    y = empty((n, k), torch.float32)
    ctx.dequant(w, y)
    assert bits_equal(host(ctx, y).reshape(-1), oracle.unpack_g32_f16(oracle.pack_g32_f16(wf, n, k)))


def test_upload_golden_groups(ctx, oracle):
    torch = pytest.importorskip("torch")
    g = GOLDEN["q4_group"]
    v = np.array(g["values"] * g["repeat"], np.float32)
    packed = np.frombuffer(bytes.fromhex(g["bytes_hex"]) * g["bytes_repeat"] + np.float32(1.0).tobytes(), np.uint8)
    w = ctx.upload(packed, rocm.Q4_G64_F32, 1, 64)
    y = empty((1, 64), torch.float32)
    ctx.dequant(w, y)
    want = np.array([7, -7, 0, 0, 2, -2, 2, -2] * 8, np.float32)
    assert bits_equal(host(ctx, y).reshape(-1), want)
    assert np.allclose(want, np.clip(np.rint(v), -7, 7))


def test_upload_rejects_invalid_checkpoints(ctx, oracle):
    packed = oracle.pack_g64(_bf16_weights(oracle, 2, 128, 0), 2, 128, 4)
    for bad_scale in (-1.0, 0.0, np.nan, np.inf):
        bad = packed.copy()
        bad[36 + 32:36 + 36] = np.frombuffer(np.float32(bad_scale).tobytes(), np.uint8)
        with pytest.raises(rocm.DzError) as e:
            ctx.upload(bad, rocm.Q4_G64_F32, 2, 128)
        assert e.value.code == "INVALID_CHECKPOINT"
    with pytest.raises(rocm.DzError) as e:
        ctx.upload(packed[:-1], rocm.Q4_G64_F32, 2, 128)
    assert e.value.code == "INVALID_CHECKPOINT"
    with pytest.raises(rocm.DzError) as e:
        ctx.upload(packed, 9, 2, 128)
    assert e.value.code == "INVALID_PARAMETERS"


def test_quantizer_rejects_nonfinite(ctx):
    x = np.zeros((2, 64), np.float32)
    x[1, 5] = np.nan
    with pytest.raises(rocm.DzError) as e:
        ctx.quantize(dev(x), rocm.F32, 2, 64, 4, 64)
    assert e.value.code == "INVALID_CHECKPOINT"


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("m,k", [(1, 1), (3, 63), (7, 65), (9, 129), (33, 1025), (128, 4096)])
def test_activation_quantizer_bit_exact(ctx, oracle, bits, m, k):
    torch = pytest.importorskip("torch")
    x = (((np.arange(m * k) * 13 % 255) - 127.0) / 17.0).astype(np.float32)
    if m > 4:
        x = np.random.default_rng(m).standard_normal(m * k).astype(np.float32)
    g = (k + 63) // 64
    q = empty((m, g * 64), torch.int8)
    s = empty((m, g), torch.float32)
    ctx.act_quantize(dev(x), m, k, bits, q, s)
    wq, ws = oracle.act_quantize(x, m, k, bits)
    assert np.array_equal(host(ctx, q), wq)
    assert bits_equal(host(ctx, s), ws)


def test_activation_quantizer_boundaries(ctx, oracle):
    """int8.rs:774-798 tie/boundary values at several scales."""
    torch = pytest.importorskip("torch")
    values = [0.0, -0.0, np.finfo(np.float32).tiny, -np.finfo(np.float32).tiny]
    for i in range(-127, 127):
        h = np.float32(i + 0.5)
        values += [np.nextafter(h, np.float32(-np.inf)), h, np.nextafter(h, np.float32(np.inf))]
    values = np.array(values, np.float32)
    k = values.size
    x = np.stack([values * np.float32(s) for s in (1.0, 0.0037, 1e-30, 1e30)]).astype(np.float32)
    g = (k + 63) // 64
    q = empty((4, g * 64), torch.int8)
    s = empty((4, g), torch.float32)
    ctx.act_quantize(dev(x), 4, k, 8, q, s)
    wq, ws = oracle.act_quantize(x, 4, k, 8)
    assert np.array_equal(host(ctx, q), wq)
    assert bits_equal(host(ctx, s), ws)


@pytest.mark.parametrize("rows,k", [(1, 4), (9, 130), (64, 4096), (5, 72)])
def test_i8_row_quantizer_bit_exact(ctx, oracle, rows, k):
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(rows * k).standard_normal((rows, k)).astype(np.float32)
    x[0] = 0.0
    q = empty((rows, k), torch.int8)
    sc = empty(rows, torch.float32)
    su = empty(rows, torch.int32)
    ctx.i8_quantize_rows(dev(x), rows, k, q, sc, su)
    wq, ws, wsum = oracle.i8_quantize_rows(x, rows, k)
    assert np.array_equal(host(ctx, q), wq)
    assert bits_equal(host(ctx, sc), ws)
    assert np.array_equal(host(ctx, su), wsum)


def test_dequant_rows_gathers_and_rejects_bad_ids(ctx, oracle):
    torch = pytest.importorskip("torch")
    n, k = 40, 256
    raw = _bf16_weights(oracle, n, k, 5)
    packed = oracle.pack_g64(raw, n, k, 4)
    w = ctx.upload(packed, rocm.Q4_G64_F32, n, k)
    ids = np.array([3, 39, 0, 3, 17], np.int32)
    y = empty((ids.size, k), torch.float32)
    ctx.dequant_rows(w, dev(ids), ids.size, y, rocm.F32)
    full = oracle.unpack_g64(packed, 4).reshape(n, k)
    assert bits_equal(host(ctx, y), full[ids])
    yh = empty((ids.size, k), torch.float16)
    ctx.dequant_rows(w, dev(ids), ids.size, yh, rocm.F16)
    assert bits_equal(host(ctx, yh), full[ids].astype(np.float16))
    with pytest.raises(rocm.DzError) as e:
        ctx.dequant_rows(w, dev(np.array([1, 40], np.int32)), 2, y, rocm.F32)
    assert e.value.code == "INVALID_REQUEST"


# ---- per-row Q4 (webgpu/q4.rs) --------------------------------------------------------

@pytest.mark.parametrize("rows,k", [(7, 72), (4, 64), (33, 1000), (128, 4096), (1, 8)])
def test_q4_rows_quantizer_bit_exact(ctx, oracle, rows, k):
    """webgpu/q4.rs:48-73 from f16 weights: every code word, scale and sum."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(rows * k)
    w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
    w[0, :] = 0.0  # a zero row: scale 0, codes 0
    bits16 = oracle.f32_to_f16_bits(w)
    out = empty((rows * (k // 8) + 2 * rows,), torch.int32)
    ctx.q4_quantize_rows(dev(bits16.view(np.float16)), rocm.F16, rows, k, out)
    got = host(ctx, out).view(np.uint32)
    want = oracle.q4_quantize_rows(bits16, rows, k)
    assert bits_equal(got, want)
    # f32 input holding f16-representable values gives the same buffer
    out32 = empty((rows * (k // 8) + 2 * rows,), torch.int32)
    ctx.q4_quantize_rows(dev(oracle.f16_bits_to_f32(bits16)), rocm.F32, rows, k, out32)
    assert bits_equal(host(ctx, out32).view(np.uint32), want)


def test_q4_rows_quantizer_rejects_bad_input(ctx, oracle):
    torch = pytest.importorskip("torch")
    out = empty((64,), torch.int32)
    with pytest.raises(rocm.DzError) as e:
        ctx.q4_quantize_rows(dev(np.ones(12, np.float32)), rocm.F32, 1, 12, out)
    assert e.value.code == "INVALID_PARAMETERS"
    x = np.ones((2, 16), np.float32)
    x[1, 3] = np.nan
    with pytest.raises(rocm.DzError) as e:
        ctx.q4_quantize_rows(dev(x), rocm.F32, 2, 16, out)
    assert e.value.code == "INVALID_CHECKPOINT"
