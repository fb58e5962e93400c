"""Pins the CPU oracle before it is trusted as the checker.

Each test checks the oracle against something other than its own formula: the
reference's committed known-answer vectors, numpy/torch IEEE conversions,
integer brute force, float64 closed forms, or the reference tests' own
invariants (src/models/pplx_flash/int8.rs:591-962, packed.rs:121-208).
"""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def bf16_bytes(values):
    """The reference tests build BF16 by truncating f32 bits (packed.rs:135-138)."""
    v = np.asarray(values, np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def half_bf16(values, o):
    """half::bf16::from_f32 (round to nearest even), as int8.rs:692 uses."""
    return o.f32_to_bf16(np.asarray(values, np.float32))


# ---- IEEE conversions against independent libraries -------------------------

def test_f16_conversion_matches_numpy(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(100),
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-5),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.96e-08, 2.98e-08,
                  2.9802322e-08, 8.9406967e-08, np.inf, -np.inf, 1e-30], np.float32),
    ])
    got = oracle.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = oracle.f16_bits_to_f32(got)
    assert np.array_equal(back.view(np.uint32), want.view(np.float16).astype(np.float32).view(np.uint32))


def test_bf16_conversion_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    x = rng.standard_normal(50000).astype(np.float32) * np.float32(3)
    x[:4] = [0.0, -0.0, 3.4e38, 1e-40]
    got = oracle.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


# ---- golden vectors held by the reference --------------------------------------

def test_q4_golden_group(oracle):
    g = GOLDEN["q4_group"]
    raw = bf16_bytes(g["values"] * g["repeat"])
    packed = oracle.pack_g64(raw, 1, 64, 4)
    assert packed.tobytes() == bytes.fromhex(g["bytes_hex"]) * g["bytes_repeat"] + struct.pack("<f", g["scale"])
    z = GOLDEN["q4_zero_group"]
    packed = oracle.pack_g64(np.zeros(64, np.uint16), 1, 64, 4)
    assert packed.tobytes() == bytes.fromhex(z["bytes_hex"]) * z["bytes_repeat"] + struct.pack("<f", 2.0 ** z["scale_exponent"])


def test_q8_golden_group(oracle):
    g = GOLDEN["q8_group"]
    packed = oracle.pack_g64(bf16_bytes(g["values"] * g["repeat"]), 1, 64, 8)
    assert packed.tobytes() == bytes(g["bytes"] * g["bytes_repeat"]) + struct.pack("<f", g["scale"])
    packed = oracle.pack_g64(np.zeros(64, np.uint16), 1, 64, 8)
    assert packed.tobytes() == bytes(64) + struct.pack("<f", 2.0 ** -126)


def test_quantized_rows_ties_to_even_and_signed_zero(oracle):
    for case in GOLDEN["quantized_rows"]["cases"]:
        x = np.array(case["input"], np.float32)
        for div in (1.0, 16.0):
            v = x / np.float32(div)
            s = oracle.group_scale(v, case["bits"])
            codes = oracle.group_codes(v, s, case["bits"])
            deq = codes.astype(np.float32) * np.float32(s)
            assert np.array_equal(deq, np.array(case["expected"], np.float32) / np.float32(div))
        zeros = np.array([0.0, -0.0, 0.0, -0.0], np.float32)
        s = oracle.group_scale(zeros, case["bits"])
        deq = oracle.group_codes(zeros, s, case["bits"]).astype(np.float32) * np.float32(s)
        assert not np.signbit(deq).any() and (deq == 0).all()


# ---- packed.rs tests restated ------------------------------------------------

def test_grouped_codes_and_scale_match_native(oracle):
    """packed.rs:124-161: wire codes/scales == Matrix codes/scales; sizes."""
    values = np.array([(i - 32.0) / 16.0 if i < 64 else (i - 96.0) * 8.0 for i in range(128)], np.float32)
    raw = bf16_bytes(values)
    for bits, group in ((4, 36), (8, 68)):
        packed = oracle.pack_g64(raw, 1, 128, bits)
        assert packed.size == 2 * group
        codes, scales = oracle.weight_quantize(raw, 1, 128, bits)
        for g in range(2):
            blk = packed[g * group:(g + 1) * group]
            assert blk[-4:].tobytes() == struct.pack("<f", scales[0, g])
            if bits == 4:
                wire = np.stack([(blk[:32] & 15), (blk[:32] >> 4)], 1).reshape(-1).astype(np.int32) - 8
            else:
                wire = blk[:64].view(np.int8).astype(np.int32)
            assert np.array_equal(wire, codes[0, g * 64:(g + 1) * 64].astype(np.int32))
        assert oracle.unpack_g64(packed, bits).size == 128
        assert np.isfinite(oracle.project(packed, bits, 128, values, 1)[0])
    assert oracle.packed_size(1, 63, 4) == 0
    assert oracle.packed_size(1, 64, 2) == 0


def test_packed_projection_and_embeddings_match_native(oracle):
    """packed.rs:162-208: project == scalar Matrix::apply exactly; unpack == append."""
    n, k = 67, 128
    i = np.arange(n * k)
    values = np.where(i % 128 >= 64, 0.0, ((i * 23 % 127) - 63) / 32.0).astype(np.float32)
    raw = bf16_bytes(values)
    x = np.array([127.0 if j == 0 else ((j % 9) - 4.0) * 0.5 for j in range(k)], np.float32)
    for bits in (4, 8):
        packed = oracle.pack_g64(raw, n, k, bits)
        codes, scales = oracle.weight_quantize(raw, n, k, bits)
        reference = oracle.matrix_apply(x, 1, codes, scales, n, k, 8, fused=False)[0]
        assert np.array_equal(oracle.project(packed, bits, k, x, 3), reference[:3])
        assert np.array_equal(oracle.project(packed, bits, k, x, n), reference)
        row = oracle.packed_size(1, k, bits)
        decoded = oracle.unpack_g64(packed[5 * row:6 * row], bits)
        append = codes[5, :k].astype(np.float32) * np.repeat(scales[5], 64)[:k]
        assert np.array_equal(decoded, append)


def test_unpack_rejects_bad_scales_and_lengths(oracle):
    packed = oracle.pack_g64(bf16_bytes(np.ones(64)), 1, 64, 4)
    bad = packed.copy()
    bad[-4:] = np.frombuffer(struct.pack("<f", -1.0), np.uint8)
    with pytest.raises(oracle.OracleError):
        oracle.unpack_g64(bad, 4)
    with pytest.raises(oracle.OracleError):
        oracle.unpack_g64(packed[:-1], 4)
    with pytest.raises(oracle.OracleError):
        oracle.pack_g64(bf16_bytes([np.nan] + [0.0] * 63), 1, 64, 4)


# ---- int8.rs tests restated ---------------------------------------------------

def _independent_grouped(x, weights, m, k, n, ab, wb):
    """int8.rs:701-733: per-group codes by numpy rint in f32, dot in float64."""
    out = np.zeros((m, n))
    for r in range(m):
        for c in range(n):
            total = 0.0
            for g in range(0, k, 64):
                xv = x[r * k + g:r * k + min(g + 64, k)]
                wv = weights[c * k + g:c * k + min(g + 64, k)]

                def quant(v, bits):
                    lim = np.float32(7 if bits == 4 else 127)
                    s = max(np.float32(np.abs(v).max() / lim), np.float32(np.finfo(np.float32).tiny))
                    inv = np.float32(1) / np.float32(s)
                    return np.clip(np.rint(v * inv), -lim, lim).astype(np.int64), s

                a, sa = quant(xv, ab)
                b, sb = quant(wv, wb)
                total += float((a * b).sum()) * float(np.float32(sa * sb))
            out[r, c] = total
    return out


@pytest.mark.parametrize("wb,ab", GOLDEN["grouped_dot_shapes"]["bits"])
def test_q4_and_q8_match_independent_grouped_dots(oracle, wb, ab):
    tol = GOLDEN["grouped_dot_shapes"]["tolerance"]
    for m, k, n in GOLDEN["grouped_dot_shapes"]["mkn"]:
        i = np.arange(k * n)
        weights = half_bf16(((i * 37 % 257) - 128.0) / 31.0, oracle)
        wf = oracle.bf16_to_f32(weights)
        x = (((np.arange(m * k) * 13 % 255) - 127.0) / 17.0).astype(np.float32)
        expected = _independent_grouped(x, wf, m, k, n, ab, wb)
        codes, scales = oracle.weight_quantize(weights, n, k, wb)
        a = oracle.matrix_apply(x, m, codes, scales, n, k, ab, fused=True)
        b = oracle.matrix_apply(x, m, codes, scales, n, k, ab, fused=False)
        assert np.all(np.abs(a - expected) <= tol["abs"] + np.abs(expected) * tol["rel"])
        assert np.all(np.abs(b - expected) <= tol["abs"] + np.abs(expected) * tol["rel"])
        if m and oracle.has_avx2() and ab == 8:
            qx, sx = oracle.act_quantize(x, m, k, ab)
            data, ps = oracle.panel_pack(codes, scales, n, k, wb)
            for threads in (1, 3):
                avx = oracle.panel_apply_avx2(data, ps, n, k, wb, qx, sx, m, threads)
                assert np.array_equal(avx.view(np.uint32), a.view(np.uint32)), (m, k, n, threads)
        z = oracle.matrix_apply(np.zeros(m * k, np.float32), m, codes, scales, n, k, ab)
        assert (z == 0).all()


def test_activation_rounding_at_boundaries(oracle):
    """int8.rs:774-798 boundary set; codes checked against numpy's rint."""
    values = [0.0, -0.0, np.finfo(np.float32).tiny, -np.finfo(np.float32).tiny]
    for i in range(-127, 127):
        h = np.float32(i + 0.5)
        values += [np.nextafter(h, np.float32(-np.inf)), h, np.nextafter(h, np.float32(np.inf))]
    values = np.array(values, np.float32)
    for s in (1.0, 0.0037, float(np.finfo(np.float32).tiny), 1e30):
        scaled = (values * np.float32(s)).astype(np.float32)
        for n in (1, 7, 8, 9, 63, 64, 65, scaled.size):
            v = scaled[:n]
            got = oracle.group_codes(v, np.float32(s), 8)
            inv = np.float32(1) / np.float32(s)
            want = np.clip(np.rint(v * inv), -127, 127).astype(np.int8)
            assert np.array_equal(got, want), (s, n)
            assert (got != -128).all()
            gs = oracle.group_scale(v, 8)
            assert gs == max(np.float32(np.abs(v).max() / np.float32(127)), np.finfo(np.float32).tiny)


def test_integer_extrema_tails(oracle):
    """int8.rs:877-949: integer-valued extremes vs float64 closed form."""
    tol = GOLDEN["extrema_shapes"]["tolerance"]
    for m, k, n in GOLDEN["extrema_shapes"]["mkn"]:
        i = np.arange(k * n)
        w = np.select([i % 5 == 0, i % 5 == 1, i % 5 == 2], [-127.0, 127.0, 0.0], (i % 31) / 8.0).astype(np.float32)
        j = np.arange(m * k)
        x = np.select([j % 7 == 0, j % 7 == 1, j % 7 == 2], [127.0, -127.0, 0.0], (j % 13) - 6.0).astype(np.float32)
        raw = half_bf16(w, oracle)
        codes, scales = oracle.weight_quantize(raw, n, k, 8)
        got = oracle.matrix_apply(x, m, codes, scales, n, k, 8, fused=False)
        expected = _independent_grouped(x, oracle.bf16_to_f32(raw), m, k, n, 8, 8)
        assert np.all(np.abs(got - expected) <= tol["abs"] + np.abs(expected) * tol["rel"])
        fused = oracle.matrix_apply(x, m, codes, scales, n, k, 8, fused=True)
        assert np.all(np.abs(fused - got) <= 0.02 + np.abs(got) * 1e-6)


def test_invalid_weights_and_nonfinite_activations(oracle):
    """int8.rs:952-962."""
    with pytest.raises(oracle.OracleError):
        oracle.weight_quantize(np.array([0x7fc0], np.uint16), 1, 1, 8)
    codes, scales = oracle.weight_quantize(np.zeros(1, np.uint16), 1, 1, 8)
    assert np.isnan(oracle.matrix_apply(np.array([np.nan], np.float32), 1, codes, scales, 1, 1)[0, 0])
    assert oracle.matrix_apply(np.zeros(1, np.float32), 1, codes, scales, 1, 1)[0, 0] == 0.0


# ---- per-row int8 (webgpu/int8.rs, webgpu/q4.rs known answers) -----------------

@pytest.mark.parametrize("m,n,k", GOLDEN["q4_raw_check_shapes"]["mnk"])
def test_i8_rows_exact_raw_dots(oracle, m, n, k):
    """webgpu/q4.rs:476-501: integer-valued inputs quantize to themselves; raw
    i32 equals the independent signed dot."""
    a = np.array([127.0 if i % k == 0 else ((i * 17 % 255) - 127.0) for i in range(m * k)], np.float32)
    b = np.array([127.0 if i % k == 0 else ((i * 11 % 15) - 7.0) for i in range(n * k)], np.float32)
    qa, sa, suma = oracle.i8_quantize_rows(a, m, k)
    qb, sb, sumb = oracle.i8_quantize_rows(b, n, k)
    assert (sa == 1.0).all() and (sb == 1.0).all()
    assert np.array_equal(qa.astype(np.float32).reshape(-1), a)
    assert np.array_equal(suma, a.reshape(m, k).sum(1).astype(np.int32))
    raw, y = oracle.i8_gemm(qa, sa, m, qb, sb, n, k)
    want = a.reshape(m, k).astype(np.int64) @ b.reshape(n, k).astype(np.int64).T
    assert np.array_equal(raw, want.astype(np.int32))
    assert np.array_equal(y, raw.astype(np.float32))


def test_i8_quantizer_division_and_zero_rows(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((9, 130)).astype(np.float32)
    x[3] = 0.0
    q, s, sums = oracle.i8_quantize_rows(x, 9, 130)
    assert s[3] == 0.0 and (q[3] == 0).all() and sums[3] == 0
    scale = (np.abs(x).max(1) / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        want = np.clip(np.rint(x / scale[:, None]), -127, 127)
    want[3] = 0
    assert np.array_equal(q.astype(np.float32), want.astype(np.float32))
    assert np.array_equal(s, scale)
    r1, y1 = oracle.i8_gemm(q, s, 9, q, s, 9, 130, threads=1)
    r3, y3 = oracle.i8_gemm(q, s, 9, q, s, 9, 130, threads=3)
    assert np.array_equal(r1, r3) and np.array_equal(y1, y3)
    assert np.array_equal(y1, (r1.astype(np.float32) * s[:, None]).astype(np.float32) * s[None, :])


def test_i8_gemm_fused_silu_epilogue(oracle):
    """webgpu/int8.rs:226-230 fused mode: the gate and up products of the same
    codes (each pinned above) feed (gate / (1 + exp(-gate))) * up; checked in
    numpy f32 operations, against the f64 closed form, and at the extremes
    (exp overflow gives a signed zero, a large gate passes gate * up)."""
    rng = np.random.default_rng(11)
    m, n, k = 13, 9, 200
    qa, sa, _ = oracle.i8_quantize_rows(rng.standard_normal((m, k)).astype(np.float32), m, k)
    qg, sg, _ = oracle.i8_quantize_rows(rng.standard_normal((n, k)).astype(np.float32), n, k)
    qu, su, _ = oracle.i8_quantize_rows(rng.standard_normal((n, k)).astype(np.float32), n, k)
    sa = sa * np.float32(4.0)  # gates of a few units, both signs
    y = oracle.i8_gemm_fused(qa, sa, m, qg, sg, qu, su, n, k)
    _, gate = oracle.i8_gemm(qa, sa, m, qg, sg, n, k)
    _, up = oracle.i8_gemm(qa, sa, m, qu, su, n, k)
    e = np.exp(-gate.astype(np.float64)).astype(np.float32)
    want = ((gate / (np.float32(1.0) + e)).astype(np.float32) * up).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))
    g64 = gate.astype(np.float64)
    closed = g64 / (1.0 + np.exp(-g64)) * up.astype(np.float64)
    assert np.allclose(y, closed, rtol=1e-6, atol=1e-30)
    assert np.abs(gate).max() > 4.0 and (gate < 0).any() and (gate > 0).any()
    # extremes: one-element products with scales chosen to hit exp overflow
    one = np.ones((1, 1), np.int8)
    big = oracle.i8_gemm_fused(one, np.float32([1.0]), 1, one, np.float32([-200.0]), one, np.float32([3.0]), 1, 1)
    assert big[0, 0] == 0.0 and np.signbit(big[0, 0])  # -200 / inf * 3 = -0
    pos = oracle.i8_gemm_fused(one, np.float32([1.0]), 1, one, np.float32([200.0]), one, np.float32([3.0]), 1, 1)
    assert pos[0, 0] == np.float32(600.0)


# ---- g32/f16 layout (D1) --------------------------------------------------------

def test_g32_f16_layout_invariants(oracle):
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    w[2, :32] = 0.0
    w[3, 32:64] = 0.35
    packed = oracle.pack_g32_f16(w, 8, 256)
    assert packed.size == 8 * 8 * 18
    groups = packed.reshape(-1, 18)
    codes = np.stack([groups[:, :16] & 15, groups[:, :16] >> 4], 2).reshape(-1, 32).astype(np.int32) - 8
    assert (np.abs(codes) <= 7).all()
    scales = groups[:, 16:18].copy().view(np.float16).astype(np.float32).reshape(-1)
    deq = oracle.unpack_g32_f16(packed).reshape(-1, 32)
    assert np.array_equal(deq, codes.astype(np.float32) * scales[:, None])
    # an all-zero run keeps the smallest f16 subnormal and decodes to zeros
    assert scales[2 * 8] == np.float32(2.0 ** -24) and (deq[2 * 8] == 0).all()
    # a constant run is exact: code 7 with scale v/7 rounded to f16
    assert (codes[3 * 8 + 1] == 7).all()
    assert np.allclose(deq[3 * 8 + 1], 0.35, rtol=2 ** -10)
    # per-group error bound: |w - deq| <= scale/2 (+ the f16 scale rounding)
    err = np.abs(w.reshape(-1, 32) - deq)
    assert (err <= scales[:, None] * 0.5 + np.abs(w.reshape(-1, 32)) * 2 ** -10 + 1e-12).all()


# ---- closed forms and epilogues -------------------------------------------------

def test_w4a16_closed_form_matches_numpy(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    xh = oracle.f32_to_f16_bits(x)
    w = rng.standard_normal((5, 96)).astype(np.float32)
    got = oracle.w4a16(xh, 3, 96, w, 5)
    want = oracle.f16_bits_to_f32(xh).astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(got, want, rtol=1e-13, atol=1e-13)


def test_epilogues_match_float64(oracle):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    ln = (xd - mu) / np.sqrt(((xd - mu) ** 2).mean(1, keepdims=True) + 1e-12) * w + b
    assert np.allclose(oracle.layernorm(x, w, b, 1e-12), ln, atol=2e-5)
    g = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xd.reshape(-1)]).reshape(x.shape)
    assert np.allclose(oracle.gelu(x), g, atol=1e-6)
    rms = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * (1 + w)
    assert np.allclose(oracle.rmsnorm(x, w, 1e-6), rms, atol=2e-5)
    up = rng.standard_normal(x.shape).astype(np.float32)
    assert np.allclose(oracle.silu_mul(x, up), xd / (1 + np.exp(-xd)) * up, atol=1e-5)
    sm = np.exp(xd[0] - xd[0].max())
    assert np.allclose(oracle.softmax(x[0]), sm / sm.sum(), atol=1e-7)
    assert np.allclose(oracle.mean_rows(x), xd.mean(0), atol=1e-6)


def test_attention_closed_form(oracle):
    rng = np.random.default_rng(8)
    seq, heads, dh = 7, 2, 8
    q, k, v = (rng.standard_normal((seq, heads * dh)).astype(np.float32) for _ in range(3))
    out = oracle.attention(q, k, v, heads, 1 / math.sqrt(dh))
    for h in range(heads):
        sl = slice(h * dh, (h + 1) * dh)
        s = q[:, sl].astype(np.float64) @ k[:, sl].astype(np.float64).T / math.sqrt(dh)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        assert np.allclose(out[:, sl], p @ v[:, sl].astype(np.float64), atol=1e-6)


def test_silu_requant_is_unfused_composition(oracle):
    """grouped_q4.rs:27-41 + the a4 quantizer per 64-column block."""
    rng = np.random.default_rng(9)
    gate = rng.standard_normal((3, 128)).astype(np.float32)
    up = rng.standard_normal((3, 128)).astype(np.float32)
    q, s = oracle.silu_requant(gate, up)
    v = oracle.silu_mul(gate, up)
    q2, s2 = oracle.act_quantize(v, 3, 128, 8)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)
    assert np.allclose(q.astype(np.float64) * np.repeat(s, 64, 1), v, atol=np.repeat(s, 64, 1) * 0.5 + 1e-12)


# ---- per-row Q4 (webgpu/q4.rs) ----------------------------------------------------------

@pytest.mark.parametrize("m,n,k", GOLDEN["q4_raw_check_shapes"]["mnk"])
def test_q4_rows_known_answer(oracle, m, n, k):
    """webgpu/q4.rs:107-142: integer weights in [-7, 7] with a 7 in every row
    quantize to themselves (scale exactly 1.0, sums = row sums) and the raw
    int32 dots against int8-quantized integer activations are exact."""
    i = np.arange(m * k)
    a = np.where(i % k == 0, 127.0, ((i * 17 % 255) - 127.0)).astype(np.float32)
    j = np.arange(n * k)
    b = np.where(j % k == 0, 7.0, ((j * 11 % 15) - 7.0)).astype(np.float32)
    words = oracle.q4_quantize_rows(oracle.f32_to_f16_bits(b), n, k)
    codes, scales, sums = oracle.q4_rows_split(words, n, k)
    assert np.array_equal(codes.astype(np.float32), b.reshape(n, k))
    assert np.array_equal(scales.view(np.uint32), np.full(n, np.float32(1.0)).view(np.uint32))
    assert np.array_equal(sums, b.reshape(n, k).sum(1).astype(np.int32))
    qa, sa, _ = oracle.i8_quantize_rows(a, m, k)
    raw, _ = oracle.i8_gemm(qa, sa, m, codes, scales, n, k, scaled=False)
    expected = a.reshape(m, k).astype(np.int64) @ b.reshape(n, k).astype(np.int64).T
    assert np.array_equal(raw.astype(np.int64), expected)


def test_q4_rows_rounding_and_zero_rows(oracle):
    """x/scale rounded half to even (q4.rs:60 even), clamped to +-7; an all-zero
    row has scale 0 and codes 0 (stored as 8)."""
    k = 16
    row0 = np.array([7, 3.5, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 6.5, -6.5, 0, 1, 2, 3, 4, 5], np.float32)
    row1 = np.zeros(k, np.float32)
    words = oracle.q4_quantize_rows(oracle.f32_to_f16_bits(np.concatenate([row0, row1])), 2, k)
    codes, scales, sums = oracle.q4_rows_split(words, 2, k)
    assert codes[0].tolist() == [7, 4, 2, -2, 0, 0, 2, -2, 6, -6, 0, 1, 2, 3, 4, 5]
    assert scales[1] == 0.0 and not codes[1].any() and sums[1] == 0
    assert words[2] == 0x88888888 and words[3] == 0x88888888
    with pytest.raises(oracle.OracleError):
        oracle.q4_quantize_rows(np.zeros(12, np.uint16), 1, 12)


def test_readout_rms_is_the_sequential_sum(oracle):
    """The oracle's RMSNorm adds the squares in row order (the reference's
    iterator sum): on a row where order matters, a pairwise sum differs."""
    x = np.zeros((1, 4096), np.float32)
    x[0, 0] = 4096.0
    x[0, 1:] = 0.5
    got = oracle.rmsnorm(x, np.zeros(4096, np.float32), 1e-6)
    seq = np.float32(0)
    for v in x[0]:
        seq = np.float32(seq + np.float32(v * v))
    scale = np.float32(1) / np.sqrt(np.float32(seq / np.float32(4096) + np.float32(1e-6)), dtype=np.float32)
    assert np.array_equal(got[0].view(np.uint32), (x[0] * scale).astype(np.float32).view(np.uint32))
    pair = np.float32(np.sum(x[0].astype(np.float32) ** 2, dtype=np.float32))
    assert pair != seq


# ---- Pplx decoder layer ops (backbone.rs, cpu.rs), pinned by properties ----

def _silu64(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def test_conv_silu_taps_are_causal_and_in_order(oracle):
    """A one-hot tap shifts the sequence: tap 3 is the current token, tap 0
    the token three back, and rows before the start are zero (backbone.rs:271-283)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((9, 24)).astype(np.float32)
    for tap in range(4):
        w = np.zeros((4, 24), np.float32)
        w[tap] = 1.0
        got = oracle.conv_silu(x, w)
        shifted = np.zeros_like(x)
        lag = 3 - tap
        shifted[lag:] = x[:9 - lag]
        assert np.allclose(got, _silu64(shifted), rtol=1e-6, atol=1e-7), tap
    # linear in the taps before the activation
    w = rng.standard_normal((4, 24)).astype(np.float32)
    pre = sum(np.pad(x, ((3 - t, 0), (0, 0)))[:9] * w[t] for t in range(4))
    assert np.allclose(oracle.conv_silu(x, w), _silu64(pre), rtol=1e-5, atol=1e-6)


def _delta_inputs(n, lh, lk, ld, keys, values, queries=None, a=None, b=None, decay=None, dt=None):
    """conv rows holding q heads, k heads, v heads; keys/queries per (t, kh)."""
    lkv = lk * ld
    conv = np.zeros((n, 2 * lkv + lh * ld), np.float32)
    for t in range(n):
        for kh in range(lk):
            conv[t, lkv + kh * ld:lkv + (kh + 1) * ld] = keys[t][kh]
            conv[t, kh * ld:(kh + 1) * ld] = (queries if queries is not None else keys)[t][kh]
        for h in range(lh):
            conv[t, 2 * lkv + h * ld:2 * lkv + (h + 1) * ld] = values[t][h]
    a = np.zeros((n, lh), np.float32) if a is None else a
    b = np.full((n, lh), 40.0, np.float32) if b is None else b     # beta = sigmoid(40) = 1 in f32
    decay = np.zeros(lh, np.float32) if decay is None else decay    # g = exp(-0 * softplus) = 1
    dt = np.zeros(lh, np.float32) if dt is None else dt
    return conv, a, b, decay, dt


def test_delta_scan_reads_back_what_it_wrote(oracle):
    """beta = 1, g = 1, orthonormal keys: the state stores k v^T, so a query
    equal to a key written earlier (or now) returns that value / sqrt(ld),
    and an unwritten key returns 0 (the delta rule with the readout after
    the update, backbone.rs:382-407). Heads 2h and 2h+1 share key head h."""
    lh, lk, ld, n = 4, 2, 16, 6
    rng = np.random.default_rng(1)
    e = np.eye(ld, dtype=np.float32)
    keys = [[e[(3 * t + kh) % ld] * (1.0 + t) for kh in range(lk)] for t in range(n)]  # scale is normalized away
    values = [[rng.standard_normal(ld).astype(np.float32) for _ in range(lh)] for _ in range(n)]
    queries = [[e[(3 * max(t - 2, 0) + kh) % ld] for kh in range(lk)] for t in range(n)]
    conv, a, b, decay, dt = _delta_inputs(n, lh, lk, ld, keys, values, queries)
    out = oracle.delta_scan(conv, lh, lk, ld, a, b, decay, dt)
    for h in range(lh):
        for t in range(n):
            want = values[max(t - 2, 0)][h] / np.sqrt(ld)
            assert np.allclose(out[h, t], want, rtol=1e-5, atol=1e-6), (h, t)
    # a query no key has touched reads zero
    queries = [[e[2 + 3 * kh] for kh in range(lk)] for _ in range(n)]  # keys 3t + kh never hit 2 or 5
    conv, a, b, decay, dt = _delta_inputs(n, lh, lk, ld, keys, values, queries)
    assert np.abs(oracle.delta_scan(conv, lh, lk, ld, a, b, decay, dt)).max() == 0.0


def test_delta_scan_decays_and_overwrites(oracle):
    """g = exp(-decay * softplus(a + dt)) scales the old state before each
    step; beta < 1 writes beta * (v - old read): writing v1 then v2 to one key
    leaves beta*v2 + beta*(1 - beta)*g*v1 (the erase-then-write of the delta rule)."""
    lh, lk, ld = 2, 1, 8
    e = np.eye(ld, dtype=np.float32)
    v1, v2 = np.arange(1, ld + 1, dtype=np.float32), np.linspace(-1, 1, ld).astype(np.float32)
    keys = [[e[0]], [e[0]]]
    values = [[v1, v1], [v2, v2]]
    a = np.full((2, lh), 0.3, np.float32)
    dt = np.array([0.2, -0.4], np.float32)
    decay = np.array([0.5, 1.5], np.float32)
    b = np.full((2, lh), 0.25, np.float32)
    conv, a, b, decay, dt = _delta_inputs(2, lh, lk, ld, keys, values, None, a, b, decay, dt)
    out = oracle.delta_scan(conv, lh, lk, ld, a, b, decay, dt)
    beta = 1.0 / (1.0 + np.exp(-0.25))
    for h in range(lh):
        g = np.exp(-decay[h] * np.log1p(np.exp(0.3 + dt[h])))
        first = beta * v1                      # written at t = 0 (state starts at zero)
        second = g * first + beta * (v2 - g * first)
        assert np.allclose(out[h, 0], first / np.sqrt(ld), rtol=1e-5, atol=1e-6)
        assert np.allclose(out[h, 1], second / np.sqrt(ld), rtol=1e-5, atol=1e-6), h


def test_delta_gate_and_attention_gate_closed_forms(oracle):
    rng = np.random.default_rng(2)
    lh, ld, n = 3, 16, 5
    heads = rng.standard_normal((lh, n, ld)).astype(np.float32) * 3
    norm = rng.standard_normal(ld).astype(np.float32)
    z = rng.standard_normal((n, lh * ld)).astype(np.float32)
    got = oracle.delta_gate(heads, norm, z)
    h64 = heads.astype(np.float64)
    scale = 1.0 / np.sqrt((h64 ** 2).mean(axis=2, keepdims=True) + 1e-6)
    want = (h64 * scale * norm).transpose(1, 0, 2).reshape(n, lh * ld) * _silu64(z)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    got = oracle.attention_gate(heads, z)
    want = h64.transpose(1, 0, 2).reshape(n, lh * ld) / (1.0 + np.exp(-z.astype(np.float64)))
    assert np.allclose(got, want, rtol=1e-6, atol=1e-7)


def test_rope_rotates_the_first_64_dims_by_position(oracle):
    """Pairs (i, i + 32) rotate by pos * freq[i]; dims from 64 on and position
    0 are unchanged; the dot of two rotated vectors depends only on the
    position difference (backbone.rs:415-428, :227-229)."""
    rng = np.random.default_rng(3)
    freq = oracle.rope_freq()
    assert freq[0] == 1.0 and abs(freq[31] - 1e7 ** (-62 / 64)) < 1e-9
    q = rng.standard_normal((1, 256)).astype(np.float32)
    k = rng.standard_normal((1, 256)).astype(np.float32)
    assert np.array_equal(oracle.rope(q, 1, 256, [0], freq), q)
    r = oracle.rope(q, 1, 256, [7], freq)
    assert np.array_equal(r[:, 64:], q[:, 64:])
    pairs = lambda x: x[0, :32].astype(np.float64) ** 2 + x[0, 32:64].astype(np.float64) ** 2
    assert np.allclose(pairs(r), pairs(q), rtol=1e-5)
    d1 = float((oracle.rope(q, 1, 256, [9], freq) @ oracle.rope(k, 1, 256, [4], freq).T)[0, 0])
    d2 = float((oracle.rope(q, 1, 256, [5], freq) @ k.T)[0, 0])
    assert abs(d1 - d2) < 1e-3 * (1 + abs(d2))


def test_attention_gqa_maps_heads_to_kv_heads(oracle):
    """Head h attends with key/value head h / (ah/akv); zero queries give the
    mean of the values; permuting the keys with their values changes nothing."""
    rng = np.random.default_rng(4)
    ah, akv, ad, nq, nk = 4, 2, 8, 3, 5
    q = rng.standard_normal((nq, ah * ad)).astype(np.float32)
    k = rng.standard_normal((nk, akv * ad)).astype(np.float32)
    v = rng.standard_normal((nk, akv * ad)).astype(np.float32)
    out = oracle.attention_gqa(q, k, v, ah, akv, ad, 0.5)
    for h in range(ah):
        kh = h // (ah // akv)
        qh, kk, vv = (q[:, h * ad:(h + 1) * ad].astype(np.float64), k[:, kh * ad:(kh + 1) * ad].astype(np.float64),
                      v[:, kh * ad:(kh + 1) * ad].astype(np.float64))
        s = qh @ kk.T * 0.5
        p = np.exp(s - s.max(axis=1, keepdims=True))
        want = (p / p.sum(axis=1, keepdims=True)) @ vv
        assert np.allclose(out[h], want, rtol=1e-5, atol=1e-6), h
    zero = oracle.attention_gqa(np.zeros_like(q), k, v, ah, akv, ad, 0.5)
    assert np.allclose(zero[0, 0], v[:, :ad].mean(axis=0), rtol=1e-5, atol=1e-6)
    perm = rng.permutation(nk)
    assert np.allclose(oracle.attention_gqa(q, k[perm], v[perm], ah, akv, ad, 0.5), out, rtol=1e-5, atol=1e-6)


# ---- fitted Q4 weights: quantization.rs fits and the affine fold -------------

def _fit_modes(oracle):
    return [False, True] if oracle.has_avx2() else [False]


def test_affine_fit_preserves_constants_and_offset_grids(oracle):
    """quantization.rs:306-325: constant groups reconstruct exactly, and values
    on a 16-level grid with an offset reconstruct to 1e-5."""
    for avx2 in _fit_modes(oracle):
        for n in (1, 7, 16, 63, 64):
            for v in (0.0, -3.25, 12.0):
                codes, s, b = oracle.fit_affine(np.full(n, v, np.float32), avx2)
                assert (codes.astype(np.float32) * s + b == np.float32(v)).all(), (avx2, n, v)
            values = np.array([4.0 + (i * 15 // max(n - 1, 1)) * 0.25 for i in range(n)], np.float32)
            codes, s, b = oracle.fit_affine(values, avx2)
            assert s > 0
            assert (codes >= -8).all() and (codes <= 7).all()
            assert np.all(np.abs(values - (codes.astype(np.float32) * s + b)) < 1e-5), (avx2, n)


def test_mse_fit_reduces_error_and_handles_tails(oracle):
    """quantization.rs:327-356: the fit never reconstructs worse than the
    symmetric Q4 quantizer (int8.rs group_scale_bits/pack_bits), keeps codes in
    [-8, 7] and maps a zero group to zero codes and a finite scale."""
    for avx2 in _fit_modes(oracle):
        for n in (1, 7, 8, 31, 63, 64):
            for seed in range(32):
                i = np.arange(n)
                values = (((i * 137 + seed * 19) % 101) - 50.0).astype(np.float32)
                values[0] *= np.float32(3.7)
                s = oracle.group_scale(values, 4)
                base = oracle.group_codes(values, s, 4)
                codes, fit = oracle.fit_mse(values, avx2)

                def error(q, scale):
                    return float(((values.astype(np.float64) - q.astype(np.float64) * float(scale)) ** 2).sum())

                assert error(codes, fit) <= error(base, s) + 1e-5, (avx2, n, seed)
                assert (codes >= -8).all() and (codes <= 7).all()
        codes, s = oracle.fit_mse(np.zeros(64, np.float32), avx2)
        assert np.isfinite(s) and (codes == 0).all()


def _dequantized_dots(codes, scales, offsets, q, sx, m, n, k):
    """f64 sum over k of (code * scale + offset) * q * sx, int8.rs:612-637."""
    g = (k + 63) // 64
    w = (codes.astype(np.float64).reshape(n, g, 64) * scales.astype(np.float64)[:, :, None]
         + offsets.astype(np.float64)[:, :, None])
    a = q.astype(np.float64).reshape(m, g, 64) * sx.astype(np.float64)[:, :, None]
    wk = w.reshape(n, g * 64)[:, :k]
    ak = a.reshape(m, g * 64)[:, :k]
    return ak @ wk.T


def test_affine_offsets_match_independent_dequantized_dots(oracle):
    """int8.rs:591-642: k = 65, n = 9; both fold orders within
    1e-3 + |expected| * 4e-6 of the float64 dequantized product, and the fused
    order bit-for-bit equal to the AVX2 panel kernel with its offset term."""
    k, n = 65, 9
    i = np.arange(k * n)
    vals = np.where(i // k % 3 == 0, (i // k) + 3.0, (((i * 31) % 97) - 48.0) / 17.0 + 9.0)
    bf16 = half_bf16(vals, oracle)
    for avx2 in _fit_modes(oracle):
        codes, scales, offsets = oracle.weight_quantize_fitted(bf16, n, k, "affine", avx2)
        assert (scales > 0).all() and np.isfinite(offsets).all()
        assert (codes.reshape(n, 2, 64)[:, 1, 1:] == 0).all()  # the group tail past k
        for m in (1, 15, 16, 17):
            x = ((((np.arange(m * k) * 13) % 255) - 127.0) / 17.0 + 3.0).astype(np.float32)
            q, sx = oracle.act_quantize(x, m, k)
            expected = _dequantized_dots(codes, scales, offsets, q, sx, m, n, k)
            for fused in (True, False):
                got = oracle.grouped_gemm_affine(q, sx, m, codes, scales, offsets, n, k, fused)
                assert np.all(np.abs(got - expected) < 1e-3 + np.abs(expected) * 4e-6), (avx2, m, fused)
            # the offset term is live: without it the product is far off
            plain = oracle.grouped_gemm(q, sx, m, codes, scales, n, k)
            assert np.abs(plain - expected).max() > 1.0
            if oracle.has_avx2():
                data, ps = oracle.panel_pack(codes, scales, n, k, 4)
                _, po = oracle.panel_pack(codes, offsets, n, k, 4)
                fused = oracle.grouped_gemm_affine(q, sx, m, codes, scales, offsets, n, k, True)
                for threads in (1, 3):
                    avx = oracle.panel_apply_avx2(data, ps, n, k, 4, q, sx, m, threads, poffsets=po)
                    assert np.array_equal(avx.view(np.uint32), fused.view(np.uint32)), (m, threads)


def test_fitted_signed_scales_and_full_code_range(oracle):
    """int8.rs:645-676: the MSE fit gives negative scales and -8 codes; the
    scalar and fused folds agree within 1e-4 + |a| * 2e-6; the fused fold is
    bit-for-bit the AVX2 panel kernel and within tolerance of float64."""
    for k, n in ((65, 9), (128, 33)):
        i = np.arange(k * n)
        bf16 = half_bf16((((i * 37) % 251) - 125.0) / 31.0, oracle)
        codes, scales, offsets = oracle.weight_quantize_fitted(bf16, n, k, "mse", True)
        assert (scales < 0).any()
        assert (codes == -8).any()
        assert (offsets == 0).all()
        for m in (1, 15, 16, 17):
            x = ((((np.arange(m * k) * 13) % 255) - 127.0) / 17.0).astype(np.float32)
            q, sx = oracle.act_quantize(x, m, k)
            scalar = oracle.grouped_gemm(q, sx, m, codes, scales, n, k, fused=False)
            simd = oracle.grouped_gemm(q, sx, m, codes, scales, n, k, fused=True)
            assert np.all(np.abs(scalar - simd) < 1e-4 + np.abs(scalar) * 2e-6), (k, m)
            expected = _dequantized_dots(codes, scales, offsets, q, sx, m, n, k)
            assert np.all(np.abs(simd - expected) < 1e-3 + np.abs(expected) * 4e-6)
            if oracle.has_avx2():
                data, ps = oracle.panel_pack(codes, scales, n, k, 4)
                avx = oracle.panel_apply_avx2(data, ps, n, k, 4, q, sx, m, 1)
                assert np.array_equal(avx.view(np.uint32), simd.view(np.uint32)), (k, m)


def test_fitted_weights_reject_nonfinite_and_wire_pack_round_trips(oracle):
    """int8.rs:98-101 refuses non-finite weights; the wire packing of fitted
    codes decodes (packed.rs:59-73) to code * scale, signed scales included."""
    with pytest.raises(oracle.OracleError):
        oracle.weight_quantize_fitted(np.array([0x7f80] + [0] * 63, np.uint16), 1, 64, "mse")
    rng = np.random.default_rng(3)
    n, k = 5, 128
    codes = rng.integers(-8, 8, (n, k)).astype(np.int8)
    scales = (rng.standard_normal((n, k // 64)) * 0.1).astype(np.float32)
    wire = oracle.pack_wire_codes(codes, scales, n, k)
    assert wire.size == n * (k // 64) * 36
    # packed.rs's decoder takes positive scales only: decode the same codes
    # with |scale| and check the signed scale bytes separately
    positive = oracle.pack_wire_codes(codes, np.abs(scales), n, k)
    got = oracle.unpack_g64(positive, 4).reshape(n, k)
    want = codes.astype(np.float32).reshape(n, 2, 64) * np.abs(scales)[:, :, None]
    assert np.array_equal(got.view(np.uint32), want.reshape(n, k).view(np.uint32))
    runs = wire.reshape(n, k // 64, 36)
    assert np.array_equal(runs[..., :32], positive.reshape(n, k // 64, 36)[..., :32])
    assert np.array_equal(runs[..., 32:].copy().view("<f4")[..., 0], scales)


def test_nf4_table_is_the_normal_quantile_codebook(oracle):
    """quantization.rs:3-20 against its definition (QLoRA's NF4): 8 positive
    and 7 negative quantiles of N(0, 1) at evenly spaced probabilities from
    0.9677083 to 1/2, an exact zero, normalized to [-1, 1]."""
    from scipy.stats import norm
    top = 0.9677083
    positive = norm.ppf(np.linspace(top, 0.5, 9)[:-1])
    negative = -norm.ppf(np.linspace(top, 0.5, 8)[:-1])
    want = np.sort(np.concatenate([positive, [0.0], negative]))
    want /= np.abs(want).max()
    table = oracle.nf4_table()
    assert np.all(np.diff(table) > 0)
    assert table[0] == -1.0 and table[7] == 0.0 and table[15] == 1.0
    assert np.abs(table.astype(np.float64) - want).max() < 2e-7


def test_nf4_fit_round_trips_codebook_and_zero(oracle):
    """quantization.rs:358-369, and the fit never reconstructs worse than its
    start at scale 1 (the codebook spread to the largest magnitude)."""
    table = oracle.nf4_table()
    codes, s = oracle.fit_nf4(table)
    assert np.all(np.abs(table[codes.astype(np.int64) + 8] * s - table) < 1e-6)
    codes, s = oracle.fit_nf4(np.zeros(16, np.float32))
    assert np.isfinite(s) and (table[codes.astype(np.int64) + 8] == 0).all()
    rng = np.random.default_rng(5)
    for n in (1, 7, 64):
        x = rng.standard_normal(n).astype(np.float32)
        codes, s = oracle.fit_nf4(x)
        m = np.abs(x).max()
        mids = (table[:-1] + table[1:]) / 2
        first = table[np.searchsorted(mids, x / m, side="left")] * m
        err = lambda y: float(((x.astype(np.float64) - y) ** 2).sum())
        assert err(table[codes.astype(np.int64) + 8].astype(np.float64) * s) <= err(first) * (1 + 1e-5) + 1e-12


def test_affine_embedding_rows_reconstruct(oracle):
    """quantized_rows.rs:121-137: rows of i / 64 through the affine fit decode
    within 0.04, each group's offset added after the scale."""
    values = (np.arange(256) / 64.0).astype(np.float32)
    bf16 = half_bf16(values, oracle)
    codes, scales, offsets = oracle.weight_quantize_fitted(bf16, 2, 128, "affine", avx2=False)
    rows = oracle.rows_decode(codes, scales, offsets, False, 2, 128)
    assert np.all(np.abs(rows - values.reshape(2, 128)) < 0.04)
    # the offset term is what centres the rows: without it they are far off
    assert np.abs(oracle.rows_decode(codes, scales, None, False, 2, 128) - values.reshape(2, 128)).max() > 0.5


def test_fitted_embedding_rows_decode_group_by_group(oracle):
    """quantized_rows.rs:139-175: NF4 and MSE rows decode per group as the
    group fit's value_code * scale, and reconstruct the inputs closely."""
    i = np.arange(256)
    bf16 = half_bf16((((i * 37) % 101) - 50.0) / 37.0, oracle)
    x = oracle.bf16_to_f32(bf16).reshape(2, 128)
    table = oracle.nf4_table()
    for mode in ("nf4", "mse"):
        codes, scales, offsets = oracle.weight_quantize_fitted(bf16, 2, 128, mode, avx2=False)
        rows = oracle.rows_decode(codes, scales, None, mode == "nf4", 2, 128)
        for r in range(2):
            for g in range(2):
                v = x[r, g * 64:(g + 1) * 64]
                c, s = oracle.fit_nf4(v) if mode == "nf4" else oracle.fit_mse(v, avx2=False)
                vc = table[c.astype(np.int64) + 8] if mode == "nf4" else c.astype(np.float32)
                assert np.array_equal(rows[r, g * 64:(g + 1) * 64], vc * s)
        assert np.abs(rows - x).max() < 0.2 * np.abs(x).max()
