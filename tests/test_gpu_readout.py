"""The decision readout (pplx_flash/mod.rs:149-185 logits): the zero-centred
RMSNorm of the selected hidden rows, summed in row order as cpu::rms is
(cpu.rs:310-333), then packed::project (packed.rs:75-119). Bit-exact against
the oracle's restatement of both; the encoder's readout equals dz_readout of
its own hidden rows."""
import struct

import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, cosine, dev, empty, host

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _weight(ctx, oracle, n, k, bits, seed):
    rng = np.random.default_rng(seed)
    raw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    packed = oracle.pack_g64(raw, n, k, bits)
    w = ctx.upload(packed, rocm.Q4_G64_F32 if bits == 4 else rocm.Q8_G64_F32, n, k)
    return packed, w


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,d,n", [(1, 2560, 255), (3, 1024, 255), (20, 512, 40), (1, 64, 7), (17, 192, 255)])
def test_readout_is_rms_then_project_bit_for_bit(ctx, oracle, bits, rows, d, n):
    torch = pytest.importorskip("torch")
    packed, w = _weight(ctx, oracle, n, d, bits, rows * 7 + d + n)
    rng = np.random.default_rng(rows + d)
    hidden = (rng.standard_normal((rows, d)) * rng.uniform(0.1, 30, (rows, 1))).astype(np.float32)
    norm = (rng.standard_normal(d) * 0.1).astype(np.float32)
    logits = empty((rows, n), torch.float32)
    ctx.readout(w, dev(norm), dev(hidden), rows, EPS, logits)
    got = host(ctx, logits)
    x = oracle.rmsnorm(hidden, norm, EPS, zero_centered=True)
    for r in range(rows):
        want = oracle.project(packed, bits, d, x[r], n)
        assert bits_equal(got[r], want), (r, float(np.abs(got[r] - want).max()))


def test_readout_rejects_nonfinite_activations_and_logits(ctx, oracle):
    torch = pytest.importorskip("torch")
    _, w = _weight(ctx, oracle, 16, 128, 4, 5)
    hidden = np.ones((2, 128), np.float32)
    hidden[1, 3] = np.inf
    logits = empty((2, 16), torch.float32)
    with pytest.raises(rocm.DzError) as e:
        ctx.readout(w, dev(np.zeros(128, np.float32)), dev(hidden), 2, EPS, logits)
    assert e.value.code == "INFERENCE_FAILED" and "nonfinite readout activation" in str(e.value)
    # finite activations whose logit overflows: codes 7 everywhere, scale 3e38
    group = bytes([0xFF]) * 32 + struct.pack("<f", 3e38)
    big = ctx.upload(np.frombuffer(group * 2, np.uint8), rocm.Q4_G64_F32, 1, 128)
    one_hot = np.zeros((1, 128), np.float32)
    one_hot[0, 0] = 1.0
    with pytest.raises(rocm.DzError) as e:
        ctx.readout(big, dev(np.zeros(128, np.float32)), dev(one_hot), 1, EPS, empty((1, 1), torch.float32))
    assert e.value.code == "INFERENCE_FAILED" and "non-finite packed logits" in str(e.value)
    w32 = ctx.quantize(dev(np.ones((16, 64), np.float32)), rocm.F32, 16, 64, 4, 32)
    with pytest.raises(rocm.DzError) as e:
        ctx.readout(w32, dev(np.zeros(64, np.float32)), dev(np.ones((1, 64), np.float32)), 1, EPS,
                    empty((1, 16), torch.float32))
    assert e.value.code == "INVALID_PARAMETERS"


def test_encoder_readout_is_the_readout_of_its_hidden_rows(ctx, oracle):
    torch = pytest.importorskip("torch")
    cfg = rocm.EncoderConfig(layers=2, hidden=256, heads=4, head_dim=64, ffn=512, vocab=1000, ln_eps=1e-5)
    enc = ctx.encoder_random(cfg, 5)
    seq = 100
    ids = np.random.default_rng(9).integers(0, cfg.vocab, seq).astype(np.int32)
    rows = enc.read_rows(ids)
    hidden = empty((seq, cfg.hidden), torch.float32)
    enc.hidden_rows(rows, seq, hidden)
    h = host(ctx, hidden)
    # the hidden rows are what the mean pool reduces
    pooled = empty((1, cfg.hidden), torch.float32)
    enc.forward_rows(rows, 1, seq, pooled)
    assert cosine(h.mean(axis=0), host(ctx, pooled)[0]) >= 0.99999
    assert np.abs(h.mean(axis=0) - host(ctx, pooled)[0]).max() <= 1e-4
    markers = np.array([5, 50, 99, 0], np.int32)
    got = enc.readout_rows(rows, seq, markers)
    assert got.shape == (4, rocm.Encoder.READOUT_CODES) and np.isfinite(got).all()
    w, norm = enc.readout_params()
    sel = np.ascontiguousarray(h[markers])
    want = empty((len(markers), rocm.Encoder.READOUT_CODES), torch.float32)
    ctx.readout(w, norm, dev(sel), len(markers), EPS, want)
    assert bits_equal(got, host(ctx, want))
    # different rows give different logits (the markers select rows)
    assert not np.array_equal(got[0], got[1])
    enc.close()


def test_encoder_readout_rejects_bad_markers(ctx):
    cfg = rocm.EncoderConfig(layers=1, hidden=128, heads=2, head_dim=64, ffn=256, vocab=100, ln_eps=1e-5)
    enc = ctx.encoder_random(cfg, 3)
    ids = np.arange(10, dtype=np.int32)
    rows = enc.read_rows(ids)
    for markers, code in [([10], "INVALID_REQUEST"), ([-1], "INVALID_REQUEST"), ([], "INVALID_REQUEST"),
                          ([0] * 257, "INPUT_TOO_LONG")]:
        with pytest.raises(rocm.DzError) as e:
            enc.readout_rows(rows, 10, np.array(markers, np.int32))
        assert e.value.code == code, markers
    enc.close()
