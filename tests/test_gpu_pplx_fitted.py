"""The Pplx decider with fitted weights, as the reference's optimized
precisions load it (native.rs:125-128: q4-w4a8-e4-r4-g64-mse and
q4-w4a8-e4-r4-g64-mse-nf4): every projection and the readout fitted by
quantization.rs:25-71 (mse: signed scales, codes -8..7), the embedding rows
MSE-fitted or NF4 (quantized_rows.rs:56-66). The layers and the chunk forward
are compared with the oracle's composition over the same fitted codes and
scales: the forward with the packed model's bound (tests/test_gpu_pplx.py),
each layer row by row (layer_close)."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests import pplx_model
from tests.gpu_util import cosine, dev, host

pytestmark = pytest.mark.gpu

SMALL = dict(layers=4, hidden=256, ff=512, delta_heads=4, delta_key_heads=2, delta_head_dim=128,
             attn_heads=4, attn_kv_heads=2, attn_head_dim=256)


def close(got, want, rel=2e-3):
    scale = max(float(np.abs(want).max()), 1e-6)
    return cosine(got, want) >= 0.9999 and float(np.abs(got - want).max()) <= rel * scale


def layer_close(got, want):
    """A layer is a chain of A8 quantizations: an ulp of difference in a layer
    op flips one code of a row now and then, which moves that row by about
    1e-3 of the output's largest value. Held: cosine >= 0.99999, every row
    within 1e-2 and at most one row in 16 beyond 2e-3 of the largest value."""
    scale = max(float(np.abs(want).max()), 1e-6)
    rows = np.abs(got - want).max(axis=1) / scale
    return (cosine(got, want) >= 0.99999 and rows.max() <= 1e-2
            and int((rows > 2e-3).sum()) <= max(1, got.shape[0] // 16))


@pytest.fixture(scope="module", params=["mse", "nf4"])
def fitted(ctx, oracle, request):
    model = pplx_model.random_model(oracle, SMALL, seed=5, fit="mse", rows_fit=request.param)
    p = pplx_model.load(ctx, rocm, model)
    yield model, p, request.param
    p.close()


def test_the_fits_use_the_whole_code_range_and_signed_scales(fitted):
    model, _, rows = fitted
    codes = np.concatenate([q[0].ravel() for q in model.quant.values()])
    scales = np.concatenate([q[1].ravel() for q in model.quant.values()])
    assert (codes == -8).any() and (scales < 0).any()
    assert model.rows[2] == (rows == "nf4")


@pytest.mark.parametrize("layer", [0, 3])
@pytest.mark.parametrize("n", [5, 37])
def test_fitted_layer_matches_the_reference_layer(ctx, oracle, fitted, layer, n):
    torch = pytest.importorskip("torch")
    model, p, _ = fitted
    h = np.random.default_rng(n + 10 * layer).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    hd = dev(h)
    p.layer(layer, hd, n)
    got = host(ctx, hd)
    want = pplx_model.ref_layer(oracle, model, layer, h)
    assert layer_close(got, want), (float(cosine(got, want)), float(np.abs(got - want).max()))


@pytest.mark.parametrize("n", [6, 130])
def test_fitted_forward_logits_match_the_reference_chunk(ctx, oracle, fitted, n):
    """The fitted rows decode as quantized_rows.rs:89-110 appends them (NF4
    through its codebook), then every layer and the fitted readout."""
    model, p, _ = fitted
    ids = np.random.default_rng(n).integers(0, 64, n)
    markers = [n - 1, 0, n // 2]
    got = p.forward_rows(model.embedding[ids], n, markers)
    want = pplx_model.ref_forward(oracle, model, ids, markers)
    assert got.shape == (3, 255) and np.isfinite(got).all()
    assert close(got, want, rel=1e-2), (float(cosine(got, want)), float(np.abs(got - want).max()))


def test_forms_the_decider_does_not_take_are_refused(ctx, oracle, fitted):
    model, p, rows = fitted
    name = "language_model.layers.0.mlp.up_proj.weight"
    wire, r, c = model.packed[name]

    def refused(code, fn):
        with pytest.raises(rocm.DzError) as e:
            fn()
        assert e.value.code == code

    refused("INVALID_PARAMETERS", lambda: p.set_weight_fitted(name, wire, r, c, rocm.FIT_AFFINE))
    refused("INVALID_PARAMETERS", lambda: p.set_weight_fitted(name, wire, r, c, rocm.FIT_NF4))
    refused("INVALID_PARAMETERS", lambda: p.set_rows_form(rocm.FIT_AFFINE))
    # packed.rs's validation still holds on the plain entry point: negative scales are refused
    refused("INVALID_CHECKPOINT", lambda: p.set_weight(name, wire, rocm.Q4_G64_F32, r, c))
    if rows == "mse":  # MSE rows with negative scales are not packed rows
        neg = np.flatnonzero((model.rows[1] < 0).any(axis=1))[:8]
        assert neg.size
        p.set_rows_form(rocm.ROWS_PACKED)
        try:
            refused("INVALID_CHECKPOINT", lambda: p.forward_rows(model.embedding[neg], neg.size, [0]))
        finally:
            p.set_rows_form(rocm.FIT_SCALED)
    # the refusals changed nothing: the model still answers as before
    got = p.forward_rows(model.embedding[:6], 6, [5])
    want = pplx_model.ref_forward(oracle, model, np.arange(6), [5])
    assert close(got, want, rel=1e-2)
