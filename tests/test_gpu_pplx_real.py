"""The Pplx decider's layers at the reference model's real shape
(backbone.rs:11-22: hidden 2560, 32 delta heads over 16 key heads of dim 128,
16 query heads over 4 key/value heads of dim 256, FFN 9216) on a 1024-token
chunk, against the oracle's composition of the reference layer
(tests/pplx_model.py ref_layer). One delta layer and one attention layer are
random (seed 11); the other two delta layers of the 4-layer model share the
first one's tensors.

The bound. The projections are bit-exact, but the ops between them (scan,
attention, gates, SiLU) round differently from the oracle in the last ulp,
and each layer re-quantizes its activations to A8 codes several times. At
this width an ulp now and then moves a value across a code boundary, and one
such flip at the MLP input moves the 9216 SiLU*up values enough to flip about
1% of their codes (step ~0.4), so a few percent of the rows end up ~1% of
the output's largest value away while the rest agree to f32 rounding. The
oracle is exactly as sensitive: the same layer on an input with one ulp added
to every seventh element moves by 0.6-1.1% of the largest value. So each case
asserts (1) cosine >= 0.9999, (2) a median row error <= 1e-5 of the largest
value, and (3) no row error above twice the oracle's own one-ulp
sensitivity, computed in the test. A wrong op (a sign, a head mapping, a
scale) fails (1) and (2) by orders of magnitude."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests import pplx_model
from tests.gpu_util import cosine, dev, host

pytestmark = pytest.mark.gpu

REAL = dict(layers=4, hidden=2560, ff=9216, delta_heads=32, delta_key_heads=16, delta_head_dim=128,
            attn_heads=16, attn_kv_heads=4, attn_head_dim=256)
N = 1024


def row_errors(got, want):
    scale = max(float(np.abs(want).max()), 1e-6)
    return np.abs(got - want).max(1) / scale


def one_ulp_sensitivity(oracle, model, layer, h, markers):
    """The oracle layer's own largest row change when one ulp is added to
    every seventh input element."""
    hp = h.copy()
    flat = hp.reshape(-1)
    flat[::7] = np.nextafter(flat[::7], np.float32(np.inf))
    base = pplx_model.ref_layer(oracle, model, layer, h, markers)
    return base, float(row_errors(pplx_model.ref_layer(oracle, model, layer, hp, markers), base).max())


def check(got, want, noise):
    rows = row_errors(got, want)
    facts = dict(cos=float(cosine(got, want)), median=float(np.median(rows)), worst=float(rows.max()),
                 oracle_one_ulp=noise)
    assert facts["cos"] >= 0.9999, facts
    assert facts["median"] <= 1e-5, facts
    assert facts["worst"] <= max(2e-3, 2 * noise), facts


@pytest.fixture(scope="module")
def real(ctx, oracle):
    model = pplx_model.random_model(oracle, REAL, seed=11, reuse={1: 0, 2: 0})
    p = pplx_model.load(ctx, rocm, model)
    h = np.random.default_rng(12).standard_normal((N, REAL["hidden"])).astype(np.float32)
    yield model, p, h, {}
    p.close()


@pytest.mark.parametrize("scan", ["chunked64", "recurrent"])
def test_real_delta_layer_matches_the_reference_layer(ctx, oracle, real, scan):
    torch = pytest.importorskip("torch")
    model, p, h, wants = real
    hd = dev(h)
    ctx.select_variant("delta_scan", scan)
    try:
        p.layer(0, hd, N)
    finally:
        ctx.select_variant("delta_scan", "chunked64")
    got = host(ctx, hd)
    if "delta" not in wants:
        wants["delta"] = one_ulp_sensitivity(oracle, model, 0, h, None)
    check(got, *wants["delta"])


@pytest.mark.parametrize("markers", [None, "40"])
def test_real_attention_layer_matches_the_reference_layer(ctx, oracle, real, markers):
    """The full layer, and the marker-pruned form with 40 markers in a
    scrambled order (o_proj, its residual and the MLP then run on 40 rows, the
    pipelined products' path)."""
    torch = pytest.importorskip("torch")
    model, p, h, _ = real
    mk = None if markers is None else [int(t) for t in np.random.default_rng(13).permutation(N)[:40]]
    hd = dev(h)
    p.layer(3, hd, N, mk)
    got = host(ctx, hd)[:N if mk is None else len(mk)]
    check(got, *one_ulp_sensitivity(oracle, model, 3, h, mk))
