"""The Pplx decider on the GPU (dz_pplx_*): each decoder layer and the whole
chunk forward against the oracle's composition of the reference's layer
(backbone.rs:207-250) on a random model at test sizes. The projections are
the bit-exact W4A8 products; the layer ops between them (SiLU conv, delta
rule, RMSNorms, rotary embedding, softmax attention, gates) use device exp/sin
and fused multiply-adds, so the comparison is to a tolerance: cosine >=
0.9999 and max-abs <= 2e-3 relative to the output's largest value for a
layer. Through a whole chunk the decoder is a chain of A8 quantizations; an
ulp of difference in a layer op flips an activation code now and then, and
the logits are held to 1% of their largest value."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests import pplx_model
from tests.gpu_util import bits_equal, cosine, dev, empty, host

pytestmark = pytest.mark.gpu

# two query heads per key/value head on both mixers, so a wrong head mapping shows
SMALL = dict(layers=4, hidden=256, ff=512, delta_heads=4, delta_key_heads=2, delta_head_dim=128,
             attn_heads=4, attn_kv_heads=2, attn_head_dim=256)


def close(got, want, rel=2e-3):
    scale = max(float(np.abs(want).max()), 1e-6)
    return cosine(got, want) >= 0.9999 and float(np.abs(got - want).max()) <= rel * scale


@pytest.fixture(scope="module")
def small(ctx, oracle):
    model = pplx_model.random_model(oracle, SMALL, seed=3)
    p = pplx_model.load(ctx, rocm, model)
    yield model, p
    p.close()


@pytest.mark.parametrize("layer", [0, 1, 3])
@pytest.mark.parametrize("n", [1, 5, 37])
def test_layer_matches_the_reference_layer(ctx, oracle, small, layer, n):
    torch = pytest.importorskip("torch")
    model, p = small
    h = np.random.default_rng(n + layer).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    hd = dev(h)
    p.layer(layer, hd, n)
    got = host(ctx, hd)
    want = pplx_model.ref_layer(oracle, model, layer, h)
    assert close(got, want), (float(cosine(got, want)), float(np.abs(got - want).max()))


def test_attention_layer_prunes_to_the_markers_in_order(ctx, oracle, small):
    torch = pytest.importorskip("torch")
    model, p = small
    n, markers = 23, [17, 2, 22, 9]
    h = np.random.default_rng(8).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    hd = dev(h)
    p.layer(3, hd, n, markers)
    got = host(ctx, hd)[:len(markers)]
    want = pplx_model.ref_layer(oracle, model, 3, h, markers)
    assert close(got, want)
    # a recurrent layer cannot be cut
    with pytest.raises(rocm.DzError) as e:
        p.layer(0, dev(h), n, markers)
    assert e.value.code == "INVALID_REQUEST"


@pytest.mark.parametrize("n", [6, 64, 400])  # 400: seven 64-token chunks of the delta scan, the last ragged
def test_forward_logits_match_the_reference_chunk(ctx, oracle, small, n):
    model, p = small
    ids = np.random.default_rng(n).integers(0, 64, n)
    markers = [n - 1, 0, n // 2]
    got = p.forward_rows(model.embedding[ids], n, markers)
    want = pplx_model.ref_forward(oracle, model, ids, markers)
    assert got.shape == (3, 255) and np.isfinite(got).all()
    assert close(got, want, rel=1e-2), (float(cosine(got, want)), float(np.abs(got - want).max()))


@pytest.mark.parametrize("scan", ["chunked64", "chunked64-c32", "recurrent", "recurrent-rolled"])
@pytest.mark.parametrize("n", [1, 37, 64, 130, 257])
def test_delta_layer_matches_the_reference_for_both_scans(ctx, oracle, small, scan, n):
    """The chunked scan (64-token chunks: one partial chunk, exact chunks, a
    ragged tail; 16 or 32 state columns per block) and the token-by-token one
    (its unrolled and rolled forms) against the oracle's sequential rule. Both regroup the rule's
    arithmetic, so an ulp now and then flips one A8 code of out_proj's input;
    the bound is a cosine of 0.99999 with max-abs within 1% (a wrong scan
    lands far below 0.9999)."""
    torch = pytest.importorskip("torch")
    model, p = small
    h = np.random.default_rng(100 + n).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    hd = dev(h)
    ctx.select_variant("delta_scan", scan)
    try:
        p.layer(1, hd, n)
    finally:
        ctx.select_variant("delta_scan", "chunked64")
    got = host(ctx, hd)
    want = pplx_model.ref_layer(oracle, model, 1, h)
    assert cosine(got, want) >= 0.99999 and close(got, want, rel=1e-2), (float(cosine(got, want)),
                                                                         float(np.abs(got - want).max()))


@pytest.mark.parametrize("n", [1, 16, 17, 130, 400])
def test_scan_forms_are_bitwise_equal(ctx, oracle, small, n):
    """Each scan's forms run the same arithmetic in the same order: the two
    chunked forms (16 or 32 state columns per block) give the same bits, and
    so do the unrolled and rolled token scans, at lengths inside one 16-token
    stage and one chunk, across them and past the 384 tokens where "auto"
    switches from the token scan to the chunked one, whose bits it then gives."""
    torch = pytest.importorskip("torch")
    model, p = small
    h = np.random.default_rng(300 + n).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    got = {}
    try:
        for scan in ("chunked64", "chunked64-c32", "recurrent", "recurrent-rolled", "auto"):
            ctx.select_variant("delta_scan", scan)
            hd = dev(h)
            p.layer(1, hd, n)
            got[scan] = host(ctx, hd).copy()
    finally:
        ctx.select_variant("delta_scan", "chunked64")
    assert bits_equal(got["chunked64"], got["chunked64-c32"])
    assert bits_equal(got["recurrent"], got["recurrent-rolled"])
    assert bits_equal(got["auto"], got["recurrent" if n < 384 else "chunked64"])


@pytest.mark.parametrize("n", [5, 64, 200])
def test_chunked_scan_outputs_do_not_depend_on_the_chunk_length(ctx, oracle, small, n):
    """The default scan is causal in its arithmetic too: the first n tokens of
    a 257-token layer are the bits of an n-token layer (masked terms add exact
    zeros), so a decider's outputs do not depend on where its chunk ends."""
    torch = pytest.importorskip("torch")
    model, p = small
    h = np.random.default_rng(900).standard_normal((257, SMALL["hidden"])).astype(np.float32)
    long, short = dev(h), dev(h[:n])
    p.layer(1, long, 257)
    p.layer(1, short, n)
    assert bits_equal(host(ctx, short), host(ctx, long)[:n])


# four query heads per key/value head, as the reference model has
GQA4 = dict(SMALL, attn_heads=8, attn_kv_heads=2)


@pytest.mark.parametrize("n,markers", [(300, None), (77, [76, 3, 40])])
def test_attention_layer_with_head_groups_of_four(ctx, oracle, n, markers):
    """Several 32-key blocks with a ragged tail, every query block, and the
    marker-pruned form, with the reference's group of four query heads."""
    torch = pytest.importorskip("torch")
    model = pplx_model.random_model(oracle, dict(GQA4, layers=4), seed=9)
    p = pplx_model.load(ctx, rocm, model)
    h = np.random.default_rng(n).standard_normal((n, GQA4["hidden"])).astype(np.float32)
    hd = dev(h)
    p.layer(3, hd, n, markers)
    got = host(ctx, hd)[:n if markers is None else len(markers)]
    want = pplx_model.ref_layer(oracle, model, 3, h, markers)
    p.close()
    assert close(got, want), (float(cosine(got, want)), float(np.abs(got - want).max()))


def test_delta_scan_state_carries_across_tokens(ctx, oracle, small):
    """The last token's output depends on the first token (the recurrent
    state): changing only token 0 changes the output at token n-1."""
    torch = pytest.importorskip("torch")
    model, p = small
    n = 12
    h = np.random.default_rng(2).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    h2 = h.copy()
    h2[0] *= -1
    a, b = dev(h), dev(h2)
    p.layer(0, a, n)
    p.layer(0, b, n)
    assert not np.allclose(host(ctx, a)[n - 1], host(ctx, b)[n - 1])


def test_missing_weights_and_bad_names_are_rejected(ctx, oracle):
    torch = pytest.importorskip("torch")
    cfg = dict(SMALL, layers=1)
    p = ctx.pplx_create(rocm.PplxConfig(**cfg))
    with pytest.raises(rocm.DzError) as e:
        p.layer(0, dev(np.zeros((2, 256), np.float32)), 2)
    assert e.value.code == "INVALID_CHECKPOINT" and "missing" in str(e.value)
    with pytest.raises(rocm.DzError) as e:
        p.set_vector("language_model.layers.0.nope", np.zeros(4, np.float32))
    assert e.value.code == "INVALID_CHECKPOINT"
    with pytest.raises(rocm.DzError) as e:
        p.set_vector("language_model.layers.7.input_layernorm.weight", np.zeros(256, np.float32))
    assert e.value.code == "INVALID_CHECKPOINT"
    # layer 0 is a delta layer: attention weights do not belong there
    wire = oracle.pack_g64(oracle.f32_to_bf16(np.zeros((256, 256), np.float32) + 0.01), 256, 256, 4)
    with pytest.raises(rocm.DzError) as e:
        p.set_weight("language_model.layers.0.self_attn.o_proj.weight", wire, rocm.Q4_G64_F32, 256, 256)
    assert e.value.code == "INVALID_CHECKPOINT"
    with pytest.raises(rocm.DzError) as e:
        ctx.pplx_create(rocm.PplxConfig(**dict(SMALL, delta_head_dim=64)))
    assert e.value.code == "INVALID_PARAMETERS"
    p.close()


MANY = [int(t) for t in np.random.default_rng(40).permutation(130)[:40]]  # more than 16 rows after pruning


@pytest.mark.parametrize("layer,n,markers", [(1, 37, None), (1, 130, None), (3, 77, None), (3, 77, [76, 3, 40]),
                                             (3, 130, MANY)])
def test_residual_added_in_the_product_epilogue_gives_the_same_bits(ctx, oracle, small, layer, n, markers):
    """The pipelined W4A8 kernels add the residual in their epilogue (out_proj,
    o_proj and down_proj onto the hidden rows); the one-wave kernel leaves it
    to a separate add. The grouped products are bitwise equal across variants
    and the add is the same float add, so the layer outputs match bit for bit."""
    torch = pytest.importorskip("torch")
    model, p = small
    h = np.random.default_rng(500 + n).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    out = {}
    for v in ("wave16x16", "pipe128x128w4", "pipe64x128w2", "pipe32x128w8g4", "fewrow16"):
        hd = dev(h)
        ctx.select_variant("grouped", v)
        try:
            p.layer(layer, hd, n, markers)
        finally:
            ctx.select_variant("grouped", "pipe-auto")
        out[v] = host(ctx, hd)[:n if markers is None else len(markers)]
    assert np.array_equal(out["wave16x16"].view(np.uint32), out["pipe128x128w4"].view(np.uint32))
    assert np.array_equal(out["wave16x16"].view(np.uint32), out["pipe64x128w2"].view(np.uint32))
    assert np.array_equal(out["wave16x16"].view(np.uint32), out["pipe32x128w8g4"].view(np.uint32))
    assert np.array_equal(out["wave16x16"].view(np.uint32), out["fewrow16"].view(np.uint32))
    want = pplx_model.ref_layer(oracle, model, layer, h, markers)
    assert close(out["pipe128x128w4"], want)


@pytest.mark.parametrize("layer,n,markers", [(1, 37, None), (1, 130, None), (3, 77, None), (3, 130, MANY), (0, 400, None)])
def test_fused_norm_codes_give_the_separate_norms_bits(ctx, oracle, small, layer, n, markers):
    """The "fused" norm writes the RMSNorm and the A8 codes its products share
    in one kernel; the "separate" norm writes the normed rows and each product
    quantizes them (act_quantize). Both are bit-exact with cpu::rms_from and
    int8.rs's quantizer, so the layers give the same bits."""
    torch = pytest.importorskip("torch")
    model, p = small
    h = np.random.default_rng(900 + n).standard_normal((n, SMALL["hidden"])).astype(np.float32)
    out = {}
    for v in ("fused", "separate"):
        hd = dev(h)
        ctx.select_variant("norm", v)
        try:
            p.layer(layer, hd, n, markers)
        finally:
            ctx.select_variant("norm", "fused")
        out[v] = host(ctx, hd)[:n if markers is None else len(markers)]
    assert np.array_equal(out["fused"].view(np.uint32), out["separate"].view(np.uint32))
    want = pplx_model.ref_layer(oracle, model, layer, h, markers)
    assert close(out["fused"], want, rel=1e-2), (float(cosine(out["fused"], want)),)


def test_fused_norm_forward_and_nonfinite_rows(ctx, oracle, small):
    """A whole chunk forward gives the same logits under both norms; a
    non-finite hidden value makes the fused norm's products NaN as the
    separate quantizer's flag does (int8.rs:170-173)."""
    torch = pytest.importorskip("torch")
    model, p = small
    n = 300
    ids = np.random.default_rng(31).integers(0, 64, n)
    markers = [n - 1, 5, n // 2]
    got = {}
    for v in ("fused", "separate"):
        ctx.select_variant("norm", v)
        try:
            got[v] = p.forward_rows(model.embedding[ids], n, markers)
        finally:
            ctx.select_variant("norm", "fused")
    assert np.array_equal(got["fused"].view(np.uint32), got["separate"].view(np.uint32))
    h = np.random.default_rng(32).standard_normal((40, SMALL["hidden"])).astype(np.float32)
    h[7, 3] = np.inf
    outs = {}
    for v in ("fused", "separate"):
        hd = dev(h)
        ctx.select_variant("norm", v)
        try:
            p.layer(0, hd, 40)
        finally:
            ctx.select_variant("norm", "fused")
        outs[v] = host(ctx, hd)
    assert np.isnan(outs["fused"]).all() and np.isnan(outs["separate"]).all()
