"""Streamed residency of the Pplx decider (dz_pplx_set_residency, the
reference's two-bank weight buffers of webgpu/streaming.rs:16-369): the layer
projections live in pinned host memory and layer i runs from device bank
i % 2 while the next layer is copied into the other bank. The kernels and the
weight bytes are the same as in resident memory, so every output must be
bitwise equal to the resident model's (which the decider's parity tests pin
against the oracle's composition)."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests import pplx_model
from tests.gpu_util import dev, host

pytestmark = pytest.mark.gpu

# eight layers: two of them attention layers (3 and 7), so bank 1 alternates kinds
CFG = dict(layers=8, hidden=256, ff=512, delta_heads=4, delta_key_heads=2, delta_head_dim=128,
           attn_heads=4, attn_kv_heads=2, attn_head_dim=256)


def bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


@pytest.fixture(scope="module")
def model(oracle):
    return pplx_model.random_model(oracle, CFG, seed=11)


def _forward(p, model, n, seed):
    ids = np.random.default_rng(seed).integers(0, 64, n)
    return p.forward_rows(model.embedding[ids], n, [n - 1, 0, n // 2])


@pytest.mark.parametrize("n", [6, 64, 400])  # 400 tokens: the chunked delta scan
def test_streamed_forward_equals_the_resident_forward(ctx, model, n):
    p = pplx_model.load(ctx, rocm, model)
    try:
        want = _forward(p, model, n, n)
        resident = p.residency_info()
        assert resident["residency"] == "resident" and resident["banks"] == 0
        p.set_residency(rocm.PPLX_STREAMED)
        info = p.residency_info()
        assert info["residency"] == "streamed" and info["banks"] == 2
        assert info["host_layer_weight_bytes"] >= info["layer_weight_bytes"] == resident["layer_weight_bytes"]
        # two banks of the largest layer instead of every layer
        assert info["device_layer_weight_bytes"] == 2 * info["bank_bytes"] < info["layer_weight_bytes"]
        for rep in range(2):  # the second forward refills banks that hold the previous forward's last layers
            got = _forward(p, model, n, n)
            assert np.array_equal(bits(got), bits(want)), rep
        info = p.residency_info()
        layers = CFG["layers"]
        assert info["layer_uploads"] == 2 * layers and info["bank_reuses"] == 2 * layers - 2
        assert info["bank_layers"] == [layers - 2, layers - 1]
        p.set_residency(rocm.PPLX_RESIDENT)
        assert p.residency_info()["residency"] == "resident"
        assert np.array_equal(bits(_forward(p, model, n, n)), bits(want))
    finally:
        p.close()


def test_streamed_layers_in_any_order(ctx, model):
    """Single layers in an order that reuses a bank's current layer (no copy)
    and switches the other bank between a delta and an attention layer."""
    torch = pytest.importorskip("torch")
    n = 37
    order = [3, 0, 3, 1, 2, 7, 6, 7]
    h = np.random.default_rng(5).standard_normal((n, CFG["hidden"])).astype(np.float32)
    p = pplx_model.load(ctx, rocm, model)
    try:
        want = {}
        for i in sorted(set(order)):
            hd = dev(h)
            p.layer(i, hd, n)
            want[i] = host(ctx, hd).copy()
        p.set_residency(rocm.PPLX_STREAMED)
        for i in order:
            hd = dev(h)
            p.layer(i, hd, n)
            assert np.array_equal(bits(host(ctx, hd)), bits(want[i])), i
        info = p.residency_info()
        # each run copies its layer unless its bank holds it, then the next layer behind it:
        # 3+4, 0+1, 3+4, 1+2, (2)+3, 7, 6+(7), (7)
        assert info["bank_layers"] == [6, 7]
        assert info["layer_uploads"] == 11
    finally:
        p.close()


def test_streamed_weight_replacement_and_layout_rule(ctx, oracle, model):
    """Under streaming, dz_pplx_set_weight replaces the host copy, also of the
    layer a bank holds at that moment: the next run equals a resident model
    that holds the new weight. A different layout (Q8 for a Q4 projection) is
    refused and changes nothing."""
    torch = pytest.importorskip("torch")
    n = 64
    name = "language_model.layers.6.mlp.down_proj.weight"
    rows, cols = CFG["hidden"], CFG["ff"]
    raw = oracle.f32_to_bf16((np.random.default_rng(77).standard_normal((rows, cols)) * 0.03).astype(np.float32))
    wire4 = oracle.pack_g64(raw, rows, cols, 4)
    h = np.random.default_rng(6).standard_normal((n, CFG["hidden"])).astype(np.float32)
    streamed = pplx_model.load(ctx, rocm, model)
    resident = pplx_model.load(ctx, rocm, model)

    def run(p):
        hd = dev(h)
        p.layer(6, hd, n)
        return host(ctx, hd).copy()

    try:
        streamed.set_residency(rocm.PPLX_STREAMED)
        before = run(streamed)
        assert streamed.residency_info()["bank_layers"][0] == 6
        streamed.set_weight(name, wire4, rocm.Q4_G64_F32, rows, cols)
        resident.set_weight(name, wire4, rocm.Q4_G64_F32, rows, cols)
        want = run(resident)
        assert not np.array_equal(bits(want), bits(before))
        assert np.array_equal(bits(run(streamed)), bits(want))
        with pytest.raises(rocm.DzError) as e:
            streamed.set_weight(name, oracle.pack_g64(raw, rows, cols, 8), rocm.Q8_G64_F32, rows, cols)
        assert e.value.code == "INVALID_REQUEST"
        assert np.array_equal(bits(run(streamed)), bits(want))
        assert np.array_equal(bits(_forward(streamed, model, n, 2)), bits(_forward(resident, model, n, 2)))
    finally:
        streamed.close()
        resident.close()


def test_streaming_needs_every_layer_projection(ctx, model):
    p = ctx.pplx_create(rocm.PplxConfig(**CFG))
    try:
        for name, (wire, rows, cols) in model.packed.items():
            if "layers.5." not in name:
                p.set_weight(name, wire, rocm.Q4_G64_F32, rows, cols)
        with pytest.raises(rocm.DzError) as e:
            p.set_residency(rocm.PPLX_STREAMED)
        assert e.value.code == "INVALID_CHECKPOINT"
        with pytest.raises(rocm.DzError) as e:
            p.set_residency(7)
        assert e.value.code == "INVALID_PARAMETERS"
        assert p.residency_info()["residency"] == "resident"
    finally:
        p.close()


def test_joined_delta_input_projections_follow_replacement(ctx, oracle, model):
    """A resident model keeps each delta layer's in_proj_z, in_proj_a and
    in_proj_b joined as one weight, which a streamed model does not: after a
    and b of layer 0 are replaced, the resident run (one product over the
    rebuilt joined weight) equals the streamed run (three products) bit for bit.
    A part in another layout leaves the layer unjoined until it is replaced by
    one in the common layout again."""
    torch = pytest.importorskip("torch")
    n = 77
    hidden, heads = CFG["hidden"], CFG["delta_heads"]
    rng = np.random.default_rng(91)
    new = {}
    for part in ("a", "b"):
        raw = oracle.f32_to_bf16((rng.standard_normal((heads, hidden)) * 0.05).astype(np.float32))
        new[part] = (f"language_model.layers.0.linear_attn.in_proj_{part}.weight", raw)
    h = rng.standard_normal((n, hidden)).astype(np.float32)
    resident = pplx_model.load(ctx, rocm, model)
    streamed = pplx_model.load(ctx, rocm, model)

    def run(p):
        hd = dev(h)
        p.layer(0, hd, n)
        return host(ctx, hd).copy()

    try:
        joined = resident.residency_info()
        assert joined["device_layer_weight_bytes"] > joined["layer_weight_bytes"]
        before = run(resident)
        streamed.set_residency(rocm.PPLX_STREAMED)
        assert np.array_equal(bits(run(streamed)), bits(before))
        for name, raw in new.values():
            wire = oracle.pack_g64(raw, heads, hidden, 4)
            resident.set_weight(name, wire, rocm.Q4_G64_F32, heads, hidden)
            streamed.set_weight(name, wire, rocm.Q4_G64_F32, heads, hidden)
        after = run(resident)
        assert not np.array_equal(bits(after), bits(before))
        assert np.array_equal(bits(after), bits(run(streamed)))
        # b in Q8: layer 0 runs three products; back in Q4, joined again
        name, raw = new["b"]
        resident.set_weight(name, oracle.pack_g64(raw, heads, hidden, 8), rocm.Q8_G64_F32, heads, hidden)
        split = resident.residency_info()
        assert split["device_layer_weight_bytes"] - split["layer_weight_bytes"] < \
            joined["device_layer_weight_bytes"] - joined["layer_weight_bytes"]
        run(resident)
        resident.set_weight(name, oracle.pack_g64(raw, heads, hidden, 4), rocm.Q4_G64_F32, heads, hidden)
        assert resident.residency_info()["device_layer_weight_bytes"] == joined["device_layer_weight_bytes"]
        assert np.array_equal(bits(run(resident)), bits(after))
    finally:
        resident.close()
        streamed.close()
