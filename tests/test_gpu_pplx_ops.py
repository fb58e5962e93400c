"""The Pplx decider's layer ops one by one at the reference model's real shape
(backbone.rs:11-22: hidden 2560, 32 delta heads over 16 key heads of dim 128,
16 query heads over 4 key/value heads of dim 256, FFN 9216; 1024 tokens),
each checked against the oracle fed the GPU's own input to that op (teacher
forcing), so an A8 code that flips in one op cannot carry into the next.

dz_pplx_layer_part runs one half of a layer and dz_pplx_activation reads the
activations it left. Per op:
  - the norms and the products: the oracle's RMSNorm + A8 quantizer
    (cpu.rs:310-333, int8.rs:178-202) and W4A8 fold (int8.rs:524-585) on the
    GPU's inputs give the GPU's codes, scales and outputs bit for bit, the
    residual adds included;
  - the ops between them (causal conv + SiLU, the delta rule's prep and scan,
    its gated norm, head norm + rotary, GQA attention, the attention gate):
    max-abs <= 1e-2 and cosine >= 0.9999 against the oracle on the GPU's
    inputs (the north star's bound), with the measured errors printed;
  - where an op's output is A8 codes (the gates, the fused MLP's SiLU * up),
    the GPU's codes are within one code of the oracle's quantization of its
    own f32 output, in at most 1e-3 of the positions, and the scales agree
    to 1e-5 relative.
"""
import numpy as np
import pytest

from decisive_amd import rocm
from tests import pplx_model
from tests.gpu_util import bits_equal, cosine, dev, host

pytestmark = pytest.mark.gpu

REAL = dict(layers=4, hidden=2560, ff=9216, delta_heads=32, delta_key_heads=16, delta_head_dim=128,
            attn_heads=16, attn_kv_heads=4, attn_head_dim=256)
N = 1024
LD, AD = pplx_model.LD, pplx_model.AD


@pytest.fixture(scope="module")
def real(ctx, oracle):
    model = pplx_model.random_model(oracle, REAL, seed=21, reuse={1: 0, 2: 0})
    p = pplx_model.load(ctx, rocm, model)
    h = np.random.default_rng(22).standard_normal((N, REAL["hidden"])).astype(np.float32)
    yield model, p, h
    p.close()


def act(ctx, p, name, shape, dtype):
    torch = pytest.importorskip("torch")
    t = torch.empty(shape, dtype=dtype, device="cuda")
    p.activation(name, t)
    return host(ctx, t).copy()


def north_star(got, want, what):
    err = float(np.abs(got.astype(np.float64) - want).max())
    cos = float(cosine(got, want))
    print(f"{what}: max |d| {err:.3e} (largest |value| {float(np.abs(want).max()):.3f}), cosine {cos:.9f}")
    assert err <= 1e-2 and cos >= 0.9999, (what, err, cos)


def codes_close(codes, scales, want_f32, what):
    """GPU A8 codes/scales against the oracle's quantization of the oracle's
    f32 output: at most one code apart, in at most 1e-3 of the positions."""
    from oracle import oracle as o
    rows, k = want_f32.shape
    qw, sw = o.act_quantize(want_f32, rows, k, 8)
    diff = np.abs(codes.astype(np.int32) - qw[:, :k].astype(np.int32))
    frac = float((diff > 0).mean())
    print(f"{what}: codes differing {frac:.2e}, largest difference {int(diff.max())}")
    assert diff.max() <= 1 and frac <= 1e-3, (what, int(diff.max()), frac)
    rel = np.abs(scales - sw) / np.maximum(np.abs(sw), 1e-30)
    assert float(rel.max()) <= 1e-5, (what, float(rel.max()))


def product(oracle, model, name, codes, scales):
    """The W4A8 product of the given A8 codes: the oracle's threaded AVX2
    panel path (int8.rs:229-585), which equals its scalar fused order bit for
    bit (tests/test_oracle.py), or that scalar order without AVX2."""
    qw, sw, rows, cols = model.quant[name]
    m = codes.shape[0]
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    if not oracle.has_avx2():
        return oracle.grouped_gemm(codes, scales, m, qw, sw, rows, cols, fused=True)
    if name not in model.panels:
        model.panels[name] = oracle.panel_pack(qw, sw, rows, cols, model.bits)
    data, ps = model.panels[name]
    return oracle.panel_apply_avx2(data, ps, rows, cols, model.bits, codes, scales, m, oracle.nprocs_env_default())


def norm_codes_exact(ctx, oracle, p, h, w, d):
    """The layer norm's A8 codes and scales against rmsnorm + act_quantize of
    the same rows: bit for bit."""
    torch = pytest.importorskip("torch")
    n = h.shape[0]
    nc = act(ctx, p, "norm_codes", (n, d), torch.int8)
    ns = act(ctx, p, "norm_scales", (n, d // 64), torch.float32)
    want = oracle.rmsnorm(h, w, 1e-6, zero_centered=True)
    qc, qs = oracle.act_quantize(want, n, d, 8)
    assert bits_equal(nc, qc[:, :d]) and bits_equal(ns, qs)
    return nc, ns


def test_delta_mixer_ops_against_the_oracle_on_the_gpus_inputs(ctx, oracle, real):
    """Input norm, the four input projections, conv + SiLU, the delta rule's
    prep and scan, its gated norm and out_proj with the residual."""
    torch = pytest.importorskip("torch")
    model, p, h = real
    c, v = model.cfg, model.vectors
    d, lh, lk = c["hidden"], c["delta_heads"], c["delta_key_heads"]
    cw, lv = pplx_model.conv_width(c), lh * LD
    pre = "language_model.layers.0."
    hd = dev(h)
    p.layer_part(0, rocm.PPLX_MIXER, hd, N)
    h1 = host(ctx, hd).copy()
    nc, ns = norm_codes_exact(ctx, oracle, p, h, v[pre + "input_layernorm.weight"], d)
    qkv = act(ctx, p, "qkv", (N, cw), torch.float32)
    z = act(ctx, p, "z", (N, lv), torch.float32)
    a = act(ctx, p, "a", (N, lh), torch.float32)
    b = act(ctx, p, "b", (N, lh), torch.float32)
    for name, got in (("in_proj_qkv", qkv), ("in_proj_z", z), ("in_proj_a", a), ("in_proj_b", b)):
        assert bits_equal(got, product(oracle, model, pre + f"linear_attn.{name}.weight", nc, ns)), name
    conv = act(ctx, p, "conv", (N, cw), torch.float32)
    taps = v[pre + "linear_attn.conv1d.weight"].reshape(cw, 4).T.copy()
    north_star(conv, oracle.conv_silu(qkv, taps), "conv + SiLU")
    heads = act(ctx, p, "heads", (lh, N, LD), torch.float32)
    decay = np.exp(v[pre + "linear_attn.A_log"]).astype(np.float32)
    want = oracle.delta_scan(conv, lh, lk, LD, a, b, decay, v[pre + "linear_attn.dt_bias"])
    north_star(heads, want, "delta prep + scan")
    gc = act(ctx, p, "gate_codes", (N, lv), torch.int8)
    gs = act(ctx, p, "gate_scales", (N, lv // 64), torch.float32)
    gated = oracle.delta_gate(heads, v[pre + "linear_attn.norm.weight"], z)
    codes_close(gc, gs, gated, "delta gate codes")
    want_h1 = (h + product(oracle, model, pre + "linear_attn.out_proj.weight", gc, gs)).astype(np.float32)
    assert bits_equal(h1, want_h1)


@pytest.mark.parametrize("markers", [None, "40"])
def test_attention_mixer_ops_against_the_oracle_on_the_gpus_inputs(ctx, oracle, real, markers):
    """Input norm, q/k/v projections, head norm + rotary of queries and keys,
    GQA attention, the attention gate and o_proj with the residual; with 40
    markers in a scrambled order the queries and residual rows are the
    markers' (prune_last)."""
    torch = pytest.importorskip("torch")
    model, p, h = real
    c, v = model.cfg, model.vectors
    d, ah, akv = c["hidden"], c["attn_heads"], c["attn_kv_heads"]
    pre = "language_model.layers.3."
    mk = None if markers is None else [int(t) for t in np.random.default_rng(23).permutation(N)[:40]]
    nq = N if mk is None else len(mk)
    pos = np.arange(N) if mk is None else np.asarray(mk)
    hd = dev(h)
    p.layer_part(3, rocm.PPLX_MIXER, hd, N, mk)
    h1 = host(ctx, hd)[:nq].copy()
    w_norm = v[pre + "input_layernorm.weight"]
    nc, ns = norm_codes_exact(ctx, oracle, p, h, w_norm, d)
    value = act(ctx, p, "value", (N, akv * AD), torch.float32)
    assert bits_equal(value, product(oracle, model, pre + "self_attn.v_proj.weight", nc, ns))
    key_raw = product(oracle, model, pre + "self_attn.k_proj.weight", nc, ns)  # bit-exact with the GPU's
    q = act(ctx, p, "q", (nq, ah * 2 * AD), torch.float32)
    if mk is None:
        assert bits_equal(q, product(oracle, model, pre + "self_attn.q_proj.weight", nc, ns))
    else:
        # the marker rows' queries come from their f32 normed rows (quantized by the product)
        normed = oracle.rmsnorm(h, w_norm, 1e-6, zero_centered=True)[mk]
        qc, qs = oracle.act_quantize(normed, nq, d, 8)
        assert bits_equal(q, product(oracle, model, pre + "self_attn.q_proj.weight", qc[:, :d], qs))
    freq = oracle.rope_freq()
    qz = q.reshape(nq, ah, 2 * AD)
    q_part = np.ascontiguousarray(qz[:, :, :AD]).reshape(nq, ah * AD)
    z = np.ascontiguousarray(qz[:, :, AD:]).reshape(nq, ah * AD)
    query = act(ctx, p, "query", (nq, ah * AD), torch.float32)
    want_q = oracle.rope(pplx_model._head_norm(oracle, q_part, ah, v[pre + "self_attn.q_norm.weight"]), ah, AD, pos,
                         freq)
    north_star(query, want_q, "query head norm + rotary")
    key = act(ctx, p, "key", (N, akv * AD), torch.float32)
    want_k = oracle.rope(pplx_model._head_norm(oracle, key_raw, akv, v[pre + "self_attn.k_norm.weight"]), akv, AD,
                         np.arange(N), freq)
    north_star(key, want_k, "key head norm + rotary")
    heads = act(ctx, p, "heads", (ah, nq, AD), torch.float32)
    north_star(heads, oracle.attention_gqa(query, key, value, ah, akv, AD, 1.0 / 16.0), "GQA attention")
    gated = oracle.attention_gate(heads, z)
    if mk is None:
        gc = act(ctx, p, "gate_codes", (nq, ah * AD), torch.int8)
        gs = act(ctx, p, "gate_scales", (nq, ah * AD // 64), torch.float32)
        codes_close(gc, gs, gated, "attention gate codes")
        proj = product(oracle, model, pre + "self_attn.o_proj.weight", gc, gs)
    else:
        g = act(ctx, p, "gate", (nq, ah * AD), torch.float32)
        north_star(g, gated, "attention gate")
        gq, gsq = oracle.act_quantize(g, nq, ah * AD, 8)  # the product quantizes its f32 input
        proj = product(oracle, model, pre + "self_attn.o_proj.weight", gq, gsq)
    rows = h if mk is None else h[mk]
    assert bits_equal(h1, (rows + proj).astype(np.float32))


@pytest.mark.parametrize("layer", [0, 3])
def test_mlp_half_against_the_oracle_and_halves_equal_the_whole_layer(ctx, oracle, real, layer):
    """Post norm, the fused gate/up + SiLU * up + A8 requant, and down_proj
    with the residual, on the GPU's mixer output; and the two halves run in
    turn give dz_pplx_layer's bits."""
    torch = pytest.importorskip("torch")
    model, p, h = real
    c, v = model.cfg, model.vectors
    d, ff = c["hidden"], c["ff"]
    pre = f"language_model.layers.{layer}."
    hd = dev(h)
    p.layer_part(layer, rocm.PPLX_MIXER, hd, N)
    h1 = host(ctx, hd).copy()
    p.layer_part(layer, rocm.PPLX_MLP, hd, N)
    h2 = host(ctx, hd).copy()
    nc, ns = norm_codes_exact(ctx, oracle, p, h1, v[pre + "post_attention_layernorm.weight"], d)
    mc = act(ctx, p, "mlp_codes", (N, ff), torch.int8)
    ms = act(ctx, p, "mlp_scales", (N, ff // 64), torch.float32)
    gate = product(oracle, model, pre + "mlp.gate_proj.weight", nc, ns)
    up = product(oracle, model, pre + "mlp.up_proj.weight", nc, ns)
    codes_close(mc, ms, oracle.silu_mul(gate, up), "SiLU * up codes")
    want_h2 = (h1 + product(oracle, model, pre + "mlp.down_proj.weight", mc, ms)).astype(np.float32)
    assert bits_equal(h2, want_h2)
    whole = dev(h)
    p.layer(layer, whole, N)
    assert bits_equal(host(ctx, whole), h2)


def test_activation_names_and_sizes_are_checked(ctx, oracle, real):
    """Unknown names, names of the other layer kind and wrong sizes are
    INVALID_PARAMETERS; the mixer's activations after an MLP half alone, and
    markers on the MLP half, are INVALID_REQUEST."""
    torch = pytest.importorskip("torch")
    model, p, h = real
    hd = dev(h[:64])
    p.layer_part(0, rocm.PPLX_MIXER, hd, 64)
    for name, shape in (("nope", (4,)), ("query", (64, 4096)), ("qkv", (3,))):
        with pytest.raises(rocm.DzError) as e:
            p.activation(name, torch.empty(shape, device="cuda"))
        assert e.value.code == "INVALID_PARAMETERS", name
    p.layer_part(0, rocm.PPLX_MLP, hd, 64)
    with pytest.raises(rocm.DzError) as e:
        p.activation("conv", torch.empty((64, pplx_model.conv_width(model.cfg)), device="cuda"))
    assert e.value.code == "INVALID_REQUEST"
    with pytest.raises(rocm.DzError) as e:
        p.layer_part(3, rocm.PPLX_MLP, hd, 64, [1, 2])
    assert e.value.code == "INVALID_REQUEST"
