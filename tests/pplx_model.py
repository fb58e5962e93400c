"""A random Pplx decider (the hybrid decoder of src/models/pplx_flash/
backbone.rs) at test sizes, and its forward composed from the oracle's
restatements: the checker for decisive_amd's dz_pplx_* entry points.

Tensor names and shapes are the checkpoint's (backbone.rs:101-199). 2-D
weights are BF16 values packed to the group-64 wire layout (what a packed
checkpoint stores); the oracle multiplies with the same codes and scales
(int8.rs W4A8, bit-exact with the GPU product). Vectors are BF16-rounded f32.
"""
from dataclasses import dataclass, field

import numpy as np

LD, AD = 128, 256


@dataclass
class Model:
    cfg: dict
    packed: dict = field(default_factory=dict)   # name -> (wire bytes, rows, cols)
    quant: dict = field(default_factory=dict)    # name -> (codes, scales, rows, cols)
    vectors: dict = field(default_factory=dict)  # name -> f32 values (checkpoint order)
    embedding: np.ndarray = None                 # packed wire rows [vocab x hidden]
    panels: dict = field(default_factory=dict)   # name -> the oracle's AVX2 panel form of quant[name]
    bits: int = 4                                # weight code bits
    fit: str = None                              # projections fitted by quantization.rs ("mse") or packed
    rows: tuple = None                           # fitted rows (codes, scales, nf4), else the packed embedding


def conv_width(c):
    return 2 * c["delta_key_heads"] * LD + c["delta_heads"] * LD


def random_model(oracle, cfg, vocab=64, seed=0, bits=4, reuse=None, fit=None, rows_fit=None):
    """`reuse` maps a layer index to an earlier layer of the same kind whose
    tensors it shares (real-size models with one layer of each kind). `fit`
    "mse" fits every projection and the readout as native.rs:125-128's
    optimized precisions do (quantization.rs:25-71); `rows_fit` "mse" or
    "nf4" fits the embedding rows (quantized_rows.rs:56-66)."""
    rng = np.random.default_rng(seed)
    m = Model(cfg=dict(cfg), bits=bits, fit=fit)
    d, ff, lh, ah, akv = cfg["hidden"], cfg["ff"], cfg["delta_heads"], cfg["attn_heads"], cfg["attn_kv_heads"]
    cw, lv = conv_width(cfg), lh * LD

    def bf(x):
        return oracle.bf16_to_f32(oracle.f32_to_bf16(np.asarray(x, np.float32)))

    def mat(name, rows, cols, std):
        raw = oracle.f32_to_bf16((rng.standard_normal((rows, cols)) * std).astype(np.float32))
        if fit:
            codes, scales, _ = oracle.weight_quantize_fitted(raw, rows, cols, fit)
            m.packed[name] = (oracle.pack_wire_codes(codes, scales, rows, cols), rows, cols)
        else:
            m.packed[name] = (oracle.pack_g64(raw, rows, cols, bits), rows, cols)
            codes, scales = oracle.weight_quantize(raw, rows, cols, bits)
        m.quant[name] = (codes, scales, rows, cols)

    def vec(name, values):
        m.vectors[name] = bf(values)

    for i in range(cfg["layers"]):
        p = f"language_model.layers.{i}."
        src = (reuse or {}).get(i)
        if src is not None:
            sp = f"language_model.layers.{src}."
            for table in (m.packed, m.quant, m.vectors):
                for name in [t for t in table if t.startswith(sp)]:
                    table[p + name[len(sp):]] = table[name]
            continue
        vec(p + "input_layernorm.weight", rng.standard_normal(d) * 0.1)
        vec(p + "post_attention_layernorm.weight", rng.standard_normal(d) * 0.1)
        if i % 4 == 3:
            mat(p + "self_attn.q_proj.weight", 2 * ah * AD, d, 0.05)
            mat(p + "self_attn.k_proj.weight", akv * AD, d, 0.05)
            mat(p + "self_attn.v_proj.weight", akv * AD, d, 0.05)
            mat(p + "self_attn.o_proj.weight", d, ah * AD, 0.03)
            vec(p + "self_attn.q_norm.weight", rng.standard_normal(AD) * 0.1)
            vec(p + "self_attn.k_norm.weight", rng.standard_normal(AD) * 0.1)
        else:
            mat(p + "linear_attn.in_proj_qkv.weight", cw, d, 0.05)
            mat(p + "linear_attn.in_proj_z.weight", lv, d, 0.05)
            mat(p + "linear_attn.in_proj_a.weight", lh, d, 0.05)
            mat(p + "linear_attn.in_proj_b.weight", lh, d, 0.05)
            mat(p + "linear_attn.out_proj.weight", d, lv, 0.03)
            vec(p + "linear_attn.conv1d.weight", rng.standard_normal(cw * 4) * 0.4)  # [width, 1, 4]
            vec(p + "linear_attn.A_log", np.log(rng.uniform(1.0, 16.0, lh)))
            vec(p + "linear_attn.dt_bias", rng.standard_normal(lh) * 0.5)
            vec(p + "linear_attn.norm.weight", 1.0 + rng.standard_normal(LD) * 0.1)
        mat(p + "mlp.gate_proj.weight", ff, d, 0.05)
        mat(p + "mlp.up_proj.weight", ff, d, 0.05)
        mat(p + "mlp.down_proj.weight", d, ff, 0.03)
    vec("language_model.norm.weight", rng.standard_normal(d) * 0.1)
    mat("readout", 255, d, 0.05)
    emb = oracle.f32_to_bf16(rng.standard_normal((vocab, d)).astype(np.float32))
    if rows_fit:
        codes, scales, _ = oracle.weight_quantize_fitted(emb, vocab, d, rows_fit)
        m.embedding = oracle.pack_wire_codes(codes, scales, vocab, d).reshape(vocab, -1)
        m.rows = (codes, scales, rows_fit == "nf4")
    else:
        m.embedding = oracle.pack_g64(emb, vocab, d, bits).reshape(vocab, -1)
    return m


def load(ctx, rocm, model):
    p = ctx.pplx_create(rocm.PplxConfig(**model.cfg))
    layout = rocm.Q4_G64_F32
    for name, (wire, rows, cols) in model.packed.items():
        if model.fit:
            p.set_weight_fitted(name, wire, rows, cols, rocm.FIT_SCALED)
        else:
            p.set_weight(name, wire, layout, rows, cols)
    if model.rows is not None:
        p.set_rows_form(rocm.FIT_NF4 if model.rows[2] else rocm.FIT_SCALED)
    for name, values in model.vectors.items():
        p.set_vector(name, values)
    return p


# ---- the oracle forward (backbone.rs:207-250, mod.rs:149-185) ----

def _apply(oracle, model, name, x):
    """int8.rs:166-176 apply. From 16 rows of finite input the oracle's
    threaded AVX2 panel path runs (int8.rs:229-585), which equals the scalar
    fused order bit for bit (tests/test_oracle.py); below, the scalar one."""
    codes, scales, rows, cols = model.quant[name]
    m = x.shape[0]
    if m < 16 or not oracle.has_avx2() or not np.isfinite(x).all():
        return oracle.matrix_apply(x, m, codes, scales, rows, cols)
    if name not in model.panels:
        model.panels[name] = oracle.panel_pack(codes, scales, rows, cols, model.bits)
    data, ps = model.panels[name]
    qx, sx = oracle.act_quantize(x, m, cols, 8)
    return oracle.panel_apply_avx2(data, ps, rows, cols, model.bits, qx, sx, m, oracle.nprocs_env_default())


def _head_norm(oracle, x, heads, w):
    rows = x.shape[0]
    return oracle.rmsnorm(x.reshape(rows * heads, AD), w, 1e-6, zero_centered=True).reshape(rows, heads * AD)


def ref_layer(oracle, model, i, h, markers=None):
    c = model.cfg
    p = f"language_model.layers.{i}."
    v = model.vectors
    n = h.shape[0]
    norm = oracle.rmsnorm(h, v[p + "input_layernorm.weight"], 1e-6, zero_centered=True)
    if i % 4 == 3:
        ah, akv = c["attn_heads"], c["attn_kv_heads"]
        key = _apply(oracle, model, p + "self_attn.k_proj.weight", norm)
        value = _apply(oracle, model, p + "self_attn.v_proj.weight", norm)
        qin = norm if markers is None else norm[markers]
        pos = np.arange(n) if markers is None else np.asarray(markers)
        qz = _apply(oracle, model, p + "self_attn.q_proj.weight", qin).reshape(len(qin), ah, 2 * AD)
        q = np.ascontiguousarray(qz[:, :, :AD]).reshape(len(qin), ah * AD)
        z = np.ascontiguousarray(qz[:, :, AD:]).reshape(len(qin), ah * AD)
        freq = oracle.rope_freq()
        q = oracle.rope(_head_norm(oracle, q, ah, v[p + "self_attn.q_norm.weight"]), ah, AD, pos, freq)
        key = oracle.rope(_head_norm(oracle, key, akv, v[p + "self_attn.k_norm.weight"]), akv, AD, np.arange(n), freq)
        heads = oracle.attention_gqa(q, key, value, ah, akv, AD, 1.0 / 16.0)
        ctx = oracle.attention_gate(heads, z)
        proj = _apply(oracle, model, p + "self_attn.o_proj.weight", ctx)
        if markers is not None:
            h = h[markers]
    else:
        lh, lk = c["delta_heads"], c["delta_key_heads"]
        cw = conv_width(c)
        qkv = _apply(oracle, model, p + "linear_attn.in_proj_qkv.weight", norm)
        z = _apply(oracle, model, p + "linear_attn.in_proj_z.weight", norm)
        a = _apply(oracle, model, p + "linear_attn.in_proj_a.weight", norm)
        b = _apply(oracle, model, p + "linear_attn.in_proj_b.weight", norm)
        taps = v[p + "linear_attn.conv1d.weight"].reshape(cw, 4).T.copy()   # backbone.rs:170-178
        conv = oracle.conv_silu(qkv, taps)
        decay = np.exp(v[p + "linear_attn.A_log"]).astype(np.float32)
        heads = oracle.delta_scan(conv, lh, lk, LD, a, b, decay, v[p + "linear_attn.dt_bias"])
        ctx = oracle.delta_gate(heads, v[p + "linear_attn.norm.weight"], z)
        proj = _apply(oracle, model, p + "linear_attn.out_proj.weight", ctx)
    h = (h + proj).astype(np.float32)
    norm = oracle.rmsnorm(h, v[p + "post_attention_layernorm.weight"], 1e-6, zero_centered=True)
    gate = _apply(oracle, model, p + "mlp.gate_proj.weight", norm)
    up = _apply(oracle, model, p + "mlp.up_proj.weight", norm)
    act = oracle.silu_mul(gate, up)
    return (h + _apply(oracle, model, p + "mlp.down_proj.weight", act)).astype(np.float32)


def ref_forward(oracle, model, ids, markers):
    """native.rs:193-274 for one chunk: embedding rows, every layer (the last
    one cut to the markers when it is an attention layer), readout logits."""
    if model.rows is not None:  # quantized_rows.rs:89-110 over the fitted rows
        codes, scales, nf4 = model.rows
        h = oracle.rows_decode(codes[ids], scales[ids], None, nf4, len(ids), model.cfg["hidden"])
    else:
        rows = model.embedding[ids]
        h = oracle.unpack_g64(rows.reshape(-1), 4).reshape(len(ids), -1)
    layers = model.cfg["layers"]
    prune = (layers - 1) % 4 == 3
    for i in range(layers):
        h = ref_layer(oracle, model, i, h, markers if (prune and i == layers - 1) else None)
    if not prune:
        h = h[markers]
    x = oracle.rmsnorm(h, model.vectors["language_model.norm.weight"], 1e-6, zero_centered=True)
    wire = model.packed["readout"][0]
    return np.stack([oracle.project(wire, 4, model.cfg["hidden"], x[r], 255) for r in range(len(markers))])
