// encoder.hip -- the encoder forward of BASELINE configuration 3 on the
// quantized-product kernels.
//
// Layer order follows the reference's post-LayerNorm encoder
// (src/models/decima/mod.rs:492-560: projections, attention, output
// projection + residual, LayerNorm, GELU feed-forward + residual, LayerNorm),
// with the Pplx-style Q4 projections (all linear weights Q4, f16 activations)
// and mean pooling (src/models/decima/cpu.rs:574-586). Token rows come from a
// Q4 group-64 embedding table (quantized_rows.rs) either by id on the device or
// as packed rows handed over by the embedding-row cache.
#include <string.h>

#include <string>
#include <vector>

#include "../../include/decisive_rocm.h"
#include "kernels.hpp"

namespace dz {

int32_t ctx_fail(dz_ctx *ctx, int32_t code, const std::string &msg);
int32_t ctx_hip_fail(dz_ctx *ctx, hipError_t e, const char *what);
hipStream_t ctx_stream(dz_ctx *ctx);
int *ctx_flag(dz_ctx *ctx);
int ctx_variant(dz_ctx *ctx, const char *family);
const Weight &weight_of(const dz_weight *h);
int32_t weight_quantize(dz_ctx *ctx, const void *values, int dtype, size_t rows, size_t cols, int bits,
                        int group, dz_weight **out);
void weight_free(dz_weight *h);
int32_t weight_upload(dz_ctx *ctx, const void *packed, size_t bytes, int32_t layout, size_t rows, size_t cols,
                      dz_weight **out);
int32_t ctx_readout_rows(dz_ctx *ctx, const Weight &w, const float *norm, const void *hidden, int dtype,
                         const int32_t *select, size_t rows, float eps, float *logits);

}  // namespace dz

namespace dz {
constexpr int kReadoutCodes = DZ_READOUT_CODES;
constexpr int kReadoutMarkers = DZ_READOUT_MAX_MARKERS;
constexpr float kReadoutEps = DZ_READOUT_EPS;
}  // namespace dz

struct dz_encoder {
    dz_encoder_config cfg{};
    struct Layer {
        dz_weight *qkv = nullptr, *o = nullptr, *up = nullptr, *down = nullptr;
        float *ln1w = nullptr, *ln1b = nullptr, *ln2w = nullptr, *ln2b = nullptr;
    };
    std::vector<Layer> layers;
    dz_weight *embed = nullptr;          // [vocab x hidden] Q4 group-64
    // the decision readout (pplx_flash/mod.rs:149-185): 255 rows x hidden, Q4
    // group-64 as the packed readout, after a zero-centred RMSNorm
    dz_weight *readout = nullptr;
    float *readout_norm = nullptr;
    int32_t *markers = nullptr;          // device copy of the readout rows of one request
    float *logits = nullptr;             // [kReadoutMarkers x 255]
    std::vector<uint8_t> embed_wire;     // the same table in the packed.rs layout (host)
    float *ln0w = nullptr, *ln0b = nullptr;
    // activations (f16) sized for `capacity` tokens
    size_t capacity = 0;
    dz::half_t *h = nullptr, *qkv = nullptr, *att = nullptr, *t = nullptr, *ff = nullptr;
    int32_t *ids = nullptr;
    // packed rows staging for the cache path
    uint8_t *rows_dev = nullptr;
    dz::Weight rows_weight;
};

namespace dz {

namespace {

void free_buffers(dz_encoder *e) {
    for (void *p : {(void *)e->h, (void *)e->qkv, (void *)e->att, (void *)e->t, (void *)e->ff,
                    (void *)e->ids, (void *)e->rows_dev, (void *)e->rows_weight.codes,
                    (void *)e->rows_weight.scales})
        if (p) hipFree(p);
    e->h = e->qkv = e->att = e->t = e->ff = nullptr;
    e->ids = nullptr;
    e->rows_dev = nullptr;
    e->rows_weight.codes = e->rows_weight.scales = nullptr;
    e->capacity = 0;
}

int32_t ensure_capacity(dz_ctx *ctx, dz_encoder *e, size_t tokens) {
    if (e->capacity >= tokens) return DZ_OK;
    hipStreamSynchronize(ctx_stream(ctx));
    free_buffers(e);
    const dz_encoder_config &c = e->cfg;
    size_t d = (size_t)c.hidden;
    hipError_t err = hipSuccess;
    auto get = [&](void **p, size_t bytes) {
        if (err == hipSuccess) err = hipMalloc(p, bytes);
    };
    get((void **)&e->h, tokens * d * 2);
    get((void **)&e->qkv, tokens * d * 3 * 2);
    get((void **)&e->att, tokens * d * 2);
    get((void **)&e->t, tokens * d * 2);
    get((void **)&e->ff, tokens * (size_t)c.ffn * 2);
    get((void **)&e->ids, tokens * 4);
    // a scratch Q4 group-64 weight of `tokens` rows receives cache-provided packed rows
    Weight &w = e->rows_weight;
    w.kind = WeightKind::Q4G64;
    w.bits = 4;
    w.group = 64;
    w.rows = (int)tokens;
    w.cols = c.hidden;
    w.groups = c.hidden / 64;
    w.np = (int)((tokens + 15) / 16 * 16);
    w.kp = (c.hidden + 127) / 128 * 128;
    w.code_bytes = (size_t)w.np * w.kp / 2;
    w.scale_bytes = (size_t)w.np * (w.kp / 128) * 8;
    get((void **)&w.codes, w.code_bytes);
    get((void **)&w.scales, w.scale_bytes);
    get((void **)&e->rows_dev, tokens * (d / 64) * 36);
    if (err != hipSuccess) {
        free_buffers(e);
        return ctx_hip_fail(ctx, err, "encoder activations");
    }
    e->capacity = tokens;
    return DZ_OK;
}

int32_t random_weight(dz_ctx *ctx, float *scratch, size_t rows, size_t cols, uint64_t seed, int bits,
                      int group, dz_weight **out) {
    launch_fill_normal_f32(scratch, rows * cols, seed, 0.02f, ctx_stream(ctx));
    return weight_quantize(ctx, scratch, 0, rows, cols, bits, group, out);
}

int32_t const_vec(dz_ctx *ctx, float **p, size_t n, float v) {
    hipError_t e = hipMalloc(p, n * sizeof(float));
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "encoder parameters");
    launch_fill_f32(*p, n, v, ctx_stream(ctx));
    return DZ_OK;
}

}  // namespace

void encoder_destroy(dz_ctx *ctx, dz_encoder *e) {
    if (!e) return;
    hipStreamSynchronize(ctx_stream(ctx));
    for (auto &l : e->layers) {
        weight_free(l.qkv);
        weight_free(l.o);
        weight_free(l.up);
        weight_free(l.down);
        for (float *p : {l.ln1w, l.ln1b, l.ln2w, l.ln2b})
            if (p) hipFree(p);
    }
    weight_free(e->embed);
    weight_free(e->readout);
    for (void *p : {(void *)e->ln0w, (void *)e->ln0b, (void *)e->readout_norm, (void *)e->markers,
                    (void *)e->logits})
        if (p) hipFree(p);
    free_buffers(e);
    delete e;
}

int32_t encoder_create_random(dz_ctx *ctx, const dz_encoder_config *cfg, uint64_t seed,
                              dz_encoder **out) {
    if (!cfg || !out) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    *out = nullptr;
    const dz_encoder_config c = *cfg;
    if (c.layers < 1 || c.hidden < 64 || c.hidden % 128 != 0 || c.heads < 1 || c.head_dim != 64 ||
        c.heads * c.head_dim != c.hidden || c.ffn < 128 || c.ffn % 128 != 0 || c.vocab < 1)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS,
                        "encoder needs head_dim 64, hidden = heads*64, hidden and ffn multiples of 128");
    dz_encoder *e = new dz_encoder();
    e->cfg = c;
    size_t d = (size_t)c.hidden, f = (size_t)c.ffn;
    size_t biggest = std::max(std::max(3 * d * d, f * d), (size_t)c.vocab * d);
    float *scratch = nullptr;
    hipError_t err = hipMalloc(&scratch, biggest * sizeof(float));
    if (err != hipSuccess) {
        delete e;
        return ctx_hip_fail(ctx, err, "encoder init scratch");
    }
    int32_t rc = DZ_OK;
    uint64_t s = seed * 1000003ull;
    rc = random_weight(ctx, scratch, (size_t)c.vocab, d, s++, 4, 64, &e->embed);
    if (!rc) rc = const_vec(ctx, &e->ln0w, d, 1.0f);
    if (!rc) rc = const_vec(ctx, &e->ln0b, d, 0.0f);
    e->layers.resize(c.layers);
    for (int l = 0; l < c.layers && !rc; l++) {
        auto &L = e->layers[l];
        rc = random_weight(ctx, scratch, 3 * d, d, s++, 4, 32, &L.qkv);
        if (!rc) rc = random_weight(ctx, scratch, d, d, s++, 4, 32, &L.o);
        if (!rc) rc = random_weight(ctx, scratch, f, d, s++, 4, 32, &L.up);
        if (!rc) rc = random_weight(ctx, scratch, d, f, s++, 4, 32, &L.down);
        if (!rc) rc = const_vec(ctx, &L.ln1w, d, 1.0f);
        if (!rc) rc = const_vec(ctx, &L.ln1b, d, 0.0f);
        if (!rc) rc = const_vec(ctx, &L.ln2w, d, 1.0f);
        if (!rc) rc = const_vec(ctx, &L.ln2b, d, 0.0f);
    }
    if (!rc) rc = random_weight(ctx, scratch, kReadoutCodes, d, s++, 4, 64, &e->readout);
    if (!rc) {
        // zero-centred norm weights near zero, as a trained model's are
        hipError_t err2 = hipMalloc(&e->readout_norm, d * sizeof(float));
        if (err2 == hipSuccess) err2 = hipMalloc(&e->markers, kReadoutMarkers * sizeof(int32_t));
        if (err2 == hipSuccess) err2 = hipMalloc(&e->logits, (size_t)kReadoutMarkers * kReadoutCodes * sizeof(float));
        if (err2 != hipSuccess) rc = ctx_hip_fail(ctx, err2, "encoder readout");
        else launch_fill_normal_f32(e->readout_norm, d, s++, 0.02f, ctx_stream(ctx));
    }
    if (!rc) {
        // host copy of the embedding table in the wire layout (the cache's source)
        size_t wire_bytes = (size_t)c.vocab * (d / 64) * 36;
        e->embed_wire.resize(wire_bytes);
        uint8_t *wire = (uint8_t *)scratch;  // scratch holds >= vocab*d floats
        launch_export_q4g64(weight_of(e->embed), wire, ctx_stream(ctx));
        err = hipMemcpyAsync(e->embed_wire.data(), wire, wire_bytes, hipMemcpyDeviceToHost, ctx_stream(ctx));
        if (err == hipSuccess) err = hipStreamSynchronize(ctx_stream(ctx));
        if (err != hipSuccess) rc = ctx_hip_fail(ctx, err, "embedding export");
    }
    hipStreamSynchronize(ctx_stream(ctx));
    hipFree(scratch);
    if (rc) {
        encoder_destroy(ctx, e);
        return rc;
    }
    *out = e;
    return DZ_OK;
}

const dz_weight *encoder_weight(const dz_encoder *e, int layer, int which) {
    if (!e) return nullptr;
    if (which == 4) return e->embed;
    if (which == 5) return e->readout;
    if (layer < 0 || layer >= (int)e->layers.size()) return nullptr;
    const auto &L = e->layers[layer];
    switch (which) {
        case 0: return L.qkv;
        case 1: return L.o;
        case 2: return L.up;
        case 3: return L.down;
        default: return nullptr;
    }
}

int32_t encoder_row_bytes(const dz_encoder *e, size_t *row_bytes) {
    if (!e || !row_bytes) return DZ_INVALID_REQUEST;
    *row_bytes = (size_t)e->cfg.hidden / 64 * 36;
    return DZ_OK;
}

int32_t encoder_read_rows(dz_ctx *ctx, const dz_encoder *e, const int32_t *ids, size_t count,
                          void *out) {
    if (!e || (count && (!ids || !out))) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    size_t rb = (size_t)e->cfg.hidden / 64 * 36;
    for (size_t i = 0; i < count; i++) {
        if (ids[i] < 0 || ids[i] >= e->cfg.vocab) return ctx_fail(ctx, DZ_INVALID_REQUEST, "token ID out of range");
        memcpy((uint8_t *)out + i * rb, e->embed_wire.data() + (size_t)ids[i] * rb, rb);
    }
    return DZ_OK;
}

namespace {

// The encoder layers over batch x seq tokens, leaving the last hidden states
// (f16 [batch*seq x hidden]) in e->h.
int32_t encoder_hidden(dz_ctx *ctx, dz_encoder *e, const int32_t *ids_dev, const void *rows_host,
                       size_t batch, size_t seq) {
    if (batch == 0 || seq == 0) return ctx_fail(ctx, DZ_INVALID_REQUEST, "empty batch");
    size_t tokens = batch * seq;
    if (tokens > (1u << 20)) return ctx_fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    if (!attention_fits(seq, (size_t)e->cfg.heads)) return ctx_fail(ctx, DZ_INPUT_TOO_LONG, "sequence too long");
    int32_t rc = ensure_capacity(ctx, e, tokens);
    if (rc) return rc;
    const dz_encoder_config &c = e->cfg;
    hipStream_t s = ctx_stream(ctx);
    const int m = (int)tokens, d = c.hidden;
    const int gv = ctx_variant(ctx, "gemm_w4a16");
    // token rows -> f16 hidden
    if (rows_host) {
        size_t bytes = tokens * (size_t)(d / 64) * 36;
        hipError_t err = hipMemcpyAsync(e->rows_dev, rows_host, bytes, hipMemcpyHostToDevice, s);
        if (err != hipSuccess) return ctx_hip_fail(ctx, err, "row upload");
        Weight &w = e->rows_weight;
        w.rows = m;
        int bad = 0;
        launch_fill_i32(ctx_flag(ctx), 0, 1, s);
        launch_upload(w, e->rows_dev, ctx_flag(ctx), s);
        launch_dequant(w, nullptr, m, e->h, 1, s);
        err = hipMemcpyAsync(&bad, ctx_flag(ctx), sizeof(int), hipMemcpyDeviceToHost, s);
        if (err == hipSuccess) err = hipStreamSynchronize(s);
        if (err != hipSuccess) return ctx_hip_fail(ctx, err, "row upload");
        if (bad) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "invalid packed scale");
    } else {
        int bad = 0;
        launch_fill_i32(ctx_flag(ctx), 0, 1, s);
        launch_dequant_checked(weight_of(e->embed), ids_dev, m, e->h, 1, ctx_flag(ctx), s);
        hipError_t err = hipMemcpyAsync(&bad, ctx_flag(ctx), sizeof(int), hipMemcpyDeviceToHost, s);
        if (err == hipSuccess) err = hipStreamSynchronize(s);
        if (err != hipSuccess) return ctx_hip_fail(ctx, err, "embedding gather");
        if (bad) return ctx_fail(ctx, DZ_INVALID_REQUEST, "token ID out of range");
    }
    launch_layernorm(e->h, e->h, 1, m, d, e->ln0w, e->ln0b, c.ln_eps, s);
    const float scale = 1.0f / 8.0f;  // 1/sqrt(64)
    for (auto &L : e->layers) {
        launch_w4a16_f16(weight_of(L.qkv), e->h, m, e->qkv, 0, nullptr, gv, s);
        launch_attention(e->qkv, e->att, (int)batch, (int)seq, c.heads, 64, scale, s);
        launch_w4a16_f16(weight_of(L.o), e->att, m, e->t, 2, e->h, gv, s);
        launch_layernorm(e->t, e->h, 1, m, d, L.ln1w, L.ln1b, c.ln_eps, s);
        launch_w4a16_f16(weight_of(L.up), e->h, m, e->ff, 1, nullptr, gv, s);
        launch_w4a16_f16(weight_of(L.down), e->ff, m, e->t, 2, e->h, gv, s);
        launch_layernorm(e->t, e->h, 1, m, d, L.ln2w, L.ln2b, c.ln_eps, s);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return ctx_hip_fail(ctx, err, "encoder forward");
    return DZ_OK;
}

}  // namespace

int32_t encoder_forward(dz_ctx *ctx, dz_encoder *e, const int32_t *ids_dev, const void *rows_host,
                        size_t batch, size_t seq, float *out) {
    if (!e || !out || (!ids_dev && !rows_host)) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    int32_t rc = encoder_hidden(ctx, e, ids_dev, rows_host, batch, seq);
    if (rc) return rc;
    launch_mean_rows(e->h, 1, (int)batch, (int)seq, e->cfg.hidden, out, ctx_stream(ctx));
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return ctx_hip_fail(ctx, err, "encoder forward");
    return DZ_OK;
}

int32_t encoder_hidden_rows(dz_ctx *ctx, dz_encoder *e, const void *rows_host, size_t seq, float *hidden) {
    if (!e || !rows_host || !hidden) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    int32_t rc = encoder_hidden(ctx, e, nullptr, rows_host, 1, seq);
    if (rc) return rc;
    launch_to_f32(e->h, 1, seq * (size_t)e->cfg.hidden, hidden, ctx_stream(ctx));
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return ctx_hip_fail(ctx, err, "encoder hidden rows");
    return DZ_OK;
}

int32_t encoder_readout_params(const dz_encoder *e, const dz_weight **w, const float **norm) {
    if (!e) return DZ_INVALID_REQUEST;
    if (w) *w = e->readout;
    if (norm) *norm = e->readout_norm;
    return DZ_OK;
}

int32_t encoder_set_readout(dz_ctx *ctx, dz_encoder *e, const void *packed, size_t bytes, int32_t layout,
                            const float *norm_host) {
    if (!e || !packed || !norm_host) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (layout != DZ_Q4_G64_F32 && layout != DZ_Q8_G64_F32)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS, "the readout is a group-64 packed matrix");
    dz_weight *w = nullptr;
    int32_t rc = weight_upload(ctx, packed, bytes, layout, kReadoutCodes, (size_t)e->cfg.hidden, &w);
    if (rc) return rc;
    hipStream_t s = ctx_stream(ctx);
    hipError_t err = hipMemcpyAsync(e->readout_norm, norm_host, (size_t)e->cfg.hidden * sizeof(float),
                                    hipMemcpyHostToDevice, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err != hipSuccess) {
        weight_free(w);
        return ctx_hip_fail(ctx, err, "readout norm upload");
    }
    weight_free(e->readout);
    e->readout = w;
    return DZ_OK;
}

int32_t encoder_readout(dz_ctx *ctx, dz_encoder *e, const void *rows_host, size_t seq, const int32_t *markers,
                        size_t count, float *logits_host) {
    if (!e || !rows_host || (count && (!markers || !logits_host)))
        return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (count == 0) return ctx_fail(ctx, DZ_INVALID_REQUEST, "no readout markers");
    if (count > (size_t)kReadoutMarkers) return ctx_fail(ctx, DZ_INPUT_TOO_LONG, "too many readout markers");
    for (size_t i = 0; i < count; i++)
        if (markers[i] < 0 || (size_t)markers[i] >= seq)
            return ctx_fail(ctx, DZ_INVALID_REQUEST, "readout marker outside the sequence");
    int32_t rc = encoder_hidden(ctx, e, nullptr, rows_host, 1, seq);
    if (rc) return rc;
    hipStream_t s = ctx_stream(ctx);
    hipError_t err = hipMemcpyAsync(e->markers, markers, count * sizeof(int32_t), hipMemcpyHostToDevice, s);
    if (err != hipSuccess) return ctx_hip_fail(ctx, err, "marker upload");
    rc = ctx_readout_rows(ctx, weight_of(e->readout), e->readout_norm, e->h, 1, e->markers, count,
                          kReadoutEps, e->logits);
    if (rc) return rc;
    err = hipMemcpyAsync(logits_host, e->logits, count * (size_t)kReadoutCodes * sizeof(float),
                         hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err != hipSuccess) return ctx_hip_fail(ctx, err, "logits readback");
    return DZ_OK;
}

}  // namespace dz
