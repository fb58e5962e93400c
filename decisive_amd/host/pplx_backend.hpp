// pplx_backend.hpp -- the Pplx decider behind decisive's Backend contract
// (src/inference/mod.rs:140-154), on a packed checkpoint: the drop-in for
// `impl Backend for pplx_flash::Model` (src/inference/adapters.rs:168-194).
//
// RocmPplx::open validates the packed checkpoint (every file digest,
// prepare_hf_q4.py:71-114), uploads each decoder tensor by its checkpoint
// name (dz_pplx_set_weight for the packed 2-D projections, dz_pplx_set_vector
// for the BF16 vectors), the readout and the final norm, and reads the answer
// temperature of decision_config.json (input.rs:127-131). Requests carry the
// encoded chunks ({"chunks": [...]}, as inspect() lists them, mod.rs:186-191:
// tokenization is the reference's input.rs, outside this path); each chunk's
// embedding rows come through the EmbeddingCache from the checkpoint's
// embedding file (browser/pplx.rs:76-137), the forward and readout run on the
// device (dz_pplx_forward_rows) and the answers follow input.rs:284-326.
#pragma once

#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "chunks.hpp"
#include "decisive_rocm.h"
#include "embedding_cache.hpp"
#include "inference.hpp"
#include "packed_checkpoint.hpp"

namespace decisive {

class RocmPplx {
public:
    using Parameters = PplxParameters;
    using CacheState = EmbeddingCache;

    // The reference's decoder shape (backbone.rs:11-22) for `layers` layers.
    static dz_pplx_config reference_config(int layers = 32) {
        dz_pplx_config c{};
        c.layers = layers;
        c.hidden = 2560;
        c.ff = 9216;
        c.delta_heads = 32;
        c.delta_key_heads = 16;
        c.delta_head_dim = 128;
        c.attn_heads = 16;
        c.attn_kv_heads = 4;
        c.attn_head_dim = 256;
        return c;
    }

    // `residency` DZ_PPLX_STREAMED keeps the layer projections in pinned host
    // memory and runs each layer from one of two device banks
    // (webgpu/streaming.rs:16-369); the answers are the same bits.
    // `tuning` (parameters.rs:13-28) runs the kernel tuner's selection stages
    // on open, as checkpoint_with_tuning does on every load
    // (webgpu/checkpoint.rs:241-262): the delta scan, the norm, the grouped
    // product and the fused MLP among variants that give their reference's
    // bits, within budget_ms, reusing a cached selection whose key matches.
    // The selection JSON is tuning(); mode "off" or a zero budget keeps the
    // reference variants.
    static Result<RocmPplx> open(int device, const std::string &dir, const dz_pplx_config &config,
                                 const PackedModel &model = PackedModel{}, int32_t residency = DZ_PPLX_RESIDENT,
                                 const TuningOptions &tuning = TuningOptions{}) {
        if ((size_t)config.layers != model.layers || (size_t)config.hidden != model.hidden)
            return Error("INVALID_PARAMETERS", "decoder shape differs from the checkpoint's");
        auto ck = PackedCheckpoint::open(dir, model);
        if (!ck) return ck.error();
        if (ck.value().format().bits != 4)
            return Error("UNSUPPORTED_FORMAT", "the Rocm decider reads q4-e4 embedding rows");
        RocmPplx r;
        int32_t rc = dz_init(device, &r.ctx_);
        if (rc != DZ_OK) return Error(dz_status_name(rc), "no context");
        if (tuning.mode == TuningMode::Auto && tuning.budget_ms > 0) {
            const std::string cache_in = tuning.cache ? tuning.cache->dump() : std::string();
            std::vector<char> out(1 << 16);
            rc = dz_tune(r.ctx_, tuning.budget_ms, tuning.cache ? cache_in.c_str() : nullptr, out.data(), out.size());
            if (rc != DZ_OK) return r.fail(rc);
            r.tuning_ = Json::parse(out.data());
        }
        rc = dz_pplx_create(r.ctx_, &config, &r.model_);
        if (rc != DZ_OK) return r.fail(rc);
        const PackedCheckpoint &c = ck.value();
        for (size_t i = 0; i < c.layers().size(); i++)
            for (const PackedTensor &t : c.layers()[i].tensors) {
                auto bytes = c.tensor(i, t.name);
                if (!bytes) return bytes.error();
                if (t.shape.size() == 2) {
                    rc = dz_pplx_set_weight(r.ctx_, r.model_, t.name.c_str(), bytes.value().data(),
                                            bytes.value().size(), c.layout(), t.shape[0], t.shape[1]);
                } else {
                    std::vector<float> values = bf16_values(bytes.value());
                    rc = dz_pplx_set_vector(r.ctx_, r.model_, t.name.c_str(), values.data(), values.size());
                }
                if (rc != DZ_OK) return r.fail(rc);
            }
        auto readout = c.readout_bytes();
        if (!readout) return readout.error();
        rc = dz_pplx_set_weight(r.ctx_, r.model_, "readout", readout.value().data(), readout.value().size(),
                                c.layout(), model.readout_rows, model.hidden);
        if (rc != DZ_OK) return r.fail(rc);
        auto norm = c.norm();
        if (!norm) return norm.error();
        rc = dz_pplx_set_vector(r.ctx_, r.model_, "language_model.norm.weight", norm.value().data(), norm.value().size());
        if (rc != DZ_OK) return r.fail(rc);
        rc = dz_pplx_set_residency(r.ctx_, r.model_, residency);
        if (rc != DZ_OK) return r.fail(rc);
        auto t = c.temperature();
        if (!t) return t.error();
        r.temperature_ = t.value();
        r.checkpoint_ = std::make_shared<PackedCheckpoint>(ck.take());
        return r;
    }

    RocmPplx(RocmPplx &&o) noexcept { *this = std::move(o); }
    RocmPplx &operator=(RocmPplx &&o) noexcept {
        if (this != &o) {
            release();
            ctx_ = std::exchange(o.ctx_, nullptr);
            model_ = std::exchange(o.model_, nullptr);
            temperature_ = o.temperature_;
            checkpoint_ = std::move(o.checkpoint_);
            tuning_ = std::move(o.tuning_);
        }
        return *this;
    }
    RocmPplx(const RocmPplx &) = delete;
    RocmPplx &operator=(const RocmPplx &) = delete;
    ~RocmPplx() { release(); }

    dz_ctx *context() const { return ctx_; }
    dz_pplx *model() const { return model_; }
    float temperature() const { return temperature_; }
    // The tuner's selection JSON of the last open (null when it did not run).
    const Json &tuning() const { return tuning_; }
    const PackedCheckpoint &checkpoint() const { return *checkpoint_; }

    Capabilities capabilities() const { return Capabilities{"pplx-flash", "rocm", {"embedding"}, "auto"}; }
    Result<EmbeddingCache> create_cache(const CacheOptions &options) const { return EmbeddingCache(options.max_bytes); }
    void clear_cache(EmbeddingCache &cache) const { cache.clear(); }

    Result<Json> predict(const Request &request, const PplxParameters &parameters, EmbeddingCache &cache,
                         const Cancellation &cancellation) {
        Status s = parameters.validate();
        if (!s) return s.error();
        if (!request.state.is_object())
            return Error("INVALID_REQUEST", "state must hold the encoded chunks ({\"chunks\": [...]})");
        return answer_chunks(
            request, parameters, cache, cancellation, (uint32_t)checkpoint_->vocab(), checkpoint_->row_bytes(),
            temperature_, [this](const std::vector<uint32_t> &miss) { return checkpoint_->embedding_rows(miss); },
            [this](const std::vector<uint8_t> &rows, size_t tokens, const std::vector<int32_t> &markers) {
                return logits(rows, tokens, markers);
            });
    }

    // Logits [markers x DZ_READOUT_CODES] of one chunk of packed rows.
    Result<std::vector<float>> logits(const std::vector<uint8_t> &rows, size_t tokens,
                                      const std::vector<int32_t> &markers) {
        std::vector<float> out(markers.size() * DZ_READOUT_CODES);
        int32_t rc = dz_pplx_forward_rows(ctx_, model_, rows.data(), tokens, markers.data(), markers.size(), out.data());
        if (rc != DZ_OK) return Error(dz_status_name(rc), dz_last_error(ctx_));
        return out;
    }

private:
    RocmPplx() = default;

    static std::vector<float> bf16_values(const std::vector<uint8_t> &raw) {
        std::vector<float> out(raw.size() / 2);
        for (size_t i = 0; i < out.size(); i++) {
            const uint32_t bits = (uint32_t)(raw[2 * i] | raw[2 * i + 1] << 8) << 16;
            std::memcpy(&out[i], &bits, 4);
        }
        return out;
    }

    Error fail(int32_t rc) { return Error(dz_status_name(rc), ctx_ ? dz_last_error(ctx_) : "no context"); }

    void release() {
        if (ctx_) {
            if (model_) dz_pplx_destroy(ctx_, model_);
            dz_destroy(ctx_);
        }
        ctx_ = nullptr;
        model_ = nullptr;
    }

    dz_ctx *ctx_ = nullptr;
    dz_pplx *model_ = nullptr;
    float temperature_ = 1.0f;
    std::shared_ptr<PackedCheckpoint> checkpoint_;
    Json tuning_;
};

}  // namespace decisive
