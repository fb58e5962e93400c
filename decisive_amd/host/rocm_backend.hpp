// rocm_backend.hpp -- the Rocm backend: decisive's Backend contract
// (src/inference/mod.rs:140-154) over the C ABI of libdecisive_rocm.so.
//
// It takes the place of `impl Backend for pplx_flash::Model` (the native CPU
// backend, src/inference/adapters.rs:168-194) for the Pplx-style encoder of
// BASELINE configuration 3:
//   Parameters = PplxParameters (maxSequenceTokens, default 1024, 0 rejected)
//   CacheState = EmbeddingCache (packed Q4 g64/f32 embedding rows by token id)
//   capabilities = {model "pplx-flash", backend "rocm", caches ["embedding"], tuning "auto"}
// A request's `state` carries tokens, already encoded (tokenization, the
// reference's input.rs plan, is outside this path), in one of two forms:
//  - an array of token ids: the embedding response. Like the reference, input
//    is never truncated: a sequence longer than maxSequenceTokens is split
//    into chunks, each run as its own sequence (input.rs:227-282 splits
//    requests rather than truncating); one mean-pooled embedding per chunk.
//  - {"chunks": [{"ids", "markers", "keys", "counts"}, ...]}: the encoded
//    chunks as the reference's inspect() lists them (mod.rs:186-191,
//    input.rs:7-13 Encoded). Each chunk runs the encoder, the readout of the
//    hidden rows at its markers (mod.rs:149-185) and the answer step
//    (input.rs:284-326) for each key's question, as native.rs:193-274 does;
//    the response is {"answers", "usage"} as there.
#pragma once

#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "answer.hpp"
#include "chunks.hpp"
#include "decisive_rocm.h"
#include "embedding_cache.hpp"
#include "inference.hpp"
#include "packed_checkpoint.hpp"

namespace decisive {

// A dz_status as the reference's Error (same code strings).
inline Error status_error(const dz_ctx *ctx, int32_t status) {
    return Error(dz_status_name(status), ctx ? dz_last_error(ctx) : "no context");
}

class Rocm {
public:
    using Parameters = PplxParameters;
    using CacheState = EmbeddingCache;

    // Opens device `device`, optionally runs the kernel tuner (TuningOptions,
    // parameters.rs:13-28) and builds a random-init encoder (`seed`).
    static Result<Rocm> create(int device, const dz_encoder_config &config, uint64_t seed,
                               const TuningOptions &tuning = TuningOptions{}) {
        Rocm r;
        int32_t rc = dz_init(device, &r.ctx_);
        if (rc != DZ_OK) return status_error(nullptr, rc);
        if (tuning.mode == TuningMode::Auto && tuning.budget_ms > 0) {
            std::string cache_in = tuning.cache ? tuning.cache->dump() : std::string();
            std::vector<char> out(1 << 16);
            rc = dz_tune(r.ctx_, tuning.budget_ms, tuning.cache ? cache_in.c_str() : nullptr, out.data(), out.size());
            if (rc != DZ_OK) return status_error(r.ctx_, rc);
            r.tuning_ = Json::parse(out.data());
        }
        rc = dz_encoder_create_random(r.ctx_, &config, seed, &r.encoder_);
        if (rc != DZ_OK) return status_error(r.ctx_, rc);
        rc = dz_encoder_embedding_row_bytes(r.encoder_, &r.row_bytes_);
        if (rc != DZ_OK) return status_error(r.ctx_, rc);
        r.config_ = config;
        rc = dz_alloc(r.ctx_, (size_t)config.hidden * sizeof(float), &r.out_dev_);
        if (rc != DZ_OK) return status_error(r.ctx_, rc);
        return r;
    }

    // A backend whose embedding rows, decision readout, final norm and answer
    // temperature come from a packed checkpoint directory (validated with
    // every file digest, as prepare_hf_q4.py:71-114 does; browser/pplx.rs:
    // 140-330 loads the same parts). The embedding cache reads its misses from
    // the checkpoint's embedding file (browser/pplx.rs:76-137). The encoder
    // layers stay random-init from `seed`: the checkpoint's decoder layers
    // belong to a different architecture. config.hidden must be the
    // checkpoint's; config.vocab is taken from it. Embedding rows are read in
    // the Q4 format (q4-e4).
    static Result<Rocm> create_from_checkpoint(int device, const std::string &dir, dz_encoder_config config,
                                               uint64_t seed, const TuningOptions &tuning = TuningOptions{},
                                               const PackedModel &model = PackedModel{}) {
        auto ck = PackedCheckpoint::open(dir, model);
        if (!ck) return ck.error();
        if (ck.value().format().bits != 4)
            return Error("UNSUPPORTED_FORMAT", "the Rocm encoder reads q4-e4 embedding rows");
        if ((size_t)config.hidden != model.hidden)
            return Error("INVALID_PARAMETERS", "encoder hidden size differs from the checkpoint's");
        config.vocab = (int32_t)ck.value().vocab();
        auto made = create(device, config, seed, tuning);
        if (!made) return made.error();
        Rocm r = made.take();
        auto readout = ck.value().readout_bytes();
        if (!readout) return readout.error();
        auto norm = ck.value().norm();
        if (!norm) return norm.error();
        int32_t rc = dz_encoder_set_readout(r.ctx_, r.encoder_, readout.value().data(), readout.value().size(),
                                            ck.value().layout(), norm.value().data());
        if (rc != DZ_OK) return status_error(r.ctx_, rc);
        auto t = ck.value().temperature();
        if (t) {
            Status s = r.set_temperature(t.value());
            if (!s) return s.error();
        }
        r.checkpoint_ = std::make_shared<PackedCheckpoint>(ck.take());
        return r;
    }

    Rocm(Rocm &&o) noexcept { *this = std::move(o); }
    Rocm &operator=(Rocm &&o) noexcept {
        if (this != &o) {
            release();
            ctx_ = std::exchange(o.ctx_, nullptr);
            encoder_ = std::exchange(o.encoder_, nullptr);
            out_dev_ = std::exchange(o.out_dev_, nullptr);
            row_bytes_ = o.row_bytes_;
            config_ = o.config_;
            temperature_ = o.temperature_;
            checkpoint_ = std::move(o.checkpoint_);
            tuning_ = std::move(o.tuning_);
        }
        return *this;
    }
    Rocm(const Rocm &) = delete;
    Rocm &operator=(const Rocm &) = delete;
    ~Rocm() { release(); }

    dz_ctx *context() const { return ctx_; }
    dz_encoder *encoder() const { return encoder_; }
    size_t row_bytes() const { return row_bytes_; }
    const dz_encoder_config &config() const { return config_; }
    const Json &tuning() const { return tuning_; }

    // The decision temperature of the answer softmax (decision_config.json's
    // "temperature" in the reference, input.rs:127-131: finite and positive).
    Status set_temperature(float t) {
        if (!(std::isfinite(t) && t > 0.0f)) return Error::engine("invalid temperature");
        temperature_ = t;
        return {};
    }
    float temperature() const { return temperature_; }

    Capabilities capabilities() const { return Capabilities{"pplx-flash", "rocm", {"embedding"}, "auto"}; }
    Result<EmbeddingCache> create_cache(const CacheOptions &options) const {
        return EmbeddingCache(options.max_bytes);
    }
    void clear_cache(EmbeddingCache &cache) const { cache.clear(); }

    Result<Json> predict(const Request &request, const PplxParameters &parameters, EmbeddingCache &cache,
                         const Cancellation &cancellation) {
        Status s = parameters.validate();
        if (!s) return s.error();
        if (request.state.is_object()) return predict_answers(request, parameters, cache, cancellation);
        auto ids = token_ids(request);
        if (!ids) return ids.error();
        const std::vector<uint32_t> &all = ids.value();
        Json embeddings = Json::array();
        const size_t step = parameters.max_sequence_tokens;
        for (size_t at = 0; at < all.size(); at += step) {
            s = cancellation.check();
            if (!s) return s.error();
            std::vector<uint32_t> chunk(all.begin() + at, all.begin() + std::min(all.size(), at + step));
            auto rows = cache.load(chunk, [this](const std::vector<uint32_t> &miss) { return read_rows(miss); },
                                   row_bytes_, cancellation);
            if (!rows) return rows.error();
            auto embedding = forward(rows.value(), chunk.size());
            if (!embedding) return embedding.error();
            Json e = Json::array();
            for (float v : embedding.value()) e.push_back(Json((double)v));
            embeddings.push_back(std::move(e));
        }
        Json out = Json::object();
        out["embeddings"] = std::move(embeddings);
        out["tokens"] = Json((uint64_t)all.size());
        out["chunks"] = Json((uint64_t)((all.size() + step - 1) / step));
        return out;
    }

    // Logits [markers x DZ_READOUT_CODES] of one sequence given as packed rows.
    Result<std::vector<float>> readout(const std::vector<uint8_t> &rows, size_t tokens,
                                       const std::vector<int32_t> &markers) {
        std::vector<float> logits(markers.size() * DZ_READOUT_CODES);
        int32_t rc = dz_encoder_readout_rows(ctx_, encoder_, rows.data(), tokens, markers.data(), markers.size(),
                                             logits.data());
        if (rc != DZ_OK) return status_error(ctx_, rc);
        return logits;
    }

    // The packed rows of `ids`: from the checkpoint's embedding file when the
    // backend was opened on one, else from the encoder's own table.
    Result<std::vector<uint8_t>> read_rows(const std::vector<uint32_t> &ids) const {
        if (checkpoint_) return checkpoint_->embedding_rows(ids);
        std::vector<int32_t> as_i32(ids.begin(), ids.end());
        std::vector<uint8_t> out(ids.size() * row_bytes_);
        int32_t rc = dz_encoder_read_rows(ctx_, encoder_, as_i32.data(), ids.size(), out.data());
        if (rc != DZ_OK) return status_error(ctx_, rc);
        return out;
    }

    // Mean-pooled embedding of one sequence given as packed rows.
    Result<std::vector<float>> forward(const std::vector<uint8_t> &rows, size_t tokens) {
        int32_t rc = dz_encoder_forward_rows(ctx_, encoder_, rows.data(), 1, tokens, (float *)out_dev_);
        if (rc != DZ_OK) return status_error(ctx_, rc);
        std::vector<float> host((size_t)config_.hidden);
        rc = dz_copy_d2h(ctx_, host.data(), out_dev_, host.size() * sizeof(float));
        if (rc != DZ_OK) return status_error(ctx_, rc);
        return host;
    }

private:
    Rocm() = default;

    // native.rs:193-274 over encoded chunks, reading out with the encoder.
    Result<Json> predict_answers(const Request &request, const PplxParameters &parameters, EmbeddingCache &cache,
                                 const Cancellation &cancellation) {
        return answer_chunks(
            request, parameters, cache, cancellation, (uint32_t)config_.vocab, row_bytes_, temperature_,
            [this](const std::vector<uint32_t> &miss) { return read_rows(miss); },
            [this](const std::vector<uint8_t> &rows, size_t tokens, const std::vector<int32_t> &markers) {
                return readout(rows, tokens, markers);
            });
    }

    Result<std::vector<uint32_t>> token_ids(const Request &request) const {
        if (!request.state.is_array() || request.state.size() == 0)
            return Error("INVALID_REQUEST", "state must be a nonempty array of token ids");
        std::vector<uint32_t> ids;
        ids.reserve(request.state.size());
        for (const Json &v : request.state.as_array()) {
            double d = v.is_number() ? v.as_number() : -1.0;
            if (d < 0 || d >= (double)config_.vocab || d != (double)(uint32_t)d)
                return Error("INVALID_REQUEST", "token id outside the vocabulary");
            ids.push_back((uint32_t)d);
        }
        return ids;
    }

    void release() {
        if (ctx_) {
            if (out_dev_) dz_free(ctx_, out_dev_);
            if (encoder_) dz_encoder_destroy(ctx_, encoder_);
            dz_destroy(ctx_);
        }
        ctx_ = nullptr;
        encoder_ = nullptr;
        out_dev_ = nullptr;
    }

    dz_ctx *ctx_ = nullptr;
    dz_encoder *encoder_ = nullptr;
    void *out_dev_ = nullptr;
    size_t row_bytes_ = 0;
    dz_encoder_config config_{};
    Json tuning_;
    float temperature_ = 1.0f;
    std::shared_ptr<PackedCheckpoint> checkpoint_;
};

}  // namespace decisive
