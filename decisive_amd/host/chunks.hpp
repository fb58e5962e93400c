// chunks.hpp -- the answer path shared by the Rocm backends: a request whose
// state is {"chunks": [...]}, each chunk the reference's Encoded (input.rs:7-13:
// ids, markers, keys, counts, as inspect() lists them, mod.rs:186-191), runs
// the forward and readout of every chunk and the answer step of each key
// (native.rs:193-274), giving {"answers", "usage"} as the reference does.
#pragma once

#include <string>
#include <vector>

#include "answer.hpp"
#include "decisive_rocm.h"
#include "embedding_cache.hpp"
#include "inference.hpp"
#include "json.hpp"

namespace decisive {

struct EncodedChunk {
    std::vector<uint32_t> ids;
    std::vector<int32_t> markers;
    std::vector<std::string> keys;
    std::vector<size_t> counts;
};

inline bool whole_below(const Json &v, double limit) {
    return v.is_number() && v.as_number() >= 0 && v.as_number() < limit &&
           v.as_number() == (double)(uint64_t)v.as_number();
}

inline Result<EncodedChunk> parse_chunk(const Json &c, const Json &questions, uint32_t vocab, size_t max_tokens) {
    if (!c.is_object() || !c["ids"].is_array() || !c["markers"].is_array() || !c["keys"].is_array() ||
        !c["counts"].is_array())
        return Error("INVALID_REQUEST", "each chunk needs ids, markers, keys and counts arrays");
    EncodedChunk e;
    for (const Json &v : c["ids"].as_array()) {
        if (!whole_below(v, (double)vocab)) return Error("INVALID_REQUEST", "token id outside the vocabulary");
        e.ids.push_back((uint32_t)v.as_number());
    }
    if (e.ids.empty()) return Error("INVALID_REQUEST", "a chunk needs at least one token");
    if (e.ids.size() > max_tokens) return Error::engine("chunk exceeds token limit");
    for (const Json &v : c["markers"].as_array()) {
        if (!whole_below(v, (double)e.ids.size())) return Error("INVALID_REQUEST", "readout marker outside the chunk");
        e.markers.push_back((int32_t)v.as_number());
    }
    for (const Json &v : c["keys"].as_array()) {
        if (!v.is_string() || !questions[v.as_string()].is_object())
            return Error("INVALID_REQUEST", "chunk key without a question");
        e.keys.push_back(v.as_string());
    }
    for (const Json &v : c["counts"].as_array()) {
        if (!whole_below(v, (double)DZ_READOUT_CODES + 1) || v.as_number() < 1)
            return Error("INVALID_REQUEST", "answer count outside 1..255");
        e.counts.push_back((size_t)v.as_number());
    }
    if (e.markers.size() != e.keys.size() || e.keys.size() != e.counts.size() || e.markers.empty() ||
        e.markers.size() > DZ_READOUT_MAX_MARKERS)
        return Error("INVALID_REQUEST", "markers, keys and counts must pair up (1..256 per chunk)");
    return e;
}

// ReadRows: ids -> packed rows (the cache's miss reader). Readout: (packed
// rows, tokens, markers) -> logits [markers x DZ_READOUT_CODES].
template <class ReadRows, class Readout>
Result<Json> answer_chunks(const Request &request, const PplxParameters &parameters, EmbeddingCache &cache,
                           const Cancellation &cancellation, uint32_t vocab, size_t row_bytes, float temperature,
                           ReadRows read_rows, Readout readout) {
    const Json &chunks = request.state["chunks"];
    if (!chunks.is_array() || chunks.size() == 0 || request.state.size() != 1)
        return Error("INVALID_REQUEST", "state must hold a nonempty chunks array");
    std::vector<EncodedChunk> plan;
    for (const Json &c : chunks.as_array()) {
        auto e = parse_chunk(c, request.questions, vocab, parameters.max_sequence_tokens);
        if (!e) return e.error();
        plan.push_back(e.take());
    }
    Json answers = Json::object();
    uint64_t tokens = 0;
    for (const EncodedChunk &e : plan) {
        Status s = cancellation.check();
        if (!s) return s.error();
        auto rows = cache.load(e.ids, read_rows, row_bytes, cancellation);
        if (!rows) return rows.error();
        auto logits = readout(rows.value(), e.ids.size(), e.markers);
        if (!logits) return logits.error();
        for (size_t i = 0; i < e.keys.size(); i++) {
            const float *row = logits.value().data() + i * DZ_READOUT_CODES;
            std::vector<float> values(row, row + e.counts[i]);
            auto a = answer(request.questions[e.keys[i]], values, temperature);
            if (!a) return a.error();
            answers[e.keys[i]] = a.take();
        }
        tokens += e.ids.size();
    }
    Json usage = Json::object();
    usage["input_tokens"] = Json(tokens);
    usage["output_tokens"] = Json(0);
    usage["sequences"] = Json((uint64_t)plan.size());
    Json out = Json::object();
    out["answers"] = std::move(answers);
    out["usage"] = std::move(usage);
    return out;
}

}  // namespace decisive
