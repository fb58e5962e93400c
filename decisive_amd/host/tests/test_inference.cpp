// test_inference.cpp -- the host layer's inference API on the CPU.
//
// The first four tests port the reference's src/inference/tests.rs:17-141
// (a fake backend exercising Model<B>); the rest cover the Error code
// mapping (tests.rs:208-249 engine part), the EmbeddingCache of
// browser/pplx.rs:45-138 and the JSON value.
#include <string>
#include <vector>

#include "../embedding_cache.hpp"
#include "../inference.hpp"
#include "harness.hpp"

using namespace decisive;

namespace {

// tests.rs:17-49
struct TestBackend {
    using Parameters = size_t;
    using CacheState = std::vector<std::string>;
    Capabilities capabilities() const { return Capabilities{"test", "cpu", {"prefix"}, "off"}; }
    Result<CacheState> create_cache(const CacheOptions &) const { return CacheState{}; }
    void clear_cache(CacheState &cache) const { cache.clear(); }
    Result<Json> predict(const Request &request, const size_t &parameters, CacheState &cache,
                         const Cancellation &cancellation) {
        Status s = cancellation.check();
        if (!s) return s.error();
        cache.push_back(request.state.as_string());
        if (request.state.as_string() == "fail") return Error("TEST_FAILURE", "failed after updating scratch");
        Json out = Json::object();
        out["retained"] = Json((uint64_t)cache.size());
        out["parameter"] = Json((uint64_t)parameters);
        return out;
    }
};

// A backend without prefix caches (as the Pplx backends are).
struct PlainBackend : TestBackend {
    Capabilities capabilities() const { return Capabilities{"test", "cpu", {}, "off"}; }
};

// tests.rs:50-55
Request request(const std::string &state) {
    return Request::from_json(Json::parse("{\"state\":\"" + state + "\",\"questions\":{\"q\":{\"type\":\"noul\"}}}"))
        .take();
}

}  // namespace

// tests.rs:57-79
TEST(batches_reuse_one_cache_and_keep_order_and_per_item_failures) {
    Model<TestBackend> model(TestBackend{}, 5);
    auto cache = model.create_cache(CacheOptions{});
    CHECK(cache.ok());
    auto outcomes = model.predict_batch({request("first"), request("second"), request("fail"), request("last")},
                                        nullptr, &cache.value(), Cancellation{});
    CHECK(outcomes.ok());
    Json value = Json::array();
    for (const Outcome &o : outcomes.value()) value.push_back(o.to_json());
    CHECK_EQ(value[0]["result"]["response"]["retained"], Json(1));
    CHECK_EQ(value[1]["result"]["response"]["retained"], Json(2));
    CHECK_EQ(value[1]["result"]["response"]["parameter"], Json(5));
    CHECK_EQ(value[2]["error"]["code"], Json("TEST_FAILURE"));
    CHECK_EQ(value[2]["status"], Json("error"));
    // the failure cleared the shared cache (mod.rs:240-242)
    CHECK_EQ(value[3]["result"]["response"]["retained"], Json(1));
    CHECK_EQ(value[3]["status"], Json("success"));
}

// tests.rs:81-114
TEST(cache_ownership_ephemeral_calls_and_cancellation) {
    Model<TestBackend> first(TestBackend{});
    Model<TestBackend> second(TestBackend{});
    auto foreign = first.create_cache(CacheOptions{});
    auto r = second.predict(request("x"), nullptr, &foreign.value(), Cancellation{});
    CHECK(!r.ok());
    CHECK_EQ(r.error().code, std::string("CACHE_OWNER"));
    CHECK_EQ(second.clear_cache(foreign.value()).error().code, std::string("CACHE_OWNER"));
    for (int i = 0; i < 2; i++) {
        size_t seven = 7;
        auto ok = second.predict(request("x"), &seven, nullptr, Cancellation{});
        CHECK(ok.ok());
        CHECK_EQ(ok.value().response["retained"], Json(1));
        CHECK_EQ(ok.value().response["parameter"], Json(7));
    }
    Cancellation cancellation;
    Cancellation clone = cancellation;  // clones share the flag
    clone.cancel();
    auto batch = second.predict_batch({request("x"), request("y")}, nullptr, nullptr, cancellation);
    CHECK(batch.ok());
    for (const Outcome &o : batch.value()) {
        CHECK(!o.success());
        CHECK_EQ(o.error->code, std::string("CANCELLED"));
    }
    // a foreign cache fails the whole batch before any item (mod.rs:257-259)
    auto foreign_batch = second.predict_batch({request("x")}, nullptr, &foreign.value(), Cancellation{});
    CHECK(!foreign_batch.ok());
    CHECK_EQ(foreign_batch.error().code, std::string("CACHE_OWNER"));
}

// tests.rs:116-131
TEST(parameter_types_reject_options_from_other_models) {
    CHECK(!PplxParameters::from_json(Json::parse(R"({"long":true})")).ok());
    CHECK(PplxParameters::from_json(Json::parse(R"({"maxSequenceTokens":1024})")).ok());
    CHECK(PplxParameters::from_json(Json::parse(R"({})")).value().max_sequence_tokens == 1024);
    PplxParameters zero;
    zero.max_sequence_tokens = 0;
    CHECK(!zero.validate().ok());
    CHECK_EQ(zero.validate().error().code, std::string("INVALID_PARAMETERS"));
    CHECK(!Request::from_json(Json::parse(R"({"state":"x","questions":{},"long":true})")).ok());
    CHECK(!TuningOptions::from_json(Json::parse(R"({"budget":5})")).ok());
    CHECK(!CacheOptions::from_json(Json::parse(R"({"maxBytes":1,"prefix":true})")).ok());
    auto t = TuningOptions::from_json(Json::parse(R"({"mode":"off","budgetMs":0})"));
    CHECK(t.ok() && t.value().mode == TuningMode::Off && t.value().budget_ms == 0);
    CHECK(!TuningOptions::from_json(Json::parse(R"({"mode":"fast"})")).ok());
    // request validation (mod.rs:26-38)
    Request empty_questions = Request::from_json(Json::parse(R"({"state":"x","questions":{}})")).take();
    CHECK_EQ(empty_questions.validate().error().code, std::string("INVALID_REQUEST"));
    Request number_state = Request::from_json(Json::parse(R"({"state":3,"questions":{"q":1}})")).take();
    CHECK(!number_state.validate().ok());
    Request ids = Request::from_json(Json::parse(R"({"state":[1,2],"questions":{"q":1}})")).take();
    CHECK(ids.validate().ok());
}

// tests.rs:133-141
TEST(tuning_budget_stops_new_selection_stages) {
    CHECK(!TuningBudget(false, std::nullopt, 0.0).permits(0.0));
    CHECK(!TuningBudget(true, 0u, 10.0).permits(10.0));
    TuningBudget budget(true, 20u, 10.0);
    CHECK(budget.permits(29.0));
    CHECK(!budget.permits(30.0));
    CHECK(TuningBudget(true, std::nullopt, 0.0).permits(std::numeric_limits<double>::max()));
}

// mod.rs:174-186
TEST(prefix_cache_requires_a_prefix_backend) {
    Model<PlainBackend> model(PlainBackend{});
    CacheOptions options;
    options.require_prefix = true;
    auto cache = model.create_cache(options);
    CHECK(!cache.ok());
    CHECK_EQ(cache.error().code, std::string("UNSUPPORTED_CACHE"));
    options.require_prefix = false;
    CHECK(model.create_cache(options).ok());
}

// tests.rs:236-249 (the engine-code part) and mod.rs:56-78
TEST(engine_errors_map_to_stable_codes) {
    CHECK_EQ(Error::engine("an unrelated engine failure").code, std::string("INFERENCE_FAILED"));
    CHECK_EQ(Error::engine("mixed FP16 checkpoints require the fp16 Cargo feature").code,
             std::string("FORMAT_NOT_COMPILED"));
    CHECK_EQ(Error::engine("INT8 requires the int8 Cargo feature").code, std::string("FORMAT_NOT_COMPILED"));
    CHECK_EQ(Error::engine("input budget exceeded").code, std::string("INPUT_TOO_LONG"));
    CHECK_EQ(Error::engine("prompt exceeds token limit").code, std::string("INPUT_TOO_LONG"));
    CHECK_EQ(Error::engine("GPU storage buffer of 100 bytes exceeds device limits").code,
             std::string("RESOURCE_LIMIT"));
    CHECK_EQ(Error::engine("required WebGPU precision is unavailable").code, std::string("MISSING_GPU_FEATURE"));
    CHECK_EQ(Error::engine("no WebGPU compute adapter").code, std::string("GPU_UNAVAILABLE"));
    Error e = Error::engine("x");
    CHECK_EQ(e.to_string(), std::string("INFERENCE_FAILED: x"));
}

// ---- EmbeddingCache (browser/pplx.rs:45-138) -----------------------------------------

namespace {

struct FakeTable {
    size_t row_bytes = 4;
    std::vector<std::vector<uint32_t>> calls;
    bool truncate = false;
    Result<std::vector<uint8_t>> operator()(const std::vector<uint32_t> &ids) {
        calls.push_back(ids);
        std::vector<uint8_t> out;
        for (uint32_t id : ids)
            for (size_t b = 0; b < row_bytes; b++) out.push_back((uint8_t)(id * 7 + b));
        if (truncate) out.pop_back();
        return out;
    }
};

std::vector<uint8_t> expected_rows(const std::vector<uint32_t> &ids, size_t row_bytes) {
    std::vector<uint8_t> out;
    for (uint32_t id : ids)
        for (size_t b = 0; b < row_bytes; b++) out.push_back((uint8_t)(id * 7 + b));
    return out;
}

}  // namespace

TEST(embedding_cache_is_lru_under_a_byte_budget) {
    FakeTable table;
    EmbeddingCache cache(3 * 4);  // three rows of 4 bytes
    auto reader = [&](const std::vector<uint32_t> &ids) { return table(ids); };
    auto r = cache.load({1, 2, 3}, reader, 4, Cancellation{});
    CHECK(r.ok() && r.value() == expected_rows({1, 2, 3}, 4));
    CHECK_EQ(cache.rows(), (size_t)3);
    // touching 1 makes 2 the oldest; loading 4 evicts it
    r = cache.load({1}, reader, 4, Cancellation{});
    CHECK(r.ok());
    CHECK_EQ(table.calls.size(), (size_t)1);  // a hit reads nothing
    r = cache.load({4}, reader, 4, Cancellation{});
    CHECK(cache.contains(1) && cache.contains(3) && cache.contains(4) && !cache.contains(2));
    CHECK_EQ(cache.order().front(), 3u);
    CHECK_EQ(cache.order().back(), 4u);
    CHECK_EQ(cache.hits(), (uint64_t)1);
    CHECK_EQ(cache.misses(), (uint64_t)4);
}

TEST(embedding_cache_dedups_reads_in_chunks_of_eight_and_keeps_order) {
    FakeTable table;
    EmbeddingCache cache(1 << 20);
    auto reader = [&](const std::vector<uint32_t> &ids) { return table(ids); };
    std::vector<uint32_t> ids = {5, 9, 5, 1, 2, 3, 4, 6, 7, 8, 10, 11, 9};
    auto r = cache.load(ids, reader, 4, Cancellation{});
    CHECK(r.ok() && r.value() == expected_rows(ids, 4));
    CHECK_EQ(table.calls.size(), (size_t)2);
    CHECK_EQ(table.calls[0].size(), (size_t)8);
    CHECK_EQ(table.calls[1].size(), (size_t)3);  // 11 distinct ids
    CHECK_EQ(table.calls[0][0], 5u);
    CHECK_EQ(table.calls[0][1], 9u);
}

TEST(embedding_cache_keeps_nothing_over_budget_and_rejects_short_rows) {
    FakeTable table;
    auto reader = [&](const std::vector<uint32_t> &ids) { return table(ids); };
    EmbeddingCache zero(0);  // the ephemeral cache of Model::predict (mod.rs:214-223)
    auto r = zero.load({1, 1, 2}, reader, 4, Cancellation{});
    CHECK(r.ok() && r.value() == expected_rows({1, 1, 2}, 4));
    CHECK_EQ(zero.rows(), (size_t)0);
    EmbeddingCache small(3);  // smaller than one row
    CHECK(small.load({1}, reader, 4, Cancellation{}).ok());
    CHECK_EQ(small.rows(), (size_t)0);
    table.truncate = true;
    EmbeddingCache cache(64);
    auto bad = cache.load({1, 2}, reader, 4, Cancellation{});
    CHECK(!bad.ok());
    CHECK_EQ(bad.error().code, std::string("INVALID_CHECKPOINT"));
}

TEST(embedding_cache_checks_cancellation_before_each_read) {
    FakeTable table;
    auto reader = [&](const std::vector<uint32_t> &ids) { return table(ids); };
    EmbeddingCache cache(1 << 20);
    Cancellation c;
    c.cancel();
    auto r = cache.load({1, 2}, reader, 4, c);
    CHECK(!r.ok());
    CHECK_EQ(r.error().code, std::string("CANCELLED"));
    CHECK(table.calls.empty());
    // all hits: nothing to read, nothing to cancel
    CHECK(cache.load({}, reader, 4, c).ok());
}

TEST(json_round_trips_and_rejects_malformed_text) {
    Json j = Json::parse(R"({"b":[1,2.5,-3e2,true,null,"x\n\u00e9"],"a":{}})");
    CHECK_EQ(j.dump(), std::string("{\"a\":{},\"b\":[1,2.5,-300,true,null,\"x\\n\xc3\xa9\"]}"));
    CHECK(Json::parse(j.dump()) == j);
    for (const char *bad : {"{", "[1,]", "01", "\"\\x\"", "{\"a\" 1}", "tru", "1 2", "\"\\ud800\""}) {
        bool threw = false;
        try {
            Json::parse(bad);
        } catch (const std::exception &) {
            threw = true;
        }
        CHECK(threw);
    }
    Json copy = j;
    copy["c"] = 1;  // copy on write leaves the original alone
    CHECK(j["c"].is_null());
}

int main(int argc, char **argv) { return harness::run_all(argc, argv); }
