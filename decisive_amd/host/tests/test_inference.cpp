// test_inference.cpp -- the host layer's inference API on the CPU.
//
// The first four tests port the reference's src/inference/tests.rs:17-141
// (a fake backend exercising Model<B>); the rest cover the Error code
// mapping (tests.rs:208-249 engine part), the EmbeddingCache of
// browser/pplx.rs:45-138 and the JSON value.
#include <string>
#include <vector>

#include <fstream>
#include <sstream>
#include <unistd.h>

#include <cstdlib>
#include <filesystem>

#include "../answer.hpp"
#include "../embedding_cache.hpp"
#include "../inference.hpp"
#include "../packed_checkpoint.hpp"
#include "../sha256.hpp"
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
    // members keep their order; -3e2 is a float, written as serde_json does
    CHECK_EQ(j.dump(), std::string("{\"b\":[1,2.5,-300.0,true,null,\"x\\n\xc3\xa9\"],\"a\":{}}"));
    CHECK(j["b"][0].is_integer() && !j["b"][2].is_integer());
    CHECK_EQ(Json(0.1).dump(), std::string("0.1"));
    CHECK_EQ(Json(1e16).dump(), std::string("10000000000000000.0"));
    CHECK_EQ(Json(1e22).dump(), std::string("1e22"));
    CHECK_EQ(Json(1e-7).dump(), std::string("1e-7"));
    CHECK_EQ(Json(0.000123).dump(), std::string("0.000123"));
    CHECK_EQ(Json(-0.0).dump(), std::string("-0.0"));
    // objects compare as maps: order does not matter
    CHECK(Json::parse(R"({"x":1,"y":2})") == Json::parse(R"({"y":2,"x":1})"));
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

// ---- answer step (input.rs:21-112, :284-326) ------------------------------------

// tests/golden/<name>, found from this program's path (decisive_amd/host/build/).
static Json golden(const char *name) {
    char exe[4096];
    ssize_t n = readlink("/proc/self/exe", exe, sizeof exe - 1);
    std::string path = n > 0 ? std::string(exe, (size_t)n) : std::string();
    path = path.substr(0, path.rfind('/')) + "/../../../tests/golden/" + name;
    std::ifstream f(path);
    std::stringstream text;
    text << f.rdbuf();
    return Json::parse(text.str());
}

// pplx_flash/mod.rs compare(): numbers within tol, objects by key with equal
// sizes, everything else exactly.
static bool close(const Json &a, const Json &b, double tol) {
    if (a.is_number() && b.is_number()) return std::fabs(a.as_number() - b.as_number()) <= tol;
    if (a.is_object() && b.is_object()) {
        if (a.size() != b.size()) return false;
        for (const auto &kv : a.as_object())
            if (!close(kv.second, b[kv.first], tol)) return false;
        return true;
    }
    return a == b;
}

static std::vector<float> floats(const Json &a) {
    std::vector<float> v;
    for (const Json &x : a.as_array()) v.push_back((float)x.as_number());
    return v;
}

TEST(answers_match_the_reference_fixture_responses) {
    Json g = golden("pplx_answers.json");
    const float temperature = (float)g["temperature_fit"].as_number();
    const double tol = g["tolerance"].as_number();
    int checked = 0;
    for (const Json &c : g["cases"].as_array()) {
        for (const auto &kv : c["logits"].as_object()) {
            const Json &q = c["questions"][kv.first];
            auto a = answer(q, floats(kv.second), temperature);
            CHECK(a.ok());
            if (!a) continue;
            const Json &want = c["answers"][kv.first];
            CHECK(close(a.value(), want, tol));
            // the probabilities keep the question's order (preserve_order)
            if (want["probabilities"].is_object()) {
                std::vector<std::string> got_keys, want_keys;
                for (const auto &p : a.value()["probabilities"].as_object()) got_keys.push_back(p.first);
                for (const auto &p : want["probabilities"].as_object()) want_keys.push_back(p.first);
                CHECK(got_keys == want_keys);
            }
            // a wrong temperature is caught by the same comparison
            auto off = answer(q, floats(kv.second), 1.0f);
            CHECK(off.ok() && !close(off.value(), want, tol));
            checked++;
        }
    }
    CHECK_EQ(checked, 4);
}

TEST(answer_rejects_bad_questions_and_logit_counts) {
    Json choice = Json::parse(R"({"type":"choice","criteria":{"a":null,"b":null}})");
    CHECK(answer(choice, {1.f}, 1.f).error() == Error("INFERENCE_FAILED", "logit count mismatch"));
    CHECK(answer(Json::parse(R"({"type":"rank"})"), {1.f}, 1.f).error().message ==
          "question type must be choice, noul or score");
    CHECK(answer(Json::parse(R"({"type":"choice","criteria":[1]})"), {1.f}, 1.f).error().message ==
          "choice criteria must be an object");
    CHECK(answer(Json::parse(R"({"type":"noul","criteria":[]})"), {1.f, 2.f}, 1.f).error().message ==
          "noul criteria must be an object");
    // one option: confidence 1; ties pick the first maximum
    auto one = answer(Json::parse(R"({"type":"choice","criteria":{"only":null}})"), {3.f}, 1.f);
    CHECK(one.ok() && one.value()["confidence"].as_number() == 1.0 && one.value()["choice"].as_string() == "only");
    auto tie = answer(choice, {2.f, 2.f}, 1.f);
    CHECK(tie.ok() && tie.value()["choice"].as_string() == "a" && tie.value()["confidence"].as_number() == 0.0);
    // score: closed form on a two-level scale
    auto score = answer(Json::parse(R"({"type":"score","criteria":["low","high"]})"), {0.f, 0.f}, 1.f);
    CHECK(score.ok() && score.value()["score"].as_number() == 0.5 && score.value()["confidence"].as_number() == 0.0);
}

TEST(json_text_and_options_match_the_reference_known_answers) {
    Json g = golden("pplx_answers.json");
    for (const Json &c : g["json_text"].as_array()) CHECK_EQ(json_text(c["value"]), c["text"].as_string());
    for (const Json &c : g["options"].as_array()) {
        auto o = options(c["question"]);
        if (!c["error"].is_null()) {
            CHECK(!o.ok() && o.error().message == c["error"].as_string());
            continue;
        }
        CHECK(o.ok());
        if (!o) continue;
        std::vector<std::string> keys;
        for (const Json &k : c["keys"].as_array()) keys.push_back(k.as_string());
        CHECK(o.value().keys == keys);
        CHECK(Json(Json::Array(o.value().legend)) == c["legend"]);
    }
    CHECK_EQ(json_text(Json::parse("[1, 2.0, 0.5, 123456.75, 1e-5]")), std::string("[1, 2.0, 0.5, 123456.75, 1e-05]"));
}

// ---- SHA-256 and the packed checkpoint (prepare_hf_q4.py:31-114) ---------------------

TEST(sha256_matches_the_fips_180_known_answers) {
    CHECK_EQ(Sha256::of("", 0), std::string("e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"));
    CHECK_EQ(Sha256::of("abc", 3), std::string("ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"));
    const char *two = "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq";
    CHECK_EQ(Sha256::of(two, strlen(two)),
             std::string("248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"));
    Sha256 million;
    std::string a(1000, 'a');
    for (int i = 0; i < 1000; i++) million.update(a.data(), a.size());
    CHECK_EQ(million.hex(), std::string("cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"));
}

namespace fs = std::filesystem;

// The checkpoint that the test driver wrote (tests/test_host.py), copied to a
// fresh directory so a case may damage it.
static std::string checkpoint_copy(const char *tag) {
    const char *src = getenv("DZ_CHECKPOINT_DIR");
    if (!src) return std::string();
    fs::path dst = fs::temp_directory_path() / (std::string("dz_ck_") + tag + "_" + std::to_string(getpid()));
    fs::remove_all(dst);
    fs::copy(src, dst, fs::copy_options::recursive);
    return dst.string();
}

static Json read_json(const std::string &path) {
    std::ifstream f(path);
    std::stringstream t;
    t << f.rdbuf();
    return Json::parse(t.str());
}

static void write_json(const std::string &path, const Json &j) {
    std::ofstream f(path, std::ios::trunc);
    f << j.dump();
}

static std::string open_error(const std::string &dir) {
    auto c = PackedCheckpoint::open(dir);
    return c.ok() ? std::string("OK") : c.error().message;
}

TEST(checkpoint_accepts_the_complete_layout_and_reads_its_parts) {
    std::string dir = checkpoint_copy("ok");
    CHECK(!dir.empty());
    if (dir.empty()) return;
    auto c = PackedCheckpoint::open(dir);
    CHECK(c.ok());
    if (!c.ok()) {
        fprintf(stderr, "%s\n", c.error().message.c_str());
        return;
    }
    const PackedCheckpoint &ck = c.value();
    CHECK_EQ(ck.format().name, std::string("q4-e4"));
    CHECK_EQ(ck.row_bytes(), (size_t)1440);
    CHECK_EQ(ck.vocab(), (uint64_t)50);
    CHECK_EQ(ck.layers().size(), (size_t)32);
    // a tensor is its byte range of the layer file
    auto t = ck.tensor(7, "language_model.layers.7.norm.weight");
    CHECK(t.ok() && t.value().size() == 256);
    std::ifstream f(dir + "/q4-e4-layer-07.bin", std::ios::binary);
    std::vector<char> all((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    CHECK(t.ok() && std::memcmp(t.value().data(), all.data() + 288, 256) == 0);
    CHECK(!ck.tensor(7, "language_model.layers.8.norm.weight").ok());
    // embedding rows at id * row_bytes, in request order
    auto rows = ck.embedding_rows({3, 0, 3});
    std::ifstream e(dir + "/q4-e4-embedding.bin", std::ios::binary);
    std::vector<char> table((std::istreambuf_iterator<char>(e)), std::istreambuf_iterator<char>());
    CHECK(rows.ok() && std::memcmp(rows.value().data(), table.data() + 3 * 1440, 1440) == 0 &&
          std::memcmp(rows.value().data() + 1440, table.data(), 1440) == 0 &&
          std::memcmp(rows.value().data() + 2880, table.data() + 3 * 1440, 1440) == 0);
    CHECK(ck.embedding_rows({50}).error().code == "INVALID_REQUEST");
    auto norm = ck.norm();
    CHECK(norm.ok() && norm.value().size() == 2560 && std::isfinite(norm.value()[0]));
    auto temperature = ck.temperature();
    CHECK(temperature.ok() && temperature.value() == 1.5539091673122623f);
    CHECK(ck.readout_bytes().ok() && ck.readout_bytes().value().size() == 255 * 1440);
    fs::remove_all(dir);
}

// test_prepare_hf_q4.py:47-95: corrupt bytes, missing / duplicate /
// overlapping tensors, wrong source, extra payload, traversal and symlinks.
TEST(checkpoint_rejects_what_the_reference_validator_rejects) {
    std::string dir = checkpoint_copy("bad");
    if (dir.empty()) {
        CHECK(!dir.empty());
        return;
    }
    const std::string manifest_path = dir + "/packed-q4-e4.json";
    const Json original = read_json(manifest_path);
    auto with = [&](auto edit) {
        Json m = original;
        edit(m);
        write_json(manifest_path, m);
        std::string err = open_error(dir);
        write_json(manifest_path, original);
        return err;
    };
    CHECK_EQ(open_error(dir), std::string("OK"));
    // corrupt bytes
    {
        std::string layer = dir + "/q4-e4-layer-07.bin";
        std::ifstream in(layer, std::ios::binary);
        std::vector<char> keep((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
        std::vector<char> bad(keep.size(), 'x');
        std::ofstream(layer, std::ios::binary | std::ios::trunc).write(bad.data(), (std::streamsize)bad.size());
        CHECK(open_error(dir).find("Checksum") == 0);
        std::ofstream(layer, std::ios::binary | std::ios::trunc).write(keep.data(), (std::streamsize)keep.size());
    }
    auto tensors0 = [](Json &m) -> Json & { return m["layers"][0]["tensors"]; };
    CHECK_EQ(with([&](Json &m) { tensors0(m) = Json::array(); }), std::string("Missing layer tensors"));
    CHECK_EQ(with([&](Json &m) { tensors0(m).push_back(Json(tensors0(m)[0])); }),
             std::string("Unknown or repeated tensor"));
    CHECK_EQ(with([&](Json &m) { tensors0(m)[0]["start"] = Json(1); }), std::string("Invalid tensor range"));
    CHECK_EQ(with([&](Json &m) { m["revision"] = Json(std::string(40, '0')); }), std::string("Wrong source revision"));
    CHECK_EQ(with([&](Json &m) { m["scheme"] = Json("other"); }), std::string("Unsupported packed format"));
    CHECK_EQ(with([&](Json &m) {
                 Json extra = Json::object();
                 extra["bytes"] = Json(1);
                 extra["sha256"] = Json(std::string(64, '0'));
                 m["files"]["unexpected.bin"] = extra;
             }),
             std::string("Unexpected packed files"));
    CHECK_EQ(with([&](Json &m) { m["layers"][3]["file"] = Json("q4-e4-layer-04.bin"); }),
             std::string("Wrong layer filename/order"));
    CHECK_EQ(with([&](Json &m) { m["decoder_bytes"] = Json(1); }), std::string("Decoder total mismatch"));
    CHECK_EQ(with([&](Json &m) { m["group_bytes"] = Json(68); }), std::string("Wrong group layout"));
    CHECK_EQ(with([&](Json &m) { m["readout"] = Json("q4-e4-norm.bin"); }), std::string("Invalid readout payload"));
    // traversal and symlinks
    Json files = Json::object();
    files["../outside"] = Json::object();
    CHECK_EQ(PackedCheckpoint::verify_files(dir, files).error().message, std::string("Unsafe filename"));
    fs::create_symlink(dir + "/q4-e4-layer-00.bin", dir + "/link.bin");
    Json linked = Json::object();
    linked["link.bin"] = original["files"]["q4-e4-layer-00.bin"];
    CHECK(PackedCheckpoint::verify_files(dir, linked).error().message.find("symlink") != std::string::npos);
    // exactly one manifest
    fs::copy_file(manifest_path, dir + "/packed-q8-e8.json");
    CHECK_EQ(open_error(dir), std::string("Expected exactly one packed manifest"));
    fs::remove_all(dir);
}

TEST(checkpoint_reader_accepts_a_pplx_decoder_checkpoint) {
    const char *dir = getenv("DZ_PPLX_CHECKPOINT_DIR");
    CHECK(dir != nullptr);
    if (!dir) return;
    PackedModel pm;
    pm.layers = 4;
    pm.hidden = 256;
    auto c = PackedCheckpoint::open(dir, pm);
    CHECK(c.ok());
    if (!c.ok()) {
        fprintf(stderr, "%s\n", c.error().message.c_str());
        return;
    }
    // a delta layer holds 14 tensors, an attention layer 11 (backbone.rs:101-199)
    CHECK_EQ(c.value().layers()[0].tensors.size(), (size_t)14);
    CHECK_EQ(c.value().layers()[3].tensors.size(), (size_t)11);
    CHECK(!PackedCheckpoint::open(dir).ok());  // the reference's 32 x 2560 shape does not fit
}

int main(int argc, char **argv) { return harness::run_all(argc, argv); }
