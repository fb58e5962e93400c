// test_rocm_backend.cpp -- Model<Rocm> on an MI355X (needs the GPU).
//
// The Rocm backend behind the reference's Model<B> contract: predictions
// equal a direct dz_encoder_forward of the same token ids bit for bit, the
// embedding-row cache serves repeats without changing results, long inputs
// are split by maxSequenceTokens rather than truncated, and failures clear
// the cache (src/inference/mod.rs:240-242).
#include <cstdlib>
#include <cstring>
#include <vector>

#include <fstream>
#include <sstream>

#include "../pplx_backend.hpp"
#include "../rocm_backend.hpp"
#include "harness.hpp"

using namespace decisive;

namespace {

dz_encoder_config small_config() {
    dz_encoder_config c{};
    c.layers = 2;
    c.hidden = 256;
    c.heads = 4;
    c.head_dim = 64;
    c.ffn = 1024;
    c.vocab = 1000;
    c.ln_eps = 1e-5f;
    return c;
}

TuningOptions no_tuning() {
    TuningOptions t;
    t.mode = TuningMode::Off;
    return t;
}

std::vector<uint32_t> ids_of(size_t n, uint32_t seed) {
    std::vector<uint32_t> ids(n);
    uint32_t s = seed;
    for (auto &id : ids) {
        s = s * 1664525u + 1013904223u;
        id = (s >> 8) % 1000;
    }
    return ids;
}

Request request_of(const std::vector<uint32_t> &ids) {
    Request r;
    r.state = Json::array();
    for (uint32_t id : ids) r.state.push_back(Json((uint64_t)id));
    r.questions["embedding"] = Json::object();
    return r;
}

// Mean-pooled embedding of `ids` through dz_encoder_forward (ids on device).
std::vector<float> direct(Rocm &rocm, const std::vector<uint32_t> &ids) {
    dz_ctx *ctx = rocm.context();
    std::vector<int32_t> as_i32(ids.begin(), ids.end());
    void *ids_dev = nullptr, *out_dev = nullptr;
    std::vector<float> out((size_t)rocm.config().hidden);
    CHECK(dz_alloc(ctx, ids.size() * 4, &ids_dev) == DZ_OK);
    CHECK(dz_alloc(ctx, out.size() * 4, &out_dev) == DZ_OK);
    CHECK(dz_copy_h2d(ctx, ids_dev, as_i32.data(), ids.size() * 4) == DZ_OK);
    CHECK(dz_encoder_forward(ctx, rocm.encoder(), (const int32_t *)ids_dev, 1, ids.size(), (float *)out_dev) == DZ_OK);
    CHECK(dz_copy_d2h(ctx, out.data(), out_dev, out.size() * 4) == DZ_OK);
    dz_free(ctx, ids_dev);
    dz_free(ctx, out_dev);
    return out;
}

bool same_bits(const Json &embedding, const std::vector<float> &want) {
    if (!embedding.is_array() || embedding.size() != want.size()) return false;
    for (size_t i = 0; i < want.size(); i++) {
        float got = (float)embedding[i].as_number();
        if (std::memcmp(&got, &want[i], 4) != 0) return false;
    }
    return true;
}

Model<Rocm> make_model() {
    auto made = Rocm::create(0, small_config(), 7, no_tuning());
    if (!made.ok()) {
        fprintf(stderr, "Rocm::create failed: %s\n", made.error().to_string().c_str());
        std::exit(2);
    }
    return Model<Rocm>(made.take());
}

Json ids_json(const std::vector<uint32_t> &ids) {
    Json a = Json::array();
    for (uint32_t id : ids) a.push_back(Json((uint64_t)id));
    return a;
}

// {"chunks": [...]} state over encoded chunks with the three question kinds.
Request answer_request(const std::vector<uint32_t> &ids, std::vector<int> markers) {
    Request r;
    Json chunk = Json::object();
    chunk["ids"] = ids_json(ids);
    Json m = Json::array();
    for (int v : markers) m.push_back(Json(v));
    chunk["markers"] = m;
    chunk["keys"] = Json::parse(R"(["team","refund","tone"])");
    chunk["counts"] = Json::parse("[3,2,3]");
    r.state = Json::object();
    r.state["chunks"] = Json(Json::Array{chunk});
    r.questions = Json::parse(R"({
        "team": {"type": "choice", "criteria": {"billing": "Charges", "support": null, "sales": "Buying"}},
        "refund": {"type": "noul"},
        "tone": {"type": "score", "criteria": ["calm", "concerned", "angry"]}})");
    return r;
}

}  // namespace

TEST(rocm_answers_are_the_answer_step_over_the_readout_logits) {
    Model<Rocm> model = make_model();
    CHECK(model.backend().set_temperature(1.5539092f).ok());
    CHECK(!model.backend().set_temperature(0.0f).ok());
    auto cache = model.create_cache(CacheOptions{});
    CHECK(cache.ok());
    std::vector<uint32_t> ids = ids_of(120, 5);
    Request req = answer_request(ids, {40, 80, 119});
    auto got = model.predict(req, nullptr, &cache.value(), Cancellation{});
    CHECK(got.ok());
    if (!got.ok()) {
        fprintf(stderr, "%s\n", got.error().to_string().c_str());
        return;
    }
    const Json &resp = got.value().response;
    CHECK_EQ(resp["usage"]["input_tokens"], Json(120));
    CHECK_EQ(resp["usage"]["sequences"], Json(1));
    // the same logits through the C ABI, then the answer step on the host
    Rocm &rocm = model.backend();
    auto rows = rocm.read_rows(ids);
    CHECK(rows.ok());
    auto logits = rocm.readout(rows.value(), ids.size(), {40, 80, 119});
    CHECK(logits.ok());
    const char *keys[3] = {"team", "refund", "tone"};
    const size_t counts[3] = {3, 2, 3};
    for (int i = 0; i < 3; i++) {
        const float *row = logits.value().data() + i * DZ_READOUT_CODES;
        auto want = answer(req.questions[keys[i]], std::vector<float>(row, row + counts[i]), rocm.temperature());
        CHECK(want.ok() && resp["answers"][keys[i]] == want.value());
    }
    CHECK_EQ(resp["answers"]["team"]["type"], Json("choice"));
    CHECK(resp["answers"]["refund"]["noul"].is_number());
    CHECK(resp["answers"]["tone"]["legend"]["2"] == Json("angry"));
    // repeats come from the embedding cache and give the same answers
    uint64_t misses = cache.value().state().misses();
    auto again = model.predict(req, nullptr, &cache.value(), Cancellation{});
    CHECK(again.ok() && again.value().response == resp);
    CHECK_EQ(cache.value().state().misses(), misses);
}

TEST(rocm_backend_opened_on_a_packed_checkpoint) {
    const char *dir = getenv("DZ_CHECKPOINT_DIR");
    CHECK(dir != nullptr);
    if (!dir) return;
    dz_encoder_config cfg = small_config();
    cfg.layers = 1;
    cfg.hidden = 2560;
    cfg.heads = 40;
    cfg.ffn = 256;
    auto made = Rocm::create_from_checkpoint(0, dir, cfg, 7, no_tuning());
    CHECK(made.ok());
    if (!made.ok()) {
        fprintf(stderr, "%s\n", made.error().to_string().c_str());
        return;
    }
    Model<Rocm> model(made.take());
    Rocm &rocm = model.backend();
    auto ck = PackedCheckpoint::open(dir);
    CHECK(ck.ok());
    if (!ck.ok()) return;
    CHECK(rocm.temperature() == ck.value().temperature().value());
    CHECK_EQ(rocm.config().vocab, 50);
    std::vector<uint32_t> ids = {4, 49, 0, 4, 17, 23, 8, 31, 2, 11, 40, 6};
    // rows come from the checkpoint's embedding file
    auto rows = rocm.read_rows(ids);
    CHECK(rows.ok() && rows.value() == ck.value().embedding_rows(ids).value());
    // answers: the readout is the checkpoint's readout with its final norm
    Request req = answer_request(ids, {0, 5, 11});
    auto got = model.predict(req, nullptr, nullptr, Cancellation{});
    CHECK(got.ok());
    if (!got.ok()) {
        fprintf(stderr, "%s\n", got.error().to_string().c_str());
        return;
    }
    dz_ctx *ctx = rocm.context();
    void *hidden = nullptr, *sel = nullptr, *norm_dev = nullptr, *logits_dev = nullptr;
    const size_t d = 2560;
    CHECK(dz_alloc(ctx, ids.size() * d * 4, &hidden) == DZ_OK);
    CHECK(dz_alloc(ctx, 3 * d * 4, &sel) == DZ_OK);
    CHECK(dz_alloc(ctx, d * 4, &norm_dev) == DZ_OK);
    CHECK(dz_alloc(ctx, 3 * DZ_READOUT_CODES * 4, &logits_dev) == DZ_OK);
    CHECK(dz_encoder_hidden_rows(ctx, rocm.encoder(), rows.value().data(), ids.size(), (float *)hidden) == DZ_OK);
    std::vector<float> h(ids.size() * d), picked(3 * d);
    CHECK(dz_copy_d2h(ctx, h.data(), hidden, h.size() * 4) == DZ_OK);
    const int markers[3] = {0, 5, 11};
    for (int i = 0; i < 3; i++) std::memcpy(&picked[i * d], &h[markers[i] * d], d * 4);
    CHECK(dz_copy_h2d(ctx, sel, picked.data(), picked.size() * 4) == DZ_OK);
    auto norm = ck.value().norm();
    CHECK(dz_copy_h2d(ctx, norm_dev, norm.value().data(), d * 4) == DZ_OK);
    auto readout = ck.value().readout_bytes();
    dz_weight *w = nullptr;
    CHECK(dz_weight_upload(ctx, readout.value().data(), readout.value().size(), DZ_Q4_G64_F32, DZ_READOUT_CODES,
                           d, &w) == DZ_OK);
    CHECK(dz_readout(ctx, w, (const float *)norm_dev, (const float *)sel, 3, DZ_READOUT_EPS, (float *)logits_dev) ==
          DZ_OK);
    std::vector<float> logits(3 * DZ_READOUT_CODES);
    CHECK(dz_copy_d2h(ctx, logits.data(), logits_dev, logits.size() * 4) == DZ_OK);
    const char *keys[3] = {"team", "refund", "tone"};
    const size_t counts[3] = {3, 2, 3};
    for (int i = 0; i < 3; i++) {
        const float *row = logits.data() + i * DZ_READOUT_CODES;
        auto want = answer(req.questions[keys[i]], std::vector<float>(row, row + counts[i]), rocm.temperature());
        CHECK(want.ok() && got.value().response["answers"][keys[i]] == want.value());
    }
    dz_weight_free(ctx, w);
    for (void *p : {hidden, sel, norm_dev, logits_dev}) dz_free(ctx, p);
    // the embedding response of the same tokens is the forward of the file's rows
    auto emb = model.predict(request_of(ids), nullptr, nullptr, Cancellation{});
    CHECK(emb.ok());
    void *out_dev = nullptr;
    std::vector<float> want(d);
    CHECK(dz_alloc(ctx, d * 4, &out_dev) == DZ_OK);
    CHECK(dz_encoder_forward_rows(ctx, rocm.encoder(), rows.value().data(), 1, ids.size(), (float *)out_dev) == DZ_OK);
    CHECK(dz_copy_d2h(ctx, want.data(), out_dev, d * 4) == DZ_OK);
    dz_free(ctx, out_dev);
    CHECK(emb.ok() && same_bits(emb.value().response["embeddings"][0], want));
    // a checkpoint of another width is refused
    dz_encoder_config narrow = small_config();
    CHECK(Rocm::create_from_checkpoint(0, dir, narrow, 7, no_tuning()).error().code == "INVALID_PARAMETERS");
}

TEST(rocm_pplx_answers_from_a_packed_checkpoint) {
    const char *dir = getenv("DZ_PPLX_CHECKPOINT_DIR");
    CHECK(dir != nullptr);
    if (!dir) return;
    dz_pplx_config cfg{4, 256, 512, 4, 2, 128, 4, 2, 256};
    PackedModel pm;
    pm.layers = 4;
    pm.hidden = 256;
    // opened with the tuner (checkpoint.rs:241-262): the selection covers the
    // reference's four stages and this library's families, each selection one
    // whose output equals the reference variant's
    TuningOptions tuned;
    tuned.budget_ms = 4000;
    auto made = RocmPplx::open(0, dir, cfg, pm, DZ_PPLX_RESIDENT, tuned);
    CHECK(made.ok());
    if (!made.ok()) {
        fprintf(stderr, "%s\n", made.error().to_string().c_str());
        return;
    }
    const Json selection = made.value().tuning();
    CHECK(selection.is_object());
    for (const char *fam : {"delta_scan", "norm", "grouped", "mlp", "gemv", "gemm_w4a16", "i8_gemm"}) {
        CHECK(selection["selected"][fam].is_string());
        CHECK(selection["families"][fam].is_object());
        CHECK(selection["families"][fam]["skipped"].is_null());
    }
    CHECK(selection["families"]["delta_scan"]["candidates"].as_array().size() == 2);
    Model<RocmPplx> model(made.take());
    RocmPplx &pplx = model.backend();
    CHECK(pplx.temperature() == 1.5539091673122623f);
    std::ifstream f(std::string(dir) + "/expected_logits.json");
    std::stringstream text;
    text << f.rdbuf();
    Json expected = Json::parse(text.str());
    std::vector<uint32_t> ids;
    for (const Json &v : expected["ids"].as_array()) ids.push_back((uint32_t)v.as_number());
    std::vector<int32_t> markers;
    for (const Json &v : expected["markers"].as_array()) markers.push_back((int32_t)v.as_number());
    // the oracle's logits (tests/test_host.py) within the layer-op tolerance
    auto rows = pplx.checkpoint().embedding_rows(ids);
    CHECK(rows.ok());
    auto lg = pplx.logits(rows.value(), ids.size(), markers);
    CHECK(lg.ok());
    if (!lg.ok()) {
        fprintf(stderr, "%s\n", lg.error().to_string().c_str());
        return;
    }
    double dot = 0, gg = 0, ww = 0, maxerr = 0, scale = 0;
    for (size_t r = 0; r < markers.size(); r++)
        for (size_t c = 0; c < DZ_READOUT_CODES; c++) {
            const double g = lg.value()[r * DZ_READOUT_CODES + c], w = expected["logits"][r][c].as_number();
            dot += g * w;
            gg += g * g;
            ww += w * w;
            maxerr = std::max(maxerr, std::fabs(g - w));
            scale = std::max(scale, std::fabs(w));
        }
    // the decoder is a chain of A8 quantizations: an ulp of difference in a
    // layer op flips an activation code now and then, so the logits are
    // compared to 1% of their largest value (the layers alone match far closer)
    CHECK(dot / std::sqrt(gg * ww) >= 0.9999);
    CHECK(maxerr <= 1e-2 * scale);
    printf("pplx logits vs oracle: cos %.9f, max |d| %.5f of %.3f\n", dot / std::sqrt(gg * ww), maxerr, scale);
    {  // the same checkpoint untuned (the reference variants): the same bits
        auto plain = RocmPplx::open(0, dir, cfg, pm, DZ_PPLX_RESIDENT, no_tuning());
        CHECK(plain.ok() && plain.value().tuning().is_null());
        if (plain.ok()) {
            auto pl = plain.value().logits(rows.value(), ids.size(), markers);
            CHECK(pl.ok() && pl.value().size() == lg.value().size() &&
                  memcmp(pl.value().data(), lg.value().data(), lg.value().size() * sizeof(float)) == 0);
        }
    }
    {  // streamed layer weights, tuned from the cached selection: the same bits
        TuningOptions cached;
        cached.cache = selection;
        auto streamed = RocmPplx::open(0, dir, cfg, pm, DZ_PPLX_STREAMED, cached);
        CHECK(streamed.ok());
        if (streamed.ok()) {
            const Json &again = streamed.value().tuning();
            for (const char *fam : {"delta_scan", "norm", "grouped", "mlp"}) {
                CHECK(again["families"][fam]["cached"] == Json(true));
                CHECK(again["selected"][fam] == selection["selected"][fam]);
            }
            auto sl = streamed.value().logits(rows.value(), ids.size(), markers);
            CHECK(sl.ok() && sl.value().size() == lg.value().size() &&
                  memcmp(sl.value().data(), lg.value().data(), lg.value().size() * sizeof(float)) == 0);
        }
    }
    // answers through Model<RocmPplx>: the answer step over those logits
    Request req;
    Json chunk = Json::object();
    chunk["ids"] = ids_json(ids);
    Json m = Json::array();
    for (int32_t v : markers) m.push_back(Json(v));
    chunk["markers"] = m;
    chunk["keys"] = Json::parse(R"(["team","refund","tone"])");
    chunk["counts"] = Json::parse("[3,2,3]");
    req.state = Json::object();
    req.state["chunks"] = Json(Json::Array{chunk});
    req.questions = answer_request(ids, {0, 1, 2}).questions;
    auto cache = model.create_cache(CacheOptions{});
    auto got = model.predict(req, nullptr, &cache.value(), Cancellation{});
    CHECK(got.ok());
    if (!got.ok()) {
        fprintf(stderr, "%s\n", got.error().to_string().c_str());
        return;
    }
    const char *keys[3] = {"team", "refund", "tone"};
    const size_t counts[3] = {3, 2, 3};
    for (int i = 0; i < 3; i++) {
        const float *row = lg.value().data() + i * DZ_READOUT_CODES;
        auto want = answer(req.questions[keys[i]], std::vector<float>(row, row + counts[i]), pplx.temperature());
        CHECK(want.ok() && got.value().response["answers"][keys[i]] == want.value());
    }
    CHECK_EQ(got.value().response["usage"]["input_tokens"], Json((uint64_t)ids.size()));
    uint64_t misses = cache.value().state().misses();
    auto again = model.predict(req, nullptr, &cache.value(), Cancellation{});
    CHECK(again.ok() && again.value().response == got.value().response);
    CHECK_EQ(cache.value().state().misses(), misses);
    // token-id states are not this backend's; shapes must match the checkpoint
    CHECK_EQ(model.predict(request_of(ids), nullptr, nullptr, Cancellation{}).error().code,
             std::string("INVALID_REQUEST"));
    dz_pplx_config wide = cfg;
    wide.hidden = 512;
    CHECK(RocmPplx::open(0, dir, wide, pm, DZ_PPLX_RESIDENT, no_tuning()).error().code == "INVALID_PARAMETERS");
}

TEST(rocm_answer_requests_are_validated) {
    Model<Rocm> model = make_model();
    std::vector<uint32_t> ids = ids_of(30, 9);
    auto code_of = [&](const Request &r, const PplxParameters *p = nullptr) {
        auto out = model.predict(r, p, nullptr, Cancellation{});
        return out.ok() ? std::string("OK") : out.error().code;
    };
    CHECK_EQ(code_of(answer_request(ids, {1, 2, 29})), std::string("OK"));
    CHECK_EQ(code_of(answer_request(ids, {1, 2, 30})), std::string("INVALID_REQUEST"));  // marker past the chunk
    Request unpaired = answer_request(ids, {1, 2});
    CHECK_EQ(code_of(unpaired), std::string("INVALID_REQUEST"));
    Request unknown = answer_request(ids, {1, 2, 3});
    unknown.questions = Json::parse(R"({"team": {"type": "choice", "criteria": {"a": null}}})");
    CHECK_EQ(code_of(unknown), std::string("INVALID_REQUEST"));  // keys without questions
    PplxParameters short_limit;
    short_limit.max_sequence_tokens = 16;
    CHECK_EQ(code_of(answer_request(ids, {1, 2, 3}), &short_limit), std::string("INPUT_TOO_LONG"));
    Request bad_count = answer_request(ids, {1, 2, 3});
    bad_count.questions["team"]["criteria"] = Json::parse(R"({"a": null, "b": null})");  // 2 options, 3 logits
    CHECK_EQ(code_of(bad_count), std::string("INFERENCE_FAILED"));
}

TEST(rocm_capabilities_and_parameters) {
    Model<Rocm> model = make_model();
    Capabilities c = model.capabilities();
    CHECK_EQ(c.model, std::string("pplx-flash"));
    CHECK_EQ(c.backend, std::string("rocm"));
    CHECK(c.has_cache("embedding") && !c.has_cache("prefix"));
    CHECK_EQ(c.tuning, std::string("auto"));
    PplxParameters zero;
    zero.max_sequence_tokens = 0;
    auto r = model.predict(request_of({1, 2}), &zero, nullptr, Cancellation{});
    CHECK(!r.ok() && r.error().code == "INVALID_PARAMETERS");
    CacheOptions prefix;
    prefix.require_prefix = true;
    CHECK_EQ(model.create_cache(prefix).error().code, std::string("UNSUPPORTED_CACHE"));
}

TEST(rocm_predict_equals_direct_forward_and_cache_reuse_is_exact) {
    Model<Rocm> model = make_model();
    auto cache = model.create_cache(CacheOptions{});
    CHECK(cache.ok());
    std::vector<uint32_t> ids = ids_of(77, 3);
    ids[5] = ids[9];  // a repeated token
    auto first = model.predict(request_of(ids), nullptr, &cache.value(), Cancellation{});
    CHECK(first.ok());
    if (!first.ok()) return;
    CHECK_EQ(first.value().backend, std::string("rocm"));
    CHECK_EQ(first.value().response["tokens"], Json(77));
    CHECK_EQ(first.value().response["chunks"], Json(1));
    std::vector<float> want = direct(model.backend(), ids);
    CHECK(same_bits(first.value().response["embeddings"][0], want));
    uint64_t misses = cache.value().state().misses();
    auto second = model.predict(request_of(ids), nullptr, &cache.value(), Cancellation{});
    CHECK(second.ok());
    CHECK_EQ(cache.value().state().misses(), misses);  // every row served from the cache
    CHECK(cache.value().state().hits() > 0);
    CHECK(second.ok() && second.value().response == first.value().response);
}

TEST(rocm_splits_long_inputs_by_max_sequence_tokens) {
    Model<Rocm> model = make_model();
    PplxParameters p;
    p.max_sequence_tokens = 128;
    std::vector<uint32_t> ids = ids_of(300, 11);
    auto r = model.predict(request_of(ids), &p, nullptr, Cancellation{});
    CHECK(r.ok());
    if (!r.ok()) return;
    CHECK_EQ(r.value().response["chunks"], Json(3));
    for (size_t c = 0; c < 3; c++) {
        std::vector<uint32_t> chunk(ids.begin() + c * 128, ids.begin() + std::min<size_t>(300, (c + 1) * 128));
        CHECK(same_bits(r.value().response["embeddings"][c], direct(model.backend(), chunk)));
    }
}

TEST(rocm_failures_clear_the_cache_and_cancellation_is_checked) {
    Model<Rocm> model = make_model();
    auto cache = model.create_cache(CacheOptions{});
    CHECK(model.predict(request_of(ids_of(20, 5)), nullptr, &cache.value(), Cancellation{}).ok());
    CHECK(cache.value().state().rows() > 0);
    Request bad = request_of({1, 2, 99999});
    auto r = model.predict(bad, nullptr, &cache.value(), Cancellation{});
    CHECK(!r.ok() && r.error().code == "INVALID_REQUEST");
    CHECK_EQ(cache.value().state().rows(), (size_t)0);
    Request text;
    text.state = "not token ids";
    text.questions["q"] = 1;
    CHECK_EQ(model.predict(text, nullptr, nullptr, Cancellation{}).error().code, std::string("INVALID_REQUEST"));
    Cancellation c;
    c.cancel();
    CHECK_EQ(model.predict(request_of({1}), nullptr, nullptr, c).error().code, std::string("CANCELLED"));
    auto batch = model.predict_batch({request_of({1}), bad, request_of({2, 3})}, nullptr, &cache.value(),
                                     Cancellation{});
    CHECK(batch.ok());
    CHECK(batch.value()[0].success() && !batch.value()[1].success() && batch.value()[2].success());
}

TEST(rocm_tuning_runs_within_budget_and_is_reported) {
    TuningOptions t;
    t.budget_ms = 300;
    auto made = Rocm::create(0, small_config(), 7, t);
    CHECK(made.ok());
    if (!made.ok()) return;
    const Json &tuning = made.value().tuning();
    CHECK(tuning.is_object());
    CHECK(tuning["selected"].is_object());
    CHECK(tuning["selected"]["gemv"].is_string());
}

int main(int argc, char **argv) { return harness::run_all(argc, argv); }
