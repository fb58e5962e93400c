// inference.hpp -- the host-side inference API of the Rocm backend, in C++.
//
// Restates, over the C ABI of libdecisive_rocm.so, the reference's public
// inference surface (hyperlogue/decisive src/inference/mod.rs:18-273 and
// src/inference/parameters.rs:5-104) so the Rocm backend plugs in the same
// way the reference's Pplx CPU backend does (src/inference/adapters.rs:168-194):
//
//   Request{state, questions}          mod.rs:18-42   (validate, deny unknown fields)
//   Error{code, message}, Error::engine mod.rs:44-85
//   Cancellation                       mod.rs:87-100
//   CacheOptions{maxBytes, requirePrefix} mod.rs:102-115
//   Capabilities, Response, Outcome    mod.rs:117-138
//   Backend (a concept here)           mod.rs:140-154
//   Model<B>, Cache<B>                 mod.rs:156-273
//   PplxParameters, TuningOptions, TuningBudget  parameters.rs:5-48, :81-104
//
// The reference's predict is `async` but never suspends on the CPU backend;
// here it is a plain call. Result<T> carries a value or an Error.
#pragma once

#include <atomic>
#include <cstdint>
#include <limits>
#include <memory>
#include <optional>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "json.hpp"

namespace decisive {

// ---- Error / Result --------------------------------------------------------------

struct Error {
    std::string code;
    std::string message;

    Error() = default;
    Error(std::string c, std::string m) : code(std::move(c)), message(std::move(m)) {}

    // mod.rs:56-78: an engine failure's code is chosen from its message.
    static Error engine(const std::string &message) {
        auto has = [&](const char *s) { return message.find(s) != std::string::npos; };
        const char *code;
        if (has("STATE_TRUNCATED") || has("exceeds token limit") || has("input budget exceeded"))
            code = "INPUT_TOO_LONG";
        else if (has("required WebGPU precision is unavailable"))
            code = "MISSING_GPU_FEATURE";
        else if (has("no WebGPU") || has("request WebGPU device"))
            code = "GPU_UNAVAILABLE";
        else if (has("exceeds device limits"))
            code = "RESOURCE_LIMIT";
        else if (has("the fp16 Cargo feature") || has("the int8 Cargo feature"))
            code = "FORMAT_NOT_COMPILED";
        else
            code = "INFERENCE_FAILED";
        return Error(code, message);
    }

    std::string to_string() const { return code + ": " + message; }
    Json to_json() const {
        Json j = Json::object();
        j["code"] = code;
        j["message"] = message;
        return j;
    }
    bool operator==(const Error &o) const { return code == o.code && message == o.message; }
};

template <class T>
class Result {
public:
    Result(T value) : value_(std::move(value)) {}
    Result(Error error) : error_(std::move(error)) {}
    bool ok() const { return value_.has_value(); }
    explicit operator bool() const { return ok(); }
    T &value() { return *value_; }
    const T &value() const { return *value_; }
    const Error &error() const { return *error_; }
    T take() { return std::move(*value_); }

private:
    std::optional<T> value_;
    std::optional<Error> error_;
};

// Result<void>
template <>
class Result<void> {
public:
    Result() = default;
    Result(Error error) : error_(std::move(error)) {}
    bool ok() const { return !error_.has_value(); }
    explicit operator bool() const { return ok(); }
    const Error &error() const { return *error_; }

private:
    std::optional<Error> error_;
};

using Status = Result<void>;

// Rejects members of `j` outside `allowed` (serde's deny_unknown_fields).
inline Status deny_unknown_fields(const Json &j, const std::set<std::string> &allowed, const char *type) {
    if (!j.is_object()) return Error("INVALID_PARAMETERS", std::string(type) + " must be a JSON object");
    for (const auto &kv : j.as_object())
        if (!allowed.count(kv.first))
            return Error("INVALID_PARAMETERS", "unknown field `" + kv.first + "` in " + type);
    return {};
}

// ---- Request ------------------------------------------------------------------------

struct Request {
    Json state;
    Json questions = Json::object();  // a JSON object (serde_json::Map)

    // mod.rs:26-38
    Status validate() const {
        bool state_ok = state.is_string() || state.is_object() || state.is_array();
        if (!state_ok || !questions.is_object() || questions.size() == 0)
            return Error("INVALID_REQUEST", "state and nonempty questions are required");
        return {};
    }
    // mod.rs:39-41
    Json value() const {
        Json v = Json::object();
        v["state"] = state;
        v["questions"] = questions;
        return v;
    }
    // #[serde(deny_unknown_fields)] Request{state, questions}
    static Result<Request> from_json(const Json &j) {
        Status s = deny_unknown_fields(j, {"state", "questions"}, "Request");
        if (!s) return Error("INVALID_REQUEST", s.error().message);
        if (!j["questions"].is_object()) return Error("INVALID_REQUEST", "questions must be an object");
        Request r;
        r.state = j["state"];
        r.questions = j["questions"];
        return r;
    }
};

// ---- Cancellation -------------------------------------------------------------------

// mod.rs:87-100: clones share one flag.
class Cancellation {
public:
    Cancellation() : flag_(std::make_shared<std::atomic<bool>>(false)) {}
    void cancel() const { flag_->store(true, std::memory_order_relaxed); }
    Status check() const {
        if (flag_->load(std::memory_order_relaxed)) return Error("CANCELLED", "Inference was cancelled");
        return {};
    }

private:
    std::shared_ptr<std::atomic<bool>> flag_;
};

// ---- options, capabilities, outcomes --------------------------------------------------

struct CacheOptions {
    size_t max_bytes = 64u * 1024 * 1024;  // mod.rs:108-114
    bool require_prefix = false;

    static Result<CacheOptions> from_json(const Json &j) {
        Status s = deny_unknown_fields(j, {"maxBytes", "requirePrefix"}, "CacheOptions");
        if (!s) return s.error();
        CacheOptions o;
        if (!j["maxBytes"].is_null()) {
            if (!j["maxBytes"].is_number() || j["maxBytes"].as_number() < 0)
                return Error("INVALID_PARAMETERS", "maxBytes must be a non-negative integer");
            o.max_bytes = (size_t)j["maxBytes"].as_number();
        }
        if (!j["requirePrefix"].is_null()) {
            if (!j["requirePrefix"].is_bool()) return Error("INVALID_PARAMETERS", "requirePrefix must be a boolean");
            o.require_prefix = j["requirePrefix"].as_bool();
        }
        return o;
    }
};

struct Capabilities {
    std::string model;
    std::string backend;
    std::vector<std::string> caches;
    std::string tuning;

    bool has_cache(const std::string &kind) const {
        for (const auto &c : caches)
            if (c == kind) return true;
        return false;
    }
};

struct Response {
    Json response;
    std::string model;
    std::string backend;
    Json to_json() const {
        Json j = Json::object();
        j["response"] = response;
        j["model"] = model;
        j["backend"] = backend;
        return j;
    }
};

// mod.rs:133-138: {"status":"success","result":..} or {"status":"error","error":..}
struct Outcome {
    std::optional<Response> result;
    std::optional<Error> error;
    bool success() const { return result.has_value(); }
    Json to_json() const {
        Json j = Json::object();
        if (result) {
            j["status"] = "success";
            j["result"] = result->to_json();
        } else {
            j["status"] = "error";
            j["error"] = error->to_json();
        }
        return j;
    }
};

// ---- parameters.rs ---------------------------------------------------------------------

enum class TuningMode { Auto, Off };

struct TuningOptions {
    TuningMode mode = TuningMode::Auto;
    uint32_t budget_ms = 1000;        // parameters.rs:21-28
    std::optional<Json> cache;        // `info.tuning.cache` from an earlier load

    static Result<TuningOptions> from_json(const Json &j) {
        Status s = deny_unknown_fields(j, {"mode", "budgetMs", "cache"}, "TuningOptions");
        if (!s) return s.error();
        TuningOptions o;
        const Json &mode = j["mode"];
        if (!mode.is_null()) {
            if (mode.is_string() && mode.as_string() == "auto") o.mode = TuningMode::Auto;
            else if (mode.is_string() && mode.as_string() == "off") o.mode = TuningMode::Off;
            else return Error("INVALID_PARAMETERS", "mode must be \"auto\" or \"off\"");
        }
        const Json &budget = j["budgetMs"];
        if (!budget.is_null()) {
            double b = budget.is_number() ? budget.as_number() : -1.0;
            if (b < 0 || b > 4294967295.0 || b != (double)(uint32_t)b)
                return Error("INVALID_PARAMETERS", "budgetMs must be an unsigned 32-bit integer");
            o.budget_ms = (uint32_t)b;
        }
        if (!j["cache"].is_null()) o.cache = j["cache"];
        return o;
    }
};

// parameters.rs:31-48
class TuningBudget {
public:
    TuningBudget(bool enabled, std::optional<uint32_t> budget_ms, double start)
        : enabled_(enabled), deadline_(budget_ms ? std::optional<double>(start + (double)*budget_ms) : std::nullopt) {}
    std::optional<double> deadline() const { return deadline_; }
    bool permits(double now) const { return enabled_ && (!deadline_ || now < *deadline_); }

private:
    bool enabled_;
    std::optional<double> deadline_;
};

// parameters.rs:81-104
struct PplxParameters {
    size_t max_sequence_tokens = 1024;

    Status validate() const {
        if (max_sequence_tokens == 0) return Error("INVALID_PARAMETERS", "maxSequenceTokens must be positive");
        return {};
    }
    static Result<PplxParameters> from_json(const Json &j) {
        Status s = deny_unknown_fields(j, {"maxSequenceTokens"}, "PplxParameters");
        if (!s) return s.error();
        PplxParameters p;
        const Json &v = j["maxSequenceTokens"];
        if (!v.is_null()) {
            if (!v.is_number() || v.as_number() < 0 || v.as_number() != (double)(uint64_t)v.as_number())
                return Error("INVALID_PARAMETERS", "maxSequenceTokens must be a non-negative integer");
            p.max_sequence_tokens = (size_t)v.as_number();
        }
        return p;
    }
};

// ---- Backend / Model<B> / Cache<B> -------------------------------------------------------

// A backend B provides (mod.rs:140-154):
//   using Parameters = ...;  (default-constructible)
//   using CacheState = ...;
//   Capabilities capabilities() const;
//   Result<CacheState> create_cache(const CacheOptions&) const;
//   void clear_cache(CacheState&) const;
//   Result<Json> predict(const Request&, const Parameters&, CacheState&, const Cancellation&);

template <class B>
class Model;

template <class B>
class Cache {
public:
    typename B::CacheState &state() { return state_; }
    const typename B::CacheState &state() const { return state_; }

private:
    friend class Model<B>;
    Cache(std::shared_ptr<const int> identity, typename B::CacheState state)
        : identity_(std::move(identity)), state_(std::move(state)) {}
    std::shared_ptr<const int> identity_;
    typename B::CacheState state_;
};

template <class B>
class Model {
public:
    using Parameters = typename B::Parameters;

    explicit Model(B backend) : Model(std::move(backend), Parameters{}) {}
    Model(B backend, Parameters defaults)
        : backend_(std::move(backend)), identity_(std::make_shared<const int>(0)), defaults_(std::move(defaults)) {}

    B &backend() { return backend_; }
    Capabilities capabilities() const { return backend_.capabilities(); }

    // mod.rs:174-187
    Result<Cache<B>> create_cache(const CacheOptions &options) const {
        if (options.require_prefix && !capabilities().has_cache("prefix"))
            return Error("UNSUPPORTED_CACHE", "This model/backend does not support prefix caching");
        auto state = backend_.create_cache(options);
        if (!state) return state.error();
        return Cache<B>(identity_, state.take());
    }

    // mod.rs:188-192
    Status clear_cache(Cache<B> &cache) const {
        Status s = check_cache(cache);
        if (!s) return s;
        backend_.clear_cache(cache.state_);
        return {};
    }

    // mod.rs:206-249
    Result<Response> predict(const Request &request, const Parameters *parameters, Cache<B> *cache,
                             const Cancellation &cancellation) {
        std::optional<Cache<B>> temporary;
        if (!cache) {
            CacheOptions ephemeral;
            ephemeral.max_bytes = 0;
            auto made = create_cache(ephemeral);
            if (!made) return made.error();
            temporary.emplace(made.take());
            cache = &*temporary;
        }
        Status s = check_cache(*cache);
        if (!s) return s.error();
        s = cancellation.check();
        if (!s) return s.error();
        s = request.validate();
        if (!s) return s.error();
        Result<Json> result = backend_.predict(request, parameters ? *parameters : defaults_, cache->state_,
                                               cancellation);
        if (result.ok()) {
            Status after = cancellation.check();
            if (!after) result = Result<Json>(after.error());
        }
        if (!result.ok()) {
            backend_.clear_cache(cache->state_);
            return result.error();
        }
        Capabilities caps = capabilities();
        return Response{result.take(), caps.model, caps.backend};
    }

    // mod.rs:250-272
    Result<std::vector<Outcome>> predict_batch(const std::vector<Request> &requests,
                                               const Parameters *parameters, Cache<B> *cache,
                                               const Cancellation &cancellation) {
        if (cache) {
            Status s = check_cache(*cache);
            if (!s) return s.error();
        }
        std::vector<Outcome> outcomes;
        outcomes.reserve(requests.size());
        for (const Request &request : requests) {
            auto r = predict(request, parameters, cache, cancellation);
            Outcome o;
            if (r.ok()) o.result = r.take();
            else o.error = r.error();
            outcomes.push_back(std::move(o));
        }
        return outcomes;
    }

private:
    // mod.rs:197-205: a cache belongs to the model instance that made it.
    Status check_cache(const Cache<B> &cache) const {
        if (cache.identity_ != identity_) return Error("CACHE_OWNER", "Cache belongs to another model instance");
        return {};
    }

    B backend_;
    std::shared_ptr<const int> identity_;
    Parameters defaults_;
};

}  // namespace decisive
