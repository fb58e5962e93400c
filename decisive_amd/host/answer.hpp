// answer.hpp -- the step after the readout: question options and the answer
// JSON built from a question's logits (hyperlogue/decisive
// src/models/pplx_flash/input.rs:21-112 truthy/describe/json_text/options,
// :284-326 answer).
//
//   options(q)   the answer keys of a question, in order, with their legend
//                values: "choice" -> the criteria's keys (object order),
//                "score" -> "0".."n-1" over the criteria array (n >= 2),
//                "noul" -> ["false", "true"].
//   answer(q, logits, temperature)
//                p = softmax(logits / temperature) in f32 (max-subtracted,
//                pplx_flash/cpu.rs:519-529), renormalised in f64, then
//                  noul   {"type","noul": p[1]}
//                  choice {"type","probabilities","choice","confidence"}
//                         confidence = clamp((p_best - 1/n) / (1 - 1/n), 0, 1)
//                         (1 when n == 1); the first maximum wins ties
//                  score  {"type","probabilities","legend","score","confidence"}
//                         score = sum i*p_i; confidence =
//                         max(1 - sum p_i*|i-best| / mean_i |i-midpoint|, 0)
//   json_text(v) the reference's Python-style JSON text (", " and ": "
//                separators, exponents as e-07 / e+16) used when a legend
//                value is not a string.
// Failures carry the reference's messages; the backend reports them through
// Error::engine (INFERENCE_FAILED).
#pragma once

#include <cmath>
#include <string>
#include <utility>
#include <vector>

#include "inference.hpp"
#include "json.hpp"

namespace decisive {

// input.rs:21-30
inline bool truthy(const Json &v) {
    switch (v.kind()) {
        case Json::Kind::Null: return false;
        case Json::Kind::Bool: return v.as_bool();
        case Json::Kind::String: return !v.as_string().empty();
        case Json::Kind::Array:
        case Json::Kind::Object: return v.size() != 0;
        case Json::Kind::Number: return v.as_number() != 0.0;
    }
    return false;
}

// Rust's Display of an f64: shortest round-trip digits, never an exponent.
inline std::string rust_display(double x) {
    std::string digits;
    int e;
    bool neg;
    Json::shortest_digits(x, digits, e, neg);
    std::string out = neg ? "-" : "";
    const int n = (int)digits.size();
    if (x == 0) {
        out += "0";
    } else if (e >= n - 1) {
        out += digits + std::string((size_t)(e - n + 1), '0');
    } else if (e < 0) {
        out += "0." + std::string((size_t)(-e - 1), '0') + digits;
    } else {
        out += digits.substr(0, (size_t)e + 1) + "." + digits.substr((size_t)e + 1);
    }
    return out;
}

// input.rs:37-68
inline std::string json_text(const Json &v) {
    switch (v.kind()) {
        case Json::Kind::Number: {
            if (v.is_integer()) return v.dump();
            const double x = v.as_number();
            if (!std::isfinite(x)) return "null";
            if (x != 0.0 && (std::fabs(x) < 1e-4 || std::fabs(x) >= 1e16)) {
                std::string digits;
                int e;
                bool neg;
                Json::shortest_digits(x, digits, e, neg);
                std::string mantissa = (neg ? "-" : "") + digits.substr(0, 1);
                if (digits.size() > 1) mantissa += "." + digits.substr(1);
                char exponent[16];
                snprintf(exponent, sizeof exponent, "%+03d", e);
                return mantissa + "e" + exponent;
            }
            std::string out = rust_display(x);
            if (out.find('.') == std::string::npos) out += ".0";
            return out;
        }
        case Json::Kind::Array: {
            std::string out = "[";
            bool first = true;
            for (const Json &e : v.as_array()) {
                if (!first) out += ", ";
                first = false;
                out += json_text(e);
            }
            return out + "]";
        }
        case Json::Kind::Object: {
            std::string out = "{";
            bool first = true;
            for (const auto &kv : v.as_object()) {
                if (!first) out += ", ";
                first = false;
                out += Json(kv.first).dump() + ": " + json_text(kv.second);
            }
            return out + "}";
        }
        default: return v.dump();
    }
}

// input.rs:31-36
inline std::string describe(const Json &v) { return v.is_string() ? v.as_string() : json_text(v); }

struct Options {
    std::vector<std::string> keys;
    std::vector<Json> legend;
};

// input.rs:69-112
inline Result<Options> options(const Json &q) {
    const Json &type = q["type"];
    const std::string t = type.is_string() ? type.as_string() : std::string();
    Options o;
    if (t == "choice") {
        const Json &c = q["criteria"];
        if (!c.is_object()) return Error::engine("choice criteria must be an object");
        for (const auto &kv : c.as_object()) {
            o.keys.push_back(kv.first);
            o.legend.push_back(Json(kv.second.is_null() ? kv.first : kv.first + ": " + describe(kv.second)));
        }
        return o;
    }
    if (t == "score") {
        const Json &c = q["criteria"];
        if (!c.is_array()) return Error::engine("score criteria must be an array");
        if (c.size() < 2) return Error::engine("score requires at least two levels");
        for (size_t i = 0; i < c.size(); i++) {
            o.keys.push_back(std::to_string(i));
            o.legend.push_back(c[i]);
        }
        return o;
    }
    if (t == "noul") {
        const Json &c = q["criteria"];
        if (!(c.is_null() || c.is_object())) return Error::engine("noul criteria must be an object");
        const char *names[2][2] = {{"false", "No / false"}, {"true", "Yes / true"}};
        for (auto &kd : names) {
            o.keys.push_back(kd[0]);
            const Json &v = c[kd[0]];
            o.legend.push_back(truthy(v) ? v : Json(kd[1]));
        }
        return o;
    }
    return Error::engine("question type must be choice, noul or score");
}

// pplx_flash/cpu.rs:519-529: max-subtracted softmax in f32.
inline void softmax_f32(std::vector<float> &x) {
    float m = -INFINITY;
    for (float v : x) m = std::fmax(m, v);
    float sum = 0.f;
    for (float &v : x) {
        v = std::exp(v - m);
        sum += v;
    }
    for (float &v : x) v /= sum;
}

// input.rs:284-326
inline Result<Json> answer(const Json &q, const std::vector<float> &logits, float temperature) {
    auto opts = options(q);
    if (!opts) return opts.error();
    const std::vector<std::string> &keys = opts.value().keys;
    if (logits.size() != keys.size()) return Error::engine("logit count mismatch");
    std::vector<float> pf(logits.size());
    for (size_t i = 0; i < logits.size(); i++) pf[i] = logits[i] / temperature;
    softmax_f32(pf);
    double sum = 0.0;
    for (float v : pf) sum += (double)v;
    std::vector<double> p(pf.size());
    for (size_t i = 0; i < pf.size(); i++) p[i] = (double)pf[i] / sum;
    size_t best = 0;
    for (size_t i = 1; i < p.size(); i++)
        if (p[i] > p[best]) best = i;
    Json probabilities = Json::object();
    for (size_t i = 0; i < keys.size(); i++) probabilities[keys[i]] = Json(p[i]);
    const std::string type = q["type"].as_string();
    Json out = Json::object();
    out["type"] = type;
    if (type == "noul") {
        out["noul"] = Json(p[1]);
    } else if (type == "choice") {
        const double n = (double)p.size();
        double confidence = 1.0;
        if (p.size() != 1) {
            // f64::clamp: NaN passes through
            confidence = (p[best] - 1.0 / n) / (1.0 - 1.0 / n);
            if (confidence < 0.0) confidence = 0.0;
            if (confidence > 1.0) confidence = 1.0;
        }
        out["probabilities"] = probabilities;
        out["choice"] = keys[best];
        out["confidence"] = Json(confidence);
    } else {
        const double midpoint = (double)(p.size() - 1) / 2.0;
        double baseline = 0.0;
        for (size_t i = 0; i < p.size(); i++) baseline += std::fabs((double)i - midpoint);
        baseline /= (double)p.size();
        double distance = 0.0, score = 0.0;
        for (size_t i = 0; i < p.size(); i++) {
            distance += p[i] * std::fabs((double)i - (double)best);
            score += (double)i * p[i];
        }
        Json legend = Json::object();
        for (size_t i = 0; i < keys.size(); i++) legend[keys[i]] = opts.value().legend[i];
        out["probabilities"] = probabilities;
        out["legend"] = legend;
        out["score"] = Json(score);
        out["confidence"] = Json(std::fmax(1.0 - distance / baseline, 0.0));
    }
    return out;
}

}  // namespace decisive
