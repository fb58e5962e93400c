// tuner.hip -- bit-exact kernel variant selection.
//
// Semantics of the reference's WebGPU tuner (src/models/pplx_flash/webgpu/
// checkpoint.rs): candidates of a kernel family are timed in three rounds with
// a rotating order; after the first round only the fastest few (three for the
// products, two for the fused MLP) and the family's reference variant keep
// running, and no round starts past the deadline (:428-475). The fastest
// candidate that is at least 1% faster than the reference (MARGIN 0.99, :41)
// and whose output is bitwise equal to the reference's replaces it
// (:480-652). Selections are cached under a key that hashes the device, the
// tuning version and the kernel sources (:279-294); a cached choice is only
// re-checked for equality (:498-513). Inputs are hashed packed words with
// small positive scales (:847-852).
//
// Families, in the order they are tuned (the reference's stages first, in its
// order, checkpoint.rs:251-262):
//   delta_scan  the decider's chunked gated delta scan with 16 or 32 state
//               columns per block, the same arithmetic, over 128 tokens of
//               32 value and 16 key heads (select_delta_scan, :328-421,
//               admits bit-equal scans only: the token-by-token scans regroup
//               the rule's arithmetic and stay out)
//   norm        the decider's layer norm with its A8 codes in one kernel
//               against the norm and the quantizer apart (select_norm,
//               :652-684: 64 rows of 2560, its input and weight generators)
//   grouped     the W4A8 grouped product (select_gemm, :480-563) at
//               (M, N, K) = (256, 8192, 2560)
//   mlp         the fused gate/up + SiLU + A8 requant (select_mlp, :568-652)
//               at (128, 9216, 2560)
//   gemv, gemm_w4a16, i8_gemm   this library's W4A16 GEMV / prefill GEMM and
//               per-row int8 GEMM (no reference counterpart) at (1 or 256,
//               8192, 2560)
#include <string.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <string>
#include <vector>

#include "../../include/decisive_rocm.h"
#include "../host/json.hpp"
#include "../host/sha256.hpp"
#include "kernels.hpp"

#ifndef DZ_SOURCE_HASH
#define DZ_SOURCE_HASH "unversioned"
#endif

namespace dz {

int32_t ctx_fail(dz_ctx *ctx, int32_t code, const std::string &msg);
int32_t ctx_hip_fail(dz_ctx *ctx, hipError_t e, const char *what);
hipStream_t ctx_stream(dz_ctx *ctx);
int ctx_variant(dz_ctx *ctx, const char *family);
void ctx_set_variant(dz_ctx *ctx, const char *family, int index);
void ctx_set_tuning(dz_ctx *ctx, const std::string &json);
std::string ctx_device_key(dz_ctx *ctx);

namespace {

using decisive::Json;

constexpr double kMargin = 0.99;

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

// checkpoint.rs:847-852: hashed words.
uint32_t test_hash(size_t i, size_t seed) {
    uint32_t v = (uint32_t)(i + seed) * 2654435761u;
    v = (v << 13) | (v >> 19);
    return v * 2246822519u;
}

// checkpoint.rs:850: a small positive f32 scale, 0.001 + (hash % 1000) * 1e-5.
float test_scale(size_t i, size_t seed) { return 0.001f + (float)(test_hash(i, seed) % 1000) * 1e-5f; }

enum class Kind { DeltaScan, Grouped, Mlp, Norm, Gemv, GemmW4A16, I8Gemm };

struct Family {
    const char *name;
    Kind kind;
    int m, n, k;
    int keep;  // candidates that stay after the first round (besides the reference)
};

// The reference's stages in its order (checkpoint.rs:251-262: delta scan,
// norm, gemm, mlp), then the families of its own. The delta scan runs 128
// tokens (checkpoint.rs:331) of the decider's 32 value and 16 key heads
// (m = tokens, n = value heads, k = key heads).
const Family kFamilies[] = {
    {"delta_scan", Kind::DeltaScan, 128, 32, 16, 1},
    {"norm", Kind::Norm, 64, 2560, 2560, 2},
    {"grouped", Kind::Grouped, 256, 8192, 2560, 3},
    {"mlp", Kind::Mlp, 128, 9216, 2560, 2},
    {"gemv", Kind::Gemv, 1, 8192, 2560, 3},
    {"gemm_w4a16", Kind::GemmW4A16, 256, 8192, 2560, 3},
    {"i8_gemm", Kind::I8Gemm, 256, 8192, 2560, 3},
};

// Device buffers of one family's selection, freed when it goes out of scope.
struct DeviceBuffers {
    hipStream_t s;
    std::vector<void *> ptrs;
    hipError_t err = hipSuccess;
    explicit DeviceBuffers(hipStream_t stream) : s(stream) {}
    ~DeviceBuffers() {
        hipStreamSynchronize(s);
        for (void *p : ptrs) hipFree(p);
    }
    void *alloc(size_t bytes) {
        void *p = nullptr;
        if (err == hipSuccess) err = hipMalloc(&p, bytes);
        if (err != hipSuccess) return nullptr;
        ptrs.push_back(p);
        return p;
    }
    template <class T>
    void *upload(const std::vector<T> &host) {
        void *p = alloc(host.size() * sizeof(T));
        if (p) err = hipMemcpyAsync(p, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice, s);
        return p;
    }
};

std::vector<uint32_t> hashed_words(size_t bytes, size_t seed) {
    std::vector<uint32_t> w((bytes + 3) / 4);
    for (size_t i = 0; i < w.size(); i++) w[i] = test_hash(i, seed);
    return w;
}

std::vector<float> small_scales(size_t count, size_t seed) {
    std::vector<float> v(count);
    for (size_t i = 0; i < count; i++) v[i] = test_scale(i, seed);
    return v;
}

// A weight of the native layout over hashed codes: Q4 g32/f16 (the W4A16
// families) or Q4 g64/f32 (the grouped families).
Weight test_weight(DeviceBuffers &buf, WeightKind kind, int n, int k, size_t seed) {
    Weight w;
    w.kind = kind;
    w.bits = 4;
    w.group = kind == WeightKind::Q4G32 ? 32 : 64;
    w.rows = n;
    w.cols = k;
    w.groups = k / 64;
    w.np = n;
    w.kp = (k + 127) / 128 * 128;
    w.code_bytes = (size_t)w.np * w.kp / 2;
    w.scale_bytes = (size_t)w.np * (w.kp / 128) * 8;
    w.codes = (uint8_t *)buf.upload(hashed_words(w.code_bytes, seed));
    if (kind == WeightKind::Q4G32) {
        std::vector<uint16_t> h(w.scale_bytes / 2);
        for (size_t i = 0; i < h.size(); i++) h[i] = (uint16_t)(0x1400 + (test_hash(i, seed + 4) % 0xC00));  // 2^-10..2^-7
        w.scales = (uint8_t *)buf.upload(h);
    } else {
        w.scales = (uint8_t *)buf.upload(small_scales(w.scale_bytes / 4, seed + 4));
    }
    return w;
}

// One family's inputs, candidate outputs and launch.
struct Bench {
    Kind kind;
    int m, n, k;
    hipStream_t s;
    Weight w, w2;            // the product weight (gate and up for the MLP)
    const void *x = nullptr;  // f16 rows (W4A16), int8 A8 codes (grouped, MLP) or int8 rows (i8)
    const float *sx = nullptr, *sw = nullptr;
    const int8_t *b = nullptr;
    const float *qhat = nullptr, *khat = nullptr, *conv = nullptr, *gb = nullptr;  // the delta scan's inputs
    float *chunk_ws = nullptr;                                                      // and its chunk workspace
    std::vector<std::vector<std::pair<void *, size_t>>> outs;  // per candidate: output buffers

    void run(int v) {
        auto &o = outs[v];
        switch (kind) {
            case Kind::DeltaScan:  // the chunked scan, 16 or 32 state columns per block
                launch_delta_scan_chunked(qhat, khat, conv, gb, m, n, k, chunk_ws, (float *)o[0].first, v == 1 ? 2 : 1,
                                          s);
                break;
            case Kind::Grouped:
                launch_grouped(w, (const int8_t *)x, sx, m, (float *)o[0].first, nullptr, v, s);
                break;
            case Kind::Mlp:
                launch_mlp_requant(w, w2, (const int8_t *)x, sx, m, (int8_t *)o[0].first, (float *)o[1].first,
                                   nullptr, v, s);
                break;
            case Kind::Norm:
                if (v == 0) {
                    launch_rms_quantize((const float *)x, m, k, sw, 1e-6f, 1, nullptr, (int8_t *)o[0].first,
                                        (float *)o[1].first, nullptr, s);
                } else {
                    launch_readout_rms(x, 0, nullptr, m, k, sw, 1e-6f, 1, (float *)o[2].first, s);
                    launch_act_quantize((const float *)o[2].first, m, k, 8, (int8_t *)o[0].first,
                                        (float *)o[1].first, nullptr, s);
                }
                break;
            case Kind::Gemv:
                launch_w4a16(w, (const half_t *)x, m, (float *)o[0].first, v, 0, s);
                break;
            case Kind::GemmW4A16:
                launch_w4a16(w, (const half_t *)x, m, (float *)o[0].first, 0, v, s);
                break;
            case Kind::I8Gemm:
                launch_i8_gemm((const int8_t *)x, sx, m, b, sw, n, k, o[0].first, 1, v, s);
                break;
        }
    }

    // Every output byte of candidate v, in order.
    std::vector<uint8_t> read(int v) {
        size_t total = 0;
        for (auto &p : outs[v]) total += p.second;
        std::vector<uint8_t> h(total);
        size_t at = 0;
        for (auto &p : outs[v]) {
            hipMemcpyAsync(h.data() + at, p.first, p.second, hipMemcpyDeviceToHost, s);
            at += p.second;
        }
        hipStreamSynchronize(s);
        return h;
    }
};

bool build_bench(DeviceBuffers &buf, const Family &f, int count, Bench *b) {
    b->kind = f.kind;
    b->m = f.m;
    b->n = f.n;
    b->k = f.k;
    b->s = buf.s;
    const size_t M = f.m, N = f.n, K = f.k;
    switch (f.kind) {
        case Kind::DeltaScan: {
            // unit-scale q, k and v and decays below one, as checkpoint.rs:336-342 builds
            // them: x_i = ((i * 7919 % 2003) / 1001.5 - 1) * 0.09; g = 0.9 + (i % 7) / 100,
            // beta = 0.5, k.q from the same generator
            auto unit = [](size_t i) { return ((float)(i * 7919 % 2003) / 1001.5f - 1.0f) * 0.09f; };
            const size_t lkv = K * 128, width = 2 * lkv + N * 128;
            std::vector<float> hq(M * lkv), hk(M * lkv), hc(M * width), hg(M * N * 4);
            for (size_t i = 0; i < hq.size(); i++) {
                hq[i] = unit(i);
                hk[i] = unit(i + 4096);
            }
            for (size_t i = 0; i < hc.size(); i++) hc[i] = unit(i + 8192);
            for (size_t i = 0; i < M * N; i++) {
                hg[4 * i] = 0.9f + (float)(i % 7) * 0.01f;
                hg[4 * i + 1] = 0.5f;
                hg[4 * i + 2] = unit(i + 12288);
                hg[4 * i + 3] = 0.0f;
            }
            b->qhat = (const float *)buf.upload(hq);
            b->khat = (const float *)buf.upload(hk);
            b->conv = (const float *)buf.upload(hc);
            b->gb = (const float *)buf.upload(hg);
            b->chunk_ws = (float *)buf.alloc(delta_chunk_ws_bytes((int)M, (int)N));
            break;
        }
        case Kind::Grouped:
        case Kind::Mlp:
            b->w = test_weight(buf, WeightKind::Q4G64, f.n, f.k, 7);
            if (f.kind == Kind::Mlp) b->w2 = test_weight(buf, WeightKind::Q4G64, f.n, f.k, 11);
            b->x = buf.upload(hashed_words(M * K, 0));         // any int8 codes
            b->sx = (const float *)buf.upload(small_scales(M * K / 64, 17));
            break;
        case Kind::Norm: {
            // checkpoint.rs:655-658: x = ((i * 7919 % 2003) - 1001) / 97, w the bf16 of ((i * 13 % 97) - 48) / 50
            std::vector<float> hx(M * K), hw(K);
            for (size_t i = 0; i < hx.size(); i++) hx[i] = ((float)(i * 7919 % 2003) - 1001.0f) / 97.0f;
            for (size_t i = 0; i < K; i++) {
                const uint32_t bits = __builtin_bit_cast(uint32_t, ((float)(i * 13 % 97) - 48.0f) / 50.0f) >> 16;
                hw[i] = __builtin_bit_cast(float, bits << 16);
            }
            b->x = buf.upload(hx);
            b->sw = (const float *)buf.upload(hw);
            break;
        }
        case Kind::Gemv:
        case Kind::GemmW4A16: {
            b->w = test_weight(buf, WeightKind::Q4G32, f.n, f.k, 7);
            std::vector<uint16_t> hx(M * K);
            for (size_t i = 0; i < hx.size(); i++) {
                uint32_t v = test_hash(i, 0);
                hx[i] = (uint16_t)(0x3000 + (v % 0x0800)) | (uint16_t)((v >> 16) & 0x8000);  // |x| in [2^-3, 2^-1)
            }
            b->x = buf.upload(hx);
            break;
        }
        case Kind::I8Gemm:
            b->x = buf.upload(hashed_words(M * K, 0));
            b->b = (const int8_t *)buf.upload(hashed_words(N * K, 7));
            b->sx = (const float *)buf.upload(small_scales(M, 17));
            b->sw = (const float *)buf.upload(small_scales(N, 19));
            break;
    }
    b->outs.resize(count);
    for (int v = 0; v < count; v++) {
        if (f.kind == Kind::Mlp || f.kind == Kind::Norm) {
            // codes, scales (and for the separate norm its normed rows, not compared)
            b->outs[v].push_back({buf.alloc(M * N), M * N});
            b->outs[v].push_back({buf.alloc(M * N / 64 * 4), M * N / 64 * 4});
            if (f.kind == Kind::Norm) b->outs[v].push_back({buf.alloc(M * N * 4), 0});
        } else if (f.kind == Kind::DeltaScan) {
            b->outs[v].push_back({buf.alloc(N * M * 128 * 4), N * M * 128 * 4});
        } else {
            b->outs[v].push_back({buf.alloc(M * N * 4), M * N * 4});
        }
    }
    if (buf.err == hipSuccess) buf.err = hipStreamSynchronize(buf.s);
    return buf.err == hipSuccess;
}

// time_candidates (checkpoint.rs:428-475): the best time per run of each
// candidate and whether it stayed for the later rounds.
void time_candidates(Bench &b, int count, int keep, double deadline, std::vector<double> *best,
                     std::vector<bool> *kept) {
    for (int v = 0; v < count; v++) b.run(v);  // warm every candidate
    hipStreamSynchronize(b.s);
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    auto batch = [&](int v, int reps) {
        hipEventRecord(e0, b.s);
        for (int r = 0; r < reps; r++) b.run(v);
        hipEventRecord(e1, b.s);
        hipEventSynchronize(e1);
        float ms = 0.f;
        hipEventElapsedTime(&ms, e0, e1);
        return (double)ms / reps;
    };
    // batches of about 2 ms of GPU work (the reference's 30 ms works around
    // Safari's whole-millisecond timer; HIP events resolve microseconds)
    const double per_run = std::max(batch(0, 2), 1e-4);
    const int reps = (int)std::min(64.0, std::max(2.0, std::ceil(2.0 / per_run)));
    best->assign(count, 1e30);
    std::vector<int> active(count);
    for (int v = 0; v < count; v++) active[v] = v;
    for (int round = 0; round < 3; round++) {
        if (round == 1) {
            std::sort(active.begin(), active.end(), [&](int a, int c) { return (*best)[a] < (*best)[c]; });
            if ((int)active.size() > keep) active.resize(keep);
            if (std::find(active.begin(), active.end(), 0) == active.end()) active.push_back(0);
        }
        if (round > 0 && now_ms() >= deadline) break;
        for (size_t j = 0; j < active.size(); j++) {
            const int v = active[(j + round) % active.size()];
            (*best)[v] = std::min((*best)[v], batch(v, reps));
        }
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    kept->assign(count, false);
    for (int v : active) (*kept)[v] = true;
}

// The cached selection of `family` when the cache's key matches, else "".
std::string cached_choice(const Json &cache, const std::string &key, const char *family) {
    if (!cache.is_object() || !cache["key"].is_string() || cache["key"].as_string() != key) return "";
    const Json &sel = cache["selected"];
    if (!sel.is_object() || !sel[family].is_string()) return "";
    return sel[family].as_string();
}

}  // namespace

std::string tuning_key(dz_ctx *ctx) {
    decisive::Sha256 h;
    const std::string head = "pplx-tuning-v1\n" + ctx_device_key(ctx) + "\n" + DZ_SOURCE_HASH + "\n";
    h.update(head.data(), head.size());
    for (const Family &f : kFamilies)
        for (int i = 0; i < variant_count(f.name); i++) {
            const std::string line = std::string(f.name) + "/" + variant_name(f.name, i) + "\n";
            h.update(line.data(), line.size());
        }
    return h.hex().substr(0, 32);  // the first 16 bytes, as checkpoint.rs:293
}

int32_t tune(dz_ctx *ctx, uint32_t budget_ms, const char *cache_in, char *cache_out, size_t cap) {
    const double started = now_ms();
    const double deadline = started + budget_ms;
    hipStream_t s = ctx_stream(ctx);
    const std::string key = tuning_key(ctx);
    Json cache;
    if (cache_in && *cache_in) {
        try {
            cache = Json::parse(cache_in);
        } catch (const std::exception &) {
            cache = Json();  // an unreadable cache is ignored, as a missing one
        }
    }
    Json report = Json::object(), families = Json::object(), selected = Json::object();
    report["key"] = key;
    report["budget_ms"] = (int64_t)budget_ms;
    for (const Family &fam : kFamilies) {
        const int count = tuned_count(fam.name);
        DeviceBuffers buf(s);
        Bench bench;
        if (!build_bench(buf, fam, count, &bench)) return ctx_hip_fail(ctx, buf.err, "tuner inputs");
        int fastest = -1;
        Json detail = Json::object();
        const std::string want = cached_choice(cache, key, fam.name);
        int cached_idx = want.empty() ? -1 : variant_index(fam.name, want.c_str());
        if (cached_idx >= count) cached_idx = -1;  // not a tuned candidate: tune again
        if (cached_idx >= 0) {
            bool agrees = cached_idx == 0;
            if (!agrees) {
                bench.run(0);
                bench.run(cached_idx);
                agrees = bench.read(0) == bench.read(cached_idx);
            }
            if (agrees) {
                fastest = cached_idx;
                detail["cached"] = true;
            }
        }
        if (fastest < 0 && now_ms() >= deadline) {
            // TuningBudget::permits (parameters.rs:305-322): no new selection stage past the deadline
            detail["skipped"] = "budget";
        } else if (fastest < 0) {
            std::vector<double> best;
            std::vector<bool> kept;
            time_candidates(bench, count, fam.keep, deadline, &best, &kept);
            std::vector<int> order;
            for (int v = 1; v < count; v++)
                if (kept[v] && best[v] < best[0] * kMargin) order.push_back(v);
            std::sort(order.begin(), order.end(), [&](int a, int c) { return best[a] < best[c]; });
            // only candidates fast enough to replace the reference are read back
            Json agrees = Json::array();
            std::vector<Json> agree(count);
            agree[0] = true;
            std::vector<uint8_t> ref;
            if (!order.empty()) {
                bench.run(0);
                ref = bench.read(0);
            }
            for (int v : order) {
                bench.run(v);
                const bool eq = bench.read(v) == ref;
                agree[v] = eq;
                if (eq) {
                    fastest = v;
                    break;
                }
            }
            Json shape = Json::array(), cands = Json::array(), ms = Json::array(), keptj = Json::array();
            for (int d : {fam.m, fam.n, fam.k}) shape.push_back(d);
            for (int v = 0; v < count; v++) {
                cands.push_back(variant_name(fam.name, v));
                ms.push_back(best[v] >= 1e29 ? Json() : Json(best[v]));
                keptj.push_back((bool)kept[v]);
                agrees.push_back(agree[v]);
            }
            detail["shape"] = shape;
            detail["candidates"] = cands;
            detail["ms_per_run"] = ms;
            detail["kept"] = keptj;
            detail["agrees"] = agrees;
        }
        if (fastest < 0) fastest = 0;
        ctx_set_variant(ctx, fam.name, fastest);
        detail["selected"] = variant_name(fam.name, fastest);
        families[fam.name] = detail;
        selected[fam.name] = variant_name(fam.name, fastest);
    }
    report["families"] = families;
    report["selected"] = selected;
    report["elapsed_ms"] = now_ms() - started;
    const std::string text = report.dump();
    ctx_set_tuning(ctx, text);
    if (cache_out) {
        if (cap < text.size() + 1) return ctx_fail(ctx, DZ_RESOURCE_LIMIT, "tuning cache buffer too small");
        memcpy(cache_out, text.c_str(), text.size() + 1);
    }
    return DZ_OK;
}

}  // namespace dz
