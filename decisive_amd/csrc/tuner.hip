// tuner.hip -- bit-exact kernel variant selection.
//
// Semantics of the reference's WebGPU tuner (src/models/pplx_flash/webgpu/
// checkpoint.rs): candidates of a kernel family are timed in three rounds with
// a rotating order; after the first round only the three fastest and the
// family's reference variant keep running, and no round starts past the
// deadline (:428-475). The fastest candidate that is at least 1% faster than
// the reference (MARGIN 0.99, :41) and whose output is bitwise equal to the
// reference's replaces it (:480-563). Selections are cached under a key that
// hashes the device, the tuning version and the kernel sources (:279-294); a
// cached choice is only re-checked for equality (:498-513). Inputs are hashed
// packed words with small positive scales (:847-852).
#include <ctype.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <string>
#include <vector>

#include "../../include/decisive_rocm.h"
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

// ---- SHA-256 (FIPS 180-4) ---------------------------------------------------------

struct Sha256 {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                     0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    uint8_t buf[64];
    size_t len = 0;
    uint64_t total = 0;
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void block(const uint8_t *p) {
        static const uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; i++) {
            uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    void update(const void *data, size_t n) {
        const uint8_t *p = (const uint8_t *)data;
        total += n;
        while (n) {
            size_t take = std::min(n, (size_t)64 - len);
            memcpy(buf + len, p, take);
            len += take;
            p += take;
            n -= take;
            if (len == 64) {
                block(buf);
                len = 0;
            }
        }
    }
    void update(const std::string &s) { update(s.data(), s.size()); }
    std::string hex16() {
        uint64_t bits = total * 8;
        uint8_t pad = 0x80;
        update(&pad, 1);
        uint8_t zero = 0;
        while (len != 56) update(&zero, 1);
        uint8_t lenb[8];
        for (int i = 0; i < 8; i++) lenb[i] = (uint8_t)(bits >> (56 - 8 * i));
        update(lenb, 8);
        static const char *hexd = "0123456789abcdef";
        std::string out;
        for (int i = 0; i < 4; i++)
            for (int b = 3; b >= 0; b--) {
                uint8_t v = (uint8_t)(h[i] >> (8 * b));
                out += hexd[v >> 4];
                out += hexd[v & 15];
            }
        return out;
    }
};

double now_ms() {
    using namespace std::chrono;
    return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

// checkpoint.rs:847-852: hashed words; every `stride`-th word a small positive scale.
uint32_t test_hash(size_t i, size_t seed) {
    uint32_t v = (uint32_t)(i + seed) * 2654435761u;
    v = (v << 13) | (v >> 19);
    return v * 2246822519u;
}

struct Family {
    const char *name;
    int m, n, k;  // tuning shape
};

// The string value of the first `"name": "value"` member in s (the tuner's own
// output, possibly re-serialized with whitespace around the colon).
std::string json_field(const std::string &s, const std::string &name) {
    const std::string pat = "\"" + name + "\"";
    for (size_t at = s.find(pat); at != std::string::npos; at = s.find(pat, at + 1)) {
        size_t p = at + pat.size();
        while (p < s.size() && isspace((unsigned char)s[p])) p++;
        if (p >= s.size() || s[p] != ':') continue;
        p++;
        while (p < s.size() && isspace((unsigned char)s[p])) p++;
        if (p >= s.size() || s[p] != '"') continue;
        size_t end = s.find('"', p + 1);
        return end == std::string::npos ? "" : s.substr(p + 1, end - p - 1);
    }
    return "";
}

}  // namespace

std::string tuning_key(dz_ctx *ctx) {
    Sha256 h;
    h.update("pplx-tuning-v1\n" + ctx_device_key(ctx) + "\n" + DZ_SOURCE_HASH + "\n");
    for (const char *f : {"gemv", "gemm_w4a16", "i8_gemm", "grouped", "mlp", "delta_scan"})
        for (int i = 0; i < variant_count(f); i++) h.update(std::string(f) + "/" + variant_name(f, i) + "\n");
    return h.hex16();
}

int32_t tune(dz_ctx *ctx, uint32_t budget_ms, const char *cache_in, char *cache_out, size_t cap) {
    const double started = now_ms();
    const double deadline = started + budget_ms;
    hipStream_t s = ctx_stream(ctx);
    const std::string key = tuning_key(ctx);
    const std::string cached = cache_in ? cache_in : "";
    const bool cache_ok = !cached.empty() && json_field(cached, "key") == key;
    const Family families[] = {{"gemv", 1, 8192, 2560}, {"gemm_w4a16", 256, 8192, 2560}, {"i8_gemm", 256, 8192, 2560}};

    std::string report = "{\"key\":\"" + key + "\",\"budget_ms\":" + std::to_string(budget_ms) + ",\"families\":{";
    std::string selected_json = "\"selected\":{";
    bool first_family = true;
    for (const Family &fam : families) {
        const int count = variant_count(fam.name);
        const int M = fam.m, N = fam.n, K = fam.k;
        // synthetic inputs
        Weight w;
        w.kind = WeightKind::Q4G32;
        w.bits = 4; w.group = 32; w.rows = N; w.cols = K; w.groups = K / 64;
        w.np = N; w.kp = (K + 127) / 128 * 128;
        w.code_bytes = (size_t)w.np * w.kp / 2;
        w.scale_bytes = (size_t)w.np * (w.kp / 128) * 8;
        std::vector<uint32_t> hcodes(w.code_bytes / 4);
        for (size_t i = 0; i < hcodes.size(); i++) hcodes[i] = test_hash(i, 7);
        std::vector<uint16_t> hscales(w.scale_bytes / 2);
        for (size_t i = 0; i < hscales.size(); i++) {
            // small positive f16 scales 2^-10 .. 2^-7
            hscales[i] = (uint16_t)(0x1400 + (test_hash(i, 11) % 0xC00));
        }
        size_t abytes = strcmp(fam.name, "i8_gemm") == 0 ? (size_t)M * K : (size_t)M * K * 2;
        (void)0;
        std::vector<uint16_t> hx(abytes / 2);
        for (size_t i = 0; i < hx.size(); i++) {
            uint32_t v = test_hash(i, 0);
            hx[i] = (uint16_t)(0x3000 + (v % 0x0800)) | (uint16_t)((v >> 16) & 0x8000);  // |x| in [2^-3, 2^-1)
        }
        const bool i8 = strcmp(fam.name, "i8_gemm") == 0;
        // int8 rows of B for the i8 family, packed Q4 codes otherwise
        const size_t bbytes = i8 ? (size_t)N * K : w.code_bytes;
        if (hcodes.size() * 4 < bbytes) hcodes.resize(bbytes / 4 + 1);
        for (size_t i = 0; i < hcodes.size(); i++) hcodes[i] = test_hash(i, 7);
        void *dcodes = nullptr, *dscales = nullptr, *dx = nullptr, *dsa = nullptr, *dsb = nullptr;
        std::vector<void *> outs(count, nullptr);
        hipError_t err = hipMalloc(&dcodes, bbytes);
        if (err == hipSuccess) err = hipMalloc(&dscales, w.scale_bytes);
        if (err == hipSuccess) err = hipMalloc(&dx, abytes);
        if (err == hipSuccess) err = hipMalloc(&dsa, (size_t)std::max(M, N) * 4);
        if (err == hipSuccess) err = hipMalloc(&dsb, (size_t)std::max(M, N) * 4);
        for (int i = 0; i < count && err == hipSuccess; i++) err = hipMalloc(&outs[i], (size_t)M * N * 4);
        if (err == hipSuccess) err = hipMemcpyAsync(dcodes, hcodes.data(), bbytes, hipMemcpyHostToDevice, s);
        if (err == hipSuccess) err = hipMemcpyAsync(dscales, hscales.data(), w.scale_bytes, hipMemcpyHostToDevice, s);
        if (err == hipSuccess) err = hipMemcpyAsync(dx, hx.data(), abytes, hipMemcpyHostToDevice, s);
        if (err == hipSuccess) {
            launch_fill_f32((float *)dsa, (size_t)std::max(M, N), 0.01f, s);
            launch_fill_f32((float *)dsb, (size_t)std::max(M, N), 0.02f, s);
            err = hipStreamSynchronize(s);
        }
        auto cleanup = [&]() {
            hipStreamSynchronize(s);
            for (void *p : {dcodes, dscales, dx, dsa, dsb})
                if (p) hipFree(p);
            for (void *p : outs)
                if (p) hipFree(p);
        };
        if (err != hipSuccess) {
            cleanup();
            return ctx_hip_fail(ctx, err, "tuner inputs");
        }
        w.codes = (uint8_t *)dcodes;
        w.scales = (uint8_t *)dscales;
        auto run = [&](int v) {
            if (strcmp(fam.name, "gemv") == 0)
                launch_w4a16(w, (const half_t *)dx, M, (float *)outs[v], v, 0, s);
            else if (strcmp(fam.name, "gemm_w4a16") == 0)
                launch_w4a16(w, (const half_t *)dx, M, (float *)outs[v], 0, v, s);
            else
                launch_i8_gemm((const int8_t *)dx, (const float *)dsa, M, (const int8_t *)dcodes,
                               (const float *)dsb, N, K, outs[v], 1, v, s);
        };
        auto read = [&](int v) {
            std::vector<uint32_t> h((size_t)M * N);
            hipMemcpyAsync(h.data(), outs[v], h.size() * 4, hipMemcpyDeviceToHost, s);
            hipStreamSynchronize(s);
            return h;
        };
        int fastest = -1;
        std::string detail;
        // a cached choice is only checked for equality again
        std::string want = cache_ok ? json_field(cached.substr(cached.find("\"selected\"") == std::string::npos ? 0 : cached.find("\"selected\"")), fam.name) : "";
        int cached_idx = want.empty() ? -1 : variant_index(fam.name, want.c_str());
        if (cached_idx >= 0) {
            bool agrees = cached_idx == 0;
            if (!agrees) {
                run(0);
                run(cached_idx);
                agrees = read(0) == read(cached_idx);
            }
            if (agrees) {
                fastest = cached_idx;
                detail = "{\"cached\":true";
            }
        }
        if (fastest < 0 && now_ms() >= deadline) {
            // TuningBudget::permits (parameters.rs:305-322): no new selection stage past the deadline
            detail = "{\"skipped\":\"budget\"";
        } else if (fastest < 0) {
            // warm every candidate, size timed batches to ~2 ms of GPU work
            for (int v = 0; v < count; v++) run(v);
            hipStreamSynchronize(s);
            hipEvent_t e0, e1;
            hipEventCreate(&e0);
            hipEventCreate(&e1);
            auto time_batch = [&](int v, int reps) {
                hipEventRecord(e0, s);
                for (int r = 0; r < reps; r++) run(v);
                hipEventRecord(e1, s);
                hipEventSynchronize(e1);
                float ms = 0.f;
                hipEventElapsedTime(&ms, e0, e1);
                return (double)ms / reps;
            };
            double per_run = std::max(time_batch(0, 2), 1e-4);
            int reps = (int)std::min(64.0, std::max(2.0, std::ceil(2.0 / per_run)));
            std::vector<double> best(count, 1e30);
            std::vector<int> active(count);
            for (int v = 0; v < count; v++) active[v] = v;
            for (int round = 0; round < 3; round++) {
                if (round == 1) {
                    std::sort(active.begin(), active.end(), [&](int a, int b) { return best[a] < best[b]; });
                    if ((int)active.size() > 3) active.resize(3);
                    if (std::find(active.begin(), active.end(), 0) == active.end()) active.push_back(0);
                }
                if (round > 0 && now_ms() >= deadline) break;
                for (size_t jdx = 0; jdx < active.size(); jdx++) {
                    int v = active[(jdx + round) % active.size()];
                    best[v] = std::min(best[v], time_batch(v, reps));
                }
            }
            hipEventDestroy(e0);
            hipEventDestroy(e1);
            std::vector<int> order;
            for (int v = 1; v < count; v++)
                if (std::find(active.begin(), active.end(), v) != active.end() && best[v] < best[0] * 0.99)
                    order.push_back(v);
            std::sort(order.begin(), order.end(), [&](int a, int b) { return best[a] < best[b]; });
            std::vector<std::string> agrees(count, "null");
            agrees[0] = "true";
            std::vector<uint32_t> ref;
            if (!order.empty()) {
                run(0);
                ref = read(0);
            }
            for (int v : order) {
                run(v);
                bool eq = read(v) == ref;
                agrees[v] = eq ? "true" : "false";
                if (eq) {
                    fastest = v;
                    break;
                }
            }
            detail = "{\"shape\":[" + std::to_string(M) + "," + std::to_string(N) + "," + std::to_string(K) +
                     "],\"candidates\":[";
            for (int v = 0; v < count; v++) detail += std::string(v ? "," : "") + "\"" + variant_name(fam.name, v) + "\"";
            detail += "],\"ms_per_run\":[";
            for (int v = 0; v < count; v++)
                detail += std::string(v ? "," : "") + (best[v] >= 1e29 ? std::string("null") : std::to_string(best[v]));
            detail += "],\"kept\":[";
            for (int v = 0; v < count; v++)
                detail += std::string(v ? "," : "") +
                          (std::find(active.begin(), active.end(), v) != active.end() ? "true" : "false");
            detail += "],\"agrees\":[";
            for (int v = 0; v < count; v++) detail += std::string(v ? "," : "") + agrees[v];
            detail += "]";
        }
        if (fastest < 0) fastest = 0;
        ctx_set_variant(ctx, fam.name, fastest);
        detail += ",\"selected\":\"" + std::string(variant_name(fam.name, fastest)) + "\"}";
        report += std::string(first_family ? "" : ",") + "\"" + fam.name + "\":" + detail;
        selected_json += std::string(first_family ? "" : ",") + "\"" + fam.name + "\":\"" +
                         variant_name(fam.name, fastest) + "\"";
        first_family = false;
        cleanup();
    }
    report += "}," + selected_json + "},\"elapsed_ms\":" + std::to_string(now_ms() - started) + "}";
    ctx_set_tuning(ctx, report);
    if (cache_out) {
        if (cap < report.size() + 1) return ctx_fail(ctx, DZ_RESOURCE_LIMIT, "tuning cache buffer too small");
        memcpy(cache_out, report.c_str(), report.size() + 1);
    }
    return DZ_OK;
}

}  // namespace dz
