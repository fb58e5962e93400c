// runtime.hip -- the extern "C" boundary of libdecisive_rocm.so.
//
// Every entry point validates its arguments on the host, records a message in
// the context on failure and returns a dz_status whose names follow the
// reference's error codes (src/inference/mod.rs:44-85). Kernels run on the
// context stream; device-side validation (scales, non-finite inputs, token
// ids) reports through a device flag that the synchronous entry points read.
#include <float.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <set>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/decisive_rocm.h"
#include "kernels.hpp"

struct dz_weight {
    dz::Weight w;
    int device = 0;
};

struct dz_ctx {
    int device = 0;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    std::string error;
    std::string arch;
    int cus = 0;
    int clock_khz = 0;
    // device ints: [0] validation / non-finite flag, [1..62] the product flag
    // ring, [kCaptureSlot0 ..] one flag per product recorded under stream capture
    int *flag = nullptr;
    uint64_t product_calls = 0;  // ring products since the last stream change (picks the slot)
    int captured_flags = 0;      // capture slots ever handed out (the high-water mark)
    std::vector<int> free_capture_slots;                          // slots given back, reused first
    std::map<unsigned long long, std::vector<int>> capture_slots;  // capture id -> slots it holds
    void *work = nullptr; // activation quantization workspace
    size_t work_bytes = 0;
    uint8_t *scratch = nullptr;        // device address of this device's `scratch` array
    // workspace -> ids of the captures that recorded it; a workspace replaced
    // while a capture still holds it is retired, and freed when the last of
    // its captures is released (or at dz_destroy)
    std::map<void *, std::set<unsigned long long>> work_users;
    std::vector<void *> retired_work;
    std::map<std::string, int> variants;
    std::string tuning;   // JSON of the last selection
};

// The workspace of dz_linear_noalloc: the A8 codes and scales of its
// activations and its non-finite flag, in a device array that the library
// never allocates or frees (each device holds its own copy until the process
// ends). Host code must not use the name `scratch` as an address: dz_init
// looks up this device's address of the array once (hipGetSymbolAddress) and
// every kernel argument uses that address.
constexpr size_t kScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace dz {
int32_t encoder_create_random(dz_ctx *ctx, const dz_encoder_config *cfg, uint64_t seed,
                              dz_encoder **out);
void encoder_destroy(dz_ctx *ctx, dz_encoder *enc);
int32_t encoder_row_bytes(const dz_encoder *enc, size_t *row_bytes);
const dz_weight *encoder_weight(const dz_encoder *enc, int layer, int which);
int32_t encoder_read_rows(dz_ctx *ctx, const dz_encoder *enc, const int32_t *ids, size_t count,
                          void *out);
int32_t encoder_hidden_rows(dz_ctx *ctx, dz_encoder *e, const void *rows_host, size_t seq, float *hidden);
int32_t encoder_readout_params(const dz_encoder *e, const dz_weight **w, const float **norm);
int32_t encoder_set_readout(dz_ctx *ctx, dz_encoder *e, const void *packed, size_t bytes, int32_t layout,
                            const float *norm_host);
int32_t encoder_readout(dz_ctx *ctx, dz_encoder *e, const void *rows_host, size_t seq, const int32_t *markers,
                        size_t count, float *logits_host);
int32_t pplx_create(dz_ctx *ctx, const dz_pplx_config *cfg, dz_pplx **out);
void pplx_destroy(dz_ctx *ctx, dz_pplx *p);
int32_t pplx_set_weight(dz_ctx *ctx, dz_pplx *p, const char *name, const void *packed, size_t bytes, int32_t layout,
                        size_t rows, size_t cols, int32_t form);
int32_t pplx_set_rows_form(dz_ctx *ctx, dz_pplx *p, int32_t form);
int32_t pplx_set_vector(dz_ctx *ctx, dz_pplx *p, const char *name, const float *values, size_t count);
int32_t pplx_layer(dz_ctx *ctx, dz_pplx *p, int index, float *hidden, size_t n, const int32_t *markers_host,
                   size_t count, int part);
int32_t pplx_activation(dz_ctx *ctx, dz_pplx *p, const char *name, void *out, size_t bytes);
int32_t pplx_set_residency(dz_ctx *ctx, dz_pplx *p, int32_t residency);
int32_t pplx_residency_info(dz_ctx *ctx, dz_pplx *p, char *json, size_t cap);
int32_t pplx_forward_rows(dz_ctx *ctx, dz_pplx *p, const void *rows_host, size_t n, const int32_t *markers,
                          size_t count, float *logits_host);
int32_t encoder_forward(dz_ctx *ctx, dz_encoder *enc, const int32_t *ids_dev, const void *rows_host,
                        size_t batch, size_t seq, float *out);
int32_t tune(dz_ctx *ctx, uint32_t budget_ms, const char *cache_in, char *cache_out, size_t cap);
}  // namespace dz

namespace {

int32_t fail(dz_ctx *ctx, int32_t code, const std::string &msg) {
    if (ctx) ctx->error = msg;
    return code;
}

int32_t hip_fail(dz_ctx *ctx, hipError_t e, const char *what) {
    std::string msg = std::string(what) + ": " + hipGetErrorString(e);
    int32_t code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? DZ_RESOURCE_LIMIT
                                                                               : DZ_INFERENCE_FAILED;
    if (code == DZ_RESOURCE_LIMIT) msg += " (exceeds device limits)";
    return fail(ctx, code, msg);
}

#define DZ_HIP(ctx, expr, what)                  \
    do {                                         \
        hipError_t e_ = (expr);                  \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, what); \
    } while (0)

#define DZ_BEGIN(ctx)                                                              \
    do {                                                                           \
        if (!(ctx)) return DZ_INVALID_REQUEST;                                      \
        (ctx)->error.clear();                                                       \
        hipError_t e_ = hipSetDevice((ctx)->device);                                \
        if (e_ != hipSuccess) return hip_fail(ctx, e_, "hipSetDevice");             \
    } while (0)

// Entry points that wait for the stream, allocate, or read host memory: under
// stream capture they return before enqueueing anything, so nothing of theirs
// lands in the recorded graph.
#define DZ_NOT_CAPTURING(ctx)                                                      \
    do {                                                                           \
        if (capturing(ctx))                                                        \
            return fail(ctx, DZ_INVALID_REQUEST, "synchronous call during stream capture"); \
    } while (0)

// Launch status of the kernels just enqueued.
int32_t launched(dz_ctx *ctx, const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, what);
    return DZ_OK;
}

int variant(dz_ctx *ctx, const char *family) {
    auto it = ctx->variants.find(family);
    return it == ctx->variants.end() ? 0 : it->second;
}

constexpr int kRingSlots = 62;
constexpr int kCaptureSlot0 = 64;
constexpr int kCaptureSlots = 4032;  // 16 KiB flag buffer
constexpr size_t kFlagBytes = (size_t)(kCaptureSlot0 + kCaptureSlots) * sizeof(int);

// True while the context stream records a graph (hipStreamBeginCapture).
bool capturing(dz_ctx *ctx) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(ctx->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

// The id of the capture the context stream is recording (valid while capturing).
unsigned long long capture_id(dz_ctx *ctx) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    if (hipStreamGetCaptureInfo(ctx->stream, &st, &id) != hipSuccess || st == hipStreamCaptureStatusNone) return 0;
    return id;
}

// Frees the retired workspaces no capture holds any more. Not while the
// context stream records: a free during a global-mode capture invalidates it.
void free_unused_retired(dz_ctx *ctx) {
    if (capturing(ctx)) return;
    bool synced = false;
    for (size_t i = 0; i < ctx->retired_work.size();) {
        void *p = ctx->retired_work[i];
        auto it = ctx->work_users.find(p);
        if (it != ctx->work_users.end() && !it->second.empty()) {
            i++;
            continue;
        }
        if (!synced) {
            hipStreamSynchronize(ctx->stream);
            synced = true;
        }
        hipFree(p);
        if (it != ctx->work_users.end()) ctx->work_users.erase(it);
        ctx->retired_work.erase(ctx->retired_work.begin() + i);
    }
}

// Resets the flag, then returns its value after running `enqueue` and syncing.
// Synchronous calls cannot be recorded into a graph.
template <class F>
int32_t flagged_sync(dz_ctx *ctx, F enqueue, int *value) {
    if (capturing(ctx)) return fail(ctx, DZ_INVALID_REQUEST, "synchronous call during stream capture");
    dz::launch_fill_i32(ctx->flag, 0, 1, ctx->stream);
    enqueue();
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(ctx, e, "kernel launch");
    DZ_HIP(ctx, hipMemcpyAsync(value, ctx->flag, sizeof(int), hipMemcpyDeviceToHost, ctx->stream),
           "flag readback");
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    return DZ_OK;
}

// The non-finite-activation flag of one asynchronous product.
//  - Eager calls take slot 1 + (call % 62) of the flag buffer, so a call never
//    reads a flag an earlier call set. The 62 slots are cleared together, by
//    one launch the stream orders after every earlier product, each time the
//    ring starts over (instead of one clearing launch per product).
//  - A call recorded under stream capture takes a slot of its own, which no
//    other call uses until dz_capture_release gives back the slots of its
//    capture, and clears it with a fill kernel recorded just before the
//    product, so every replay starts from a clear flag. Replays of one graph
//    must not overlap each other. At most kCaptureSlots recorded products hold
//    slots at once.
int32_t product_flag(dz_ctx *ctx, int **out) {
    if (capturing(ctx)) {
        int index;
        if (!ctx->free_capture_slots.empty()) {
            index = ctx->free_capture_slots.back();
            ctx->free_capture_slots.pop_back();
        } else if (ctx->captured_flags < kCaptureSlots) {
            index = ctx->captured_flags++;
        } else {
            return fail(ctx, DZ_RESOURCE_LIMIT,
                        "4032 products recorded under stream capture hold flag slots on this context: release the "
                        "captures of destroyed graphs with dz_capture_release");
        }
        ctx->capture_slots[capture_id(ctx)].push_back(index);
        int *slot = ctx->flag + kCaptureSlot0 + index;
        dz::launch_fill_i32(slot, 0, 1, ctx->stream);
        *out = slot;
        return DZ_OK;
    }
    const int slot = (int)(ctx->product_calls++ % kRingSlots);
    if (slot == 0) dz::launch_fill_i32(ctx->flag + 1, 0, kRingSlots, ctx->stream);
    *out = ctx->flag + 1 + slot;
    return DZ_OK;
}

// Makes the context workspace at least `bytes` long. Growing it waits for the
// context stream; a workspace that a captured graph refers to is retired
// instead of freed, and freed once every capture that recorded it has been
// released (dz_capture_release) or at dz_destroy. Under capture the workspace
// cannot grow: the caller runs the same call once before capturing it.
int32_t ensure_work(dz_ctx *ctx, size_t bytes) {
    const bool cap = capturing(ctx);
    if (ctx->work_bytes >= bytes) {
        if (cap) ctx->work_users[ctx->work].insert(capture_id(ctx));
        return DZ_OK;
    }
    if (cap)
        return fail(ctx, DZ_INVALID_REQUEST,
                    "the workspace cannot grow during stream capture: run the call once before capturing it");
    if (ctx->work) {
        DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
        auto it = ctx->work_users.find(ctx->work);
        if (it != ctx->work_users.end() && !it->second.empty()) {
            ctx->retired_work.push_back(ctx->work);
        } else {
            if (it != ctx->work_users.end()) ctx->work_users.erase(it);
            hipFree(ctx->work);
        }
        ctx->work = nullptr;
        ctx->work_bytes = 0;
    }
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    DZ_HIP(ctx, hipMalloc(&ctx->work, want), "workspace allocation");
    ctx->work_bytes = want;
    return DZ_OK;
}

// Workspace bytes that enqueue_project needs for m rows.
size_t project_work_bytes(const dz::Weight &w, size_t m) {
    if (m <= 16) return 0;
    return m * (size_t)w.groups * 64 + 256 + m * (size_t)w.groups * sizeof(float);
}

// packed.rs:75-119 project of x [m x cols] into y [m x rows(w)]; `work` holds
// project_work_bytes(w, m). A non-finite activation sets bit 0 of the flag.
void enqueue_project(dz_ctx *ctx, const dz::Weight &w, const float *x, size_t m, float *y, uint8_t *work) {
    if (m <= 16) {
        dz::launch_grouped_small(w, x, (int)m, 8, y, ctx->flag, true, ctx->stream);
        return;
    }
    size_t qbytes = m * (size_t)w.groups * 64;
    int8_t *q = (int8_t *)work;
    float *sx = (float *)(work + (qbytes + 255) / 256 * 256);
    dz::launch_act_quantize(x, (int)m, w.cols, 8, q, sx, ctx->flag, ctx->stream);
    dz::launch_grouped_codes(w, q, sx, (int)m, y, ctx->flag, true, ctx->stream);
}

// pplx_flash/mod.rs:149-185 logits: the zero-centred RMSNorm of the selected
// hidden rows (f32 dtype 0 or f16 dtype 1; `select` a device index array or
// null), then project. Synchronous; logits on the device.
int32_t readout_rows(dz_ctx *ctx, const dz::Weight &w, const float *norm, const void *hidden, int dtype,
                     const int32_t *select, size_t rows, float eps, float *logits) {
    const size_t xbytes = (rows * (size_t)w.cols * sizeof(float) + 255) / 256 * 256;
    int32_t rc = ensure_work(ctx, xbytes + project_work_bytes(w, rows));
    if (rc) return rc;
    float *xn = (float *)ctx->work;
    int bad = 0;
    rc = flagged_sync(ctx, [&] {
        dz::launch_readout_rms(hidden, dtype, select, (int)rows, w.cols, norm, eps, 1, xn, ctx->stream);
        enqueue_project(ctx, w, xn, rows, logits, (uint8_t *)ctx->work + xbytes);
        dz::launch_flag_nonfinite(logits, rows * (size_t)w.rows, ctx->flag, 2, ctx->stream);
    }, &bad);
    if (rc) return rc;
    if (bad & 1) return fail(ctx, DZ_INFERENCE_FAILED, "nonfinite readout activation");
    if (bad & 2) return fail(ctx, DZ_INFERENCE_FAILED, "non-finite packed logits");
    return DZ_OK;
}

// This device's address of `scratch`, looked up once per device with that
// device current.
hipError_t scratch_address(int device, uint8_t **out) {
    static std::mutex mu;
    static std::map<int, uint8_t *> addresses;
    std::lock_guard<std::mutex> lock(mu);
    auto it = addresses.find(device);
    if (it != addresses.end()) {
        *out = it->second;
        return hipSuccess;
    }
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    addresses[device] = (uint8_t *)p;
    *out = (uint8_t *)p;
    return hipSuccess;
}

bool valid_dtype(int32_t d) { return d == DZ_F32 || d == DZ_F16 || d == DZ_BF16; }

int32_t alloc_weight(dz_ctx *ctx, dz::WeightKind kind, size_t rows, size_t cols, dz_weight **out) {
    if (rows == 0 || cols == 0 || rows > (1u << 28) || cols > (1u << 28))
        return fail(ctx, DZ_INVALID_PARAMETERS, "invalid weight shape");
    dz_weight *h = new dz_weight();
    dz::Weight &w = h->w;
    w.kind = kind;
    w.rows = (int)rows;
    w.cols = (int)cols;
    w.bits = kind == dz::WeightKind::Q8G64 ? 8 : 4;
    w.group = kind == dz::WeightKind::Q4G32 ? 32 : 64;
    w.groups = (int)((cols + 63) / 64);
    w.np = (int)((rows + 15) / 16 * 16);
    w.kp = w.bits == 4 ? (int)((cols + 127) / 128 * 128) : (int)((cols + 63) / 64 * 64);
    w.code_bytes = (size_t)w.np * w.kp / (w.bits == 4 ? 2 : 1);
    w.scale_bytes = w.bits == 4 ? (size_t)w.np * (w.kp / 128) * 8 : (size_t)w.np * (w.kp / 64) * 4;
    h->device = ctx->device;
    hipError_t e = hipMalloc(&w.codes, w.code_bytes);
    if (e == hipSuccess) e = hipMalloc(&w.scales, w.scale_bytes);
    if (e == hipSuccess) e = hipMemsetAsync(w.codes, w.bits == 4 ? 0x88 : 0, w.code_bytes, ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(w.scales, 0, w.scale_bytes, ctx->stream);
    if (e != hipSuccess) {
        if (w.codes) hipFree(w.codes);
        if (w.scales) hipFree(w.scales);
        delete h;
        return hip_fail(ctx, e, "weight allocation");
    }
    *out = h;
    return DZ_OK;
}

void free_weight(dz_weight *h) {
    if (!h) return;
    if (h->w.codes) hipFree(h->w.codes);
    if (h->w.scales) hipFree(h->w.scales);
    if (h->w.offsets) hipFree(h->w.offsets);
    delete h;
}

// The fitted forms (bit DZ_FIT_*) a product takes; weights that are not
// fitted run everywhere.
constexpr int kFitGrouped = 1 << DZ_FIT_SCALED | 1 << DZ_FIT_AFFINE;
constexpr int kFitScaled = 1 << DZ_FIT_SCALED;  // signed scales and -8 codes: any fold takes them
constexpr int kFitNone = 0;
const char *const kFitNames[] = {"scaled", "affine", "NF4"};

int32_t fitted_form_ok(dz_ctx *ctx, const dz_weight *w, int forms, const char *what) {
    if (!w || !w->w.fitted) return DZ_OK;
    const int form = w->w.nf4 ? DZ_FIT_NF4 : w->w.offsets ? DZ_FIT_AFFINE : DZ_FIT_SCALED;
    if (forms >> form & 1) return DZ_OK;
    return fail(ctx, DZ_INVALID_PARAMETERS,
                std::string(what) + " does not take " + kFitNames[form] + " fitted weights");
}

}  // namespace

extern "C" {

const char *dz_status_name(int32_t status) {
    switch (status) {
        case DZ_OK: return "OK";
        case DZ_INVALID_REQUEST: return "INVALID_REQUEST";
        case DZ_INVALID_PARAMETERS: return "INVALID_PARAMETERS";
        case DZ_CANCELLED: return "CANCELLED";
        case DZ_CACHE_OWNER: return "CACHE_OWNER";
        case DZ_INPUT_TOO_LONG: return "INPUT_TOO_LONG";
        case DZ_GPU_UNAVAILABLE: return "GPU_UNAVAILABLE";
        case DZ_RESOURCE_LIMIT: return "RESOURCE_LIMIT";
        case DZ_MISSING_GPU_FEATURE: return "MISSING_GPU_FEATURE";
        case DZ_INFERENCE_FAILED: return "INFERENCE_FAILED";
        case DZ_INVALID_CHECKPOINT: return "INVALID_CHECKPOINT";
        case DZ_UNSUPPORTED_CACHE: return "UNSUPPORTED_CACHE";
        default: return "UNKNOWN";
    }
}

int32_t dz_init(int32_t device, dz_ctx **out) {
    if (!out) return DZ_INVALID_REQUEST;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return DZ_GPU_UNAVAILABLE;
    if (device < 0 || device >= count) return DZ_GPU_UNAVAILABLE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return DZ_GPU_UNAVAILABLE;
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) return DZ_MISSING_GPU_FEATURE;
    dz_ctx *ctx = new dz_ctx();
    ctx->device = device;
    ctx->arch = prop.gcnArchName;
    ctx->cus = prop.multiProcessorCount;
    ctx->clock_khz = prop.clockRate;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&ctx->own, hipStreamNonBlocking) != hipSuccess ||
        hipMalloc(&ctx->flag, kFlagBytes) != hipSuccess || hipMemset(ctx->flag, 0, kFlagBytes) != hipSuccess) {
        delete ctx;
        return DZ_GPU_UNAVAILABLE;
    }
    if (scratch_address(device, &ctx->scratch) != hipSuccess) {
        hipStreamDestroy(ctx->own);
        hipFree(ctx->flag);
        delete ctx;
        return DZ_GPU_UNAVAILABLE;
    }
    ctx->stream = ctx->own;
    *out = ctx;
    return DZ_OK;
}

void dz_destroy(dz_ctx *ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    if (ctx->work) hipFree(ctx->work);
    for (void *p : ctx->retired_work) hipFree(p);
    if (ctx->flag) hipFree(ctx->flag);
    if (ctx->own) hipStreamDestroy(ctx->own);
    delete ctx;
}

const char *dz_last_error(const dz_ctx *ctx) { return ctx ? ctx->error.c_str() : "no context"; }

int32_t dz_set_stream(dz_ctx *ctx, void *hip_stream) {
    DZ_BEGIN(ctx);
    hipStream_t next = hip_stream ? (hipStream_t)hip_stream : ctx->own;
    if (next == ctx->stream) return DZ_OK;
    // The workspace and the product flag ring are shared by every call on the
    // context: work still queued on the old stream must finish before calls on
    // the new one may reuse them.
    if (capturing(ctx)) return fail(ctx, DZ_INVALID_REQUEST, "stream change while the stream records a graph");
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    ctx->stream = next;
    ctx->product_calls = 0;
    return DZ_OK;
}

int32_t dz_sync(dz_ctx *ctx) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    return DZ_OK;
}

int32_t dz_capture_id(dz_ctx *ctx, uint64_t *id) {
    DZ_BEGIN(ctx);
    if (!id) return fail(ctx, DZ_INVALID_REQUEST, "null output");
    if (!capturing(ctx)) return fail(ctx, DZ_INVALID_REQUEST, "the context stream is not recording a graph");
    *id = capture_id(ctx);
    return DZ_OK;
}

int32_t dz_capture_release(dz_ctx *ctx, uint64_t id) {
    DZ_BEGIN(ctx);
    if (capturing(ctx) && capture_id(ctx) == id)
        return fail(ctx, DZ_INVALID_REQUEST, "the capture is still recording: release it after hipStreamEndCapture");
    auto it = ctx->capture_slots.find(id);
    if (it != ctx->capture_slots.end()) {
        for (int index : it->second) ctx->free_capture_slots.push_back(index);
        ctx->capture_slots.erase(it);
    }
    for (auto &kv : ctx->work_users) kv.second.erase(id);
    free_unused_retired(ctx);
    return DZ_OK;
}

int32_t dz_capture_release_all(dz_ctx *ctx) {
    DZ_BEGIN(ctx);
    if (capturing(ctx)) return fail(ctx, DZ_INVALID_REQUEST, "the context stream is recording a graph");
    ctx->capture_slots.clear();
    ctx->free_capture_slots.clear();
    ctx->captured_flags = 0;
    ctx->work_users.clear();
    free_unused_retired(ctx);
    return DZ_OK;
}

int32_t dz_info(dz_ctx *ctx, char *buf, size_t cap) {
    DZ_BEGIN(ctx);
    std::string s = "{\"arch\":\"" + ctx->arch + "\",\"compute_units\":" + std::to_string(ctx->cus) +
                    ",\"clock_khz\":" + std::to_string(ctx->clock_khz) + ",\"variants\":{";
    bool first = true;
    for (const char *f : {"gemv", "gemm_w4a16", "i8_gemm", "grouped", "mlp", "delta_scan", "norm"}) {
        if (!first) s += ",";
        first = false;
        s += std::string("\"") + f + "\":\"" + dz::variant_name(f, variant(ctx, f)) + "\"";
    }
    s += "},\"tuning\":" + (ctx->tuning.empty() ? std::string("null") : ctx->tuning);
    size_t held = 0;
    for (const auto &kv : ctx->capture_slots) held += kv.second.size();
    s += ",\"capture_slots\":{\"held\":" + std::to_string(held) + ",\"limit\":" + std::to_string(kCaptureSlots) +
         ",\"captures\":" + std::to_string(ctx->capture_slots.size()) +
         ",\"retired_workspaces\":" + std::to_string(ctx->retired_work.size()) + "}}";
    if (!buf || cap < s.size() + 1) return fail(ctx, DZ_RESOURCE_LIMIT, "info buffer too small");
    memcpy(buf, s.c_str(), s.size() + 1);
    return DZ_OK;
}

int32_t dz_alloc(dz_ctx *ctx, size_t bytes, void **dev) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (!dev) return fail(ctx, DZ_INVALID_REQUEST, "null output");
    DZ_HIP(ctx, hipMalloc(dev, bytes ? bytes : 1), "hipMalloc");
    return DZ_OK;
}

int32_t dz_free(dz_ctx *ctx, void *dev) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    if (dev) DZ_HIP(ctx, hipFree(dev), "hipFree");
    return DZ_OK;
}

int32_t dz_copy_h2d(dz_ctx *ctx, void *dst, const void *src, size_t bytes) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (bytes && (!dst || !src)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    DZ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "copy to device");
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    return DZ_OK;
}

int32_t dz_copy_d2h(dz_ctx *ctx, void *dst, const void *src, size_t bytes) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (bytes && (!dst || !src)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    DZ_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "copy to host");
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    return DZ_OK;
}

// ---- weights ------------------------------------------------------------------------

namespace {

int32_t upload_weight(dz_ctx *ctx, const void *packed, size_t bytes, int32_t layout, size_t rows, size_t cols,
                      bool fitted, dz_weight **out) {
    if (!out || (!packed && bytes)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    *out = nullptr;
    dz::WeightKind kind;
    size_t run, gbytes;
    switch (layout) {
        case DZ_Q4_G64_F32: kind = dz::WeightKind::Q4G64; run = 64; gbytes = 36; break;
        case DZ_Q8_G64_F32: kind = dz::WeightKind::Q8G64; run = 64; gbytes = 68; break;
        case DZ_Q4_G32_F16: kind = dz::WeightKind::Q4G32; run = 32; gbytes = 18; break;
        default: return fail(ctx, DZ_INVALID_PARAMETERS, "unknown packed layout");
    }
    if (rows == 0 || cols == 0 || cols % run != 0)
        return fail(ctx, DZ_INVALID_CHECKPOINT, "invalid packed matrix shape");
    if (bytes != rows * (cols / run) * gbytes)
        return fail(ctx, DZ_INVALID_CHECKPOINT, "packed byte count does not match the shape");
    dz_weight *h = nullptr;
    int32_t rc = alloc_weight(ctx, kind, rows, cols, &h);
    if (rc) return rc;
    uint8_t *staging = nullptr;
    hipError_t e = hipMalloc(&staging, bytes);
    if (e != hipSuccess) {
        free_weight(h);
        return hip_fail(ctx, e, "staging allocation");
    }
    e = hipMemcpyAsync(staging, packed, bytes, hipMemcpyHostToDevice, ctx->stream);
    int bad = 0;
    if (e == hipSuccess) {
        rc = flagged_sync(ctx, [&] { dz::launch_upload(h->w, staging, ctx->flag, ctx->stream, fitted); }, &bad);
    } else {
        rc = hip_fail(ctx, e, "copy to device");
    }
    hipFree(staging);
    if (rc) {
        free_weight(h);
        return rc;
    }
    if (bad) {
        free_weight(h);
        return fail(ctx, DZ_INVALID_CHECKPOINT, "invalid packed scale");
    }
    *out = h;
    return DZ_OK;
}

}  // namespace

int32_t dz_weight_upload(dz_ctx *ctx, const void *packed, size_t bytes, int32_t layout,
                         size_t rows, size_t cols, dz_weight **out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return upload_weight(ctx, packed, bytes, layout, rows, cols, false, out);
}

int32_t dz_weight_upload_fitted(dz_ctx *ctx, const void *packed, size_t bytes, size_t rows, size_t cols,
                                int32_t form, const float *offsets, dz_weight **out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (form != DZ_FIT_SCALED && form != DZ_FIT_AFFINE && form != DZ_FIT_NF4)
        return fail(ctx, DZ_INVALID_PARAMETERS, "unknown fitted form");
    if ((form == DZ_FIT_AFFINE) != (offsets != nullptr))
        return fail(ctx, DZ_INVALID_REQUEST, "affine weights take offsets and the other forms none");
    dz_weight *h = nullptr;
    int32_t rc = upload_weight(ctx, packed, bytes, DZ_Q4_G64_F32, rows, cols, true, &h);
    if (rc) return rc;
    h->w.fitted = true;
    h->w.nf4 = form == DZ_FIT_NF4;
    if (offsets) {
        // [rows x groups] -> the group-64 scale layout: [tile][k-block][16 rows][2]
        dz::Weight &w = h->w;
        const size_t groups = cols / 64, kbs = (size_t)w.kblocks();
        std::vector<float> native(w.scale_bytes / sizeof(float), 0.0f);
        for (size_t r = 0; r < rows; r++)
            for (size_t g = 0; g < groups; g++) {
                const float v = offsets[r * groups + g];
                if (!isfinite(v)) {
                    free_weight(h);
                    return fail(ctx, DZ_INVALID_CHECKPOINT, "non-finite affine offset");
                }
                native[(((r / 16) * kbs + g / 2) * 16 + r % 16) * 2 + g % 2] = v;
            }
        hipError_t e = hipMalloc(&w.offsets, w.scale_bytes);
        if (e == hipSuccess)
            e = hipMemcpyAsync(w.offsets, native.data(), w.scale_bytes, hipMemcpyHostToDevice, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            free_weight(h);
            return hip_fail(ctx, e, "affine offsets");
        }
    }
    *out = h;
    return DZ_OK;
}

int32_t dz_weight_quantize(dz_ctx *ctx, const void *values, int32_t dtype, size_t rows,
                           size_t cols, int32_t bits, int32_t group, dz_weight **out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (!out || !values) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    *out = nullptr;
    if (!valid_dtype(dtype)) return fail(ctx, DZ_INVALID_PARAMETERS, "unknown dtype");
    dz::WeightKind kind;
    if (bits == 4 && group == 64)
        kind = dz::WeightKind::Q4G64;
    else if (bits == 8 && group == 64)
        kind = dz::WeightKind::Q8G64;
    else if (bits == 4 && group == 32)
        kind = dz::WeightKind::Q4G32;
    else
        return fail(ctx, DZ_INVALID_PARAMETERS, "unsupported quantization bits");
    dz_weight *h = nullptr;
    int32_t rc = alloc_weight(ctx, kind, rows, cols, &h);
    if (rc) return rc;
    int bad = 0;
    rc = flagged_sync(ctx, [&] { dz::launch_quantize_weight(h->w, values, dtype, ctx->flag, ctx->stream); }, &bad);
    if (rc || bad) {
        free_weight(h);
        return rc ? rc : fail(ctx, DZ_INVALID_CHECKPOINT, "non-finite INT8 weight");
    }
    *out = h;
    return DZ_OK;
}

int32_t dz_weight_free(dz_ctx *ctx, dz_weight *w) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    DZ_HIP(ctx, hipStreamSynchronize(ctx->stream), "stream synchronize");
    free_weight(w);
    return DZ_OK;
}

int32_t dz_weight_info(const dz_weight *h, size_t *rows, size_t *cols, int32_t *bits,
                       int32_t *group, size_t *device_bytes) {
    if (!h) return DZ_INVALID_REQUEST;
    if (rows) *rows = (size_t)h->w.rows;
    if (cols) *cols = (size_t)h->w.cols;
    if (bits) *bits = h->w.bits;
    if (group) *group = h->w.group;
    if (device_bytes) *device_bytes = h->w.code_bytes + h->w.scale_bytes + (h->w.offsets ? h->w.scale_bytes : 0);
    return DZ_OK;
}

int32_t dz_dequant(dz_ctx *ctx, const dz_weight *w, float *y) {
    DZ_BEGIN(ctx);
    if (!w || !y) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    dz::launch_dequant(w->w, nullptr, w->w.rows, y, 0, ctx->stream);
    return launched(ctx, "dequant");
}

int32_t dz_dequant_rows(dz_ctx *ctx, const dz_weight *w, const int32_t *ids, size_t count, void *y,
                        int32_t dtype) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (!w || (count && (!ids || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (dtype != DZ_F32 && dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "dtype must be f32 or f16");
    int bad = 0;
    int32_t rc = flagged_sync(ctx, [&] {
        dz::launch_dequant_checked(w->w, ids, (int)count, y, dtype == DZ_F16 ? 1 : 0, ctx->flag, ctx->stream);
    }, &bad);
    if (rc) return rc;
    if (bad) return fail(ctx, DZ_INVALID_REQUEST, "token ID out of range");
    return DZ_OK;
}

// ---- quantized products ------------------------------------------------------------

int32_t dz_act_quantize(dz_ctx *ctx, const float *x, size_t m, size_t k, int32_t bits, int8_t *q,
                        float *s) {
    DZ_BEGIN(ctx);
    if (bits != 4 && bits != 8) return fail(ctx, DZ_INVALID_PARAMETERS, "unsupported quantization bits");
    if (k == 0) return fail(ctx, DZ_INVALID_PARAMETERS, "invalid activation shape");
    if (m && (!x || !q || !s)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    dz::launch_act_quantize(x, (int)m, (int)k, bits, q, s, nullptr, ctx->stream);
    return launched(ctx, "act_quantize");
}

namespace {

// Up to four rows, and up to 16 for fitted affine weights (whose code sums
// only the few-row kernel takes itself), the few-row kernel quantizes x in
// every block. From five rows one quantization and the few-row kernel over
// the codes are faster: its blocks re-quantized every row of x (M = 16,
// K = 2560, N = 9216: 15.1 against 37.6 us; M = 8: 10.5 against 20.8 us).
bool grouped_quantizes_in_kernel(size_t m, bool affine) { return m <= 4 || (m <= 16 && affine); }

// The grouped product of A8 codes: the few-row kernel up to 16 rows, the
// pipelined or tiled kernels above (launch_grouped).
void grouped_of_codes(dz_ctx *ctx, const dz::Weight &w, const int8_t *q, const float *s, size_t m, float *y,
                      const int *bad, const float *sq) {
    if (m <= 16)
        dz::launch_grouped_codes(w, q, s, (int)m, y, bad, false, ctx->stream);
    else
        dz::launch_grouped(w, q, s, (int)m, y, bad, variant(ctx, "grouped"), ctx->stream, nullptr, sq);
}

int32_t grouped_linear(dz_ctx *ctx, const dz_weight *a, const dz_weight *b, const float *x,
                       size_t m, float *ya, float *yb, int32_t mode) {
    const dz::Weight &w = a->w;
    if (w.kind == dz::WeightKind::Q4G32)
        return fail(ctx, DZ_INVALID_PARAMETERS, "grouped int8 mode needs a group-64 weight");
    if (b && (b->w.cols != w.cols || b->w.kind == dz::WeightKind::Q4G32))
        return fail(ctx, DZ_INVALID_PARAMETERS, "paired weights must share the input width");
    if (int32_t rc = fitted_form_ok(ctx, a, kFitGrouped, "the grouped product")) return rc;
    if (int32_t rc = fitted_form_ok(ctx, b, kFitGrouped, "the grouped product")) return rc;
    if (m == 0) return DZ_OK;
    const int abits = mode == DZ_W4A4 ? 4 : 8;
    const bool sums = w.offsets || (b && b->w.offsets);
    if (grouped_quantizes_in_kernel(m, sums)) {
        // one launch per weight: the kernel quantizes x itself (same codes as act_quantize)
        dz::launch_grouped_small(w, x, (int)m, abits, ya, nullptr, false, ctx->stream);
        if (b) dz::launch_grouped_small(b->w, x, (int)m, abits, yb, nullptr, false, ctx->stream);
        return launched(ctx, "grouped linear");
    }
    // codes, their scales and, for affine weights, sx * f32(sum of the codes) per group
    size_t qbytes = m * (size_t)w.groups * 64, sbytes = m * (size_t)w.groups * sizeof(float);
    const size_t sq_at = (qbytes + 255) / 256 * 256 + (sbytes + 255) / 256 * 256;
    int32_t rc = ensure_work(ctx, sums ? sq_at + sbytes : qbytes + sbytes + 256);
    if (rc) return rc;
    int8_t *q = (int8_t *)ctx->work;
    float *s = (float *)((uint8_t *)ctx->work + (qbytes + 255) / 256 * 256);
    float *sq = sums ? (float *)((uint8_t *)ctx->work + sq_at) : nullptr;
    int *bad = nullptr;
    rc = product_flag(ctx, &bad);
    if (rc) return rc;
    dz::launch_act_quantize(x, (int)m, w.cols, abits, q, s, bad, ctx->stream);
    if (sums) dz::launch_act_sums(q, s, (int)m, w.groups, sq, ctx->stream);
    grouped_of_codes(ctx, w, q, s, m, ya, bad, sq);
    if (b) grouped_of_codes(ctx, b->w, q, s, m, yb, bad, sq);
    return launched(ctx, "grouped linear");
}

}  // namespace

int32_t dz_linear(dz_ctx *ctx, const dz_weight *w, const void *x, int32_t x_dtype, size_t m,
                  float *y, int32_t mode) {
    DZ_BEGIN(ctx);
    if (!w || (m && (!x || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (m > (1u << 24)) return fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    if (mode == DZ_W4A8 || mode == DZ_W4A4) {
        if (x_dtype != DZ_F32) return fail(ctx, DZ_INVALID_PARAMETERS, "grouped int8 mode takes f32 activations");
        return grouped_linear(ctx, w, nullptr, (const float *)x, m, y, nullptr, mode);
    }
    if (mode == DZ_W4A16) {
        if (x_dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 takes f16 activations");
        if (w->w.bits != 4) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 needs a Q4 weight");
        if (w->w.cols % 8 != 0) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 needs cols % 8 == 0");
        if (((uintptr_t)x & 15) != 0) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 activations must be 16-byte aligned");
        if (int32_t rc = fitted_form_ok(ctx, w, kFitScaled, "W4A16")) return rc;
        if (m == 0) return DZ_OK;
        dz::launch_w4a16(w->w, (const dz::half_t *)x, (int)m, y, variant(ctx, "gemv"),
                         variant(ctx, "gemm_w4a16"), ctx->stream);
        return launched(ctx, "w4a16 linear");
    }
    return fail(ctx, DZ_INVALID_PARAMETERS, "unknown mode");
}

int32_t dz_linear_noalloc(dz_ctx *ctx, const dz_weight *w, const void *x, int32_t x_dtype, size_t m, float *y,
                          int32_t mode) {
    DZ_BEGIN(ctx);
    if (!w || (m && (!x || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (m > (1u << 24)) return fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    if (mode == DZ_W4A16 || (m <= 16 && grouped_quantizes_in_kernel(m, w->w.offsets != nullptr)))
        return dz_linear(ctx, w, x, x_dtype, m, y, mode);  // no workspace on these paths
    if (mode != DZ_W4A8 && mode != DZ_W4A4) return fail(ctx, DZ_INVALID_PARAMETERS, "unknown mode");
    if (x_dtype != DZ_F32) return fail(ctx, DZ_INVALID_PARAMETERS, "grouped int8 mode takes f32 activations");
    const dz::Weight &wt = w->w;
    if (wt.kind == dz::WeightKind::Q4G32)
        return fail(ctx, DZ_INVALID_PARAMETERS, "grouped int8 mode needs a group-64 weight");
    if (int32_t rc = fitted_form_ok(ctx, w, kFitGrouped, "the grouped product")) return rc;
    // [0, 256) the flag, then the codes, then the scales, then for affine
    // weights sx * sum of the codes (each part 256-byte aligned)
    const size_t qbytes = m * (size_t)wt.groups * 64, sbytes = m * (size_t)wt.groups * sizeof(float);
    const size_t sq_at = 256 + (qbytes + 255) / 256 * 256 + (sbytes + 255) / 256 * 256;
    const size_t need = wt.offsets ? sq_at + sbytes : 256 + (qbytes + 255) / 256 * 256 + sbytes;
    if (need > kScratchBytes)
        return fail(ctx, DZ_RESOURCE_LIMIT,
                    "dz_linear_noalloc: " + std::to_string(m) + " rows of " + std::to_string(wt.cols) +
                        " need " + std::to_string(need) + " bytes of its " + std::to_string(kScratchBytes) +
                        "-byte scratch");
    int *bad = (int *)ctx->scratch;
    int8_t *q = (int8_t *)(ctx->scratch + 256);
    float *sx = (float *)(ctx->scratch + 256 + (qbytes + 255) / 256 * 256);
    const int abits = mode == DZ_W4A4 ? 4 : 8;
    dz::launch_fill_i32(bad, 0, 1, ctx->stream);  // a kernel, not a memset: graph replays clear it too
    float *sq = wt.offsets ? (float *)(ctx->scratch + sq_at) : nullptr;
    dz::launch_act_quantize((const float *)x, (int)m, wt.cols, abits, q, sx, bad, ctx->stream);
    if (sq) dz::launch_act_sums(q, sx, (int)m, wt.groups, sq, ctx->stream);
    grouped_of_codes(ctx, wt, q, sx, m, y, bad, sq);
    return launched(ctx, "grouped linear (no allocation)");
}

int32_t dz_linear_f16(dz_ctx *ctx, const dz_weight *w, const void *x, size_t m, void *y, int32_t epilogue,
                      const void *residual) {
    DZ_BEGIN(ctx);
    if (!w || (m && (!x || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (epilogue < DZ_EPI_NONE || epilogue > DZ_EPI_RESIDUAL)
        return fail(ctx, DZ_INVALID_PARAMETERS, "unknown epilogue");
    if (epilogue == DZ_EPI_RESIDUAL && m && !residual) return fail(ctx, DZ_INVALID_REQUEST, "null residual");
    if (w->w.bits != 4) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 needs a Q4 weight");
    if (int32_t rc = fitted_form_ok(ctx, w, kFitScaled, "dz_linear_f16")) return rc;
    if (w->w.cols % 8 != 0) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 needs cols % 8 == 0");
    if (((uintptr_t)x & 15) != 0) return fail(ctx, DZ_INVALID_PARAMETERS, "W4A16 activations must be 16-byte aligned");
    if (m == 0) return DZ_OK;
    if (m > (1u << 24)) return fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    if (m <= 16) {
        // the GEMV's f32 products (dz_linear's few-row arithmetic), then the epilogue
        const size_t count = m * (size_t)w->w.rows;
        int32_t rc = ensure_work(ctx, count * sizeof(float));
        if (rc) return rc;
        dz::launch_w4a16(w->w, (const dz::half_t *)x, (int)m, (float *)ctx->work, variant(ctx, "gemv"),
                         variant(ctx, "gemm_w4a16"), ctx->stream);
        dz::launch_f16_epilogue((const float *)ctx->work, epilogue, (const dz::half_t *)residual,
                                (dz::half_t *)y, count, ctx->stream);
    } else {
        dz::launch_w4a16_f16(w->w, (const dz::half_t *)x, (int)m, (dz::half_t *)y, epilogue,
                             (const dz::half_t *)residual, variant(ctx, "gemm_w4a16"), ctx->stream);
    }
    return launched(ctx, "w4a16 f16 linear");
}

int32_t dz_linear_pair(dz_ctx *ctx, const dz_weight *a, const dz_weight *b, const float *x, size_t m,
                       float *ya, float *yb, int32_t mode) {
    DZ_BEGIN(ctx);
    if (!a || !b || (m && (!x || !ya || !yb))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (mode != DZ_W4A8 && mode != DZ_W4A4) return fail(ctx, DZ_INVALID_PARAMETERS, "pair takes a grouped int8 mode");
    return grouped_linear(ctx, a, b, x, m, ya, yb, mode);
}

int32_t dz_mlp_requant(dz_ctx *ctx, const dz_weight *gate, const dz_weight *up, const float *x,
                       size_t m, int8_t *qo, float *so) {
    DZ_BEGIN(ctx);
    if (!gate || !up || (m && (!x || !qo || !so))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    const dz::Weight &g = gate->w, &u = up->w;
    if (g.kind != dz::WeightKind::Q4G64 || u.kind != dz::WeightKind::Q4G64)
        return fail(ctx, DZ_INVALID_PARAMETERS, "fused MLP needs Q4 group-64 weights");
    if (int32_t rc = fitted_form_ok(ctx, gate, kFitScaled, "dz_mlp_requant")) return rc;
    if (int32_t rc = fitted_form_ok(ctx, up, kFitScaled, "dz_mlp_requant")) return rc;
    if (g.rows != u.rows || g.cols != u.cols || g.rows % 64 != 0)
        return fail(ctx, DZ_INVALID_PARAMETERS, "fused MLP shapes must match with rows % 64 == 0");
    if (m == 0) return DZ_OK;
    size_t qbytes = m * (size_t)g.groups * 64, sbytes = m * (size_t)g.groups * sizeof(float);
    int32_t rc = ensure_work(ctx, qbytes + sbytes + 256);
    if (rc) return rc;
    int8_t *q = (int8_t *)ctx->work;
    float *s = (float *)((uint8_t *)ctx->work + (qbytes + 255) / 256 * 256);
    int *bad = nullptr;
    rc = product_flag(ctx, &bad);
    if (rc) return rc;
    dz::launch_act_quantize(x, (int)m, g.cols, 8, q, s, bad, ctx->stream);
    dz::launch_mlp_requant(g, u, q, s, (int)m, qo, so, bad, variant(ctx, "mlp"), ctx->stream);
    return launched(ctx, "fused MLP");
}

int32_t dz_linear_q8(dz_ctx *ctx, const dz_weight *w, const int8_t *q, const float *s, size_t m,
                     float *y) {
    DZ_BEGIN(ctx);
    if (!w || (m && (!q || !s || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (w->w.kind == dz::WeightKind::Q4G32)
        return fail(ctx, DZ_INVALID_PARAMETERS, "grouped int8 mode needs a group-64 weight");
    if (int32_t rc = fitted_form_ok(ctx, w, kFitScaled, "dz_linear_q8")) return rc;
    if (m <= 16)
        dz::launch_grouped_codes(w->w, q, s, (int)m, y, nullptr, false, ctx->stream);
    else
        dz::launch_grouped(w->w, q, s, (int)m, y, nullptr, variant(ctx, "grouped"), ctx->stream);
    return launched(ctx, "grouped linear");
}

int32_t dz_project(dz_ctx *ctx, const dz_weight *w, const float *x, size_t m, float *y) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (!w || (m && (!x || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (w->w.kind == dz::WeightKind::Q4G32 || w->w.cols % 64 != 0)
        return fail(ctx, DZ_INVALID_PARAMETERS, "invalid packed readout shape");
    if (int32_t rc = fitted_form_ok(ctx, w, kFitScaled, "dz_project")) return rc;
    if (m == 0) return DZ_OK;
    if (m > (1u << 24)) return fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    int32_t rc = ensure_work(ctx, project_work_bytes(w->w, m));
    if (rc) return rc;
    int bad = 0;
    rc = flagged_sync(ctx, [&] { enqueue_project(ctx, w->w, x, m, y, (uint8_t *)ctx->work); }, &bad);
    if (rc) return rc;
    if (bad) return fail(ctx, DZ_INFERENCE_FAILED, "nonfinite readout activation");
    return DZ_OK;
}

int32_t dz_readout(dz_ctx *ctx, const dz_weight *w, const float *norm, const float *hidden, size_t rows,
                   float eps, float *logits) {
    DZ_BEGIN(ctx);
    if (!w || !norm || (rows && (!hidden || !logits))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (w->w.kind == dz::WeightKind::Q4G32 || w->w.cols % 64 != 0 || w->w.cols > dz::kReadoutMaxCols)
        return fail(ctx, DZ_INVALID_PARAMETERS, "invalid packed readout shape");
    if (int32_t rc = fitted_form_ok(ctx, w, kFitScaled, "dz_readout")) return rc;
    if (rows == 0) return DZ_OK;
    if (rows > (1u << 20)) return fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    return readout_rows(ctx, w->w, norm, hidden, 0, nullptr, rows, eps, logits);
}

int32_t dz_act_quantize_records(dz_ctx *ctx, const float *x, size_t m, size_t k, uint32_t *records) {
    DZ_BEGIN(ctx);
    if (k == 0 || k % 64 != 0) return fail(ctx, DZ_INVALID_PARAMETERS, "records need k % 64 == 0");
    if (m && (!x || !records)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    dz::launch_act_quantize_records(x, (int)m, (int)k, records, nullptr, ctx->stream);
    return launched(ctx, "act_quantize_records");
}

int32_t dz_linear_records(dz_ctx *ctx, const dz_weight *w, const uint32_t *records, size_t m, float *y) {
    DZ_BEGIN(ctx);
    if (!w || (m && (!records || !y))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (w->w.kind == dz::WeightKind::Q4G32 || w->w.cols % 64 != 0)
        return fail(ctx, DZ_INVALID_PARAMETERS, "records products need a group-64 weight with cols % 64 == 0");
    if (int32_t rc = fitted_form_ok(ctx, w, kFitNone, "dz_linear_records")) return rc;
    if (m > (1u << 24)) return fail(ctx, DZ_INPUT_TOO_LONG, "input budget exceeded");
    dz::launch_grouped_records(w->w, records, (int)m, y, ctx->stream);
    return launched(ctx, "grouped records linear");
}

int32_t dz_i8_quantize_rows(dz_ctx *ctx, const float *x, size_t rows, size_t k, int8_t *q,
                            float *scales, int32_t *sums) {
    DZ_BEGIN(ctx);
    if (rows && (!x || !q || !scales)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (k == 0 || k > 32768) return fail(ctx, DZ_INVALID_PARAMETERS, "INT8 reduction must be 1..32768");
    dz::launch_i8_quantize_rows(x, (int)rows, (int)k, q, scales, sums, ctx->stream);
    return launched(ctx, "i8 quantize");
}

int32_t dz_i8_gemm(dz_ctx *ctx, const int8_t *a, const float *sa, size_t m, const int8_t *w,
                   const float *sw, size_t n, size_t k, void *y, int32_t raw) {
    DZ_BEGIN(ctx);
    if ((m && n) && (!a || !w || !y || (!raw && (!sa || !sw))))
        return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (k == 0 || k > 32768) return fail(ctx, DZ_INVALID_PARAMETERS, "INT8 reduction must be 1..32768");
    dz::launch_i8_gemm(a, sa, (int)m, w, sw, (int)n, (int)k, y, raw ? 1 : 0, variant(ctx, "i8_gemm"), ctx->stream);
    return launched(ctx, "i8 gemm");
}

int32_t dz_i8_gemm_fused(dz_ctx *ctx, const int8_t *a, const float *sa, size_t m, const int8_t *wg,
                         const float *sg, const int8_t *wu, const float *su, size_t n, size_t k, float *y) {
    DZ_BEGIN(ctx);
    if ((m && n) && (!a || !sa || !wg || !sg || !wu || !su || !y)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (k == 0 || k > 32768) return fail(ctx, DZ_INVALID_PARAMETERS, "INT8 reduction must be 1..32768");
    dz::launch_i8_gemm_fused(a, sa, (int)m, wg, sg, wu, su, (int)n, (int)k, y, ctx->stream);
    return launched(ctx, "i8 gemm fused");
}

int32_t dz_q4_quantize_rows(dz_ctx *ctx, const void *values, int32_t dtype, size_t rows, size_t k,
                            uint32_t *out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (dtype != DZ_F32 && dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "dtype must be f32 or f16");
    if (k == 0 || k % 8 != 0 || k > 32768)
        return fail(ctx, DZ_INVALID_PARAMETERS, "Q4 reduction must be a multiple of eight, at most 32768");
    if (rows && (!values || !out)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (rows == 0) return DZ_OK;
    int bad = 0;
    int32_t rc = flagged_sync(ctx, [&] {
        dz::launch_q4_quantize_rows(values, dtype == DZ_F16 ? 1 : 0, (int)rows, (int)k, out, ctx->flag, ctx->stream);
    }, &bad);
    if (rc) return rc;
    if (bad) return fail(ctx, DZ_INVALID_CHECKPOINT, "non-finite Q4 weight");
    return DZ_OK;
}

int32_t dz_q4_rows_gemm(dz_ctx *ctx, const int8_t *a, const float *sa, size_t m, const uint32_t *w, size_t n,
                        size_t k, void *y, int32_t raw) {
    DZ_BEGIN(ctx);
    if ((m && n) && (!a || !w || !y || (!raw && !sa))) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (k == 0 || k % 8 != 0 || k > 32768)
        return fail(ctx, DZ_INVALID_PARAMETERS, "Q4 reduction must be a multiple of eight, at most 32768");
    const float *sw = (const float *)(w + n * (k / 8));  // the row scales follow the code words
    dz::launch_i8_gemm(a, sa, (int)m, (const int8_t *)w, sw, (int)n, (int)k, y, raw ? 1 : 0, variant(ctx, "i8_gemm"),
                       ctx->stream, true);
    return launched(ctx, "q4 rows gemm");
}

// ---- epilogues --------------------------------------------------------------------------

int32_t dz_layernorm(dz_ctx *ctx, const void *x, void *y, int32_t dtype, size_t rows, size_t d,
                     const float *w, const float *b, float eps) {
    DZ_BEGIN(ctx);
    if (dtype != DZ_F32 && dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "dtype must be f32 or f16");
    if (rows && (!x || !y || !w || !b || d == 0)) return fail(ctx, DZ_INVALID_REQUEST, "invalid layernorm arguments");
    dz::launch_layernorm(x, y, dtype == DZ_F16 ? 1 : 0, (int)rows, (int)d, w, b, eps, ctx->stream);
    return launched(ctx, "layernorm");
}

int32_t dz_rmsnorm(dz_ctx *ctx, const float *x, float *y, size_t rows, size_t d, const float *w,
                   float eps, int32_t zero_centered) {
    DZ_BEGIN(ctx);
    if (rows && (!x || !y || !w || d == 0)) return fail(ctx, DZ_INVALID_REQUEST, "invalid rmsnorm arguments");
    dz::launch_rmsnorm(x, y, (int)rows, (int)d, w, eps, zero_centered, ctx->stream);
    return launched(ctx, "rmsnorm");
}

int32_t dz_gelu(dz_ctx *ctx, void *x, int32_t dtype, size_t n) {
    DZ_BEGIN(ctx);
    if (dtype != DZ_F32 && dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "dtype must be f32 or f16");
    if (n && !x) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    dz::launch_gelu(x, dtype == DZ_F16 ? 1 : 0, n, ctx->stream);
    return launched(ctx, "gelu");
}

int32_t dz_silu_mul(dz_ctx *ctx, float *g, const float *u, size_t n) {
    DZ_BEGIN(ctx);
    if (n && (!g || !u)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    dz::launch_silu_mul(g, u, n, ctx->stream);
    return launched(ctx, "silu_mul");
}

int32_t dz_add(dz_ctx *ctx, void *x, const void *y, int32_t dtype, size_t n) {
    DZ_BEGIN(ctx);
    if (dtype != DZ_F32 && dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "dtype must be f32 or f16");
    if (n && (!x || !y)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    dz::launch_add(x, y, dtype == DZ_F16 ? 1 : 0, n, ctx->stream);
    return launched(ctx, "add");
}

int32_t dz_softmax_rows(dz_ctx *ctx, float *x, size_t rows, size_t n) {
    DZ_BEGIN(ctx);
    if (rows && (!x || n == 0)) return fail(ctx, DZ_INVALID_REQUEST, "invalid softmax arguments");
    dz::launch_softmax_rows(x, (int)rows, (int)n, ctx->stream);
    return launched(ctx, "softmax");
}

int32_t dz_mean_rows(dz_ctx *ctx, const void *x, int32_t dtype, size_t batch, size_t rows, size_t d,
                     float *out) {
    DZ_BEGIN(ctx);
    if (dtype != DZ_F32 && dtype != DZ_F16) return fail(ctx, DZ_INVALID_PARAMETERS, "dtype must be f32 or f16");
    if (batch && (!x || !out || rows == 0 || d == 0)) return fail(ctx, DZ_INVALID_REQUEST, "invalid mean arguments");
    dz::launch_mean_rows(x, dtype == DZ_F16 ? 1 : 0, (int)batch, (int)rows, (int)d, out, ctx->stream);
    return launched(ctx, "mean");
}

int32_t dz_attention(dz_ctx *ctx, const void *qkv, void *out, size_t batch, size_t seq, size_t heads,
                     size_t dh, float scale) {
    DZ_BEGIN(ctx);
    if (dh != 64) return fail(ctx, DZ_INVALID_PARAMETERS, "attention needs head_dim 64");
    if (batch && seq && (!qkv || !out || heads == 0)) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (!dz::attention_fits(seq, heads)) return fail(ctx, DZ_INPUT_TOO_LONG, "attention sequence too long");
    dz::launch_attention((const dz::half_t *)qkv, (dz::half_t *)out, (int)batch, (int)seq, (int)heads,
                         (int)dh, scale, ctx->stream);
    return launched(ctx, "attention");
}

// ---- encoder --------------------------------------------------------------------------

int32_t dz_encoder_create_random(dz_ctx *ctx, const dz_encoder_config *cfg, uint64_t seed,
                                 dz_encoder **out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_create_random(ctx, cfg, seed, out);
}

void dz_encoder_destroy(dz_ctx *ctx, dz_encoder *enc) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    dz::encoder_destroy(ctx, enc);
}

int32_t dz_encoder_embedding_row_bytes(const dz_encoder *enc, size_t *row_bytes) {
    return dz::encoder_row_bytes(enc, row_bytes);
}

const dz_weight *dz_encoder_weight(const dz_encoder *enc, int32_t layer, int32_t which) {
    return dz::encoder_weight(enc, layer, which);
}

int32_t dz_encoder_read_rows(dz_ctx *ctx, const dz_encoder *enc, const int32_t *ids, size_t count,
                             void *out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_read_rows(ctx, enc, ids, count, out);
}

int32_t dz_encoder_forward(dz_ctx *ctx, dz_encoder *enc, const int32_t *ids, size_t batch, size_t seq,
                           float *out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_forward(ctx, enc, ids, nullptr, batch, seq, out);
}

int32_t dz_encoder_forward_rows(dz_ctx *ctx, dz_encoder *enc, const void *rows, size_t batch,
                                size_t seq, float *out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_forward(ctx, enc, nullptr, rows, batch, seq, out);
}

int32_t dz_encoder_hidden_rows(dz_ctx *ctx, dz_encoder *enc, const void *rows, size_t seq, float *hidden) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_hidden_rows(ctx, enc, rows, seq, hidden);
}

int32_t dz_encoder_readout_params(const dz_encoder *enc, const dz_weight **w, const float **norm) {
    return dz::encoder_readout_params(enc, w, norm);
}

int32_t dz_encoder_set_readout(dz_ctx *ctx, dz_encoder *enc, const void *packed, size_t bytes, int32_t layout,
                               const float *norm_host) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_set_readout(ctx, enc, packed, bytes, layout, norm_host);
}

int32_t dz_encoder_readout_rows(dz_ctx *ctx, dz_encoder *enc, const void *rows, size_t seq,
                                const int32_t *markers, size_t count, float *logits) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::encoder_readout(ctx, enc, rows, seq, markers, count, logits);
}

// ---- the Pplx decider ---------------------------------------------------------------

int32_t dz_pplx_create(dz_ctx *ctx, const dz_pplx_config *cfg, dz_pplx **out) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_create(ctx, cfg, out);
}

void dz_pplx_destroy(dz_ctx *ctx, dz_pplx *model) {
    if (ctx && model) dz::pplx_destroy(ctx, model);
}

int32_t dz_pplx_set_weight(dz_ctx *ctx, dz_pplx *model, const char *name, const void *packed, size_t bytes,
                           int32_t layout, size_t rows, size_t cols) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_set_weight(ctx, model, name, packed, bytes, layout, rows, cols, -1);
}

int32_t dz_pplx_set_weight_fitted(dz_ctx *ctx, dz_pplx *model, const char *name, const void *packed, size_t bytes,
                                  size_t rows, size_t cols, int32_t form) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    if (form < 0) return fail(ctx, DZ_INVALID_PARAMETERS, "unknown fitted form");
    return dz::pplx_set_weight(ctx, model, name, packed, bytes, DZ_Q4_G64_F32, rows, cols, form);
}

int32_t dz_pplx_set_rows_form(dz_ctx *ctx, dz_pplx *model, int32_t form) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_set_rows_form(ctx, model, form);
}

int32_t dz_pplx_set_vector(dz_ctx *ctx, dz_pplx *model, const char *name, const float *values, size_t count) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_set_vector(ctx, model, name, values, count);
}

int32_t dz_pplx_layer(dz_ctx *ctx, dz_pplx *model, int32_t layer, float *hidden, size_t n, const int32_t *markers,
                      size_t count) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_layer(ctx, model, layer, hidden, n, markers, count, DZ_PPLX_WHOLE);
}

int32_t dz_pplx_layer_part(dz_ctx *ctx, dz_pplx *model, int32_t layer, int32_t part, float *hidden, size_t n,
                           const int32_t *markers, size_t count) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_layer(ctx, model, layer, hidden, n, markers, count, part);
}

int32_t dz_pplx_activation(dz_ctx *ctx, dz_pplx *model, const char *name, void *out_dev, size_t bytes) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_activation(ctx, model, name, out_dev, bytes);
}

int32_t dz_pplx_forward_rows(dz_ctx *ctx, dz_pplx *model, const void *rows, size_t n, const int32_t *markers,
                             size_t count, float *logits) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::pplx_forward_rows(ctx, model, rows, n, markers, count, logits);
}

int32_t dz_pplx_set_residency(dz_ctx *ctx, dz_pplx *model, int32_t residency) {
    DZ_BEGIN(ctx);
    if (capturing(ctx)) return fail(ctx, DZ_INVALID_REQUEST, "residency change during stream capture");
    return dz::pplx_set_residency(ctx, model, residency);
}

int32_t dz_pplx_residency_info(dz_ctx *ctx, dz_pplx *model, char *json, size_t cap) {
    DZ_BEGIN(ctx);
    return dz::pplx_residency_info(ctx, model, json, cap);
}

// ---- tuner ---------------------------------------------------------------------------

int32_t dz_tune(dz_ctx *ctx, uint32_t budget_ms, const char *cache_in, char *cache_out, size_t cap) {
    DZ_BEGIN(ctx);
    DZ_NOT_CAPTURING(ctx);
    return dz::tune(ctx, budget_ms, cache_in, cache_out, cap);
}

int32_t dz_select_variant(dz_ctx *ctx, const char *family, const char *name) {
    DZ_BEGIN(ctx);
    if (!family || !name) return fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    int idx = dz::variant_index(family, name);
    if (idx < 0) return fail(ctx, DZ_INVALID_PARAMETERS, std::string("unknown variant ") + family + "/" + name);
    ctx->variants[family] = idx;
    return DZ_OK;
}

}  // extern "C"

// ---- helpers shared with encoder.hip and tuner.hip -----------------------------------

namespace dz {

int32_t ctx_fail(dz_ctx *ctx, int32_t code, const std::string &msg) { return fail(ctx, code, msg); }
int32_t ctx_hip_fail(dz_ctx *ctx, hipError_t e, const char *what) { return hip_fail(ctx, e, what); }
hipStream_t ctx_stream(dz_ctx *ctx) { return ctx->stream; }
int *ctx_flag(dz_ctx *ctx) { return ctx->flag; }
int ctx_variant(dz_ctx *ctx, const char *family) { return variant(ctx, family); }

// h += the W4A8 product of x (f32 rows, quantized here to A8 codes) or of the
// codes q with scales qs, in the product kernel's epilogue, when the
// pipelined grouped kernel takes m rows (*fused set); otherwise nothing is
// launched and the caller runs the product and the add.
int32_t ctx_product_add(dz_ctx *ctx, const dz_weight *w, const float *x, const int8_t *q, const float *qs,
                        size_t m, float *h, bool *fused, const int *qbad) {
    *fused = false;
    const int v = variant(ctx, "grouped");
    if (!dz::grouped_adds_residual(w->w, (int)m, v)) return DZ_OK;
    const int *bad = qbad;
    if (x) {
        const size_t qbytes = m * (size_t)w->w.groups * 64, sbytes = m * (size_t)w->w.groups * sizeof(float);
        int32_t rc = ensure_work(ctx, qbytes + sbytes + 256);
        if (rc) return rc;
        int8_t *codes = (int8_t *)ctx->work;
        float *scales = (float *)((uint8_t *)ctx->work + (qbytes + 255) / 256 * 256);
        int *flag = nullptr;
        rc = product_flag(ctx, &flag);
        if (rc) return rc;
        dz::launch_act_quantize(x, (int)m, w->w.cols, 8, codes, scales, flag, ctx->stream);
        q = codes;
        qs = scales;
        bad = flag;
    }
    if (!dz::launch_grouped(w->w, q, qs, (int)m, h, bad, v, ctx->stream, h))
        return fail(ctx, DZ_INFERENCE_FAILED, "residual product: no pipelined kernel takes the shape");
    *fused = true;
    return launched(ctx, "grouped linear");
}
// A non-finite flag for a product (or several sharing one set of codes).
int32_t ctx_product_flag(dz_ctx *ctx, int **flag) { return product_flag(ctx, flag); }
// y = the W4A8 product of the A8 codes q / scales qs of m > 16 rows (the
// grouped kernel dz_linear uses); NaN outputs when *bad is set.
int32_t ctx_codes_product(dz_ctx *ctx, const dz_weight *w, const int8_t *q, const float *qs, size_t m, float *y,
                          const int *bad) {
    dz::launch_grouped(w->w, q, qs, (int)m, y, bad, variant(ctx, "grouped"), ctx->stream);
    return launched(ctx, "grouped linear");
}
// dz_mlp_requant on already-quantized activations (the codes of a norm)
int32_t ctx_mlp_codes(dz_ctx *ctx, const dz_weight *gate, const dz_weight *up, const int8_t *q, const float *qs,
                      size_t m, int8_t *qo, float *so, const int *bad) {
    dz::launch_mlp_requant(gate->w, up->w, q, qs, (int)m, qo, so, bad, variant(ctx, "mlp"), ctx->stream);
    return launched(ctx, "fused MLP");
}
void ctx_set_variant(dz_ctx *ctx, const char *family, int index) { ctx->variants[family] = index; }
void ctx_set_tuning(dz_ctx *ctx, const std::string &json) { ctx->tuning = json; }
std::string ctx_device_key(dz_ctx *ctx) {
    return ctx->arch + "/" + std::to_string(ctx->cus) + "cu/" + std::to_string(ctx->clock_khz) + "khz";
}
const Weight &weight_of(const dz_weight *h) { return h->w; }
// The device pointers of a weight whose memory another owner manages (the
// decider's streamed banks): codes and scales are re-pointed, never freed here.
Weight &weight_mut(dz_weight *h) { return h->w; }
int32_t weight_quantize(dz_ctx *ctx, const void *values, int dtype, size_t rows, size_t cols, int bits,
                        int group, dz_weight **out) {
    return dz_weight_quantize(ctx, values, dtype, rows, cols, bits, group, out);
}
void weight_free(dz_weight *h) { free_weight(h); }
// One weight holding the parts' rows in order, each part starting on a
// 16-row tile: part i's rows begin at row sum_{j<i} ceil16(rows_j), and the
// rows between parts are the parts' own padding (code 0, scale 0), whose
// products are 0. Same kind and columns for all parts. The native layouts are
// tile-major, so the codes and scales are the parts' arrays one after the
// other. Synchronous.
int32_t weight_concat_rows(dz_ctx *ctx, const dz_weight *const *parts, int count, dz_weight **out) {
    *out = nullptr;
    if (count < 1) return fail(ctx, DZ_INVALID_REQUEST, "no weights to join");
    size_t rows = 0;
    for (int i = 0; i < count; i++) {
        const Weight &p = parts[i]->w;
        if (p.kind != parts[0]->w.kind || p.cols != parts[0]->w.cols)
            return fail(ctx, DZ_INVALID_PARAMETERS, "joined weights need one layout and one width");
        rows += i + 1 < count ? (size_t)p.np : (size_t)p.rows;
    }
    dz_weight *h = nullptr;
    int32_t rc = alloc_weight(ctx, parts[0]->w.kind, rows, (size_t)parts[0]->w.cols, &h);
    if (rc) return rc;
    size_t co = 0, so = 0;
    hipError_t e = hipSuccess;
    for (int i = 0; i < count && e == hipSuccess; i++) {
        const Weight &p = parts[i]->w;
        e = hipMemcpyAsync(h->w.codes + co, p.codes, p.code_bytes, hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess)
            e = hipMemcpyAsync(h->w.scales + so, p.scales, p.scale_bytes, hipMemcpyDeviceToDevice, ctx->stream);
        co += p.code_bytes;
        so += p.scale_bytes;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipStreamSynchronize(ctx->stream);
        free_weight(h);
        return hip_fail(ctx, e, "joined weight");
    }
    *out = h;
    return DZ_OK;
}
int32_t weight_upload(dz_ctx *ctx, const void *packed, size_t bytes, int32_t layout, size_t rows, size_t cols,
                      dz_weight **out) {
    return dz_weight_upload(ctx, packed, bytes, layout, rows, cols, out);
}
int32_t weight_upload_fitted(dz_ctx *ctx, const void *packed, size_t bytes, size_t rows, size_t cols, int32_t form,
                             dz_weight **out) {
    return dz_weight_upload_fitted(ctx, packed, bytes, rows, cols, form, nullptr, out);
}
int32_t ctx_readout_rows(dz_ctx *ctx, const Weight &w, const float *norm, const void *hidden, int dtype,
                         const int32_t *select, size_t rows, float eps, float *logits) {
    return readout_rows(ctx, w, norm, hidden, dtype, select, rows, eps, logits);
}
int32_t ctx_workspace(dz_ctx *ctx, size_t bytes, void **out) {
    int32_t rc = ensure_work(ctx, bytes);
    *out = rc ? nullptr : ctx->work;
    return rc;
}

}  // namespace dz
