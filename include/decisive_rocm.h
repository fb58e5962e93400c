/*
 * decisive_rocm.h -- C ABI of the MI355X (gfx950) quantized matrix-product
 * library, libdecisive_rocm.so.
 *
 * The reference (hyperlogue/decisive, Rust) has no FFI on this path: its
 * quantized products are Rust functions called in-process. Each entry point
 * below names the reference function whose behaviour it takes over; a Rust
 * `Rocm` backend binds these with `extern "C"` blocks of its own.
 *
 * Conventions
 *  - Every call returns a dz_status; on failure dz_last_error(ctx) holds a
 *    message that stays valid until the next call on the same context.
 *  - Pointers named *_dev are device memory on the context's GPU (from
 *    dz_alloc, hipMalloc or a framework allocator). *_host pointers are host
 *    memory borrowed for the duration of the call.
 *  - Work is enqueued on the context's stream (dz_set_stream may replace it)
 *    and is asynchronous unless stated; dz_sync waits for it.
 *  - A context is not thread-safe; the caller serialises calls, as the
 *    reference's `Backend::predict(&mut self, ..)` does.
 *  - Stream capture (HIP graphs): the asynchronous products may be recorded.
 *    Products that quantize their activations (dz_linear and dz_linear_pair
 *    in a grouped mode with m > 16, dz_mlp_requant) use the context workspace
 *    and a non-finite flag of their own, which the recorded graph clears on
 *    every replay; run such a call once before capturing it (the workspace
 *    cannot grow under capture: DZ_INVALID_REQUEST), and replay the graph on
 *    the context stream or ordered with it, one replay at a time. The slots
 *    and workspaces a capture holds are given back by dz_capture_release
 *    (below), else at dz_destroy. Entry points that wait
 *    for the stream, allocate, or read host memory return DZ_INVALID_REQUEST
 *    under capture before enqueueing anything: dz_sync, dz_alloc, dz_free,
 *    dz_copy_h2d, dz_copy_d2h, dz_set_stream, dz_weight_upload,
 *    dz_weight_upload_fitted, dz_weight_quantize, dz_weight_free,
 *    dz_dequant_rows, dz_project,
 *    dz_q4_quantize_rows, dz_encoder_create_random, dz_encoder_read_rows,
 *    dz_encoder_forward (it reads back the token-range flag),
 *    dz_encoder_forward_rows, dz_encoder_hidden_rows, dz_encoder_set_readout,
 *    dz_encoder_readout_rows, dz_pplx_create, dz_pplx_set_weight,
 *    dz_pplx_set_weight_fitted, dz_pplx_set_rows_form,
 *    dz_pplx_set_vector, dz_pplx_layer and dz_pplx_layer_part (they may grow
 *    the model's activation buffers), dz_pplx_activation,
 *    dz_pplx_forward_rows, dz_pplx_set_residency and dz_tune.
 */
#ifndef DECISIVE_ROCM_H
#define DECISIVE_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dz_ctx dz_ctx;
typedef struct dz_weight dz_weight;
typedef struct dz_encoder dz_encoder;

/* Status codes map 1:1 onto the reference's error codes
 * (src/inference/mod.rs:44-85, parameters.rs:368-376, browser/pplx.rs:105). */
typedef enum dz_status {
    DZ_OK = 0,
    DZ_INVALID_REQUEST = 1,     /* "INVALID_REQUEST"     mod.rs:32-35   */
    DZ_INVALID_PARAMETERS = 2,  /* "INVALID_PARAMETERS"  parameters.rs:370-373 */
    DZ_CANCELLED = 3,           /* "CANCELLED"           mod.rs:95      */
    DZ_CACHE_OWNER = 4,         /* "CACHE_OWNER"         mod.rs:199-202 */
    DZ_INPUT_TOO_LONG = 5,      /* "INPUT_TOO_LONG"      mod.rs:58-62   */
    DZ_GPU_UNAVAILABLE = 6,     /* "GPU_UNAVAILABLE"     mod.rs:65-66   */
    DZ_RESOURCE_LIMIT = 7,      /* "RESOURCE_LIMIT"      mod.rs:67-68   */
    DZ_MISSING_GPU_FEATURE = 8, /* "MISSING_GPU_FEATURE" mod.rs:63-64   */
    DZ_INFERENCE_FAILED = 9,    /* "INFERENCE_FAILED"    mod.rs:73-74   */
    DZ_INVALID_CHECKPOINT = 10, /* "INVALID_CHECKPOINT"  browser/pplx.rs:105,126 */
    DZ_UNSUPPORTED_CACHE = 11   /* "UNSUPPORTED_CACHE"   mod.rs:181-186 */
} dz_status;

/* Packed weight layouts accepted by dz_weight_upload. */
typedef enum dz_layout {
    /* packed.rs:3-56: per row, per 64-run along K: 32 bytes of code+8 nibbles
     * (low nibble = even k) then the f32 LE scale; 36 B per group. */
    DZ_Q4_G64_F32 = 0,
    /* packed.rs:3-56 with bits=8: 64 two's-complement code bytes + f32 scale. */
    DZ_Q8_G64_F32 = 1,
    /* Group-32 variant with f16 scales: 16 code bytes + f16 LE scale (18 B). */
    DZ_Q4_G32_F16 = 2
} dz_layout;

typedef enum dz_dtype { DZ_F32 = 0, DZ_F16 = 1, DZ_BF16 = 2 } dz_dtype;

/* Numeric mode of dz_linear. */
typedef enum dz_mode {
    /* Activations re-quantized per (row, 64-group) to int8 (int8.rs:178-202)
     * and multiplied with exact int32 group dots folded in the AVX2 order
     * acc = fma(f32(dot), sw*sx, acc) (int8.rs:524-585). Bit-exact with the
     * reference CPU path. x is f32. W8A8 when the weight is Q8. */
    DZ_W4A8 = 0,
    /* As DZ_W4A8 with 4-bit activation codes (int8.rs:59-69 Precision bits);
     * W8A4 when the weight is Q8 (int8.rs:61-64 takes any of the four pairs). */
    DZ_W4A4 = 1,
    /* f16 activations times dequantized Q4 weights, f32 accumulation. */
    DZ_W4A16 = 2
} dz_mode;

/* ---- context -------------------------------------------------------------- */

/* Name of a status ("OK", "INVALID_REQUEST", ...). Never NULL. */
const char *dz_status_name(int32_t status);
/* Opens a context on HIP device `device` with its own stream. Fails with
 * DZ_GPU_UNAVAILABLE when there is no device, DZ_MISSING_GPU_FEATURE when the
 * device is not gfx950. */
int32_t dz_init(int32_t device, dz_ctx **out);
void dz_destroy(dz_ctx *ctx);
const char *dz_last_error(const dz_ctx *ctx);
/* Replaces the context stream (a hipStream_t); NULL restores its own. Waits
 * for the work queued on the old stream first (the workspace and the product
 * flags are shared by the context's calls); DZ_INVALID_REQUEST while the
 * current stream is capturing. */
int32_t dz_set_stream(dz_ctx *ctx, void *hip_stream);
int32_t dz_sync(dz_ctx *ctx);
/* JSON description of the device, the selected kernel variants and the
 * capture state: "capture_slots" {"held", "limit", "captures",
 * "retired_workspaces"}. */
int32_t dz_info(dz_ctx *ctx, char *buf, size_t cap);

/* Capture bookkeeping (no reference counterpart: the reference records no
 * graphs). Each product recorded under stream capture that quantizes its
 * activations holds one of 4032 flag slots of the context, and a graph that
 * recorded the context workspace keeps it alive when it grows. These calls give
 * both back once the caller has destroyed every graph instantiated from a
 * capture (or will not replay it again) and its replays have finished:
 *  - dz_capture_id: while the context stream records, the id of that capture
 *    (hipStreamGetCaptureInfo's); DZ_INVALID_REQUEST when it is not recording;
 *  - dz_capture_release: gives back the slots and workspaces held by the
 *    capture `id`; DZ_INVALID_REQUEST while that capture is still recording;
 *    an id that holds nothing is accepted;
 *  - dz_capture_release_all: gives back everything every capture holds;
 *    DZ_INVALID_REQUEST while the context stream records.
 * Without them, a context in which more than 4032 such products have been
 * recorded fails further recordings with DZ_RESOURCE_LIMIT. Retired workspaces
 * are freed after a wait for the context stream. */
int32_t dz_capture_id(dz_ctx *ctx, uint64_t *id);
int32_t dz_capture_release(dz_ctx *ctx, uint64_t id);
int32_t dz_capture_release_all(dz_ctx *ctx);

/* Device memory for callers without an allocator of their own. */
int32_t dz_alloc(dz_ctx *ctx, size_t bytes, void **dev);
int32_t dz_free(dz_ctx *ctx, void *dev);
int32_t dz_copy_h2d(dz_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
int32_t dz_copy_d2h(dz_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);

/* ---- weights ---------------------------------------------------------------- */

/* Takes over packed.rs:59-73 (unpack validation) at load: copies `bytes` of a
 * packed [rows x cols] matrix in `layout` to the device and re-tiles it into
 * the library's HBM layout. Rejects a scale that is not finite and positive
 * (DZ_INVALID_CHECKPOINT), a byte count that does not match packed.rs:10-19
 * size() (DZ_INVALID_CHECKPOINT) and an unknown layout (DZ_INVALID_PARAMETERS).
 * Synchronous. */
int32_t dz_weight_upload(dz_ctx *ctx, const void *packed_host, size_t bytes, int32_t layout,
                         size_t rows, size_t cols, dz_weight **out);
/* Fitted Q4 forms (quantization.rs), each a [rows x cols] matrix in the
 * DZ_Q4_G64_F32 wire layout whose codes may take the whole nibble range
 * (-8..7) and whose f32 scales may be any finite nonzero value:
 *  - DZ_FIT_SCALED: y = code * scale; quantization.rs:25-71 mse (its scales
 *    may be negative), int8.rs:51-152 from_bf16_optimized with `optimized`;
 *  - DZ_FIT_AFFINE: y = code * scale + offset, one f32 offset per row and
 *    64-group; quantization.rs:147-200 affine, from_bf16_optimized with
 *    `affine`;
 *  - DZ_FIT_NF4: y = NF4[code + 8] * scale, the codebook of
 *    quantization.rs:3-20; quantization.rs:260-302 nf4, the embedding rows of
 *    quantized_rows.rs:21-87 (int8.rs Matrix has no codebook form). */
#define DZ_FIT_SCALED 0
#define DZ_FIT_AFFINE 1
#define DZ_FIT_NF4 2
/* Takes over the fitted forms above at load: `offsets_host` is f32
 * [rows x cols/64] for DZ_FIT_AFFINE and NULL otherwise (DZ_INVALID_REQUEST).
 * The fitting stays with the caller (the reference fits on the CPU at load).
 * Where each form runs:
 *  - dz_dequant / dz_dequant_rows decode every form as quantized_rows.rs:89-110
 *    append does: y = f32(value_code) * scale, then + offset (two roundings);
 *  - the grouped products (dz_linear, dz_linear_pair, dz_linear_noalloc in
 *    W4A8/W4A4 mode) take DZ_FIT_SCALED and DZ_FIT_AFFINE, folding each group
 *    as int8.rs:524-571 does:
 *      acc = fma(f32(dot), sw * sx, acc);
 *      acc = fma(offset, sx * f32(sum of the row's 64 activation codes), acc)
 *  - the other products on codes and scales (dz_linear in W4A16 mode,
 *    dz_linear_f16, dz_mlp_requant, dz_linear_q8, dz_project, dz_readout)
 *    take DZ_FIT_SCALED: signed scales and -8 codes need no other arithmetic;
 *  - dz_linear_records takes no fitted weight.
 * A product refuses a form it does not take with DZ_INVALID_PARAMETERS.
 * cols % 64 == 0 (the wire layout's); a zero or non-finite scale or a
 * non-finite offset is DZ_INVALID_CHECKPOINT; an unknown form
 * DZ_INVALID_PARAMETERS. Synchronous. */
int32_t dz_weight_upload_fitted(dz_ctx *ctx, const void *packed_host, size_t bytes, size_t rows, size_t cols,
                                int32_t form, const float *offsets_host, dz_weight **out);
/* Takes over int8.rs:51-152 Matrix::from_bf16_optimized (plain mode; bits 4
 * or 8, group 64, f32 scales; any cols, zero padded) and, with group == 32
 * and bits == 4, the group-32/f16 quantizer. `values_dev` is [rows x cols] of
 * `dtype`. Non-finite weights give DZ_INVALID_CHECKPOINT. Synchronous. */
int32_t dz_weight_quantize(dz_ctx *ctx, const void *values_dev, int32_t dtype, size_t rows,
                           size_t cols, int32_t bits, int32_t group, dz_weight **out);
int32_t dz_weight_free(dz_ctx *ctx, dz_weight *w);
/* rows, cols, bits, group and device bytes of a weight; any pointer may be NULL. */
int32_t dz_weight_info(const dz_weight *w, size_t *rows, size_t *cols, int32_t *bits,
                       int32_t *group, size_t *device_bytes);

/* packed.rs:59-73 unpack / quantized_rows.rs:89-110 append: y = f32(code)*scale,
 * [rows x cols] f32, bit-exact. */
int32_t dz_dequant(dz_ctx *ctx, const dz_weight *w, float *y_dev);
/* Dequantizes the rows listed in ids_dev (int32, count entries) into
 * y_dev [count x cols] of `dtype` (f32 exact; f16 rounds to nearest even):
 * the embedding-row gather of browser_gpu.rs:177-209 done on device. */
int32_t dz_dequant_rows(dz_ctx *ctx, const dz_weight *w, const int32_t *ids_dev, size_t count,
                        void *y_dev, int32_t dtype);

/* ---- quantized products ------------------------------------------------------ */

/* int8.rs:178-202 Matrix::prepare: per (row, 64-group) activation codes.
 * x_dev f32 [m x k]; q_dev int8 [m x G*64] (G = ceil(k/64), tail zero);
 * s_dev f32 [m x G]. bits is 8 or 4. */
int32_t dz_act_quantize(dz_ctx *ctx, const float *x_dev, size_t m, size_t k, int32_t bits,
                        int8_t *q_dev, float *s_dev);
/* int8.rs:166-176 Matrix::apply (DZ_W4A8/DZ_W4A4; x f32, a non-finite value
 * anywhere in x makes every output NaN, int8.rs:170-173) or the W4A16 product
 * (x f16). y_dev f32 [m x rows(w)]. m may be 0. */
int32_t dz_linear(dz_ctx *ctx, const dz_weight *w, const void *x_dev, int32_t x_dtype, size_t m,
                  float *y_dev, int32_t mode);
/* No counterpart in the reference: dz_linear for callers that cannot
 * allocate device memory (code recorded under graph capture, serving loops,
 * harnesses that forbid hipMalloc). Same arguments, results and bits as
 * dz_linear; it calls no allocator. The grouped modes from m = 5 (m > 16 for
 * affine fitted weights) keep the A8
 * codes, scales and non-finite flag in a static 16 MiB device array (one per
 * GPU, held until the process ends), so 256 + round256(m*G*64) + m*G*4 bytes
 * (G = ceil(cols/64)) must fit 16 MiB: up to 3,855 rows at cols 4096, 6,168 at
 * 2560; affine fitted weights add round256(m*G*4) + m*G*4 bytes for the code
 * sums (3,640 rows at cols 4096); more is DZ_RESOURCE_LIMIT with nothing
 * launched. Every call on a GPU
 * shares that array: calls that overlap on one GPU (other streams, other
 * contexts, concurrent graph replays) race; serialise them. */
int32_t dz_linear_noalloc(dz_ctx *ctx, const dz_weight *w, const void *x_dev, int32_t x_dtype, size_t m,
                          float *y_dev, int32_t mode);
/* int8.rs:204-227 Matrix::apply_pair: one activation quantization shared by
 * two weights with the same cols. */
int32_t dz_linear_pair(dz_ctx *ctx, const dz_weight *a, const dz_weight *b, const float *x_dev,
                       size_t m, float *ya_dev, float *yb_dev, int32_t mode);
/* The prefill form of DZ_W4A16 (the encoder's
 * projections): f16 activations x_dev [m x cols(w)] (16-byte aligned) ->
 * f16 y_dev [m x rows(w)]: the products accumulate in f32 as dz_linear's
 * DZ_W4A16 does, and each output is rounded to f16 once, after the epilogue:
 *   DZ_EPI_NONE      y = x W^T
 *   DZ_EPI_GELU      y = gelu(x W^T), erf form (decima/cpu.rs:542-556)
 *   DZ_EPI_RESIDUAL  y = x W^T + residual, residual_dev f16 [m x rows(w)]
 * Bits equal f16(dz_linear(..., DZ_W4A16)) after the same epilogue in f32.
 * Q4 weight (either group), cols % 8 == 0. */
#define DZ_EPI_NONE 0
#define DZ_EPI_GELU 1
#define DZ_EPI_RESIDUAL 2
int32_t dz_linear_f16(dz_ctx *ctx, const dz_weight *w, const void *x_dev, size_t m, void *y_dev,
                      int32_t epilogue, const void *residual_dev);
/* grouped_q4_mlp.wgsl:1-105 (q4_mlp): gate/up W4A8 products of one input,
 * v = silu(gate)*up, re-quantized per (row, 64-column block) to the A8 form of
 * dz_act_quantize: q_dev int8 [m x n], s_dev f32 [m x n/64]. n % 64 == 0. */
int32_t dz_mlp_requant(dz_ctx *ctx, const dz_weight *gate, const dz_weight *up,
                       const float *x_dev, size_t m, int8_t *q_dev, float *s_dev);
/* Product of already-quantized activations (the A8 form above) with a weight:
 * the down_proj consumer of dz_mlp_requant. */
int32_t dz_linear_q8(dz_ctx *ctx, const dz_weight *w, const int8_t *q_dev, const float *s_dev,
                     size_t m, float *y_dev);

/* packed.rs:75-119 project: the portable W{4,8}A8 product of the readout,
 * folding groups as sum += f32(dot) * (sx*sw) (separate multiply and add,
 * unlike dz_linear's fused fold). x_dev f32 [m x cols], y_dev f32
 * [m x rows(w)]; the weight is group-64 with cols % 64 == 0. Synchronous: a
 * non-finite activation gives DZ_INFERENCE_FAILED ("nonfinite readout
 * activation"), as the reference's ensure! does. */
int32_t dz_project(dz_ctx *ctx, const dz_weight *w, const float *x_dev, size_t m, float *y_dev);
/* webgpu/grouped_q4.rs:3-25 quantize: the activation codes and scales of
 * dz_act_quantize written as 17-word records per (row, 64-group): words 0..15
 * the int8 codes (element 4l+e in byte e of word l), word 16 the f32 scale.
 * records_dev uint32 [m x k/64 x 17]; k % 64 == 0. */
int32_t dz_act_quantize_records(dz_ctx *ctx, const float *x_dev, size_t m, size_t k,
                                uint32_t *records_dev);
/* grouped_q4_tuned.wgsl:1-84 (int8_gemm on records): the W4A8/W8A8 product of
 * dz_linear consuming 17-word records, y_dev f32 [m x rows(w)]. */
int32_t dz_linear_records(dz_ctx *ctx, const dz_weight *w, const uint32_t *records_dev, size_t m,
                          float *y_dev);
/* webgpu/int8.rs:107-145 quantize: per row scale = absmax/127 (no floor),
 * q = clamp(rne(x/scale), +-127), 0 when scale == 0; sums = sum of q.
 * q_dev int8 [rows x k] (signed), scales_dev f32 [rows], sums_dev int32 [rows]
 * (may be NULL). */
int32_t dz_i8_quantize_rows(dz_ctx *ctx, const float *x_dev, size_t rows, size_t k,
                            int8_t *q_dev, float *scales_dev, int32_t *sums_dev);
/* webgpu/int8.rs:147-242 gemm(fused=false, raw): y [m x n] = exact int32
 * sum_k a[i,k]*w[j,k] (raw != 0, y int32) or (f32(dot)*sa[i])*sw[j] (y f32). */
int32_t dz_i8_gemm(dz_ctx *ctx, const int8_t *a_dev, const float *sa_dev, size_t m,
                   const int8_t *w_dev, const float *sw_dev, size_t n, size_t k, void *y_dev,
                   int32_t raw);
/* webgpu/int8.rs:147-242 gemm(fused=true), epilogue :226-230: two per-row
 * products of the same codes a, gate = (f32(a.wg)*sa)*sg and
 * up = (f32(a.wu)*sa)*su, and y f32 [m x n] = (gate / (1 + exp(-gate))) * up.
 * exp is the f32 rounding of the f64 exponential (the reference leaves its
 * accuracy to the WGSL implementation). wg_dev, wu_dev int8 [n x k]. */
int32_t dz_i8_gemm_fused(dz_ctx *ctx, const int8_t *a_dev, const float *sa_dev, size_t m,
                         const int8_t *wg_dev, const float *sg_dev, const int8_t *wu_dev,
                         const float *su_dev, size_t n, size_t k, float *y_dev);

/* webgpu/q4.rs:48-73 quantize_q4 (the per-output-channel Q4 mode): per row
 * scale = absmax/7 (f32 division, no floor), code = clamp(rne(x/scale), +-7)
 * (0 when scale == 0). out_dev is the reference's word buffer, uint32
 * [rows*(k/8) + 2*rows]: rows*(k/8) code words (element 8j+t of a row as
 * code+8 at bits 4t of its word j), then the rows f32 scales, then the rows
 * i32 code sums. values_dev is f16 (as the reference) or f32. k % 8 == 0,
 * k <= 32768. Synchronous; a non-finite weight gives DZ_INVALID_CHECKPOINT. */
int32_t dz_q4_quantize_rows(dz_ctx *ctx, const void *values_dev, int32_t dtype, size_t rows, size_t k,
                            uint32_t *out_dev);
/* webgpu/q4.rs:99-105 gemm (int8::gemm with Q4 weights expanded): a_dev int8
 * [m x k] per-row codes (dz_i8_quantize_rows), w_dev the buffer above for n
 * rows; y_dev [m x n] = exact int32 dots (raw != 0) or (f32(dot)*sa)*sw. */
int32_t dz_q4_rows_gemm(dz_ctx *ctx, const int8_t *a_dev, const float *sa_dev, size_t m,
                        const uint32_t *w_dev, size_t n, size_t k, void *y_dev, int32_t raw);

/* ---- layer epilogues --------------------------------------------------------- */

/* decima/cpu.rs:529-540 LayerNorm over rows of d: (x-mean)*rsqrt(var+eps)*w+b.
 * x/y are f32 or f16 (dtype), w/b f32. y may alias x. */
int32_t dz_layernorm(dz_ctx *ctx, const void *x_dev, void *y_dev, int32_t dtype, size_t rows,
                     size_t d, const float *w_dev, const float *b_dev, float eps);
/* pplx_flash/cpu.rs:310-333 rms_from (zero_centered != 0 uses 1 + w). f32. */
int32_t dz_rmsnorm(dz_ctx *ctx, const float *x_dev, float *y_dev, size_t rows, size_t d,
                   const float *w_dev, float eps, int32_t zero_centered);
/* decima/cpu.rs:542-556 gelu (erf form), in place, f32 or f16. */
int32_t dz_gelu(dz_ctx *ctx, void *x_dev, int32_t dtype, size_t n);
/* pplx_flash/cpu.rs:348-371 silu_mul: gate = silu(gate)*up, f32. */
int32_t dz_silu_mul(dz_ctx *ctx, float *gate_dev, const float *up_dev, size_t n);
/* pplx_flash/cpu.rs:334-347 add: x += y, f32 or f16. */
int32_t dz_add(dz_ctx *ctx, void *x_dev, const void *y_dev, int32_t dtype, size_t n);
/* pplx_flash/cpu.rs:519-529 softmax over each row of n, f32. */
int32_t dz_softmax_rows(dz_ctx *ctx, float *x_dev, size_t rows, size_t n);
/* decima/cpu.rs:574-586 mean over rows: x [batch x rows x d] (f32/f16) ->
 * out f32 [batch x d]. */
int32_t dz_mean_rows(dz_ctx *ctx, const void *x_dev, int32_t dtype, size_t batch, size_t rows,
                     size_t d, float *out_dev);
/* Non-causal softmax attention (pplx_flash/backbone.rs:484-615 without the
 * gate/RoPE): qkv f16 [batch*seq x 3*heads*dh] (q | k | v), out f16
 * [batch*seq x heads*dh]; scores scaled by `scale`, f32 softmax. dh == 64. */
int32_t dz_attention(dz_ctx *ctx, const void *qkv_dev, void *out_dev, size_t batch, size_t seq,
                     size_t heads, size_t dh, float scale);

/* ---- encoder forward -------------------------------- */

typedef struct dz_encoder_config {
    int32_t layers;     /* 24   */
    int32_t hidden;     /* 1024 */
    int32_t heads;      /* 16   */
    int32_t head_dim;   /* 64   */
    int32_t ffn;        /* 4096 */
    int32_t vocab;      /* 32000 */
    float ln_eps;       /* LayerNorm epsilon */
} dz_encoder_config;

/* Builds an encoder with random-init weights from `seed` (all linear weights
 * N(0, 0.02) quantized to Q4 g32/f16 on device, embedding rows Q4 g64/f32,
 * LayerNorm weight 1 / bias 0). Synchronous. */
int32_t dz_encoder_create_random(dz_ctx *ctx, const dz_encoder_config *cfg, uint64_t seed,
                                 dz_encoder **out);
void dz_encoder_destroy(dz_ctx *ctx, dz_encoder *enc);
/* The packed embedding rows (Q4 g64/f32 wire layout) of ids_host, copied to
 * out_host (count * row_bytes); the EmbeddingCache source. Synchronous. */
int32_t dz_encoder_embedding_row_bytes(const dz_encoder *enc, size_t *row_bytes);
int32_t dz_encoder_read_rows(dz_ctx *ctx, const dz_encoder *enc, const int32_t *ids_host,
                             size_t count, void *out_host);
/* The encoder's weights for inspection: which = 0 qkv [3h x h], 1 output
 * [h x h], 2 ffn up [f x h], 3 ffn down [h x f] of `layer`; 4 the embedding
 * table [vocab x h]; 5 the readout [255 x h]. Owned by the encoder; NULL when
 * out of range. */
const dz_weight *dz_encoder_weight(const dz_encoder *enc, int32_t layer, int32_t which);
/* Forward over batch x seq token ids (ids_dev int32) -> mean-pooled
 * embeddings out_dev f32 [batch x hidden]. */
int32_t dz_encoder_forward(dz_ctx *ctx, dz_encoder *enc, const int32_t *ids_dev, size_t batch,
                           size_t seq, float *out_dev);
/* Same forward from packed embedding rows already gathered on the host
 * (rows_host: batch*seq rows in the Q4 g64/f32 wire layout), as the
 * EmbeddingCache hands them over (browser/pplx.rs:76-137). */
int32_t dz_encoder_forward_rows(dz_ctx *ctx, dz_encoder *enc, const void *rows_host,
                                size_t batch, size_t seq, float *out_dev);

/* The per-token output of the encoder: the last layer's hidden states of one
 * sequence of packed rows (as dz_encoder_forward_rows takes them), f32
 * [seq x hidden] in hidden_dev (exact f16 -> f32). */
int32_t dz_encoder_hidden_rows(dz_ctx *ctx, dz_encoder *enc, const void *rows_host, size_t seq,
                               float *hidden_dev);

/* ---- decision readout (pplx_flash/mod.rs:149-185 logits) ------------------------ */

#define DZ_READOUT_CODES 255       /* answer codes per readout row (input.rs:137-140) */
#define DZ_READOUT_MAX_MARKERS 256 /* readout rows per dz_encoder_readout_rows call */
#define DZ_READOUT_EPS 1e-6f       /* RMSNorm epsilon of the readout (mod.rs:155) */

/* pplx_flash/mod.rs:149-185 logits with a packed readout: for each of `rows`
 * hidden rows (hidden_dev f32 [rows x cols(w)]) the zero-centred RMSNorm of
 * pplx_flash/cpu.rs:310-333, y = (x * s) * (1 + norm), s = 1/sqrt(sum x^2 /
 * cols + eps), with the squares summed in row order as the reference's sum
 * is (bit-exact), then dz_project (packed.rs:75-119) into logits_dev f32
 * [rows x rows(w)]. w is group-64 (Q4 or Q8 wire layout), cols(w) <= 16384.
 * Synchronous. A non-finite normalised activation gives DZ_INFERENCE_FAILED
 * "nonfinite readout activation", a non-finite logit "non-finite packed
 * logits", as the reference's ensure!s. */
int32_t dz_readout(dz_ctx *ctx, const dz_weight *w, const float *norm_dev, const float *hidden_dev,
                   size_t rows, float eps, float *logits_dev);
/* The encoder's readout: weight [DZ_READOUT_CODES x hidden] (Q4 g64) and its
 * zero-centred norm weights (device f32 [hidden]); owned by the encoder. */
int32_t dz_encoder_readout_params(const dz_encoder *enc, const dz_weight **w, const float **norm_dev);
/* Replaces the encoder's readout with a loaded one (browser/pplx.rs:212-218
 * and mod.rs:126-135: the packed readout file, Q4 or Q8 by its size, and the
 * final norm of a packed checkpoint): packed_host holds DZ_READOUT_CODES x hidden in a group-64
 * wire layout (DZ_Q4_G64_F32 or DZ_Q8_G64_F32, validated as
 * dz_weight_upload does), norm_host f32 [hidden] the zero-centred norm
 * weights. The encoder owns the uploaded copy. Synchronous. */
int32_t dz_encoder_set_readout(dz_ctx *ctx, dz_encoder *enc, const void *packed_host, size_t bytes,
                               int32_t layout, const float *norm_host);
/* pplx_flash/native.rs:193-274 for one chunk: the encoder over one sequence
 * of packed rows, then dz_readout of the hidden rows at markers_host (count
 * positions < seq, count <= DZ_READOUT_MAX_MARKERS) with the encoder's
 * readout. logits_host f32 [count x DZ_READOUT_CODES]. Synchronous. */
int32_t dz_encoder_readout_rows(dz_ctx *ctx, dz_encoder *enc, const void *rows_host, size_t seq,
                                const int32_t *markers_host, size_t count, float *logits_host);

/* ---- the Pplx decider (src/models/pplx_flash: backbone.rs, mod.rs, native.rs) ---- */

typedef struct dz_pplx dz_pplx;
typedef struct dz_pplx_config {
    int32_t layers;          /* 32 (backbone.rs: layer i is full attention when i % 4 == 3) */
    int32_t hidden;          /* 2560 (D) */
    int32_t ff;              /* 9216 (FF) */
    int32_t delta_heads;     /* 32 (LH) */
    int32_t delta_key_heads; /* 16 (LK), at most 16 */
    int32_t delta_head_dim;  /* 128 (LD), fixed */
    int32_t attn_heads;      /* 16 (AH) */
    int32_t attn_kv_heads;   /* 4 (KV / AD) */
    int32_t attn_head_dim;   /* 256 (AD), fixed */
} dz_pplx_config;

/* An empty model of the given shape; weights arrive by name. */
int32_t dz_pplx_create(dz_ctx *ctx, const dz_pplx_config *cfg, dz_pplx **out);
void dz_pplx_destroy(dz_ctx *ctx, dz_pplx *model);
/* A packed projection by its checkpoint name (export_packed.rs:44-64 stores
 * every 2-D tensor this way): "language_model.layers.<i>.<linear_attn|
 * self_attn|mlp>.<proj>.weight" or "readout" (DZ_READOUT_CODES x hidden);
 * rows x cols as the checkpoint lists them. Synchronous upload, validated as
 * dz_weight_upload. An unknown name or shape is DZ_INVALID_CHECKPOINT. */
int32_t dz_pplx_set_weight(dz_ctx *ctx, dz_pplx *model, const char *name, const void *packed_host,
                           size_t bytes, int32_t layout, size_t rows, size_t cols);
/* dz_pplx_set_weight for a fitted Q4 projection of the reference's
 * `optimized` precisions (native.rs:125-128: q4-w4a8-e8-r4-g64-mse,
 * q4-w4a8-e4-r4-g64-mse, q4-w4a8-e4-r4-g64-mse-nf4; quantization.rs:25-71
 * mse): the DZ_Q4_G64_F32 wire layout with the full code range and signed
 * scales, form DZ_FIT_SCALED, validated as dz_weight_upload_fitted. The
 * decider folds it as any weight (int8.rs:524-585). DZ_FIT_AFFINE and
 * DZ_FIT_NF4 are DZ_INVALID_PARAMETERS: its products have no offset term
 * (q4-w4a8-e4-r4-g64-affine is not served) and its projections no codebook. */
int32_t dz_pplx_set_weight_fitted(dz_ctx *ctx, dz_pplx *model, const char *name, const void *packed_host,
                                  size_t bytes, size_t rows, size_t cols, int32_t form);
/* How dz_pplx_forward_rows decodes its packed embedding rows
 * (quantized_rows.rs:89-110): DZ_ROWS_PACKED, the default (packed.rs:59-73:
 * f32(code) * scale, scales positive), DZ_FIT_SCALED (MSE-fitted rows: signed
 * scales, codes -8..7) or DZ_FIT_NF4 (NF4[code + 8] * scale, the
 * q4-w4a8-e4-r4-g64-mse-nf4 rows). DZ_FIT_AFFINE is DZ_INVALID_PARAMETERS:
 * affine rows carry offsets the row bytes do not hold. */
#define DZ_ROWS_PACKED (-1)
int32_t dz_pplx_set_rows_form(dz_ctx *ctx, dz_pplx *model, int32_t form);
/* A vector by its checkpoint name, as f32 values in the checkpoint's order:
 * the layer norms, linear_attn.conv1d.weight ([width, 1, 4]), A_log, dt_bias,
 * linear_attn.norm.weight, self_attn.q_norm / k_norm, language_model.norm.weight. */
int32_t dz_pplx_set_vector(dz_ctx *ctx, dz_pplx *model, const char *name, const float *values_host,
                           size_t count);
/* One decoder layer (backbone.rs:207-250) in place on hidden_dev f32
 * [n x hidden]. With markers_host (an attention layer only) the layer keeps
 * the marker rows, in marker order (prune_last). */
int32_t dz_pplx_layer(dz_ctx *ctx, dz_pplx *model, int32_t layer, float *hidden_dev, size_t n,
                      const int32_t *markers_host, size_t count);
/* Which part of a decoder layer dz_pplx_layer_part runs. */
enum { DZ_PPLX_WHOLE = 0, DZ_PPLX_MIXER = 1, DZ_PPLX_MLP = 2 };
/* dz_pplx_layer restricted to one half of the layer (backbone.rs:207-250,
 * the two residual blocks): DZ_PPLX_MIXER runs the input norm, the mixer
 * (gated delta rule or gated attention; markers as dz_pplx_layer takes them)
 * and the output projection with its residual; DZ_PPLX_MLP the post norm and
 * the MLP with its residual (markers_host must be NULL). Running the two
 * halves in turn gives dz_pplx_layer's bits. */
int32_t dz_pplx_layer_part(dz_ctx *ctx, dz_pplx *model, int32_t layer, int32_t part, float *hidden_dev,
                           size_t n, const int32_t *markers_host, size_t count);
/* Diagnostics for op-by-op parity checks (no reference counterpart: the
 * reference's layer ops are Rust functions a test can call one by one).
 * Copies an activation that the last dz_pplx_layer / dz_pplx_layer_part call
 * left in the model's buffers into out_dev; `bytes` must be its size. n is
 * that call's rows, nq its query rows (the markers' count when it pruned,
 * else n), rows its output rows, d = hidden, W the gate's width (delta:
 * delta_heads x 128, attention: attn_heads x 256).
 *   any layer:  "hidden" f32 [rows x d]; "norm_codes" int8 [n x d] and
 *               "norm_scales" f32 [n x d/64] (the last norm's A8 codes, when
 *               it wrote codes: above 16 rows) or "normed" f32 [n x d];
 *               "gate_codes" int8 [nq x W] and "gate_scales" f32 [nq x W/64]
 *               (the mixer gate's A8 codes, when it wrote codes; a later MLP
 *               half replaces them) or "gate" f32 [nq x W]; "mlp_codes" int8
 *               [rows x ff] and "mlp_scales" f32 [rows x ff/64] (the fused
 *               MLP's codes for down_proj)
 *   delta:      "qkv" f32 [n x conv width], "z" f32 [n x delta_heads*128],
 *               "a" and "b" f32 [n x delta_heads], "conv" f32 [n x conv
 *               width] (after the causal conv and SiLU), "heads" f32
 *               [delta_heads x n x 128] (the scan's output)
 *   attention:  "q" f32 [nq x attn_heads*512] (q_proj: each head's query then
 *               its gate), "query" f32 [nq x attn_heads*256] (after the head
 *               norm and rotary), "key" f32 [n x attn_kv_heads*256] (after
 *               the head norm and rotary), "value" f32 [n x attn_kv_heads*256],
 *               "heads" f32 [attn_heads x nq x 256] (attention's output)
 * DZ_INVALID_PARAMETERS for a name this layer kind does not have or a wrong
 * size, DZ_INVALID_REQUEST when the last call did not produce it.
 * Synchronous. */
int32_t dz_pplx_activation(dz_ctx *ctx, dz_pplx *model, const char *name, void *out_dev, size_t bytes);
/* native.rs:193-274 for one chunk: packed embedding rows (rows_host, n rows
 * of the group-64 wire layout), every layer (the last one cut to the
 * markers when it is an attention layer), the final zero-centred RMSNorm
 * and the packed readout of the marker rows: logits_host f32
 * [count x DZ_READOUT_CODES]. n <= 8192. Synchronous; a non-finite hidden
 * state is DZ_INFERENCE_FAILED "non-finite hidden state" (backbone.rs:247). */
int32_t dz_pplx_forward_rows(dz_ctx *ctx, dz_pplx *model, const void *rows_host, size_t n,
                             const int32_t *markers_host, size_t count, float *logits_host);

/* Where the decider's layer projections live (webgpu/streaming.rs:16-369, the
 * reference's two-bank weight buffers; browser_gpu.rs:336-378 keeps at most
 * two layers queued).
 *  - DZ_PPLX_RESIDENT (the default): every projection in device memory.
 *  - DZ_PPLX_STREAMED: every layer projection in pinned host memory, already
 *    in the device layout, and two device banks of the largest layer's size.
 *    Layer i runs from bank i % 2 (streaming.rs:220 banks[layer % 2]). While
 *    layer i computes, a copy stream fills the other bank with layer i + 1,
 *    once the layer that used that bank last has finished; layer i + 1 waits
 *    for its copy. Device memory for layer weights drops from the whole model
 *    to two layers; a forward then moves every layer's bytes over the host
 *    link once. Outputs are bitwise equal to the resident ones.
 * Switching needs a complete model (every layer projection set) and waits
 * for the context stream. Under DZ_PPLX_STREAMED, dz_pplx_set_weight replaces
 * a layer projection's host copy (same layout and shape, else
 * DZ_INVALID_REQUEST). Not recordable under stream capture. */
#define DZ_PPLX_RESIDENT 0
#define DZ_PPLX_STREAMED 1
int32_t dz_pplx_set_residency(dz_ctx *ctx, dz_pplx *model, int32_t residency);
/* streaming.rs:176-191 diagnostics as JSON: "residency", "layer_weight_bytes"
 * (every layer projection), "device_layer_weight_bytes" (what the device
 * holds for them now: resident, the projections plus the joined z|a|b copy
 * of each delta layer; streamed, the two banks), "host_layer_weight_bytes", "banks", "bank_bytes",
 * "bank_layers" (the layer each bank holds, or null), "layer_uploads",
 * "bank_reuses" (uploads into a bank that held another layer), "upload_bytes"
 * and "max_in_flight_layers". DZ_RESOURCE_LIMIT when cap is too small. */
int32_t dz_pplx_residency_info(dz_ctx *ctx, dz_pplx *model, char *json, size_t cap);

/* ---- kernel tuner (webgpu/checkpoint.rs:95-294, 428-652) ------------------------ */

/* Times the tile variants of every tuned kernel family within budget_ms and
 * keeps the fastest variant whose output is bitwise equal to the family's
 * reference variant and faster than 0.99x it. Families, in the reference's
 * stage order (checkpoint.rs:251-262): "delta_scan" (:328-421
 * select_delta_scan: 128 tokens of 32 value and 16 key heads; only the two
 * chunked scans, which keep the default's summation order, are candidates),
 * "norm" (:652-684 select_norm: 64 rows of 2560, the fused norm and codes
 * against the separate ones), "grouped" (the W4A8 product, :480-563
 * select_gemm at M,N,K = 256, 8192, 2560), "mlp" (the fused MLP, :568-652
 * select_mlp at 128, 9216, 2560), then "gemv", "gemm_w4a16" and "i8_gemm"
 * (no reference counterpart). cache_in (JSON from an earlier
 * cache_out, or NULL; unreadable text is ignored) is reused while its key
 * still matches, re-checking equality only. The selection JSON is written to
 * cache_out (cap bytes). budget_ms == 0 keeps the reference variants. */
int32_t dz_tune(dz_ctx *ctx, uint32_t budget_ms, const char *cache_in, char *cache_out,
                size_t cap);
/* Forces a variant of a family by name (tests and benchmarks). Families and
 * variants (the first of each is the default; every variant of a family
 * gives the same bits, except the delta scan's two opt-ins below):
 *   "gemv"        auto, w16, w8, stream8, stream4, persist (w16/w8: 16 or 8 waves
 *                 share one 16-row tile, each wave a fixed chunk of K; stream8/
 *                 stream4: one wave per tile, 8 or 4 tiles per block, for K a
 *                 multiple of 2048 and up to 8 rows, else w16; persist: w16's
 *                 blocks, one per compute unit, each walking tiles with the next
 *                 tile's loads in flight, for K <= 4096 and up to 8 rows, else
 *                 w16; "auto" takes persist for up to 8 rows over four or more
 *                 tiles per compute unit at K <= 4096, else w16, or stream4 /
 *                 stream8 for 2..8 rows over eight or more tiles per compute unit)
 *   "gemm_w4a16"  pipe-auto, 256x256p2w8, 128x128p2w4, 128x256p2w8, 256x128w2x2,
 *                 128x128w2x2, 128x64w2x2, 256x256p2w8-persist, 256x192p2w8-persist,
 *                 256x128p2w8
 *   "i8_gemm"     256x256p2w8, 256x256p4k64w8, 256x128p3w8, 256x128p3, 128x128w2x2,
 *                 256x128w2x2, 64x64w2x2, 256x256p2w8-stream, 256x256p2w8-stream-mid,
 *                 256x128k64p2-stream2 (the "-stream" forms are persistent: one
 *                 or two blocks per compute unit, each walking several tiles)
 *   "grouped"     pipe-auto, pipe256x128w8, wave16x16, pipe128x128w4, pipe64x128w2,
 *                 pipe128x128m8, pipe128x128n8, pipe32x128w8, pipe64x128w8,
 *                 pipe32x128w8g4, pipe64x128w8g4 (g4: four 64-groups per
 *                 pipeline step instead of two), fewrow16 (the few-row kernel,
 *                 16 rows per block row, over the A8 codes), pipe32x64w4,
 *                 pipe64x64w8
 *   "mlp"         pipe-auto, pipe256x64w8, pipe128x64w4, wave16x64, pipe256x64n2,
 *                 pipe128x64n2
 *   "delta_scan"  chunked64, chunked64-c32, recurrent, recurrent-rolled,
 *                 auto (the decider's gated delta rule. The default runs the
 *                 rule by 64-token chunks with 16 state columns per block;
 *                 chunked64-c32 takes 32 per block, the same bits. The two
 *                 token scans (whole 16-token stages unrolled, or rolled)
 *                 give the same bits as each other; they regroup the
 *                 arithmetic, so they agree with the chunked scans to
 *                 rounding, not bit for bit. "auto" runs the token scan
 *                 below 384 tokens and the chunked one from there, so a
 *                 decider's bits then depend on its chunk length. The token
 *                 scans and auto are explicit opt-ins that the tuner never
 *                 selects, and the only variants anywhere that do not give
 *                 their family's reference bits)
 *   "norm"        fused, separate (the decider's layer norms above 16 rows:
 *                 one kernel for the RMSNorm and the A8 codes its products
 *                 share, or the norm then one quantization per product; the
 *                 same bits) */
int32_t dz_select_variant(dz_ctx *ctx, const char *family, const char *variant);

#ifdef __cplusplus
}
#endif
#endif
