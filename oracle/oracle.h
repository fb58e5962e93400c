/*
 * oracle.h -- CPU restatement of decisive's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels in
 * decisive_amd/csrc: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product never links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the hyperlogue/decisive source tree).  Floating point follows IEEE-754
 * binary32 with round-to-nearest-even; the library is compiled with
 * -ffp-contract=off so that only explicit fmaf() calls fuse.
 */
#ifndef DECISIVE_ORACLE_H
#define DECISIVE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE conversions (half 2.7.1 semantics: round to nearest even) ---- */
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
void or_f32_to_bf16_n(const float *x, size_t n, uint16_t *out);
void or_f32_to_f16_n(const float *x, size_t n, uint16_t *out);
void or_f16_to_f32_n(const uint16_t *x, size_t n, float *out);

/* ---- a1/a2: the g64 wire layout (src/models/pplx_flash/packed.rs) ---- */
/* packed.rs:10-19 size(); returns 0 when the shape is invalid. */
size_t or_packed_size(size_t rows, size_t cols, int bits);
/* packed.rs:31-56 pack(): BF16 [rows x cols] -> rows x cols/64 groups of
 * (bits*8 code bytes, f32 LE scale). Returns 0, or -1 on bad shape, -2 on a
 * non-finite weight. */
int or_pack_g64(const uint16_t *bf16, size_t rows, size_t cols, int bits, uint8_t *out);
/* packed.rs:59-73 unpack(): f32(code) * scale per value. Returns 0, -1 on bad
 * length, -3 on a scale that is not finite and positive. */
int or_unpack_g64(const uint8_t *bytes, size_t nbytes, int bits, float *out);
/* packed.rs:75-119 project(): portable W{4,8}A8 GEMV on the wire layout,
 * `sum += dot * (sx * sw)` unfused. Returns 0, -1 bad shape, -2 non-finite x. */
int or_project(const uint8_t *packed, int bits, size_t cols, const float *x,
               size_t outputs, float *y);

/* ---- D1: the g32/f16 layout quantized from f32 weights ----
 * Per 32-run along K: scale = max(absmax/7, smallest f16 subnormal) in f32,
 * codes = clamp(rne(v * (1/scale)), +-7) (packed.rs:37-45 with L=7, run 32),
 * stored as 16 code bytes (code+8 nibbles, low nibble = even k) followed by
 * the f16 LE scale f16(scale) (decima/pack.rs:134-140 precedent). */
size_t or_g32_size(size_t rows, size_t cols);
int or_pack_g32_f16(const float *w, size_t rows, size_t cols, uint8_t *out);
int or_unpack_g32_f16(const uint8_t *bytes, size_t nbytes, float *out);

/* ---- a3/a4: grouped quantizers (src/models/pplx_flash/int8.rs) ----
 * int8.rs:305-313 group_scale_bits and :347-360 pack_bits over one run.
 * Scale = max(absmax/limit, FLT_MIN); code = clamp(rne(v * recip(scale)), +-limit). */
float or_group_scale(const float *x, size_t n, int bits);
void or_group_codes(const float *x, size_t n, float scale, int bits, int8_t *out);
/* int8.rs:51-152 from_bf16_optimized (plain mode): BF16 [n x k], any k >= 1,
 * zero-padded to G=ceil(k/64) groups. codes [n x G*64], scales [n x G].
 * Returns 0, -1 on bad shape, -2 on a non-finite weight. */
int or_weight_quantize(const uint16_t *bf16, size_t n, size_t k, int bits,
                       int8_t *codes, float *scales);
/* int8.rs:178-202 prepare(): per (token, 64-group) A8 (or A4) quantization;
 * tail group zero-padded. q [m x G*64], s [m x G]. */
void or_act_quantize(const float *x, size_t m, size_t k, int bits, int8_t *q, float *s);

/* ---- a5: grouped W{4,8}A8 product ----
 * fused=1: int8.rs:524-585 rows<R,Q4> order, acc = fmaf(f32(dot), sw*sx, acc)
 * fused=0: int8.rs:259-287 scalar order, acc = acc + f32(dot) * (sx*sw).
 * Group dots are exact int32. Non-finite activations give all-NaN rows for the
 * whole call (int8.rs:170-173): the caller checks finiteness first. */
void or_grouped_gemm(const int8_t *qx, const float *sx, size_t m,
                     const int8_t *qw, const float *sw, size_t n, size_t k,
                     int fused, float *y);
/* The same with the affine offset term of a fitted matrix (offsets [n x G]):
 * fused int8.rs:566-571 acc = fmaf(off, sx*f32(sum q), acc); scalar
 * :279-282 acc = acc + off*(sx*f32(sum q)); sum q the row's group codes. */
void or_grouped_gemm_affine(const int8_t *qx, const float *sx, size_t m, const int8_t *qw, const float *sw,
                            const float *offsets, size_t n, size_t k, int fused, float *y);
/* ---- fitted Q4 quantizers (quantization.rs; avx2 selects the 8-lane sum order) ----
 * :25-71 mse over one group (n <= 64): codes [-8, 7], returns the scale (may be < 0).
 * :147-200 affine: codes [-8, 7], scale > 0 and offset.
 * int8.rs:86-117 from_bf16_optimized, mode 1 mse / 2 affine; offsets zero for mse. */
float or_fit_mse(const float *x, size_t n, int avx2, int8_t *out);
void or_fit_affine(const float *x, size_t n, int avx2, int8_t *out, float *scale, float *offset);
float or_fit_nf4(const float *x, size_t n, int8_t *out);
float or_nf4_value(int index);
void or_rows_decode(const int8_t *codes, const float *scales, const float *offsets, int nf4, size_t rows,
                    size_t cols, float *y);
int or_weight_quantize_fitted(const uint16_t *bf16, size_t n, size_t k, int mode, int avx2, int8_t *codes,
                              float *scales, float *offsets);
/* int8.rs:166-176 Matrix::apply: finiteness check + prepare + product. */
void or_matrix_apply(const float *x, size_t m, const int8_t *qw, const float *sw,
                     size_t n, size_t k, int act_bits, int fused, float *y);

/* ---- a3 panel layout + AVX2 rows<4,Q4> (CPU baseline) ---- */
/* int8.rs:121-131: panel p, group g, k, column c -> g*512 + (k/4)*32 + c*4 + k%4
 * (Q4: byte index /2, low nibble even). data bytes = ceil(n/8)*G*512/(8/bits). */
size_t or_panel_bytes(size_t n, size_t k, int bits);
void or_panel_pack(const int8_t *codes, const float *scales, size_t n, size_t k,
                   int bits, uint8_t *data, float *pscales);
/* int8.rs:229-256 + :404-585, threads over ceil(n/32) tiles; poffsets (the
 * affine offsets in the pscales layout, or NULL) adds int8.rs:566-571. Returns
 * 0, or -1 when AVX2 is not available on this CPU. */
int or_panel_apply_avx2(const uint8_t *data, const float *pscales, const float *poffsets, size_t n,
                        size_t k, int bits, const int8_t *qx, const float *sx, size_t m,
                        int threads, float *y);
int or_has_avx2(void);

/* ---- a11/a12: per-row int8 (src/models/pplx_flash/webgpu/int8.rs) ---- */
/* int8.rs:107-145 quantize(): scale = absmax/127 (no floor); q = clamp(rne(x/scale),
 * +-127) if scale > 0 else 0; sums = sum of q. */
void or_i8_quantize_rows(const float *x, size_t rows, size_t k, int8_t *q,
                         float *scales, int32_t *sums);
/* int8.rs:147-242 gemm(): exact int32 dot; raw -> i32, else (f32(dot)*sx)*sw.
 * Either output pointer may be NULL. threads >= 1 splits rows. */
/* webgpu/q4.rs:48-73 quantize (a13): per-row Q4 of f16 weights into the
 * reference's word buffer [rows*(k/8) codes | rows scales | rows sums]. */
int or_q4_quantize_rows(const uint16_t *x_f16, size_t rows, size_t k, uint32_t *out);
void or_q4_rows_codes(const uint32_t *words, size_t rows, size_t k, int8_t *codes);
void or_i8_gemm(const int8_t *qa, const float *sa, size_t m, const int8_t *qw,
                const float *sw, size_t n, size_t k, int threads, int32_t *raw,
                float *y);
void or_i8_gemm_fused(const int8_t *qa, const float *sa, size_t m, const int8_t *qg, const float *sg,
                      const int8_t *qu, const float *su, size_t n, size_t k, float *y);

/* ---- W4A16 closed form (no reference kernel; see D2) ----
 * y[m x n] = sum_k f16(x)[i,k] * w[j,k] in f64, w already dequantized f32. */
void or_w4a16(const uint16_t *x_f16, size_t m, size_t k, const float *w,
              size_t n, double *y);

/* ---- a14: layer epilogues ---- */
/* decima/cpu.rs:529-540 Norm::in_place */
void or_layernorm(float *x, size_t rows, size_t d, const float *w, const float *b, float eps);
/* decima/cpu.rs:542-556 gelu (erf form) */
void or_gelu(float *x, size_t n);
/* pplx_flash/cpu.rs:310-333 rms_from, zero_centered */
void or_rmsnorm(const float *x, size_t rows, size_t d, const float *w, float eps,
                int zero_centered, float *y);
/* pplx_flash/cpu.rs:513-518 silu and :348-371 silu_mul (portable form) */
void or_silu_mul(float *gate, const float *up, size_t n);
/* pplx_flash/cpu.rs:519-529 softmax */
void or_softmax(float *x, size_t n);
/* decima/cpu.rs:574-586 mean over rows */
void or_mean_rows(const float *x, size_t rows, size_t d, float *out);
/* Softmax attention, non-causal: q,k,v [seq x heads*dh] f32 -> out, in f64
 * accumulation (closed form for the tolerance check). */
void or_attention(const float *q, const float *k, const float *v, size_t seq,
                  size_t heads, size_t dh, float scale, float *out);

/* ---- a8/a10: fused MLP requantization (webgpu/grouped_q4.rs:27-41) ----
 * v = silu(gate)*up with silu(v) = v*(1/(1+exp(-v))), then per (row, 64-col
 * block) A8 quantization with the a4 formula. gate/up [m x n], n % 64 == 0. */
void or_silu_requant(const float *gate, const float *up, size_t m, size_t n,
                     int8_t *q, float *s);

/* ---- Pplx decoder layer ops (src/models/pplx_flash/backbone.rs, cpu.rs) ----
 * Dimensions are parameters; the reference fixes hidden 2560, FF 9216, 32
 * delta heads (lh) of ld = 128 over 16 key heads (lk), 16 attention heads
 * (ah) of ad = 256 over 4 key/value heads (akv). */
/* cpu.rs:372-391 conv_silu over a fresh sequence (backbone.rs:271-283):
 * out[t][c] = silu(sum over tap 0..3 of x[t-3+tap][c] * w[tap][c]), rows
 * before t = 0 zero (the zero history); the sum starts at 0 in tap order with
 * unfused products. x, out [n x width]; w [4 x width] (tap-major, as
 * backbone.rs:170-178 repacks conv1d.weight [width, 1, 4]). */
void or_conv_silu(const float *x, size_t n, size_t width, const float *w, float *out);
/* backbone.rs:349-408 delta_scan for every head over a fresh state: conv
 * [n x (2*lk*ld + lh*ld)] holds the q heads, k heads and v heads of each
 * token; head h reads q/k head h / (lh/lk). a, b [n x lh]; decay = exp(A_log)
 * and dt [lh]. out [lh x n x ld]. */
void or_delta_scan(const float *conv, size_t n, int lh, int lk, int ld, const float *a, const float *b,
                   const float *decay, const float *dt, float *out);
/* backbone.rs:310-326 and cpu.rs:392-414: per (t, h), s = 1/sqrt(sum(src^2)/ld
 * + 1e-6), ctx[t][h*ld + i] = ((src[i]*s)*norm[i])*silu(z[t][h*ld + i]).
 * heads [lh x n x ld], z and ctx [n x lh*ld]. */
void or_delta_gate(const float *heads, size_t n, int lh, int ld, const float *norm, const float *z,
                   float *ctx);
/* backbone.rs:415-428 rope: per row (position pos[r]) and head of width ad,
 * dims i and i+32 (i < 32) rotate by angle = f32(pos) * freq[i]. */
void or_rope(float *x, size_t rows, int heads, int ad, const size_t *pos, const float *freq);
/* backbone.rs:509-579 attention core, in f64 (closed form; the reference uses
 * matrixmultiply's sgemm): q [nq x ah x ad], k and v [nk x akv x ad]; head h
 * reads key/value head h / (ah/akv); out [ah x nq x ad] = softmax(q.k * scale) v. */
void or_attention_gqa(const float *q, const float *k, const float *v, size_t nq, size_t nk, int ah, int akv,
                      int ad, float scale, float *out);
/* cpu.rs:415-429 attention_gate: out[t][h*ad + i] = heads[h][t][i] *
 * sigmoid(z[t][h*ad + i]); heads [ah x n x ad], z and out [n x ah*ad]. */
void or_attention_gate(const float *heads, size_t n, int ah, int ad, const float *z, float *out);

#ifdef __cplusplus
}
#endif
#endif
