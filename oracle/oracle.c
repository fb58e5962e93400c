/*
 * oracle.c -- CPU restatement of decisive's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never the product.
 * Each function cites the reference file:line it restates (relative to the
 * hyperlogue/decisive tree). Built with -ffp-contract=off -fno-fast-math so the
 * only fused multiply-adds are the explicit fmaf() calls that the reference's
 * AVX2 kernel performs with _mm256_fmadd_ps.
 *
 * Parity unpinned: the AVX2 lane order of the fitted quantizers' sums
 * (or_fit_mse / or_fit_affine, quantization.rs:73-129, :202-258) is followed
 * but checked only through the reference's invariants of the fits; they make
 * test weights, and no product's parity depends on their exact bits.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <unistd.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* Runs `fn(job)` on up to `threads` threads that take their work from a shared
 * counter in `job`: joins exactly the threads that started, and runs the
 * worker on the calling thread when none could start, so every unit of work is
 * done whatever pthread_create returns. */
static void run_workers(void *(*fn)(void *), void *job, int threads) {
    pthread_t *ids = threads > 0 ? (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads) : NULL;
    int started = 0;
    for (int t = 0; ids && t < threads; t++)
        if (pthread_create(&ids[started], NULL, fn, job) == 0) started++;
    if (started == 0) fn(job);
    for (int t = 0; t < started; t++) pthread_join(ids[t], NULL);
    free(ids);
}

/* ------------------------------------------------------------------------ */
/* IEEE conversions (half 2.7.1: bf16::from_f32 / f16::from_f32 round to    */
/* nearest even; widening is exact).                                        */
/* ------------------------------------------------------------------------ */

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_bf16_to_f32(uint16_t h) { return float_of((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
    uint32_t x = bits_of(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return float_of(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        float v = (float)m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    return float_of(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x = bits_of(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    int e = (int)exp - 112; /* biased f16 exponent */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t full = man | 0x800000u;
        int shift = 14 - e;
        uint32_t q = full >> shift;
        uint32_t rem = full & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

void or_f32_to_bf16_n(const float *x, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_bf16(x[i]);
}
void or_f32_to_f16_n(const float *x, size_t n, uint16_t *out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f32_to_f16(x[i]);
}
void or_f16_to_f32_n(const uint16_t *x, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = or_f16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Grouped quantizer: int8.rs:305-313 (group_scale_bits), :347-360          */
/* (pack_bits); identical formula to packed.rs:43-45.                        */
/* ------------------------------------------------------------------------ */

static float limit_of(int bits) { return bits == 4 ? 7.0f : 127.0f; }

float or_group_scale(const float *x, size_t n, int bits) {
    float maximum = 0.0f;
    for (size_t i = 0; i < n; i++) maximum = fmaxf(maximum, fabsf(x[i]));
    float s = maximum / limit_of(bits);
    return s > FLT_MIN ? s : FLT_MIN;
}

static int8_t quantize_one(float v, float inverse, float limit) {
    float r = rintf(v * inverse); /* round_ties_even under the default mode */
    if (r < -limit) r = -limit;
    if (r > limit) r = limit;
    return (int8_t)(int)r;
}

void or_group_codes(const float *x, size_t n, float scale, int bits, int8_t *out) {
    float inverse = 1.0f / scale; /* f32::recip */
    float limit = limit_of(bits);
    for (size_t i = 0; i < n; i++) out[i] = quantize_one(x[i], inverse, limit);
}

/* ------------------------------------------------------------------------ */
/* a1/a2: the g64 wire layout, packed.rs                                    */
/* ------------------------------------------------------------------------ */

static size_t group_bytes(int bits) { return 64u * (size_t)bits / 8u + 4u; }

size_t or_packed_size(size_t rows, size_t cols, int bits) {
    if (bits != 4 && bits != 8) return 0;
    if (rows == 0 || cols == 0 || cols % 64 != 0) return 0;
    return rows * (cols / 64) * group_bytes(bits);
}

int or_pack_g64(const uint16_t *bf16, size_t rows, size_t cols, int bits, uint8_t *out) {
    if (!or_packed_size(rows, cols, bits)) return -1;
    size_t groups = rows * cols / 64;
    for (size_t g = 0; g < groups; g++) {
        float values[64];
        for (int i = 0; i < 64; i++) {
            values[i] = or_bf16_to_f32(bf16[g * 64 + i]);
            if (!isfinite(values[i])) return -2;
        }
        float scale = or_group_scale(values, 64, bits);
        int8_t codes[64];
        or_group_codes(values, 64, scale, bits, codes);
        uint8_t *dst = out + g * group_bytes(bits);
        if (bits == 4) {
            for (int i = 0; i < 32; i++)
                dst[i] = (uint8_t)((codes[2 * i] + 8) | ((codes[2 * i + 1] + 8) << 4));
            dst += 32;
        } else {
            for (int i = 0; i < 64; i++) dst[i] = (uint8_t)codes[i];
            dst += 64;
        }
        memcpy(dst, &scale, 4); /* little-endian host */
    }
    return 0;
}

static int code_at(const uint8_t *group, size_t k, int bits) {
    if (bits == 4) return (int)((group[k / 2] >> (4 * (k % 2))) & 15u) - 8;
    return (int)(int8_t)group[k];
}

int or_unpack_g64(const uint8_t *bytes, size_t nbytes, int bits, float *out) {
    size_t stride = or_packed_size(1, 64, bits);
    if (!stride || nbytes == 0 || nbytes % stride != 0) return -1;
    for (size_t g = 0; g < nbytes / stride; g++) {
        const uint8_t *group = bytes + g * stride;
        float scale;
        memcpy(&scale, group + stride - 4, 4);
        if (!(isfinite(scale) && scale > 0.0f)) return -3;
        for (size_t k = 0; k < 64; k++) out[g * 64 + k] = (float)code_at(group, k, bits) * scale;
    }
    return 0;
}

int or_project(const uint8_t *packed, int bits, size_t cols, const float *x, size_t outputs,
               float *y) {
    size_t stride = or_packed_size(1, cols, bits);
    size_t gstride = or_packed_size(1, 64, bits);
    if (!stride) return -1;
    for (size_t i = 0; i < cols; i++)
        if (!isfinite(x[i])) return -2;
    size_t groups = cols / 64;
    int32_t *codes = (int32_t *)malloc(cols * sizeof(int32_t));
    float *scales = (float *)malloc(groups * sizeof(float));
    for (size_t g = 0; g < groups; g++) {
        float s = or_group_scale(x + g * 64, 64, 8);
        float inverse = 1.0f / s;
        for (size_t i = 0; i < 64; i++) codes[g * 64 + i] = quantize_one(x[g * 64 + i], inverse, 127.0f);
        scales[g] = s;
    }
    for (size_t o = 0; o < outputs; o++) {
        const uint8_t *row = packed + o * stride;
        float sum = 0.0f;
        for (size_t g = 0; g < groups; g++) {
            const uint8_t *group = row + g * gstride;
            float scale;
            memcpy(&scale, group + gstride - 4, 4);
            int32_t dot = 0;
            for (size_t k = 0; k < 64; k++) dot += codes[g * 64 + k] * code_at(group, k, bits);
            sum = sum + (float)dot * (scales[g] * scale);
        }
        y[o] = sum;
    }
    free(codes);
    free(scales);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* D1: g32/f16 layout                                                       */
/* ------------------------------------------------------------------------ */

size_t or_g32_size(size_t rows, size_t cols) {
    if (rows == 0 || cols == 0 || cols % 32 != 0) return 0;
    return rows * (cols / 32) * 18u;
}

int or_pack_g32_f16(const float *w, size_t rows, size_t cols, uint8_t *out) {
    if (!or_g32_size(rows, cols)) return -1;
    const float smallest = 5.9604644775390625e-8f; /* f16 bits 0x0001 */
    size_t groups = rows * cols / 32;
    for (size_t g = 0; g < groups; g++) {
        const float *v = w + g * 32;
        float maximum = 0.0f;
        for (int i = 0; i < 32; i++) {
            if (!isfinite(v[i])) return -2;
            maximum = fmaxf(maximum, fabsf(v[i]));
        }
        float scale = maximum / 7.0f;
        if (!(scale > smallest)) scale = smallest;
        float inverse = 1.0f / scale;
        uint8_t *dst = out + g * 18;
        for (int i = 0; i < 16; i++) {
            int c0 = quantize_one(v[2 * i], inverse, 7.0f);
            int c1 = quantize_one(v[2 * i + 1], inverse, 7.0f);
            dst[i] = (uint8_t)((c0 + 8) | ((c1 + 8) << 4));
        }
        uint16_t h = or_f32_to_f16(scale);
        dst[16] = (uint8_t)(h & 0xff);
        dst[17] = (uint8_t)(h >> 8);
    }
    return 0;
}

int or_unpack_g32_f16(const uint8_t *bytes, size_t nbytes, float *out) {
    if (nbytes == 0 || nbytes % 18 != 0) return -1;
    for (size_t g = 0; g < nbytes / 18; g++) {
        const uint8_t *group = bytes + g * 18;
        float scale = or_f16_to_f32((uint16_t)(group[16] | (group[17] << 8)));
        if (!(isfinite(scale) && scale > 0.0f)) return -3;
        for (size_t k = 0; k < 32; k++) out[g * 32 + k] = (float)code_at(group, k, 4) * scale;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* a3/a4: grouped weight and activation quantization, int8.rs               */
/* ------------------------------------------------------------------------ */

int or_weight_quantize(const uint16_t *bf16, size_t n, size_t k, int bits, int8_t *codes,
                       float *scales) {
    if ((bits != 4 && bits != 8) || n == 0 || k == 0) return -1;
    size_t groups = (k + 63) / 64;
    for (size_t c = 0; c < n; c++) {
        for (size_t g = 0; g < groups; g++) {
            size_t count = k - g * 64 < 64 ? k - g * 64 : 64;
            float values[64] = {0};
            for (size_t i = 0; i < count; i++) {
                values[i] = or_bf16_to_f32(bf16[c * k + g * 64 + i]);
                if (!isfinite(values[i])) return -2;
            }
            float s = or_group_scale(values, 64, bits);
            scales[c * groups + g] = s;
            or_group_codes(values, 64, s, bits, codes + (c * groups + g) * 64);
        }
    }
    return 0;
}

void or_act_quantize(const float *x, size_t m, size_t k, int bits, int8_t *q, float *s) {
    size_t groups = (k + 63) / 64;
    for (size_t r = 0; r < m; r++) {
        for (size_t g = 0; g < groups; g++) {
            size_t count = k - g * 64 < 64 ? k - g * 64 : 64;
            const float *values = x + r * k + g * 64;
            float scale = or_group_scale(values, count, bits);
            s[r * groups + g] = scale;
            int8_t *out = q + (r * groups + g) * 64;
            memset(out, 0, 64);
            or_group_codes(values, count, scale, bits, out);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a5: grouped W{4,8}A8 product                                              */
/* ------------------------------------------------------------------------ */

void or_grouped_gemm(const int8_t *qx, const float *sx, size_t m, const int8_t *qw,
                     const float *sw, size_t n, size_t k, int fused, float *y) {
    size_t groups = (k + 63) / 64;
    for (size_t r = 0; r < m; r++) {
        for (size_t c = 0; c < n; c++) {
            float acc = 0.0f;
            for (size_t g = 0; g < groups; g++) {
                const int8_t *a = qx + (r * groups + g) * 64;
                const int8_t *b = qw + (c * groups + g) * 64;
                int32_t dot = 0;
                for (int i = 0; i < 64; i++) dot += (int32_t)a[i] * (int32_t)b[i];
                if (fused) {
                    float s = sw[c * groups + g] * sx[r * groups + g];
                    acc = fmaf((float)dot, s, acc);
                } else {
                    acc = acc + (float)dot * (sx[r * groups + g] * sw[c * groups + g]);
                }
            }
            y[r * n + c] = acc;
        }
    }
}

/* int8.rs:259-287 (scalar) and :524-585 (AVX2 rows) with the affine offset
 * term of a fitted matrix: per group, after the scale term,
 *   fused:  acc = fmaf(offset, sx * f32(sum q), acc)         int8.rs:566-571
 *   scalar: acc = acc + offset * (sx * f32(sum q))            int8.rs:279-282
 * where sum q is the exact sum of the row's group codes (int8.rs:191-193). */
void or_grouped_gemm_affine(const int8_t *qx, const float *sx, size_t m, const int8_t *qw, const float *sw,
                            const float *offsets, size_t n, size_t k, int fused, float *y) {
    size_t groups = (k + 63) / 64;
    for (size_t r = 0; r < m; r++) {
        for (size_t c = 0; c < n; c++) {
            float acc = 0.0f;
            for (size_t g = 0; g < groups; g++) {
                const int8_t *a = qx + (r * groups + g) * 64;
                const int8_t *b = qw + (c * groups + g) * 64;
                int32_t dot = 0, sum = 0;
                for (int i = 0; i < 64; i++) {
                    dot += (int32_t)a[i] * (int32_t)b[i];
                    sum += a[i];
                }
                const float sxv = sx[r * groups + g], off = offsets[c * groups + g];
                if (fused) {
                    acc = fmaf((float)dot, sw[c * groups + g] * sxv, acc);
                    acc = fmaf(off, sxv * (float)sum, acc);
                } else {
                    acc = acc + (float)dot * (sxv * sw[c * groups + g]);
                    acc = acc + off * (sxv * (float)sum);
                }
            }
            y[r * n + c] = acc;
        }
    }
}

/* ---- fitted Q4 quantizers (quantization.rs) -------------------------------
 * The AVX2 forms keep eight lane sums (lane l takes elements l, l+8, ... of
 * the whole 8-wide part), each a separate multiply and add, then add the
 * lanes in order to a -0.0 start (Rust's f32 Sum) and that to the scalar
 * sums of the tail. */
/* f32::clamp(-8, 7), which passes NaN through (as do the AVX2 min/max with
 * the rounded value second), and Rust's saturating `as i8`, NaN -> 0. */
static float clamp_code(float v) { return v < -8.0f ? -8.0f : (v > 7.0f ? 7.0f : v); }
static int8_t code_i8(float v) { return isnan(v) ? 0 : (int8_t)v; }

static float f32_sum_lanes(const float *lanes) {
    float s = -0.0f;
    for (int l = 0; l < 8; l++) s += lanes[l];
    return s;
}

/* quantization.rs:73-129 stats: (sum v q, sum q q, sum (v - q s)^2). */
static void mse_stats(const float *x, size_t n, float scale, int avx2, float out[3]) {
    const float inverse = 1.0f / scale;
    size_t end = avx2 ? n / 8 * 8 : 0;
    float lanes[3][8] = {{0}};
    for (size_t i = 0; i < end; i++) {
        const float q = clamp_code(rintf(x[i] * inverse));
        const float e = x[i] - q * scale;
        lanes[0][i % 8] += x[i] * q;
        lanes[1][i % 8] += q * q;
        lanes[2][i % 8] += e * e;
    }
    float t[3] = {0.0f, 0.0f, 0.0f};
    for (size_t i = end; i < n; i++) {
        const float q = clamp_code(rintf(x[i] * inverse));
        const float e = x[i] - q * scale;
        t[0] += x[i] * q;
        t[1] += q * q;
        t[2] += e * e;
    }
    for (int j = 0; j < 3; j++) out[j] = avx2 ? f32_sum_lanes(lanes[j]) + t[j] : t[j];
}

/* quantization.rs:25-71 mse: the symmetric scale, then alternating least
 * squares from six starts (signs -1, 1 x ratios 0.8, 0.95, 1.1 of 1/7), four
 * steps each, keeping the codes of the lowest error. Codes in [-8, 7]; the
 * returned scale may be negative. */
float or_fit_mse(const float *x, size_t n, int avx2, int8_t *out) {
    float maximum = 0.0f;
    for (size_t i = 0; i < n; i++) maximum = fmaxf(maximum, fabsf(x[i]));
    const float baseline = or_group_scale(x, n, 4);
    or_group_codes(x, n, baseline, 4, out);
    if (maximum == 0.0f) return baseline;
    float normalized[64];
    for (size_t i = 0; i < n; i++) normalized[i] = x[i] / maximum;
    float best_error = 0.0f;
    {
        const float ratio = baseline / maximum;
        for (size_t i = 0; i < n; i++) {
            const float e = normalized[i] - (float)out[i] * ratio;
            best_error += e * e;
        }
    }
    float best = baseline;
    const float signs[2] = {-1.0f, 1.0f}, ratios[3] = {0.8f, 0.95f, 1.1f};
    for (int si = 0; si < 2; si++) {
        for (int ri = 0; ri < 3; ri++) {
            float scale = signs[si] * ratios[ri] / 7.0f;
            for (int step = 0; step < 4; step++) {
                float st[3];
                mse_stats(normalized, n, scale, avx2, st);
                if (st[2] < best_error) {
                    best_error = st[2];
                    best = scale * maximum;
                    const float inverse = 1.0f / scale;
                    for (size_t i = 0; i < n; i++)
                        out[i] = code_i8(clamp_code(rintf(normalized[i] * inverse)));
                }
                if (st[1] == 0.0f) break;
                const float next = st[0] / st[1];
                if (!isfinite(next) || fabsf(next) < FLT_MIN || next == scale) break;
                scale = next;
            }
        }
    }
    return best;
}

/* quantization.rs:202-262 affine_stats: (sum v q, sum q q, sum e^2, sum q),
 * e = v - (q s + o). */
static void affine_stats(const float *x, size_t n, float scale, float offset, int avx2, float out[4]) {
    const float inverse = 1.0f / scale;
    size_t end = avx2 ? n / 8 * 8 : 0;
    float lanes[4][8] = {{0}};
    for (size_t i = 0; i < end; i++) {
        const float q = clamp_code(rintf((x[i] - offset) * inverse));
        const float e = x[i] - (q * scale + offset);
        lanes[0][i % 8] += x[i] * q;
        lanes[1][i % 8] += q * q;
        lanes[2][i % 8] += e * e;
        lanes[3][i % 8] += q;
    }
    float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t i = end; i < n; i++) {
        const float q = clamp_code(rintf((x[i] - offset) * inverse));
        const float e = x[i] - (q * scale + offset);
        t[0] += x[i] * q;
        t[1] += q * q;
        t[2] += e * e;
        t[3] += q;
    }
    for (int j = 0; j < 4; j++) out[j] = avx2 ? t[j] + f32_sum_lanes(lanes[j]) : t[j];
}

/* quantization.rs:147-200 affine: values normalized by the largest magnitude,
 * three starts (ratios 0.8, 1, 1.2 of the range / 15) with the offset at the
 * range's centre plus half a step, four least-squares steps each, keeping the
 * lowest error. A zero group gives (FLT_MIN, 0) and zero codes; a constant one
 * (FLT_MIN, x[0]). Codes in [-8, 7]; scale > 0. */
void or_fit_affine(const float *x, size_t n, int avx2, int8_t *out, float *scale_out, float *offset_out) {
    float maximum = 0.0f;
    for (size_t i = 0; i < n; i++) maximum = fmaxf(maximum, fabsf(x[i]));
    if (maximum == 0.0f) {
        memset(out, 0, n);
        *scale_out = FLT_MIN;
        *offset_out = 0.0f;
        return;
    }
    float v[64];
    for (size_t i = 0; i < n; i++) v[i] = x[i] / maximum;
    float low = INFINITY, high = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        low = fminf(low, v[i]);
        high = fmaxf(high, v[i]);
    }
    if (low == high) {
        memset(out, 0, n);
        *scale_out = FLT_MIN;
        *offset_out = x[0];
        return;
    }
    float total = -0.0f;
    for (size_t i = 0; i < n; i++) total += v[i];
    const float mean = total / (float)n;
    float best_error = INFINITY, best_s = 0.0f, best_o = 0.0f;
    const float ratios[3] = {0.8f, 1.0f, 1.2f};
    for (int ri = 0; ri < 3; ri++) {
        float scale = (high - low) / 15.0f * ratios[ri];
        float offset = (high + low + scale) * 0.5f;
        for (int step = 0; step < 4; step++) {
            float st[4];
            affine_stats(v, n, scale, offset, avx2, st);
            if (st[2] < best_error) {
                best_error = st[2];
                best_s = scale * maximum;
                best_o = offset * maximum;
                const float inverse = 1.0f / scale;
                for (size_t i = 0; i < n; i++)
                    out[i] = code_i8(clamp_code(rintf((v[i] - offset) * inverse)));
            }
            const float mean_q = st[3] / (float)n;
            const float denominator = st[1] - st[3] * mean_q;
            if (denominator <= 0.0f) break;
            const float next = (st[0] - st[3] * mean) / denominator;
            if (!isfinite(next) || next <= 0.0f) break;
            const float next_offset = mean - next * mean_q;
            if (next == scale && next_offset == offset) break;
            scale = next;
            offset = next_offset;
        }
    }
    *scale_out = best_s;
    *offset_out = best_o;
}

/* quantization.rs:3-20: the NF4 codebook as the reference writes it. */
static const float kNf4[16] = {-1.0f,        -0.6961928f,  -0.52507305f, -0.3949175f,
                               -0.28444138f, -0.18477343f, -0.091050036f, 0.0f,
                               0.0795803f,   0.1609302f,   0.2461123f,   0.33791524f,
                               0.44070983f,  0.562617f,    0.72295684f,  1.0f};

float or_nf4_value(int index) { return kNf4[index & 15]; }

/* quantization.rs:131-145 nf4_code: binary search over the midpoints. */
static int nf4_code(float value) {
    int low = 0, high = 15;
    while (low < high) {
        const int middle = (low + high) / 2;
        if (value > (kNf4[middle] + kNf4[middle + 1]) * 0.5f)
            low = middle + 1;
        else
            high = middle;
    }
    return low;
}

/* quantization.rs:260-302 nf4: normalized by the largest magnitude, three
 * starts (0.85, 1, 1.15), four least-squares steps each, the lowest error
 * kept. A zero group gives codes -1 (NF4 zero) and FLT_MIN. */
float or_fit_nf4(const float *x, size_t n, int8_t *out) {
    float maximum = 0.0f;
    for (size_t i = 0; i < n; i++) maximum = fmaxf(maximum, fabsf(x[i]));
    if (maximum == 0.0f) {
        memset(out, 0xff, n);
        return FLT_MIN;
    }
    float v[64];
    for (size_t i = 0; i < n; i++) v[i] = x[i] / maximum;
    float best_error = INFINITY, best_scale = maximum;
    const float initials[3] = {0.85f, 1.0f, 1.15f};
    for (int ii = 0; ii < 3; ii++) {
        float scale = initials[ii];
        for (int step = 0; step < 4; step++) {
            int8_t codes[64];
            float numerator = 0.0f, denominator = 0.0f, error = 0.0f;
            for (size_t i = 0; i < n; i++) {
                const int index = nf4_code(v[i] / scale);
                codes[i] = (int8_t)(index - 8);
                const float q = kNf4[index];
                numerator += v[i] * q;
                denominator += q * q;
                const float e = v[i] - scale * q;
                error += e * e;
            }
            if (error < best_error) {
                best_error = error;
                best_scale = scale * maximum;
                memcpy(out, codes, n);
            }
            if (denominator == 0.0f) break;
            const float next = numerator / denominator;
            if (next == scale || next <= 0.0f) break;
            scale = next;
        }
    }
    return best_scale;
}

/* quantized_rows.rs:89-110 append for a Q4 row of `cols` codes: value =
 * f32(code) or NF4[code + 8], times the group's scale, then plus its offset
 * (offsets may be NULL), each step rounded to f32. */
void or_rows_decode(const int8_t *codes, const float *scales, const float *offsets, int nf4, size_t rows,
                    size_t cols, float *y) {
    const size_t groups = cols / 64;
    for (size_t r = 0; r < rows; r++)
        for (size_t i = 0; i < cols; i++) {
            const int8_t c = codes[r * cols + i];
            const float value = nf4 ? kNf4[(c + 8) & 15] : (float)c;
            float out = value * scales[r * groups + i / 64];
            if (offsets) out = out + offsets[r * groups + i / 64];
            y[r * cols + i] = out;
        }
}

/* int8.rs:86-117 from_bf16_optimized with `optimized` (mode 1: mse) or
 * `affine` (mode 2), or quantized_rows.rs:56-66 with `nf4` (mode 3; the codes
 * index the codebook): BF16 [n x k] -> codes [n x G*64] (tail zero), scales
 * [n x G], offsets [n x G] (mode 2; zero otherwise). Returns 0, -2 on a
 * non-finite weight. */
int or_weight_quantize_fitted(const uint16_t *bf16, size_t n, size_t k, int mode, int avx2, int8_t *codes,
                              float *scales, float *offsets) {
    const size_t groups = (k + 63) / 64;
    for (size_t c = 0; c < n; c++) {
        for (size_t g = 0; g < groups; g++) {
            const size_t count = k - g * 64 < 64 ? k - g * 64 : 64;
            float values[64];
            for (size_t i = 0; i < count; i++) {
                values[i] = or_bf16_to_f32(bf16[c * k + g * 64 + i]);
                if (!isfinite(values[i])) return -2;
            }
            int8_t *out = codes + (c * groups + g) * 64;
            memset(out, 0, 64);
            float s, o = 0.0f;
            if (mode == 2)
                or_fit_affine(values, count, avx2, out, &s, &o);
            else if (mode == 3)
                s = or_fit_nf4(values, count, out);
            else
                s = or_fit_mse(values, count, avx2, out);
            scales[c * groups + g] = s;
            offsets[c * groups + g] = o;
        }
    }
    return 0;
}

void or_matrix_apply(const float *x, size_t m, const int8_t *qw, const float *sw, size_t n,
                     size_t k, int act_bits, int fused, float *y) {
    for (size_t i = 0; i < m * k; i++) {
        if (!isfinite(x[i])) {
            for (size_t j = 0; j < m * n; j++) y[j] = NAN;
            return;
        }
    }
    size_t groups = (k + 63) / 64;
    int8_t *q = (int8_t *)malloc(m * groups * 64 + 1);
    float *s = (float *)malloc(m * groups * sizeof(float) + 4);
    or_act_quantize(x, m, k, act_bits, q, s);
    or_grouped_gemm(q, s, m, qw, sw, n, k, fused, y);
    free(q);
    free(s);
}

/* ------------------------------------------------------------------------ */
/* a3 panel layout and the AVX2 rows<R,Q4> kernel (CPU baseline)             */
/* ------------------------------------------------------------------------ */

size_t or_panel_bytes(size_t n, size_t k, int bits) {
    size_t groups = (k + 63) / 64;
    return (n + 7) / 8 * groups * 512 / (bits == 4 ? 2 : 1);
}

void or_panel_pack(const int8_t *codes, const float *scales, size_t n, size_t k, int bits,
                   uint8_t *data, float *pscales) {
    size_t groups = (k + 63) / 64;
    size_t panels = (n + 7) / 8;
    memset(data, 0, or_panel_bytes(n, k, bits));
    memset(pscales, 0, panels * groups * 8 * sizeof(float));
    for (size_t p = 0; p < panels; p++) {
        uint8_t *pd = data + p * groups * 512 / (bits == 4 ? 2 : 1);
        for (size_t c = 0; c < 8 && p * 8 + c < n; c++) {
            size_t col = p * 8 + c;
            for (size_t g = 0; g < groups; g++) {
                pscales[(p * groups + g) * 8 + c] = scales[col * groups + g];
                const int8_t *src = codes + (col * groups + g) * 64;
                for (size_t kk = 0; kk < 64; kk++) {
                    size_t at = g * 512 + kk / 4 * 32 + c * 4 + kk % 4;
                    if (bits == 4) {
                        uint8_t nib = (uint8_t)(src[kk] + 8) & 15u;
                        pd[at / 2] |= (uint8_t)(nib << (4 * (at % 2)));
                    } else {
                        pd[at] = (uint8_t)src[kk];
                    }
                }
            }
        }
    }
}

int or_has_avx2(void) {
#if defined(__x86_64__)
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
#else
    return 0;
#endif
}

#if defined(__x86_64__)
struct panel_job {
    const uint8_t *data;
    const float *pscales;
    size_t n, k, m;
    int bits;
    const int8_t *qx;
    const float *sx;
    const float *poffsets; /* panel layout like pscales, NULL for none */
    float *y;
    size_t tiles;
    size_t next; /* atomic tile counter */
};

__attribute__((target("avx2"))) static __m256i unpack_q4(const uint8_t *p) {
    __m256i packed = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i *)p));
    __m256i low = _mm256_and_si256(packed, _mm256_set1_epi16(0x000f));
    __m256i high = _mm256_and_si256(_mm256_slli_epi16(packed, 4), _mm256_set1_epi16(0x0f00));
    return _mm256_sub_epi8(_mm256_or_si256(low, high), _mm256_set1_epi8(8));
}

/* int8.rs:524-585 rows<R,Q4>: R rows x one 8-column panel. `q4` selects the
 * on-the-fly nibble unpack; otherwise `pd` holds one signed byte per code. */
__attribute__((target("avx2,fma"))) static void panel_rows(const struct panel_job *j,
                                                           const uint8_t *pd, const float *ps,
                                                           int q4, size_t panel, size_t first,
                                                           size_t rows) {
    size_t groups = (j->k + 63) / 64;
    __m256i one = _mm256_set1_epi16(1);
    __m256 sums[8];
    for (size_t r = 0; r < rows; r++) sums[r] = _mm256_setzero_ps();
    for (size_t g = 0; g < groups; g++) {
        __m256i acc[8];
        for (size_t r = 0; r < rows; r++) acc[r] = _mm256_setzero_si256();
        size_t base = g * 512;
        for (size_t kk = 0; kk < 64; kk += 4) {
            __m256i b = q4 ? unpack_q4(pd + (base + kk * 8) / 2)
                           : _mm256_loadu_si256((const __m256i *)(pd + base + kk * 8));
            __m256i magnitude = _mm256_abs_epi8(b);
            for (size_t r = 0; r < rows; r++) {
                int32_t word;
                memcpy(&word, j->qx + ((first + r) * groups + g) * 64 + kk, 4);
                __m256i a = _mm256_set1_epi32(word);
                __m256i pair = _mm256_maddubs_epi16(magnitude, _mm256_sign_epi8(a, b));
                acc[r] = _mm256_add_epi32(acc[r], _mm256_madd_epi16(pair, one));
            }
        }
        __m256 sw = _mm256_loadu_ps(ps + g * 8);
        for (size_t r = 0; r < rows; r++) {
            __m256 s = _mm256_mul_ps(sw, _mm256_set1_ps(j->sx[(first + r) * groups + g]));
            sums[r] = _mm256_fmadd_ps(_mm256_cvtepi32_ps(acc[r]), s, sums[r]);
            if (j->poffsets) { /* int8.rs:566-571, with the code sums of int8.rs:197-199 */
                const int8_t *q = j->qx + ((first + r) * groups + g) * 64;
                int32_t total = 0;
                for (int i = 0; i < 64; i++) total += q[i];
                __m256 offset = _mm256_loadu_ps(j->poffsets + (panel * groups + g) * 8);
                const float sxs = j->sx[(first + r) * groups + g] * (float)total;
                sums[r] = _mm256_fmadd_ps(offset, _mm256_set1_ps(sxs), sums[r]);
            }
        }
    }
    for (size_t r = 0; r < rows; r++) {
        float *dst = j->y + (first + r) * j->n + panel * 8;
        float tail[8];
        _mm256_storeu_ps(tail, sums[r]);
        size_t count = j->n - panel * 8 < 8 ? j->n - panel * 8 : 8;
        memcpy(dst, tail, count * sizeof(float));
    }
}

__attribute__((target("avx2,fma"))) static void *panel_worker(void *arg) {
    struct panel_job *j = (struct panel_job *)arg;
    size_t groups = (j->k + 63) / 64;
    size_t panels = (j->n + 7) / 8;
    size_t panel_stride = groups * 512 / (j->bits == 4 ? 2 : 1);
    int buffered = j->bits == 4 && j->m >= 16; /* int8.rs:241 */
    uint8_t *expanded = buffered ? (uint8_t *)malloc(groups * 512) : NULL;
    for (;;) {
        size_t tile = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (tile >= j->tiles) break;
        size_t end = tile * 4 + 4 < panels ? tile * 4 + 4 : panels;
        for (size_t panel = tile * 4; panel < end; panel++) {
            const uint8_t *pd = j->data + panel * panel_stride;
            const float *ps = j->pscales + panel * groups * 8;
            int q4 = j->bits == 4;
            if (buffered) { /* int8.rs:446-480 project_buffered */
                for (size_t at = 0; at < groups * 512; at += 32)
                    _mm256_storeu_si256((__m256i *)(expanded + at), unpack_q4(pd + at / 2));
                pd = expanded;
                q4 = 0;
            }
            size_t full = j->m / 4 * 4; /* project_panel::<4>, int8.rs:496-522 */
            for (size_t r = 0; r < full; r += 4) panel_rows(j, pd, ps, q4, panel, r, 4);
            if (j->m > full) panel_rows(j, pd, ps, q4, panel, full, j->m - full);
        }
    }
    free(expanded);
    return NULL;
}
#endif

int or_panel_apply_avx2(const uint8_t *data, const float *pscales, const float *poffsets, size_t n, size_t k,
                        int bits, const int8_t *qx, const float *sx, size_t m, int threads, float *y) {
#if defined(__x86_64__)
    if (!or_has_avx2()) return -1;
    struct panel_job job = {data, pscales, n, k, m, bits, qx, sx, poffsets, y, (n + 31) / 32, 0};
    if (threads <= 1) {
        panel_worker(&job);
        return 0;
    }
    run_workers(panel_worker, &job, threads);
    return 0;
#else
    (void)data; (void)pscales; (void)poffsets; (void)n; (void)k; (void)bits; (void)qx; (void)sx; (void)m;
    (void)threads; (void)y;
    return -1;
#endif
}

/* ------------------------------------------------------------------------ */
/* a11/a12: per-row int8, webgpu/int8.rs                                     */
/* ------------------------------------------------------------------------ */

/* webgpu/int8.rs:115 even(): floor-based round half to even. */
static int32_t even(float v) {
    float lo = floorf(v);
    float f = v - lo;
    int32_t i = (int32_t)lo;
    return i + ((f > 0.5f || (f == 0.5f && (i & 1) == 1)) ? 1 : 0);
}

void or_i8_quantize_rows(const float *x, size_t rows, size_t k, int8_t *q, float *scales,
                         int32_t *sums) {
    for (size_t r = 0; r < rows; r++) {
        const float *row = x + r * k;
        float maximum = 0.0f;
        for (size_t j = 0; j < k; j++) maximum = fmaxf(maximum, fabsf(row[j]));
        float scale = maximum / 127.0f;
        int32_t total = 0;
        for (size_t j = 0; j < k; j++) {
            int32_t v = 0;
            if (scale > 0.0f) {
                v = even(row[j] / scale);
                if (v < -127) v = -127;
                if (v > 127) v = 127;
            }
            total += v;
            q[r * k + j] = (int8_t)v;
        }
        scales[r] = scale;
        if (sums) sums[r] = total;
    }
}

/* ------------------------------------------------------------------------ */
/* a13: per-row Q4 from f16 weights, webgpu/q4.rs:48-73 (the legacy         */
/* symmetric per-output-channel mode). Output words, as the reference's     */
/* buffer: rows*(k/8) code words (element 8j+t of a row at bits 4t of word  */
/* j, code+8), then rows f32 scales, then rows i32 code sums.               */
/* ------------------------------------------------------------------------ */

int or_q4_quantize_rows(const uint16_t *x_f16, size_t rows, size_t k, uint32_t *out) {
    if (k == 0 || k % 8 != 0 || k > 32768) return -1;
    const size_t words = k / 8;
    for (size_t r = 0; r < rows; r++) {
        const uint16_t *row = x_f16 + r * k;
        float maximum = 0.0f;
        for (size_t j = 0; j < k; j++) maximum = fmaxf(maximum, fabsf(or_f16_to_f32(row[j])));
        float scale = maximum / 7.0f;
        int32_t total = 0;
        for (size_t j = 0; j < words; j++) {
            uint32_t packed = 0;
            for (size_t t = 0; t < 8; t++) {
                int32_t q = 0;
                if (scale > 0.0f) {
                    q = even(or_f16_to_f32(row[j * 8 + t]) / scale);
                    if (q < -7) q = -7;
                    if (q > 7) q = 7;
                }
                total += q;
                packed |= (uint32_t)(q + 8) << (4 * t);
            }
            out[r * words + j] = packed;
        }
        uint32_t bits;
        memcpy(&bits, &scale, 4);
        out[rows * words + r] = bits;
        out[rows * words + rows + r] = (uint32_t)total;
    }
    return 0;
}

/* The signed codes of that buffer, [rows x k] int8 (q4.rs:81-97 expand). */
void or_q4_rows_codes(const uint32_t *words, size_t rows, size_t k, int8_t *codes) {
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < k; j++)
            codes[r * k + j] = (int8_t)((int)((words[r * (k / 8) + j / 8] >> (4 * (j % 8))) & 15u) - 8);
}

struct i8_job {
    const int8_t *qa, *qw;
    const float *sa, *sw;
    size_t m, n, k;
    int32_t *raw;
    float *y;
    size_t next;
};

static void *i8_worker(void *arg) {
    struct i8_job *j = (struct i8_job *)arg;
    for (;;) {
        size_t r = __atomic_fetch_add(&j->next, 1, __ATOMIC_RELAXED);
        if (r >= j->m) break;
        const int8_t *a = j->qa + r * j->k;
        for (size_t c = 0; c < j->n; c++) {
            const int8_t *b = j->qw + c * j->k;
            int32_t dot = 0;
            for (size_t i = 0; i < j->k; i++) dot += (int32_t)a[i] * (int32_t)b[i];
            if (j->raw) j->raw[r * j->n + c] = dot;
            if (j->y) j->y[r * j->n + c] = ((float)dot * j->sa[r]) * j->sw[c];
        }
    }
    return NULL;
}

void or_i8_gemm(const int8_t *qa, const float *sa, size_t m, const int8_t *qw, const float *sw,
                size_t n, size_t k, int threads, int32_t *raw, float *y) {
    struct i8_job job = {qa, qw, sa, sw, m, n, k, raw, y, 0};
    if (threads <= 1) {
        i8_worker(&job);
        return;
    }
    run_workers(i8_worker, &job, threads);
}

/* webgpu/int8.rs:226-230, gemm(fused=true): gate and up are two rescaled
 * per-row products of the same codes (the f32 epilogue above), and
 * y = (gate / (1 + exp(-gate))) * up in f32 operations, exp being the f32
 * rounding of the f64 exponential. */
void or_i8_gemm_fused(const int8_t *qa, const float *sa, size_t m, const int8_t *qg, const float *sg,
                      const int8_t *qu, const float *su, size_t n, size_t k, float *y) {
    for (size_t r = 0; r < m; r++) {
        const int8_t *a = qa + r * k;
        for (size_t c = 0; c < n; c++) {
            int32_t dg = 0, du = 0;
            for (size_t i = 0; i < k; i++) {
                dg += (int32_t)a[i] * (int32_t)qg[c * k + i];
                du += (int32_t)a[i] * (int32_t)qu[c * k + i];
            }
            const float gate = ((float)dg * sa[r]) * sg[c];
            const float up = ((float)du * sa[r]) * su[c];
            const float e = (float)exp(-(double)gate);
            y[r * n + c] = (gate / (1.0f + e)) * up;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* W4A16 closed form                                                         */
/* ------------------------------------------------------------------------ */

void or_w4a16(const uint16_t *x_f16, size_t m, size_t k, const float *w, size_t n, double *y) {
    double *xr = (double *)malloc(k * sizeof(double));
    for (size_t r = 0; r < m; r++) {
        for (size_t i = 0; i < k; i++) xr[i] = (double)or_f16_to_f32(x_f16[r * k + i]);
        for (size_t c = 0; c < n; c++) {
            const float *wr = w + c * k;
            double acc = 0.0;
            for (size_t i = 0; i < k; i++) acc += xr[i] * (double)wr[i];
            y[r * n + c] = acc;
        }
    }
    free(xr);
}

/* ------------------------------------------------------------------------ */
/* a14: epilogues                                                            */
/* ------------------------------------------------------------------------ */

void or_layernorm(float *x, size_t rows, size_t d, const float *w, const float *b, float eps) {
    for (size_t r = 0; r < rows; r++) {
        float *row = x + r * d;
        float sum = 0.0f;
        for (size_t i = 0; i < d; i++) sum = sum + row[i];
        float mean = sum / (float)d;
        float var = 0.0f;
        for (size_t i = 0; i < d; i++) var = var + (row[i] - mean) * (row[i] - mean);
        var = var / (float)d;
        float inv = 1.0f / sqrtf(var + eps);
        for (size_t i = 0; i < d; i++) row[i] = (row[i] - mean) * inv * w[i] + b[i];
    }
}

void or_gelu(float *x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = 0.5f * x[i] * (1.0f + erff(x[i] * 0.70710678118654752f));
}

void or_rmsnorm(const float *x, size_t rows, size_t d, const float *w, float eps, int zero_centered,
                float *y) {
    for (size_t r = 0; r < rows; r++) {
        const float *src = x + r * d;
        float ss = 0.0f;
        for (size_t i = 0; i < d; i++) ss = ss + src[i] * src[i];
        float scale = 1.0f / sqrtf(ss / (float)d + eps);
        for (size_t i = 0; i < d; i++) y[r * d + i] = (src[i] * scale) * (zero_centered ? 1.0f + w[i] : w[i]);
    }
}

static float silu(float v) { return v * (1.0f / (1.0f + expf(-v))); }

void or_silu_mul(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; i++) gate[i] = silu(gate[i]) * up[i];
}

void or_softmax(float *x, size_t n) {
    float maximum = -INFINITY;
    for (size_t i = 0; i < n; i++) maximum = fmaxf(maximum, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - maximum);
        sum = sum + x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] = x[i] / sum;
}

void or_mean_rows(const float *x, size_t rows, size_t d, float *out) {
    for (size_t i = 0; i < d; i++) out[i] = 0.0f;
    for (size_t r = 0; r < rows; r++)
        for (size_t i = 0; i < d; i++) out[i] = out[i] + x[r * d + i];
    for (size_t i = 0; i < d; i++) out[i] = out[i] / (float)rows;
}

void or_attention(const float *q, const float *k, const float *v, size_t seq, size_t heads,
                  size_t dh, float scale, float *out) {
    size_t width = heads * dh;
    double *p = (double *)malloc(seq * sizeof(double));
    for (size_t h = 0; h < heads; h++) {
        for (size_t i = 0; i < seq; i++) {
            double maximum = -INFINITY;
            for (size_t j = 0; j < seq; j++) {
                double dot = 0.0;
                for (size_t d = 0; d < dh; d++)
                    dot += (double)q[i * width + h * dh + d] * (double)k[j * width + h * dh + d];
                p[j] = dot * (double)scale;
                if (p[j] > maximum) maximum = p[j];
            }
            double sum = 0.0;
            for (size_t j = 0; j < seq; j++) {
                p[j] = exp(p[j] - maximum);
                sum += p[j];
            }
            for (size_t d = 0; d < dh; d++) {
                double acc = 0.0;
                for (size_t j = 0; j < seq; j++) acc += p[j] * (double)v[j * width + h * dh + d];
                out[i * width + h * dh + d] = (float)(acc / sum);
            }
        }
    }
    free(p);
}

void or_silu_requant(const float *gate, const float *up, size_t m, size_t n, int8_t *q, float *s) {
    size_t blocks = n / 64;
    float values[64];
    for (size_t r = 0; r < m; r++) {
        for (size_t b = 0; b < blocks; b++) {
            for (int i = 0; i < 64; i++) {
                size_t at = r * n + b * 64 + (size_t)i;
                values[i] = silu(gate[at]) * up[at];
            }
            float scale = or_group_scale(values, 64, 8);
            s[r * blocks + b] = scale;
            or_group_codes(values, 64, scale, 8, q + (r * blocks + b) * 64);
        }
    }
}

/* ---- Pplx decoder layer ops ---- */

static float sigmoidf_ref(float v) { return 1.0f / (1.0f + expf(-v)); }

void or_conv_silu(const float *x, size_t n, size_t width, const float *w, float *out) {
    for (size_t t = 0; t < n; t++)
        for (size_t c = 0; c < width; c++) {
            float sum = 0.0f;
            for (size_t tap = 0; tap < 4; tap++) {
                const long row = (long)t - 3 + (long)tap;
                const float v = row < 0 ? 0.0f : x[(size_t)row * width + c];
                sum = sum + v * w[tap * width + c];
            }
            out[t * width + c] = silu(sum);
        }
}

void or_delta_scan(const float *conv, size_t n, int lh, int lk, int ld, const float *a, const float *b,
                   const float *decay, const float *dt, float *out) {
    const size_t lkv = (size_t)lk * ld, width = 2 * lkv + (size_t)lh * ld;
    const int group = lh / lk;
    float *state = (float *)calloc((size_t)ld * ld, sizeof(float));
    float *q = (float *)malloc(ld * sizeof(float)), *k = (float *)malloc(ld * sizeof(float));
    float *memory = (float *)malloc(ld * sizeof(float)), *delta = (float *)malloc(ld * sizeof(float));
    for (int h = 0; h < lh; h++) {
        memset(state, 0, (size_t)ld * ld * sizeof(float));
        const int kh = h / group;
        for (size_t t = 0; t < n; t++) {
            const float *row = conv + t * width;
            memcpy(q, row + (size_t)kh * ld, ld * sizeof(float));
            memcpy(k, row + lkv + (size_t)kh * ld, ld * sizeof(float));
            float qs = 0.0f, ks = 0.0f;
            for (int i = 0; i < ld; i++) qs = qs + q[i] * q[i];
            for (int i = 0; i < ld; i++) ks = ks + k[i] * k[i];
            const float qi = 1.0f / sqrtf(qs + 1e-6f), ki = 1.0f / sqrtf(ks + 1e-6f);
            const float root = 1.0f / sqrtf((float)ld);
            for (int i = 0; i < ld; i++) {
                q[i] = (q[i] * qi) * root;
                k[i] = k[i] * ki;
            }
            const float x = a[t * lh + h] + dt[h];
            const float softplus = x > 20.0f ? x : log1pf(expf(x));
            const float g = expf(-decay[h] * softplus);
            const float beta = sigmoidf_ref(b[t * lh + h]);
            for (int j = 0; j < ld; j++) memory[j] = 0.0f;
            for (int i = 0; i < ld; i++)
                for (int j = 0; j < ld; j++) {
                    state[i * ld + j] = state[i * ld + j] * g;
                    memory[j] = memory[j] + state[i * ld + j] * k[i];
                }
            const float *v = row + 2 * lkv + (size_t)h * ld;
            for (int j = 0; j < ld; j++) delta[j] = (v[j] - memory[j]) * beta;
            float *dst = out + ((size_t)h * n + t) * ld;
            for (int j = 0; j < ld; j++) dst[j] = 0.0f;
            for (int i = 0; i < ld; i++)
                for (int j = 0; j < ld; j++) {
                    state[i * ld + j] = state[i * ld + j] + k[i] * delta[j];
                    dst[j] = dst[j] + state[i * ld + j] * q[i];
                }
        }
    }
    free(state);
    free(q);
    free(k);
    free(memory);
    free(delta);
}

void or_delta_gate(const float *heads, size_t n, int lh, int ld, const float *norm, const float *z,
                   float *ctx) {
    for (size_t t = 0; t < n; t++)
        for (int h = 0; h < lh; h++) {
            const float *src = heads + ((size_t)h * n + t) * ld;
            float ss = 0.0f;
            for (int i = 0; i < ld; i++) ss = ss + src[i] * src[i];
            const float scale = 1.0f / sqrtf(ss / (float)ld + 1e-6f);
            for (int i = 0; i < ld; i++) {
                const size_t at = t * (size_t)lh * ld + (size_t)h * ld + i;
                ctx[at] = ((src[i] * scale) * norm[i]) * silu(z[at]);
            }
        }
}

void or_rope(float *x, size_t rows, int heads, int ad, const size_t *pos, const float *freq) {
    for (size_t r = 0; r < rows; r++)
        for (int h = 0; h < heads; h++) {
            float *head = x + (r * heads + h) * (size_t)ad;
            for (int i = 0; i < 32; i++) {
                const float angle = (float)pos[r] * freq[i];
                const float c = cosf(angle), sn = sinf(angle);
                const float a = head[i], b = head[i + 32];
                head[i] = a * c - b * sn;
                head[i + 32] = b * c + a * sn;
            }
        }
}

typedef struct {
    const float *q, *k, *v;
    size_t nq, nk;
    int ah, akv, ad, next_head;
    float scale;
    float *out;
    pthread_mutex_t mu;
} gqa_job;

// One head of or_attention_gqa: every query row against every key, in f64.
static void gqa_head(const gqa_job *j, int h, double *p, double *acc) {
    const int kh = h / (j->ah / j->akv), ad = j->ad, ah = j->ah, akv = j->akv;
    for (size_t t = 0; t < j->nq; t++) {
        const float *qr = j->q + (t * ah + h) * (size_t)ad;
        double mx = -INFINITY;
        for (size_t s = 0; s < j->nk; s++) {
            const float *kr = j->k + (s * akv + kh) * (size_t)ad;
            double d = 0.0;
            for (int i = 0; i < ad; i++) d += (double)qr[i] * kr[i];
            p[s] = d * j->scale;
            if (p[s] > mx) mx = p[s];
        }
        double sum = 0.0;
        for (size_t s = 0; s < j->nk; s++) {
            p[s] = exp(p[s] - mx);
            sum += p[s];
        }
        // each output sums p[s] * v[s][i] over s in key order; the key loop is
        // outermost so that the value rows are read contiguously
        float *o = j->out + ((size_t)h * j->nq + t) * ad;
        for (int i = 0; i < ad; i++) acc[i] = 0.0;
        for (size_t s = 0; s < j->nk; s++) {
            const float *vr = j->v + (s * akv + kh) * (size_t)ad;
            const double ps = p[s];
            for (int i = 0; i < ad; i++) acc[i] += ps * vr[i];
        }
        for (int i = 0; i < ad; i++) o[i] = (float)(acc[i] / sum);
    }
}

static void *gqa_worker(void *arg) {
    gqa_job *j = (gqa_job *)arg;
    double *p = (double *)malloc(j->nk * sizeof(double));
    double *acc = (double *)malloc((size_t)j->ad * sizeof(double));
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int h = j->next_head++;
        pthread_mutex_unlock(&j->mu);
        if (h >= j->ah) break;
        gqa_head(j, h, p, acc);
    }
    free(acc);
    free(p);
    return NULL;
}

// Heads are independent, so they run on up to 16 threads; each head's
// arithmetic does not depend on the thread count.
void or_attention_gqa(const float *q, const float *k, const float *v, size_t nq, size_t nk, int ah, int akv,
                      int ad, float scale, float *out) {
    gqa_job job = {q, k, v, nq, nk, ah, akv, ad, 0, scale, out, PTHREAD_MUTEX_INITIALIZER};
    long cpus = sysconf(_SC_NPROCESSORS_ONLN);
    int threads = cpus < 1 ? 1 : (cpus > 16 ? 16 : (int)cpus);
    if (threads > ah) threads = ah;
    run_workers(gqa_worker, &job, threads);
}

void or_attention_gate(const float *heads, size_t n, int ah, int ad, const float *z, float *out) {
    for (size_t t = 0; t < n; t++)
        for (int h = 0; h < ah; h++)
            for (int i = 0; i < ad; i++) {
                const size_t at = t * (size_t)ah * ad + (size_t)h * ad + i;
                out[at] = heads[((size_t)h * n + t) * ad + i] * sigmoidf_ref(z[at]);
            }
}
