// products.hip -- quantized matrix products on CDNA4 matrix cores.
//
//  grouped   : W{4,8}A{8,4}, the reference's numeric mode. One
//              v_mfma_i32_16x16x64_i8 per 64-run gives the exact int32 group
//              dot; outputs fold groups in order with
//              acc = fma(f32(dot), sw*sx, acc), the AVX2 rows<R,Q4> order of
//              src/models/pplx_flash/int8.rs:524-585, so results are bit-exact.
//  gemv      : W4A16 for M <= 16 rows, HBM bound. Each lane streams one 128-bit
//              word of packed codes per 128-k block; codes become exact f16 and
//              feed v_mfma_f32_16x16x32_f16; per-32-run scales are applied to the
//              f32 partials. K is split into 16 fixed chunks reduced in order, so
//              every variant is bitwise equal.
//  gemm      : W4A16 for large M, MFMA bound. The activation tile is staged in
//              LDS; each wave dequantizes its weight fragments (code * scale in
//              f16) straight from HBM and accumulates in f32.
//  i8_gemm   : per-row int8 (webgpu/int8.rs:147-242): exact int32 dots on
//              v_mfma_i32_16x16x64_i8, epilogue (f32(dot)*sa)*sw.
#include <float.h>

#include <algorithm>
#include <type_traits>

#include "kernels.hpp"

namespace dz {

namespace {

__device__ __forceinline__ size_t q4_lane(int t, int kb, int kbs, int q, int j) {
    return ((((size_t)t * kbs + kb) * 64) + q * 16 + j) * 16;
}

// ============================================================================
// grouped W{4,8}A{8,4}
// ============================================================================

// One wave per 16x16 output tile; a block of 4 waves covers 64 columns.
// AFF (fitted affine Q4, int8.rs:566-571): after each group's fold,
// acc = fma(offset[c][g], sxq[r][g], acc), sxq = sx * f32(sum of the codes).
template <int BITS, bool AFF = false>
__global__ __launch_bounds__(256) void grouped_kernel(const uint8_t *__restrict__ codes,
                                                      const uint8_t *__restrict__ scales,
                                                      const int8_t *__restrict__ q,
                                                      const float *__restrict__ sx, int m, int n,
                                                      int groups, int kbs, float *__restrict__ y,
                                                      const int *__restrict__ bad,
                                                      const uint8_t *__restrict__ offsets = nullptr,
                                                      const float *__restrict__ sxq = nullptr) {
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int t = blockIdx.x * 4 + wave;
    const int mt = blockIdx.y;
    if (t * 16 >= n) return;
    const int qd = lane / 16, i = lane % 16, j = i;
    const int arow = mt * 16 + i;
    const bool arow_ok = arow < m;
    const bool nan_out = bad != nullptr && *bad != 0;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    const int4_t zero = {0, 0, 0, 0};
    const int8_t *qrow = q + (size_t)arow * groups * 64;
    // Groups go in batches of B; batch i+1's loads are issued before batch i's
    // products and folds, so each wait covers B groups. The fold stays in
    // group order.
    constexpr int B = 4;
    struct Batch {
        int4_t a[B], b[B];
        float sw[B], sx[B][4];
        float ofs[AFF ? B : 1], sq[AFF ? B : 1][4];
    };
    auto fetch = [&](Batch &bt, int g0) {
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int g = min(g0 + u, groups - 1);  // past the end: a valid group, never folded
            int4_t a = zero, b;
            float sw;
            if (BITS == 4) {
                const int kb = g >> 1, s0 = (g & 1) * 2;
                uint2_t wds = *(const uint2_t *)(codes + q4_lane(t, kb, kbs, qd, j) + s0 * 4);
                b = q4_operand16(wds[0], wds[1]);
                if (arow_ok) {
                    uint2_t a0 = *(const uint2_t *)(qrow + g * 64 + qd * 8);
                    uint2_t a1 = *(const uint2_t *)(qrow + g * 64 + 32 + qd * 8);
                    a = int4_t{(int)a0[0], (int)a0[1], (int)a1[0], (int)a1[1]};
                }
                sw = ((const float *)(scales + (((size_t)t * kbs + kb) * 16 + j) * 8))[g & 1];
            } else {
                b = *(const int4_t *)(codes + q4_lane(t, g, kbs, qd, j));
                if (arow_ok) a = *(const int4_t *)(qrow + g * 64 + qd * 16);
                sw = ((const float *)scales)[((size_t)t * kbs + g) * 16 + j];
            }
            bt.a[u] = a;
            bt.b[u] = b;
            bt.sw[u] = sw;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = mt * 16 + qd * 4 + v;
                bt.sx[u][v] = r < m ? sx[(size_t)r * groups + g] : 0.0f;
            }
            if (AFF) {  // Q4 only: offsets share the group-64 scale layout
                bt.ofs[u] = ((const float *)(offsets + (((size_t)t * kbs + (g >> 1)) * 16 + j) * 8))[g & 1];
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = mt * 16 + qd * 4 + v;
                    bt.sq[u][v] = r < m ? sxq[(size_t)r * groups + g] : 0.0f;
                }
            }
        }
    };
    auto fold = [&](const Batch &bt, int g0) {
#pragma unroll
        for (int u = 0; u < B; u++) {
            if (g0 + u >= groups) break;
            const int4_t d = mfma_dot<BITS>(bt.a[u], bt.b[u]);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                acc[v] = __builtin_fmaf(dot_of<BITS>(d[v]), __fmul_rn(bt.sw[u], bt.sx[u][v]), acc[v]);
                if (AFF) acc[v] = __builtin_fmaf(bt.ofs[AFF ? u : 0], bt.sq[AFF ? u : 0][v], acc[v]);
            }
        }
    };
    if (!nan_out) {
        Batch x0, x1;
        fetch(x0, 0);
        for (int g0 = 0; g0 < groups; g0 += 2 * B) {
            if (g0 + B < groups) fetch(x1, g0 + B);
            fold(x0, g0);
            if (g0 + B >= groups) break;
            if (g0 + 2 * B < groups) fetch(x0, g0 + 2 * B);
            fold(x1, g0 + B);
        }
    }
    const int col = t * 16 + j;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        int r = mt * 16 + qd * 4 + v;
        if (r < m && col < n) y[(size_t)r * n + col] = nan_out ? __builtin_nanf("") : acc[v];
    }
}

// ============================================================================
// grouped W{4,8}A{8,4}, few rows (M <= 16 per block row)
// ============================================================================
//
// One block per 16-column tile. The 64-groups are taken in windows of
// kGvWindow; in a window each of the kGvWaves waves owns kGvSub consecutive
// groups: it loads their weight codes, weight scales and activation codes
// (or f32 activations, quantized here with the a4 formula), takes each
// group's exact int32 dot with one v_mfma_i32_16x16x64_i8 and leaves it in
// LDS. After a barrier, lane (r, c) folds the window's groups into its output
// in group order, so the result is the reference's fold whatever the split:
//   fused   acc = fma(f32(dot), sw*sx, acc)        int8.rs:524-585 (AVX2 rows)
//   project acc = acc + f32(dot) * (sx*sw)          packed.rs:102-116
// Activation sources (AMODE): 0 f32 x quantized in the kernel (every block
// sees all of x, so a non-finite value anywhere makes every output NaN, as
// int8.rs:170-173 requires); 1 int8 codes + f32 scales (the dz_act_quantize
// layout); 2 the 17-word records of grouped_q4.rs:3-25.

constexpr int kGvWaves = 16;
constexpr int kGvSub = 4;
constexpr int kGvWindow = kGvWaves * kGvSub;

template <int MPAD, bool AFF = false>
struct GvShape {
    static constexpr int ASTRIDE = kGvSub * 64 + 16;           // staged codes per row (+ pad)
    static constexpr int ACODE = MPAD * ASTRIDE;                // per wave
    static constexpr int ACODE_ALL = kGvWaves * ACODE;
    static constexpr int ASX = MPAD * kGvWindow * 4;            // activation scales of a window
    static constexpr int SW = kGvWindow * 16 * 4;               // weight scales of a window
    static constexpr int DOTS = kGvWindow * MPAD * 16 * 4;      // int32 group dots of a window
    static constexpr int AFFB = AFF ? ASX + SW : 0;             // sx * sum q and the offsets of a window
    static constexpr int BYTES = ACODE_ALL + ASX + SW + DOTS + 16 + AFFB;
};

// AFF (fitted affine Q4 weights, AMODE 0): each group's fold is followed by
// acc = fma(offset, sx * f32(sum of the row's group codes), acc), the term
// int8.rs:566-571 adds; the code sums come from the quantization here.
template <int BITS, int MPAD, int AMODE, bool PROJECT, bool AFF = false>
__global__ __launch_bounds__(kGvWaves * 64) void grouped_gemv_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, const void *__restrict__ a,
    const float *__restrict__ sa, int m, int k, int n, int groups, int kbs, int abits,
    float *y, const int *__restrict__ bad_in, int *__restrict__ bad_out,
    const uint8_t *__restrict__ offsets = nullptr, const float *res = nullptr) {
    static_assert(!AFF || (AMODE == 0 && !PROJECT && BITS == 4), "affine offsets: Q4 weights, f32 activations");
    // Q4 codes as the 16 * code operand (q4_operand16) where it keeps the
    // kernel within 64 VGPRs (8 waves per SIMD); from MPAD 4 its extra
    // register costs a wave per SIMD (M = 4: 10.4 against 13.6 us at
    // K = 2560, N = 9216), so the plain codes go in there. Same dots either way.
    constexpr bool X16 = BITS == 4 && MPAD <= 2;
    using S = GvShape<MPAD, AFF>;
    extern __shared__ __align__(16) uint8_t lds[];
    float *asx = (float *)(lds + S::ACODE_ALL);
    float *sw = (float *)(lds + S::ACODE_ALL + S::ASX);
    int32_t *dots = (int32_t *)(lds + S::ACODE_ALL + S::ASX + S::SW);
    int *flag = (int *)(lds + S::ACODE_ALL + S::ASX + S::SW + S::DOTS);
    float *asq = (float *)(lds + S::ACODE_ALL + S::ASX + S::SW + S::DOTS + 16);  // AFF only
    float *ofs = asq + MPAD * kGvWindow;                                         // AFF only
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int t = blockIdx.x, row0 = blockIdx.y * 16;
    const int qd = lane / 16, i = lane % 16, j = i;
    uint8_t *acode = lds + wave * S::ACODE;
    const int fr = threadIdx.x / 16, fc = threadIdx.x % 16;  // fold lane -> output (row, column)
    const bool folds = threadIdx.x < MPAD * 16;
    const float limit = abits == 4 ? 7.0f : 127.0f;
    if (threadIdx.x == 0) *flag = (bad_in != nullptr && *bad_in != 0) ? 1 : 0;
    float acc = 0.0f;
    __syncthreads();

    for (int w0 = 0; w0 < groups; w0 += kGvWindow) {
        const int g0 = w0 + wave * kGvSub;
        // ---- weight codes: Q4 one 16-byte lane word per k-block (two groups), Q8 one per group
        constexpr int BLOADS = BITS == 4 ? kGvSub / 2 : kGvSub;
        uint4_t bq[BLOADS];
#pragma unroll
        for (int u = 0; u < BLOADS; u++) {
            int blk = BITS == 4 ? g0 / 2 + u : g0 + u;
            blk = blk < kbs ? blk : 0;  // past the end: a valid block whose dots are never folded
            bq[u] = *(const uint4_t *)(codes + q4_lane(t, blk, kbs, qd, j));
        }
        // ---- weight scales of the wave's groups: 256 contiguous bytes, 16 lanes x 16 B
        uint4_t swv = {0u, 0u, 0u, 0u}, ofv = {0u, 0u, 0u, 0u};
        const int first_blk = BITS == 4 ? g0 / 2 : g0;
        const int blk_of_lane = BITS == 4 ? first_blk + lane / 8 : first_blk + lane / 4;
        if (lane < 16 && blk_of_lane < kbs) swv = *(const uint4_t *)(scales + ((size_t)t * kbs + first_blk) * (BITS == 4 ? 128 : 64) + lane * 16);
        if (AFF && lane < 16 && blk_of_lane < kbs) ofv = *(const uint4_t *)(offsets + ((size_t)t * kbs + first_blk) * 128 + lane * 16);
        // ---- activation codes and scales
        if (AMODE == 0) {
            const float *x = (const float *)a;
            float4_t xv[MPAD];
#pragma unroll
            for (int r = 0; r < MPAD; r++) {
                const int row = row0 + r, g = g0 + lane / 16, kk = g * 64 + (lane % 16) * 4;
                float4_t v = {0.f, 0.f, 0.f, 0.f};
                if (row < m && g < groups) {
                    const float *p = x + (size_t)row * k + kk;
                    if ((k & 3) == 0 && kk + 4 <= k) {
                        v = *(const float4_t *)p;
                    } else {
                        for (int e = 0; e < 4; e++) v[e] = kk + e < k ? p[e] : 0.0f;
                    }
                }
                xv[r] = v;
            }
#pragma unroll
            for (int r = 0; r < MPAD; r++) {
                float maximum = 0.0f;
                bool finite = true;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    finite = finite && __builtin_isfinite(xv[r][e]);
                    maximum = fmaxf(maximum, fabsf(xv[r][e]));
                }
                for (int off = 8; off > 0; off >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off, 16));
                if (!finite) atomicOr(flag, 1);
                const float scale = fmaxf(__fdiv_rn(maximum, limit), FLT_MIN);
                const float inverse = __frcp_rn(scale);
                uint32_t word = 0;
                int qsum = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float q = fminf(fmaxf(__builtin_rintf(__fmul_rn(xv[r][e], inverse)), -limit), limit);
                    word |= ((uint32_t)(uint8_t)(int8_t)(int)q) << (8 * e);
                    qsum += (int)q;
                }
                *(uint32_t *)(acode + r * S::ASTRIDE + (lane / 16) * 64 + (lane % 16) * 4) = word;
                if (lane % 16 == 0) asx[r * kGvWindow + (g0 - w0) + lane / 16] = scale;
                if (AFF) {
                    for (int off = 8; off > 0; off >>= 1) qsum += __shfl_xor(qsum, off, 16);
                    if (lane % 16 == 0) asq[r * kGvWindow + (g0 - w0) + lane / 16] = __fmul_rn(scale, (float)qsum);
                }
            }
        } else if (AMODE == 1) {
            const int8_t *q = (const int8_t *)a;
            constexpr int UNITS = MPAD * 16;  // 16-byte units: row, group, quarter
#pragma unroll
            for (int L = 0; L < (UNITS + 63) / 64; L++) {
                const int u = L * 64 + lane;
                const int r = u / 16, gg = (u % 16) / 4, part = u % 4, row = row0 + r, g = g0 + gg;
                uint4_t v = {0u, 0u, 0u, 0u};
                if (u < UNITS && row < m && g < groups) v = *(const uint4_t *)(q + ((size_t)row * groups + g) * 64 + part * 16);
                if (u < UNITS) *(uint4_t *)(acode + r * S::ASTRIDE + gg * 64 + part * 16) = v;
            }
            if (lane < MPAD * kGvSub) {
                const int r = lane / kGvSub, gg = lane % kGvSub, row = row0 + r, g = g0 + gg;
                asx[r * kGvWindow + (g0 - w0) + gg] = (row < m && g < groups) ? sa[(size_t)row * groups + g] : 0.0f;
            }
        } else {
            const uint32_t *rec = (const uint32_t *)a;
            constexpr int WORDS = MPAD * kGvSub * 17;
#pragma unroll
            for (int L = 0; L < (WORDS + 63) / 64; L++) {
                const int u = L * 64 + lane;
                const int r = u / (kGvSub * 17), gg = (u / 17) % kGvSub, wd = u % 17, row = row0 + r, g = g0 + gg;
                uint32_t v = 0u;
                if (u < WORDS && row < m && g < groups) v = rec[((size_t)row * groups + g) * 17 + wd];
                if (u < WORDS) {
                    if (wd < 16) *(uint32_t *)(acode + r * S::ASTRIDE + gg * 64 + wd * 4) = v;
                    else asx[r * kGvWindow + (g0 - w0) + gg] = __builtin_bit_cast(float, v);
                }
            }
        }
        // weight scales to LDS as sw[group in window][column]
        if (lane < 16) {
            if (BITS == 4) {
                // record (kb, column) holds the f32 scales of groups 2kb and 2kb+1
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int col = (lane % 8) * 2 + h;
                    const int gl = g0 - w0 + (lane / 8) * 2;
                    sw[gl * 16 + col] = word_as_float(swv[h * 2]);
                    sw[(gl + 1) * 16 + col] = word_as_float(swv[h * 2 + 1]);
                    if (AFF) {
                        ofs[gl * 16 + col] = word_as_float(ofv[h * 2]);
                        ofs[(gl + 1) * 16 + col] = word_as_float(ofv[h * 2 + 1]);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) sw[(g0 - w0 + lane / 4) * 16 + (lane % 4) * 4 + e] = word_as_float(swv[e]);
            }
        }
        // ---- exact group dots
#pragma unroll
        for (int gg = 0; gg < kGvSub; gg++) {
            if (g0 + gg >= groups) break;
            int4_t av = {0, 0, 0, 0}, bv;
            if (BITS == 4) {
                const uint4_t w = bq[gg / 2];
                if (X16) {
                    bv = q4_operand16(w[(gg % 2) * 2], w[(gg % 2) * 2 + 1]);
                } else {
                    const uint2_t lo = nibbles_to_i8(w[(gg % 2) * 2]), hi = nibbles_to_i8(w[(gg % 2) * 2 + 1]);
                    bv = int4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
                }
                if (i < MPAD) {
                    const uint2_t a0 = *(const uint2_t *)(acode + i * S::ASTRIDE + gg * 64 + qd * 8);
                    const uint2_t a1 = *(const uint2_t *)(acode + i * S::ASTRIDE + gg * 64 + 32 + qd * 8);
                    av = int4_t{(int)a0[0], (int)a0[1], (int)a1[0], (int)a1[1]};
                }
            } else {
                bv = __builtin_bit_cast(int4_t, bq[gg]);
                if (i < MPAD) av = *(const int4_t *)(acode + i * S::ASTRIDE + gg * 64 + qd * 16);
            }
            const int4_t d = X16 ? mfma_i8_biased16(av, bv) : mfma_i8_biased(av, bv);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = qd * 4 + v;
                if (r < MPAD) dots[((g0 - w0 + gg) * MPAD + r) * 16 + j] = d[v];
            }
        }
        __syncthreads();
        if (folds) {
            const int end = min(groups - w0, kGvWindow);
            for (int gw = 0; gw < end; gw++) {
                const int32_t biased = dots[(gw * MPAD + fr) * 16 + fc];
                const float dot = X16 ? dot_value16(biased) : dot_value(biased);
                const float sxv = asx[fr * kGvWindow + gw], swv2 = sw[gw * 16 + fc];
                if (PROJECT)
                    acc = __fadd_rn(acc, __fmul_rn(dot, __fmul_rn(sxv, swv2)));
                else
                    acc = __builtin_fmaf(dot, __fmul_rn(swv2, sxv), acc);
                if (AFF) acc = __builtin_fmaf(ofs[gw * 16 + fc], asq[fr * kGvWindow + gw], acc);
            }
        }
        __syncthreads();
    }
    const bool nan_out = *flag != 0;
    if (nan_out && bad_out != nullptr && threadIdx.x == 0) atomicOr(bad_out, 1);
    if (folds) {
        // with `res` (which may be y itself) res + Y, the same float add as a separate residual pass
        const int row = row0 + fr, col = t * 16 + fc;
        const size_t at = (size_t)row * n + col;
        if (row < m && col < n) y[at] = nan_out ? __builtin_nanf("") : res ? __fadd_rn(res[at], acc) : acc;
    }
}

// Fused gate/up + SiLU + A8 requantization (grouped_q4_mlp.wgsl:78-105): a
// block is 16 rows x one 64-column block; the four waves hold 16 columns each.
__global__ __launch_bounds__(256) void mlp_requant_kernel(
    const uint8_t *__restrict__ gcodes, const uint8_t *__restrict__ gscales,
    const uint8_t *__restrict__ ucodes, const uint8_t *__restrict__ uscales,
    const int8_t *__restrict__ q, const float *__restrict__ sx, int m, int n, int groups, int kbs,
    int8_t *__restrict__ qo, float *__restrict__ so, const int *__restrict__ bad) {
    __shared__ float rmax[4][16];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int t = blockIdx.x * 4 + wave;
    const int mt = blockIdx.y;
    const int qd = lane / 16, i = lane % 16, j = i;
    const int arow = mt * 16 + i;
    const bool arow_ok = arow < m;
    const bool nan_out = bad != nullptr && *bad != 0;
    float4_t ga = {0.f, 0.f, 0.f, 0.f}, ua = {0.f, 0.f, 0.f, 0.f};
    const int4_t zero = {0, 0, 0, 0};
    const int8_t *qrow = q + (size_t)arow * groups * 64;
    for (int g = 0; g < groups; g++) {
        const int kb = g >> 1, s0 = (g & 1) * 2;
        int4_t a = zero;
        if (arow_ok) {
            uint2_t a0 = *(const uint2_t *)(qrow + g * 64 + qd * 8);
            uint2_t a1 = *(const uint2_t *)(qrow + g * 64 + 32 + qd * 8);
            a = int4_t{(int)a0[0], (int)a0[1], (int)a1[0], (int)a1[1]};
        }
        uint2_t gw = *(const uint2_t *)(gcodes + q4_lane(t, kb, kbs, qd, j) + s0 * 4);
        uint2_t uw = *(const uint2_t *)(ucodes + q4_lane(t, kb, kbs, qd, j) + s0 * 4);
        const int4_t gb = q4_operand16(gw[0], gw[1]), ub = q4_operand16(uw[0], uw[1]);
        const int4_t gd = mfma_i8_biased16(a, gb), ud = mfma_i8_biased16(a, ub);
        size_t rec = (((size_t)t * kbs + kb) * 16 + j) * 8;
        float gs = ((const float *)(gscales + rec))[g & 1];
        float us = ((const float *)(uscales + rec))[g & 1];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            int r = mt * 16 + qd * 4 + v;
            float sxv = r < m ? sx[(size_t)r * groups + g] : 0.0f;
            ga[v] = __builtin_fmaf(dot_value16(gd[v]), __fmul_rn(gs, sxv), ga[v]);
            ua[v] = __builtin_fmaf(dot_value16(ud[v]), __fmul_rn(us, sxv), ua[v]);
        }
    }
    float4_t val;
    float local[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
        float gv = ga[v];
        float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gv)));
        val[v] = __fmul_rn(__fmul_rn(gv, sig), ua[v]);
        local[v] = fabsf(val[v]);
    }
    // row maxima over the 16 columns of this wave (lanes with equal qd)
#pragma unroll
    for (int v = 0; v < 4; v++)
        for (int off = 8; off > 0; off >>= 1) local[v] = fmaxf(local[v], __shfl_xor(local[v], off, 16));
    if (j == 0)
        for (int v = 0; v < 4; v++) rmax[wave][qd * 4 + v] = local[v];
    __syncthreads();
    const int col = t * 16 + j;
    const int blocks = n / 64;
#pragma unroll
    for (int v = 0; v < 4; v++) {
        int rr = qd * 4 + v;
        int r = mt * 16 + rr;
        float maximum = fmaxf(fmaxf(rmax[0][rr], rmax[1][rr]), fmaxf(rmax[2][rr], rmax[3][rr]));
        float scale = fmaxf(__fdiv_rn(maximum, 127.0f), FLT_MIN);
        float inverse = __frcp_rn(scale);
        float c = fminf(fmaxf(__builtin_rintf(__fmul_rn(val[v], inverse)), -127.0f), 127.0f);
        if (r < m) {
            if (nan_out) {
                qo[(size_t)r * n + col] = 0;
                if (wave == 0 && j == 0) so[(size_t)r * blocks + blockIdx.x] = __builtin_nanf("");
            } else {
                qo[(size_t)r * n + col] = (int8_t)(int)c;
                if (wave == 0 && j == 0) so[(size_t)r * blocks + blockIdx.x] = scale;
            }
        }
    }
}

// ============================================================================
// W4A16 skinny-M GEMV
// ============================================================================
//
// HBM bound: a launch is one pass over the packed weight, so its time is the
// load latency plus whatever runs after the last bytes land. The kernel is
// shaped so that every load of a wave is in flight at once and little work
// follows them:
//  - one block per 16-row tile; K is split into kGemvChunks fixed chunks,
//    chunk c holding the k-blocks c, c + 16, c + 32, ... (interleaved: the
//    16 waves' first loads then cover 16 adjacent KiB of the tile, which
//    streams faster than each wave reading adjacent k-blocks); a wave owns PW
//    chunks and takes their k-blocks two at a time ("pairs");
//  - a round issues every load of up to NP pairs before using any: per pair
//    ONE full-width staging load for the activation rows and the two scale
//    records, then one 16-byte code load per k-block, each in a straight line
//    with no branch or select between them (out-of-range lanes read a zero page
//    or a clamped valid block), so the compiler waits for each load just before
//    its first use;
//  - codes become exact f16 with 9 VALU ops per 8 codes (v_and_or with the
//    1024 exponent, one shift per word, packed add/fma to remove the bias);
//    the MFMAs of a pair are issued back to back and their scale FMAs after
//    them. Every lane reads an activation row for the MFMA (row i % MPAD):
//    rows >= MPAD only feed output rows that are never stored;
//  - only the MFMA output rows that hold live activation rows get the scale
//    FMA; chunk partials are summed in chunk order by wave 0.
// Every output is  sum_c ( sum_{kb in c, ascending} sum_s fma(p_s, scale_s, .) ),
// chunks added in order, whatever WAVES, MPAD or NP is, so all variants and row
// counts give the same bits.

constexpr int kGemvChunks = 16;

// Read by staged lanes whose unit lies outside the activations or scales.
__device__ __align__(16) uint4_t g_zero_unit[1];

__device__ __forceinline__ uint32_t and_or(uint32_t v, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(bits));
    return r;
}

// 8 (code + 8) nibbles in the tile16x128 order -> 8 exact f16 codes.
// Pairs at bits (0,16) and (8,24) give 1024 + nib; pairs at (4,20), (12,28)
// give 1024 + 16*nib, turned into nib - 8 by one exact fma (x/16 - 72).
__device__ __forceinline__ uint4_t unpack_codes(uint32_t w, uint32_t magic) {
    const half2_t bias = {(half_t)-1032.0f, (half_t)-1032.0f};
    const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
    const half2_t bias16 = {(half_t)-72.0f, (half_t)-72.0f};
    const uint32_t w8 = w >> 8;
    uint4_t out;
    out[0] = half2_as_word(word_as_half2(and_or(w, 0x000F000Fu, magic)) + bias);
    out[1] = half2_as_word(__builtin_elementwise_fma(word_as_half2(and_or(w, 0x00F000F0u, magic)), sixteenth, bias16));
    out[2] = half2_as_word(word_as_half2(and_or(w8, 0x000F000Fu, magic)) + bias);
    out[3] = half2_as_word(__builtin_elementwise_fma(word_as_half2(and_or(w8, 0x00F000F0u, magic)), sixteenth, bias16));
    return out;
}

template <int MPAD>
struct GemvShape {
    static constexpr int LIVE = MPAD < 4 ? MPAD : 4;     // MFMA output rows per lane that are live
    static constexpr int XROW = 512 + 16;                // staged activation row: 256 f16 + pad
    static constexpr int SLICE = MPAD * XROW + 256;      // per wave: rows, then 2 scale records
    static constexpr int UNITS = MPAD * 32 + 16;         // 16-byte units staged per pair
    static constexpr int LOADS = (UNITS + 63) / 64;
    static constexpr int NPMAX = MPAD >= 16 ? 1 : (MPAD >= 8 ? 2 : 4);  // pairs per round (staging VGPRs)
};

template <int WAVES, int MPAD, bool G32, int NP>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(const uint8_t *__restrict__ codes,
                                                          const uint8_t *__restrict__ scales,
                                                          const half_t *__restrict__ x, int m,
                                                          int k, int n, int kbs,
                                                          float *__restrict__ y) {
    using S = GemvShape<MPAD>;
    constexpr int PW = kGemvChunks / WAVES;
    constexpr int C = kGemvChunks;
    extern __shared__ __align__(16) uint8_t lds[];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int t = blockIdx.x;
    const int qd = lane / 16, i = lane % 16, j = i;
    uint8_t *slice = lds + wave * S::SLICE;
    const uint8_t *cbase = codes + q4_lane(t, 0, kbs, qd, j);
    const uint8_t *arow = slice + (i % MPAD) * S::XROW + qd * 16;
    const uint32_t magic = 0x64006400u;
    const float4_t fz = {0.f, 0.f, 0.f, 0.f};
    float part[PW][S::LIVE];
#pragma unroll
    for (int cc = 0; cc < PW; cc++) {
        const int chunk = wave * PW + cc;
        const int count = chunk < kbs ? (kbs - chunk + C - 1) / C : 0;  // k-blocks of the chunk
        float acc[S::LIVE];
#pragma unroll
        for (int v = 0; v < S::LIVE; v++) acc[v] = 0.0f;
        for (int p0 = 0; 2 * p0 < count; p0 += NP) {
            uint4_t st[NP][S::LOADS], cw[NP][2];
            // pair q holds k-blocks chunk + (2q)C and chunk + (2q+1)C; a k-block past K
            // reads k-block `chunk` (valid) with zero activations and scales: it adds 0
#pragma unroll
            for (int q = 0; q < NP; q++) {
#pragma unroll
                for (int L = 0; L < S::LOADS; L++) {
                    const int u = L * 64 + lane;
                    const uint8_t *p = (const uint8_t *)g_zero_unit;
                    if (u < MPAD * 32) {
                        const int r = u / 32, kbu = chunk + (2 * (p0 + q) + (u % 32) / 16) * C;
                        const int kk = kbu * 128 + (u % 16) * 8;
                        if (r < m && kbu < kbs && kk < k) p = (const uint8_t *)(x + (size_t)r * k + kk);
                    } else if (u < S::UNITS) {
                        const int v = u - MPAD * 32, kbq = chunk + (2 * (p0 + q) + v / 8) * C;
                        if (kbq < kbs) p = scales + ((size_t)t * kbs + kbq) * 128 + (v % 8) * 16;
                    }
                    st[q][L] = *(const uint4_t *)p;
                }
                __builtin_amdgcn_sched_barrier(0);  // the staging load leaves first: it is used first
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int kb = chunk + (2 * (p0 + q) + h) * C;
                    cw[q][h] = __builtin_nontemporal_load((const uint4_t *)(cbase + (size_t)(kb < kbs ? kb : chunk) * 1024));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int q = 0; q < NP; q++) {
                if (2 * (p0 + q) >= count) break;
                // the previous pair's LDS reads completed before its MFMAs: the slice is free
#pragma unroll
                for (int L = 0; L < S::LOADS; L++) {
                    const int u = L * 64 + lane;
                    if (u < MPAD * 32) *(uint4_t *)(slice + (u / 32) * S::XROW + (u % 32) * 16) = st[q][L];
                    else if (u < S::UNITS) *(uint4_t *)(slice + MPAD * S::XROW + (u - MPAD * 32) * 16) = st[q][L];
                }
                // One k-block's four MFMAs at a time where four output rows are live
                // (fewer registers, more resident waves); both k-blocks' eight back to
                // back otherwise. The scale FMAs run in the same order either way.
                constexpr int HB = S::LIVE >= 4 ? 1 : 2;
#pragma unroll
                for (int h0 = 0; h0 < 2; h0 += HB) {
                    half8_t a[HB][4];
                    uint2_t sc[HB];
#pragma unroll
                    for (int hh = 0; hh < HB; hh++) {
                        const int h = h0 + hh;
                        sc[hh] = *(const uint2_t *)(slice + MPAD * S::XROW + h * 128 + j * 8);
#pragma unroll
                        for (int s = 0; s < 4; s++) a[hh][s] = *(const half8_t *)(arow + (h * 128 + s * 32) * 2);
                    }
                    float4_t pr[HB][4];
#pragma unroll
                    for (int hh = 0; hh < HB; hh++)
#pragma unroll
                        for (int s = 0; s < 4; s++)
                            pr[hh][s] = mfma_f16(a[hh][s], as_half8(unpack_codes(cw[q][h0 + hh][s], magic)), fz);
                    // Every register of every MFMA result stays allocated until here. Left
                    // to itself the compiler hands the registers of the unused result rows
                    // to the next unpack while the MFMA is still writing them.
#pragma unroll
                    for (int hh = 0; hh < HB; hh++)
#pragma unroll
                        for (int s = 0; s < 4; s++) asm volatile("" : "+v"(pr[hh][s]));
#pragma unroll
                    for (int hh = 0; hh < HB; hh++)
#pragma unroll
                        for (int s = 0; s < 4; s++) {
                            float scale;
                            if (G32)
                                scale = f16_bits_to_float((sc[hh][s >> 1] >> (16 * (s & 1))) & 0xffffu);
                            else
                                scale = word_as_float(sc[hh][s >> 1]);
#pragma unroll
                            for (int v = 0; v < S::LIVE; v++) acc[v] = __builtin_fmaf(pr[hh][s][v], scale, acc[v]);
                        }
                }
            }
        }
#pragma unroll
        for (int v = 0; v < S::LIVE; v++) part[cc][v] = acc[v];
    }
    // chunk partials replace the wave's staged data (each wave only reuses its own slice)
    float *mine = (float *)slice;
#pragma unroll
    for (int cc = 0; cc < PW; cc++)
#pragma unroll
        for (int v = 0; v < S::LIVE; v++) mine[(cc * S::LIVE + v) * 64 + lane] = part[cc][v];
    __syncthreads();
    if (wave != 0 || qd * 4 >= MPAD) return;
    float total[S::LIVE];
#pragma unroll
    for (int c = 0; c < kGemvChunks; c++) {
        const float *src = (const float *)(lds + (c / PW) * S::SLICE) + (c % PW) * S::LIVE * 64;
#pragma unroll
        for (int v = 0; v < S::LIVE; v++) total[v] = c == 0 ? src[v * 64 + lane] : __fadd_rn(total[v], src[v * 64 + lane]);
    }
    const int col = t * 16 + j;
#pragma unroll
    for (int v = 0; v < S::LIVE; v++) {
        const int r = qd * 4 + v;
        if (r < m && col < n) y[(size_t)r * n + col] = total[v];
    }
}

// Persistent form of gemv_kernel<16, MPAD, G32, 1> for weights whose chunks
// hold at most one k-block pair (K <= 4096): one block per compute unit,
// block b taking tiles b, b + gridDim.x, ... The activation rows are staged
// once. A wave issues the next tile's loads (the staging load of its scale
// records and its two code loads) as soon as this tile's MFMAs and scale FMAs
// are done with their operands, so every wave keeps its loads in flight
// through the chunk reduction and the barrier instead of ending and handing
// the unit to a new block. The chunk partials go to an LDS area of
// their own, double-buffered by tile parity, so one barrier per tile orders
// them. The arithmetic is gemv_kernel's, so the outputs are bitwise equal.
template <int MPAD, bool G32>
__global__ __launch_bounds__(kGemvChunks * 64) void gemv_persist_kernel(const uint8_t *__restrict__ codes,
                                                                        const uint8_t *__restrict__ scales,
                                                                        const half_t *__restrict__ x, int m,
                                                                        int k, int n, int kbs,
                                                                        float *__restrict__ y) {
    using S = GemvShape<MPAD>;
    constexpr int C = kGemvChunks, LIVE = S::LIVE;
    extern __shared__ __align__(16) uint8_t lds[];
    float *const partials = (float *)(lds + C * S::SLICE);  // [2][C][LIVE][64]
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int qd = lane / 16, i = lane % 16, j = i;
    const int chunk = wave;
    const bool live = chunk < kbs;  // the chunk's one pair (or nothing past K)
    uint8_t *slice = lds + wave * S::SLICE;
    const uint8_t *arow = slice + (i % MPAD) * S::XROW + qd * 16;
    const uint32_t magic = 0x64006400u;
    const float4_t fz = {0.f, 0.f, 0.f, 0.f};
    const int tiles = (n + 15) / 16;
    // Staging units as gemv_kernel's first round (k-blocks chunk, chunk + C):
    // the activation units are the same for every tile, so they are staged
    // once; a tile loads only the loads that hold its scale units.
    constexpr int L0 = MPAD * 32 / 64;
    if (live) {
#pragma unroll
        for (int L = 0; L < S::LOADS; L++) {
            const int u = L * 64 + lane;
            if (u < MPAD * 32) {
                const int r = u / 32, kbu = chunk + ((u % 32) / 16) * C;
                const int kk = kbu * 128 + (u % 16) * 8;
                const uint8_t *p = (const uint8_t *)g_zero_unit;
                if (r < m && kbu < kbs && kk < k) p = (const uint8_t *)(x + (size_t)r * k + kk);
                *(uint4_t *)(slice + r * S::XROW + (u % 32) * 16) = *(const uint4_t *)p;
            }
        }
    }
    // one tile of loads in flight beside the tile being computed (two or
    // three tiles ahead, and two blocks per compute unit, measured slower)
    uint4_t st[S::LOADS - L0], cw[2];
    auto issue = [&](int t) {
#pragma unroll
        for (int L = L0; L < S::LOADS; L++) {
            const int u = L * 64 + lane;
            const uint8_t *p = (const uint8_t *)g_zero_unit;
            if (u >= MPAD * 32 && u < S::UNITS) {
                const int v = u - MPAD * 32, kbq = chunk + (v / 8) * C;
                if (kbq < kbs) p = scales + ((size_t)t * kbs + kbq) * 128 + (v % 8) * 16;
            }
            st[L - L0] = *(const uint4_t *)p;
        }
        const uint8_t *cbase = codes + q4_lane(t, 0, kbs, qd, j);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int kb = chunk + h * C;
            cw[h] = __builtin_nontemporal_load((const uint4_t *)(cbase + (size_t)(kb < kbs ? kb : chunk) * 1024));
        }
    };
    auto tile = [&](int t, int it) {
        float acc[LIVE];
#pragma unroll
        for (int v = 0; v < LIVE; v++) acc[v] = 0.0f;
        if (live) {
            // only this wave reads its slice, and its reads of the last tile are done
#pragma unroll
            for (int L = L0; L < S::LOADS; L++) {
                const int u = L * 64 + lane;
                if (u >= MPAD * 32 && u < S::UNITS)
                    *(uint4_t *)(slice + MPAD * S::XROW + (u - MPAD * 32) * 16) = st[L - L0];
            }
            // one k-block's four MFMAs at a time, their scale FMAs in gemv_kernel's order
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint2_t sc = *(const uint2_t *)(slice + MPAD * S::XROW + h * 128 + j * 8);
                half8_t a[4];
#pragma unroll
                for (int s = 0; s < 4; s++) a[s] = *(const half8_t *)(arow + (h * 128 + s * 32) * 2);
                float4_t pr[4];
#pragma unroll
                for (int s = 0; s < 4; s++) pr[s] = mfma_f16(a[s], as_half8(unpack_codes(cw[h][s], magic)), fz);
#pragma unroll
                for (int s = 0; s < 4; s++) asm volatile("" : "+v"(pr[s]));
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const float scale = G32 ? f16_bits_to_float((sc[s >> 1] >> (16 * (s & 1))) & 0xffffu)
                                            : word_as_float(sc[s >> 1]);
#pragma unroll
                    for (int v = 0; v < LIVE; v++) acc[v] = __builtin_fmaf(pr[s][v], scale, acc[v]);
                }
            }
            // this tile's codes and staging are used up: the next tile's loads leave now
            if (t + (int)gridDim.x < tiles) issue(t + (int)gridDim.x);
        }
        float *pb = partials + (it & 1) * (C * LIVE * 64);
#pragma unroll
        for (int v = 0; v < LIVE; v++) pb[(chunk * LIVE + v) * 64 + lane] = acc[v];
        __syncthreads();  // every chunk's partial of tile t; the other buffer is free
        if (wave == 0 && qd * 4 < MPAD) {
            float total[LIVE];
#pragma unroll
            for (int c = 0; c < C; c++)
#pragma unroll
                for (int v = 0; v < LIVE; v++) {
                    const float pc = pb[(c * LIVE + v) * 64 + lane];
                    total[v] = c == 0 ? pc : __fadd_rn(total[v], pc);
                }
            const int col = t * 16 + j;
#pragma unroll
            for (int v = 0; v < LIVE; v++) {
                const int r = qd * 4 + v;
                if (r < m && col < n) y[(size_t)r * n + col] = total[v];
            }
        }
    };
    if (live && (int)blockIdx.x < tiles) issue(blockIdx.x);
    for (int t = blockIdx.x, it = 0; t < tiles; t += gridDim.x, it++) tile(t, it);
}

// Streaming form for wide products (several 16-row tiles per SIMD): one wave
// owns a whole tile, so no partial sum crosses waves, and it keeps D k-blocks
// of codes and scale records in flight while it computes. The block's
// activation rows are staged in LDS once. The wave walks the tile chunk by
// chunk (chunk c = k-blocks c, c + 16, ...; K a multiple of 2048, so every
// chunk holds kbs / 16 of them), folds each chunk into one accumulator with
// the per-32-run scale FMAs, and adds a finished chunk to the total in chunk
// order: the arithmetic of gemv_kernel, so the outputs are bitwise equal.
template <int WAVES, int MPAD, bool G32, int D>
__global__ __launch_bounds__(WAVES * 64) void gemv_stream_kernel(const uint8_t *__restrict__ codes,
                                                                 const uint8_t *__restrict__ scales,
                                                                 const half_t *__restrict__ x, int m,
                                                                 int k, int n, int kbs,
                                                                 float *__restrict__ y) {
    constexpr int LIVE = GemvShape<MPAD>::LIVE;
    extern __shared__ __align__(16) uint8_t lds[];
    const int xrow = kbs * 256 + 16;  // staged row: kbs * 128 f16 + 16 bytes of pad
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int qd = lane / 16, j = lane % 16;
    const int units = MPAD * kbs * 16;  // 16-byte units of the MPAD staged rows
    for (int u = threadIdx.x; u < units; u += WAVES * 64) {
        const int r = u / (kbs * 16), c = u % (kbs * 16);
        uint4_t v = {0u, 0u, 0u, 0u};
        if (r < m && c * 8 < k) v = *(const uint4_t *)(x + (size_t)r * k + c * 8);
        *(uint4_t *)(lds + r * xrow + c * 16) = v;
    }
    __syncthreads();
    const int t = blockIdx.x * WAVES + wave;
    if (t * 16 >= n) return;
    const uint8_t *cbase = codes + q4_lane(t, 0, kbs, qd, j);
    const uint8_t *sbase = scales + (size_t)t * kbs * 128 + j * 8;
    const uint8_t *arow = lds + (j % MPAD) * xrow + qd * 16;
    const int per = kbs / kGemvChunks;  // k-blocks per chunk (kbs % 16 == 0)
    const uint32_t magic = 0x64006400u;
    const float4_t fz = {0.f, 0.f, 0.f, 0.f};
    uint4_t cw[D];
    uint2_t sc[D];
#pragma unroll
    for (int r = 0; r < D; r++) {
        const int kb = r < kbs ? r / per + kGemvChunks * (r % per) : 0;
        cw[r] = __builtin_nontemporal_load((const uint4_t *)(cbase + (size_t)kb * 1024));
        sc[r] = *(const uint2_t *)(sbase + (size_t)kb * 128);
    }
    float acc[LIVE], total[LIVE];
#pragma unroll
    for (int v = 0; v < LIVE; v++) acc[v] = total[v] = 0.0f;
    for (int p0 = 0; p0 < kbs; p0 += D) {
#pragma unroll
        for (int r = 0; r < D; r++) {
            const int p = p0 + r;
            if (p >= kbs) break;
            const int kb = p / per + kGemvChunks * (p % per);
            half8_t a[4];
#pragma unroll
            for (int s = 0; s < 4; s++) a[s] = *(const half8_t *)(arow + (kb * 128 + s * 32) * 2);
            float4_t pr[4];
#pragma unroll
            for (int s = 0; s < 4; s++) pr[s] = mfma_f16(a[s], as_half8(unpack_codes(cw[r][s], magic)), fz);
#pragma unroll
            for (int s = 0; s < 4; s++) asm volatile("" : "+v"(pr[s]));
            const uint2_t scr = sc[r];
            // refill the slot with the k-block D positions ahead (a valid block past the end)
            const int pn = p + D;
            const int kbn = pn < kbs ? pn / per + kGemvChunks * (pn % per) : 0;
            cw[r] = __builtin_nontemporal_load((const uint4_t *)(cbase + (size_t)kbn * 1024));
            sc[r] = *(const uint2_t *)(sbase + (size_t)kbn * 128);
#pragma unroll
            for (int s = 0; s < 4; s++) {
                float scale;
                if (G32)
                    scale = f16_bits_to_float((scr[s >> 1] >> (16 * (s & 1))) & 0xffffu);
                else
                    scale = word_as_float(scr[s >> 1]);
#pragma unroll
                for (int v = 0; v < LIVE; v++) acc[v] = __builtin_fmaf(pr[s][v], scale, acc[v]);
            }
            if (p % per == per - 1) {
#pragma unroll
                for (int v = 0; v < LIVE; v++) {
                    total[v] = p == per - 1 ? acc[v] : __fadd_rn(total[v], acc[v]);
                    acc[v] = 0.0f;
                }
            }
        }
    }
    if (qd * 4 >= MPAD) return;
    const int col = t * 16 + j;
#pragma unroll
    for (int v = 0; v < LIVE; v++) {
        const int r = qd * 4 + v;
        if (r < m && col < n) y[(size_t)r * n + col] = total[v];
    }
}

// ============================================================================
// W4A16 large-M GEMM
// ============================================================================

// Block tile BM x BN, waves WM x WN, wave tile (BM/WM) x (BN/WN). One k-step
// is a 128-k block. The activation tile lives in LDS as BM rows of sixteen
// 16-byte chunks; chunk c of row r sits at slot c ^ (r & 15) so the 16 rows a
// ds_read_b128 touches fall in distinct banks.
// Epilogue: 0 -> f32 out; 1 -> f16 out; 2 -> f16 GELU; 3 -> f16 + residual.
template <int BM, int BN, int WM, int WN, bool G32, int EPI>
__global__ __launch_bounds__(WM *WN * 64) void gemm_w4a16_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales,
    const half_t *__restrict__ x, int m, int k, int n, int kbs, void *__restrict__ out,
    const half_t *__restrict__ residual) {
    constexpr int THREADS = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int MB = TM / 16, NT = TN / 16;
    constexpr int CHUNKS = BM * 16;  // 16-byte chunks of the A tile
    constexpr int PER_THREAD = CHUNKS / THREADS;
    static_assert(CHUNKS % THREADS == 0, "tile/threads mismatch");
    extern __shared__ __align__(16) uint8_t lds[];

    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int wm = wave / WN, wn = wave % WN;
    const int qd = lane / 16, i = lane % 16, j = i;
    const int bn = blockIdx.x, bm = blockIdx.y;
    const int row0 = bm * BM, col0 = bn * BN;
    const int tile0 = (col0 + wn * TN) / 16;
    const int tiles = (n + 15) / 16;

    float4_t acc[MB][NT];
#pragma unroll
    for (int a = 0; a < MB; a++)
#pragma unroll
        for (int b = 0; b < NT; b++) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    uint4_t pa[PER_THREAD];
    auto load_a = [&](int kb) {
#pragma unroll
        for (int p = 0; p < PER_THREAD; p++) {
            int idx = threadIdx.x + p * THREADS;
            int r = idx / 16, ch = idx % 16;
            int gr = row0 + r, gk = kb * 128 + ch * 8;
            uint4_t v = {0u, 0u, 0u, 0u};
            if (gr < m && gk < k) v = *(const uint4_t *)(x + (size_t)gr * k + gk);
            pa[p] = v;
        }
    };
    auto store_a = [&]() {
#pragma unroll
        for (int p = 0; p < PER_THREAD; p++) {
            int idx = threadIdx.x + p * THREADS;
            int r = idx / 16, ch = idx % 16;
            *(uint4_t *)(lds + r * 256 + ((ch ^ (r & 15)) * 16)) = pa[p];
        }
    };
    uint4_t pc[NT];
    uint2_t ps[NT];
    auto load_b = [&](int kb) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            int t = tile0 + nt;
            if (t < tiles) {
                pc[nt] = *(const uint4_t *)(codes + q4_lane(t, kb, kbs, qd, j));
                ps[nt] = *(const uint2_t *)(scales + (((size_t)t * kbs + kb) * 16 + j) * 8);
            } else {
                pc[nt] = uint4_t{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
                ps[nt] = uint2_t{0u, 0u};
            }
        }
    };

    load_a(0);
    load_b(0);
    for (int kb = 0; kb < kbs; kb++) {
        __syncthreads();
        store_a();
        // dequantize this k-block's weight fragments: code * scale in f16
        half8_t bf[NT][4];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int s = 0; s < 4; s++) {
                half_t sh;
                if (G32)
                    sh = __builtin_bit_cast(half_t, (unsigned short)((ps[nt][s >> 1] >> (16 * (s & 1))) & 0xffffu));
                else
                    sh = (half_t)word_as_float(ps[nt][s >> 1]);
                half2_t s2 = {sh, sh};
                uint4_t cw = nibbles_to_half8(pc[nt][s]);
#pragma unroll
                for (int p = 0; p < 4; p++) cw[p] = half2_as_word(word_as_half2(cw[p]) * s2);
                bf[nt][s] = as_half8(cw);
            }
        }
        __syncthreads();
        if (kb + 1 < kbs) {
            load_a(kb + 1);
            load_b(kb + 1);
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
#pragma unroll
            for (int mb = 0; mb < MB; mb++) {
                int r = wm * TM + mb * 16 + i;
                int ch = s * 4 + qd;
                half8_t a = *(const half8_t *)(lds + r * 256 + ((ch ^ (r & 15)) * 16));
#pragma unroll
                for (int nt = 0; nt < NT; nt++) acc[mb][nt] = mfma_f16(a, bf[nt][s], acc[mb][nt]);
            }
        }
    }
    // epilogue
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            int col = col0 + wn * TN + nt * 16 + j;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                int r = row0 + wm * TM + mb * 16 + qd * 4 + v;
                if (r < m && col < n) {
                    float val = acc[mb][nt][v];
                    size_t at = (size_t)r * n + col;
                    if (EPI == 0) {
                        ((float *)out)[at] = val;
                    } else if (EPI == 1) {
                        ((half_t *)out)[at] = (half_t)val;
                    } else if (EPI == 2) {
                        ((half_t *)out)[at] = (half_t)f32_rounded(gelu_erf(val));
                    } else {
                        ((half_t *)out)[at] = (half_t)f32_rounded(val + (float)residual[at]);
                    }
                }
            }
        }
    }
}

// ============================================================================
// per-row int8 GEMM
// ============================================================================

// K-step 64 bytes; both tiles staged in LDS as rows of four 16-byte chunks,
// chunk c of row r at slot c ^ ((r >> 2) & 3).
// 8 (code + 8) nibbles of a per-row Q4 word (element t at bits 4t) -> two
// words of signed int8 codes in element order.
__device__ __forceinline__ uint2_t row_nibbles_to_i8(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu;         // elements 0 2 4 6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // elements 1 3 5 7
    uint2_t out;
    out[0] = (__builtin_amdgcn_perm(hi, lo, 0x05010400u) + 0x78787878u) ^ 0x80808080u;  // 0 1 2 3
    out[1] = (__builtin_amdgcn_perm(hi, lo, 0x07030602u) + 0x78787878u) ^ 0x80808080u;  // 4 5 6 7
    return out;
}

// FUSED (webgpu/int8.rs:226-230): the B tile is BN/2 rows of b (the gate
// weights) over BN/2 rows of u (the up weights) for the same BN/2 output
// columns; each wave's first NB/2 fragments are gate columns and the last NB/2
// the up rows of the same columns, so the epilogue finds both dots of an
// output in one lane: y = (g / (1 + exp(-g))) * up with g and up rescaled like
// the plain output, exp the f32 rounding of the f64 exponential.
template <int BM, int BN, int WM, int WN, bool Q4B, bool FUSED = false>
__global__ __launch_bounds__(WM *WN * 64) void i8_gemm_kernel(const int8_t *__restrict__ a,
                                                              const float *__restrict__ sa, int m,
                                                              const int8_t *__restrict__ b,
                                                              const float *__restrict__ sb, int n,
                                                              int k, void *__restrict__ y,
                                                              int raw, const int8_t *__restrict__ u = nullptr,
                                                              const float *__restrict__ su = nullptr) {
    constexpr int THREADS = WM * WN * 64;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int MB = TM / 16, NB = TN / 16;
    static_assert(!FUSED || (NB % 2 == 0 && !Q4B), "fused tiles pair gate and up fragments");
    constexpr int OUT_N = FUSED ? BN / 2 : BN;  // output columns per tile
    constexpr int ACH = BM * 4, BCH = BN * 4;
    constexpr int PA = (ACH + THREADS - 1) / THREADS, PB = (BCH + THREADS - 1) / THREADS;
    __shared__ __align__(16) uint8_t la[2][BM * 64];
    __shared__ __align__(16) uint8_t lb[2][BN * 64];

    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int wm = wave / WN, wn = wave % WN;
    const int qd = lane / 16, i = lane % 16;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * OUT_N;
    const int steps = (k + 63) / 64;

    int4_t acc[MB][NB];
#pragma unroll
    for (int x = 0; x < MB; x++)
#pragma unroll
        for (int z = 0; z < NB; z++) acc[x][z] = int4_t{0, 0, 0, 0};

    uint4_t ra[PA], rb[PB];
    auto load_chunk = [&](const int8_t *src, int rows, int r, int kk) -> uint4_t {
        uint4_t v = {0u, 0u, 0u, 0u};
        if (r < rows) {
            const int8_t *p = src + (size_t)r * k + kk;
            if (kk + 16 <= k) {
                v = *(const uint4_t *)p;
            } else if (kk < k) {
                uint8_t tmp[16] = {};
                for (int e = 0; e < 16 && kk + e < k; e++) tmp[e] = (uint8_t)p[e];
                v = *(uint4_t *)tmp;
            }
        }
        return v;
    };
    // per-row Q4 B: 16 codes = two words of row r (k % 8 == 0), expanded to int8
    auto load_q4_chunk = [&](int r, int kk) -> uint4_t {
        uint4_t v = {0u, 0u, 0u, 0u};
        if (r < n && kk < k) {
            const uint32_t *row = (const uint32_t *)b + (size_t)r * (k / 8);
            const uint2_t c0 = row_nibbles_to_i8(row[kk / 8]);
            const uint2_t c1 = kk + 8 < k ? row_nibbles_to_i8(row[kk / 8 + 1]) : uint2_t{0u, 0u};
            v = uint4_t{c0[0], c0[1], c1[0], c1[1]};
        }
        return v;
    };
    auto load = [&](int step) {
#pragma unroll
        for (int p = 0; p < PA; p++) {
            int idx = threadIdx.x + p * THREADS;
            if (idx < ACH) ra[p] = load_chunk(a, m, row0 + idx / 4, step * 64 + (idx % 4) * 16);
        }
#pragma unroll
        for (int p = 0; p < PB; p++) {
            int idx = threadIdx.x + p * THREADS;
            if (idx < BCH) {
                if (FUSED) {
                    const int r = idx / 4;
                    rb[p] = load_chunk(r < BN / 2 ? b : u, n, col0 + r % (BN / 2), step * 64 + (idx % 4) * 16);
                } else {
                    rb[p] = Q4B ? load_q4_chunk(col0 + idx / 4, step * 64 + (idx % 4) * 16)
                                : load_chunk(b, n, col0 + idx / 4, step * 64 + (idx % 4) * 16);
                }
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PA; p++) {
            int idx = threadIdx.x + p * THREADS;
            if (idx < ACH) {
                int r = idx / 4, c = idx % 4;
                *(uint4_t *)(la[buf] + r * 64 + ((c ^ ((r >> 2) & 3)) * 16)) = ra[p];
            }
        }
#pragma unroll
        for (int p = 0; p < PB; p++) {
            int idx = threadIdx.x + p * THREADS;
            if (idx < BCH) {
                int r = idx / 4, c = idx % 4;
                *(uint4_t *)(lb[buf] + r * 64 + ((c ^ ((r >> 2) & 3)) * 16)) = rb[p];
            }
        }
    };

    load(0);
    store(0);
    __syncthreads();
    for (int st = 0; st < steps; st++) {
        const int buf = st & 1;
        if (st + 1 < steps) load(st + 1);
        int4_t bfrag[NB];
#pragma unroll
        for (int z = 0; z < NB; z++) {
            const int r = FUSED ? (z < NB / 2 ? 0 : BN / 2) + wn * (TN / 2) + (z % (NB / 2)) * 16 + i
                                : wn * TN + z * 16 + i;
            bfrag[z] = *(const int4_t *)(lb[buf] + r * 64 + ((qd ^ ((r >> 2) & 3)) * 16));
        }
#pragma unroll
        for (int x = 0; x < MB; x++) {
            int r = wm * TM + x * 16 + i;
            int4_t af = *(const int4_t *)(la[buf] + r * 64 + ((qd ^ ((r >> 2) & 3)) * 16));
#pragma unroll
            for (int z = 0; z < NB; z++) acc[x][z] = mfma_i8(af, bfrag[z], acc[x][z]);
        }
        if (st + 1 < steps) store(buf ^ 1);
        __syncthreads();
    }
    if constexpr (FUSED) {
#pragma unroll
        for (int x = 0; x < MB; x++) {
#pragma unroll
            for (int z = 0; z < NB / 2; z++) {
                const int col = col0 + wn * (TN / 2) + z * 16 + i;
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const int r = row0 + wm * TM + x * 16 + qd * 4 + v;
                    if (r < m && col < n) {
                        const float g = __fmul_rn(__fmul_rn((float)acc[x][z][v], sa[r]), sb[col]);
                        const float up = __fmul_rn(__fmul_rn((float)acc[x][z + NB / 2][v], sa[r]), su[col]);
                        const float e = __double2float_rn(exp(-(double)g));
                        ((float *)y)[(size_t)r * n + col] = __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, e)), up);
                    }
                }
            }
        }
        return;
    }
#pragma unroll
    for (int x = 0; x < MB; x++) {
#pragma unroll
        for (int z = 0; z < NB; z++) {
            int col = col0 + wn * TN + z * 16 + i;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                int r = row0 + wm * TM + x * 16 + qd * 4 + v;
                if (r < m && col < n) {
                    size_t at = (size_t)r * n + col;
                    if (raw)
                        ((int32_t *)y)[at] = acc[x][z][v];
                    else
                        ((float *)y)[at] = __fmul_rn(__fmul_rn((float)acc[x][z][v], sa[r]), sb[col]);
                }
            }
        }
    }
}


// Tiles are assigned XCD-aware: consecutive block ids go to different XCDs,
// so tile ids are taken in XCD-major order and grouped GROUP_M tile-rows at a
// time, keeping the blocks that share an XCD's L2 on neighbouring tiles.

__device__ __forceinline__ void xcd_tile(int bid, int nblocks, int tiles_m, int tiles_n, int &tm, int &tn) {
    constexpr int XCDS = 8, GROUP_M = 4;
    int linear = bid;
    if (nblocks % XCDS == 0) linear = (bid % XCDS) * (nblocks / XCDS) + bid / XCDS;
    const int per_group = GROUP_M * tiles_n;
    const int group = linear / per_group;
    const int first_m = group * GROUP_M;
    const int gsize = min(tiles_m - first_m, GROUP_M);
    const int in_group = linear % per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}


typedef int int16_t_v __attribute__((ext_vector_type(16)));

// Deep-pipelined per-row int8 GEMM. Block tile BM x BN over 4 waves (2 x 2),
// 32x32x32 i8 MFMAs, k-steps of BK bytes (64 or 128) in NS LDS stages filled
// by buffer_load ... lds (no VGPR staging). NS - 1 k-steps are in flight: a
// step waits only for its own stage (s_waitcnt vmcnt of the younger stages'
// loads) before the workgroup barrier, so HBM/L2 latency overlaps NS - 2
// steps of MFMA work. Stage rows are BK bytes of 16-byte chunks, XOR-swizzled
// so that the 16 rows of a fragment read (16 lanes per 256-byte LDS cycle)
// fall in distinct banks, with 256 / BK rows sharing a bank line:
//   BK = 128: slot = chunk ^ ((row >> 1) & 7); BK = 64: slot = chunk ^ ((row >> 2) & 3).
// Rows past m (n) and chunks past k read as zero (buffer range checks), so
// any m, n and k % 16 == 0 work. The f32 epilogue reads its row and column
// scales from LDS.
template <int BK>
__device__ __forceinline__ int pipe_slot(int c, int r) {
    return BK == 128 ? (c ^ ((r >> 1) & 7)) : (c ^ ((r >> 2) & 3));
}

template <int BM, int BN, int BK, int NS, int WGM, int WGN>
__global__ __launch_bounds__(WGM *WGN * 64) void i8_gemm_pipe_kernel(const int8_t *__restrict__ a, const float *__restrict__ sa,
                                                           int m, const int8_t *__restrict__ b,
                                                           const float *__restrict__ sb, int n, int k,
                                                           void *__restrict__ y, int raw) {
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    constexpr int WAVES = WGM * WGN, THREADS = WAVES * 64;
    constexpr int TM = BM / WGM, TN = BN / WGN, MB = TM / 32, NB = TN / 32;
    constexpr int CPR = BK / 16;                 // 16-byte chunks per stage row
    constexpr int RPI = 64 / CPR;                // stage rows filled by one DMA instruction
    constexpr int STAGE = (BM + BN) * BK;
    constexpr int DPW = (BM + BN) / RPI / WAVES; // DMA instructions per wave per stage
    static_assert(DPW * WAVES * RPI == BM + BN, "DMA blocks split evenly over the waves");
    constexpr int SUBS = BK / 32;                // k-substeps of one 32x32x32 MFMA
    static_assert((NS - 2) * DPW <= 63, "vmcnt range");
    static_assert(NS > 2 || SUBS >= 2, "two stages issue their loads over the first two substeps");
    __shared__ __align__(16) uint8_t st0[STAGE];
    __shared__ __align__(16) uint8_t st1[STAGE];
    __shared__ __align__(16) uint8_t st2[NS > 2 ? STAGE : 16];
    __shared__ __align__(16) uint8_t st3[NS > 3 ? STAGE : 16];
    __shared__ float scale_rows[BM], scale_cols[BN];
    uint8_t *const stages[4] = {st0, st1, st2, st3};

    // the wave index is uniform; saying so keeps the DMA's buffer resource in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int wm = wave / WGN, wn = wave % WGN;
    const int h = lane / 32, i = lane % 32;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    const int steps = (k + BK - 1) / BK;
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(a + (size_t)row0 * k), (short)0, min(BM, m - row0) * k, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(b + (size_t)col0 * k), (short)0, min(BN, n - col0) * k, 0x00020000);
    // Lane l fills slot l % CPR of stage row RPI*blk + l / CPR. That row's
    // source chunk depends on the lane only. The whole byte offset (row and
    // chunk) goes in the VGPR offset, the part the buffer range check covers,
    // so rows past m (n) and chunks past k read as zero and nothing past the
    // operands is touched; soffset stays 0.
    // The swizzle of row RPI*blk + lrow depends on blk only through its
    // parity (BK = 128) or not at all (BK = 64); DPW is even, so the parity
    // of blk is that of p.
    static_assert(DPW % 2 == 0, "instruction parity known at compile time");
    const int lrow = lane / CPR;
    const int c16[2] = {pipe_slot<BK>(lane % CPR, lrow) * 16, pipe_slot<BK>(lane % CPR, lrow + RPI) * 16};
    const uint32_t lane_off[2] = {(uint32_t)(lrow * k + c16[0]), (uint32_t)(lrow * k + c16[1])};
    // DMA instructions p0 <= p < p1 of a stage (issued in slices between MFMA groups)
    auto dma = [&](uint8_t *stage, int st, int p0, int p1) {
        const int kk = st * BK;
        // >= 2^31 stays out of range after adding a row offset (BM, BN rows * k < 2^31)
        const uint32_t voff0 = kk + c16[0] < k ? lane_off[0] + (uint32_t)kk : 0x80000000u;
        const uint32_t voff1 = kk + c16[1] < k ? lane_off[1] + (uint32_t)kk : 0x80000000u;
#pragma unroll
        for (int p = p0; p < p1; p++) {
            const int blk = wave * DPW + p;
            const uint32_t voff = (p & 1) ? voff1 : voff0;
            auto *dst = (__attribute__((address_space(3))) void *)(stage + __builtin_amdgcn_readfirstlane(blk * 1024));
            if (blk * RPI < BM)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, dst, 16, voff + (uint32_t)(blk * RPI * k), 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, dst, 16, voff + (uint32_t)((blk * RPI - BM) * k), 0, 0, 0);
        }
    };
    auto read_frags = [&](const uint8_t *stage, int sub, int4_t *af, int4_t *bf) {
        const uint8_t *la = stage, *lb = stage + BM * BK;
        const int c = sub * 2 + h;
#pragma unroll
        for (int x = 0; x < MB; x++) {
            const int r = wm * TM + x * 32 + i;
            af[x] = *(const int4_t *)(la + r * BK + pipe_slot<BK>(c, r) * 16);
        }
#pragma unroll
        for (int z = 0; z < NB; z++) {
            const int r = wn * TN + z * 32 + i;
            bf[z] = *(const int4_t *)(lb + r * BK + pipe_slot<BK>(c, r) * 16);
        }
    };
    int16_t_v acc[MB][NB];
#pragma unroll
    for (int x = 0; x < MB; x++)
#pragma unroll
        for (int z = 0; z < NB; z++) acc[x][z] = int16_t_v{};
    // compute on `stage`; when `next` is set, the loads of step `next_step`
    // into it are issued in SUBS slices, one before each substep's MFMAs.
    // With two stages they are issued in two slices, before the first two
    // substeps, so that the last of them has most of the step to land
    // (config 4, alternated on one box: 123.3-123.9 us against 126.9-128.1
    // with all of them before the first substep and 130.0-131.5 with four
    // slices; three slices 1.2% slower than two; with three stages the four
    // slices pay)
    auto compute = [&](const uint8_t *stage, uint8_t *next, int next_step) {
        int4_t af[2][MB], bf[2][NB];
        read_frags(stage, 0, af[0], bf[0]);
#pragma unroll
        for (int sub = 0; sub < SUBS; sub++) {
            const int cur = sub & 1;
            if (next) {
                if (NS > 2)
                    dma(next, next_step, sub * DPW / SUBS, (sub + 1) * DPW / SUBS);
                else if (sub < 2)
                    dma(next, next_step, sub * DPW / 2, (sub + 1) * DPW / 2);
            }
            if (sub + 1 < SUBS) read_frags(stage, sub + 1, af[cur ^ 1], bf[cur ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int x = 0; x < MB; x++)
#pragma unroll
                for (int z = 0; z < NB; z++)
                    acc[x][z] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][x], bf[cur][z], acc[x][z], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if (!raw) {
        for (int r = threadIdx.x; r < BM; r += THREADS) scale_rows[r] = row0 + r < m ? sa[row0 + r] : 0.0f;
        for (int c = threadIdx.x; c < BN; c += THREADS) scale_cols[c] = col0 + c < n ? sb[col0 + c] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NS - 1; j++)
        if (j < steps) dma(stages[j], j, 0, DPW);
    for (int base = 0; base < steps; base += NS) {
#pragma unroll
        for (int j = 0; j < NS; j++) {
            const int s2 = base + j;
            if (s2 >= steps) break;
            // this wave's loads of step s2 are done once at most the younger
            // steps' loads are outstanding; then the barrier covers every wave
            if (s2 + NS - 2 < steps)
                asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * DPW) : "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
            compute(stages[j], s2 + NS - 1 < steps ? stages[(j + NS - 1) % NS] : nullptr, s2 + NS - 1);
        }
    }
    __syncthreads();
    // Epilogue: each wave turns a 32-row slice of its tile into row-major
    // order in its own LDS region (the stage arrays are free now) and writes
    // it with 16-byte stores, four consecutive columns per lane.
    // wave w's slab: stage array w % NS, after the slabs of the waves before it there
    const int home = wave % NS;  // chosen without indexing `stages` at run time
    uint8_t *slab_stage = home == 0 ? st0 : home == 1 ? st1 : home == 2 ? st2 : st3;
    uint32_t *slab = (uint32_t *)(slab_stage + (wave / NS) * 32 * TN * 4);
    static_assert(((WAVES + NS - 1) / NS) * 32 * TN * 4 <= STAGE, "epilogue slabs fit the stage arrays");
    float cs[NB];
    if (!raw) {
#pragma unroll
        for (int z = 0; z < NB; z++) cs[z] = scale_cols[wn * TN + z * 32 + i];
    }
#pragma unroll
    for (int x = 0; x < MB; x++) {
        float rs[16];
        if (!raw) {
#pragma unroll
            for (int e = 0; e < 16; e++) rs[e] = scale_rows[wm * TM + x * 32 + 8 * (e / 4) + 4 * h + (e % 4)];
        }
#pragma unroll
        for (int z = 0; z < NB; z++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int rl = 8 * (e / 4) + 4 * h + (e % 4), cl = z * 32 + i;
                uint32_t v = (uint32_t)acc[x][z][e];
                if (!raw) v = __builtin_bit_cast(uint32_t, __fmul_rn(__fmul_rn((float)acc[x][z][e], rs[e]), cs[z]));
                slab[rl * TN + cl] = v;
            }
        }
        // the slab is this wave's alone: LDS accesses of one wave complete in order
        constexpr int QUADS = TN / 4;                   // 16-byte pieces per row
        constexpr int ROWS_PER_PASS = 64 / QUADS;
#pragma unroll
        for (int pass = 0; pass < 32 / ROWS_PER_PASS; pass++) {
            const int rl = pass * ROWS_PER_PASS + lane / QUADS, q = lane % QUADS;
            const uint4_t v = *(const uint4_t *)(slab + rl * TN + q * 4);
            const int r = row0 + wm * TM + x * 32 + rl, c = col0 + wn * TN + q * 4;
            if (r < m) {
                uint32_t *dst = (uint32_t *)y + (size_t)r * n + c;
                if (c + 4 <= n && (n & 3) == 0 && ((uintptr_t)y & 15) == 0) {
                    *(uint4_t *)dst = v;
                } else {
                    for (int e = 0; e < 4; e++)
                        if (c + e < n) dst[e] = v[e];
                }
            }
        }
    }
}

// Persistent form of i8_gemm_pipe_kernel: a grid of at most one block per
// compute unit, block b taking tiles b, b + grid, ... (xcd_tile order over all
// tiles) as ONE stream of k-steps, so the loads of a tile's first steps are in
// flight while the previous tile's last steps compute. Each tile's epilogue
// stores straight from the accumulators (lane (i, h) of a 32x32 block holds
// column i of rows 8(e/4) + 4h + e%4: a store instruction writes two 128-byte
// row pieces), which leaves the LDS stages to the next tile and lets those
// stores drain under its MFMAs. Outputs equal i8_gemm_pipe_kernel's (exact
// int32 dots; the f32 epilogue (f32(dot) * sa) * sb).
template <int BM, int BN, int BK, int NS, int WGM, int WGN, bool MID>
__global__ __launch_bounds__(WGM *WGN * 64, 2) void i8_gemm_stream_kernel(const int8_t *__restrict__ a,
                                                                     const float *__restrict__ sa, int m,
                                                                     const int8_t *__restrict__ b,
                                                                     const float *__restrict__ sb, int n, int k,
                                                                     void *__restrict__ y, int raw) {
    static_assert(NS >= 2 && NS <= 4, "2 to 4 stages");
    constexpr int WAVES = WGM * WGN, THREADS = WAVES * 64;
    constexpr int TM = BM / WGM, TN = BN / WGN, MB = TM / 32, NB = TN / 32;
    constexpr int CPR = BK / 16;
    constexpr int RPI = 64 / CPR;
    constexpr int STAGE = (BM + BN) * BK;
    constexpr int DPW = (BM + BN) / RPI / WAVES;
    static_assert(DPW * WAVES * RPI == BM + BN, "DMA blocks split evenly over the waves");
    constexpr int SUBS = BK / 32;
    static_assert((NS - 2) * DPW <= 63, "vmcnt range");
    __shared__ __align__(16) uint8_t stages[NS * STAGE];
    __shared__ __align__(16) float scale_rows[2][BM], scale_cols[2][BN];  // by tile parity

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int wm = wave / WGN, wn = wave % WGN;
    const int h = lane / 32, i = lane % 32;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN, total = tiles_m * tiles_n;
    const int grid = gridDim.x, blk = blockIdx.x;
    if (blk >= total) return;
    const int my_tiles = (total - blk + grid - 1) / grid;
    const int steps = (k + BK - 1) / BK;
    const int stream = my_tiles * steps;
    auto tile_origin = [&](int j, int &row0, int &col0) {
        int tm, tn;
        xcd_tile(blk + j * grid, total, tiles_m, tiles_n, tm, tn);
        row0 = tm * BM;
        col0 = tn * BN;
    };
    static_assert(DPW % 2 == 0, "instruction parity known at compile time");
    const int lrow = lane / CPR;
    const int c16[2] = {pipe_slot<BK>(lane % CPR, lrow) * 16, pipe_slot<BK>(lane % CPR, lrow + RPI) * 16};
    const uint32_t lane_off[2] = {(uint32_t)(lrow * k + c16[0]), (uint32_t)(lrow * k + c16[1])};
    // the tile the loads are filling (they run NS - 1 steps ahead of the MFMAs)
    __amdgpu_buffer_rsrc_t rsa, rsb;
    auto load_tile = [&](int j) {
        int row0, col0;
        tile_origin(j, row0, col0);
        rsa = __builtin_amdgcn_make_buffer_rsrc((void *)(a + (size_t)row0 * k), (short)0, min(BM, m - row0) * k,
                                                0x00020000);
        rsb = __builtin_amdgcn_make_buffer_rsrc((void *)(b + (size_t)col0 * k), (short)0, min(BN, n - col0) * k,
                                                0x00020000);
    };
    auto dma = [&](uint8_t *stage, int st, int p0, int p1) {
        const int kk = st * BK;
        const uint32_t voff0 = kk + c16[0] < k ? lane_off[0] + (uint32_t)kk : 0x80000000u;
        const uint32_t voff1 = kk + c16[1] < k ? lane_off[1] + (uint32_t)kk : 0x80000000u;
#pragma unroll
        for (int p = p0; p < p1; p++) {
            const int bl = wave * DPW + p;
            const uint32_t voff = (p & 1) ? voff1 : voff0;
            auto *dst = (__attribute__((address_space(3))) void *)(stage + __builtin_amdgcn_readfirstlane(bl * 1024));
            if (bl * RPI < BM)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, dst, 16, voff + (uint32_t)(bl * RPI * k), 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsb, dst, 16, voff + (uint32_t)((bl * RPI - BM) * k), 0, 0, 0);
        }
    };
    auto read_frags = [&](const uint8_t *stage, int sub, int4_t *af, int4_t *bf) {
        const uint8_t *la = stage, *lb = stage + BM * BK;
        const int c = sub * 2 + h;
#pragma unroll
        for (int x = 0; x < MB; x++) {
            const int r = wm * TM + x * 32 + i;
            af[x] = *(const int4_t *)(la + r * BK + pipe_slot<BK>(c, r) * 16);
        }
#pragma unroll
        for (int z = 0; z < NB; z++) {
            const int r = wn * TN + z * 32 + i;
            bf[z] = *(const int4_t *)(lb + r * BK + pipe_slot<BK>(c, r) * 16);
        }
    };
    int16_t_v acc[MB][NB];
    auto compute = [&](const uint8_t *stage, uint8_t *next, int next_step) {
        int4_t af[2][MB], bf[2][NB];
        read_frags(stage, 0, af[0], bf[0]);
#pragma unroll
        for (int sub = 0; sub < SUBS; sub++) {
            const int cur = sub & 1;
            if (next) dma(next, next_step, sub * DPW / SUBS, (sub + 1) * DPW / SUBS);
            if (sub + 1 < SUBS) read_frags(stage, sub + 1, af[cur ^ 1], bf[cur ^ 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int x = 0; x < MB; x++)
#pragma unroll
                for (int z = 0; z < NB; z++)
                    acc[x][z] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][x], bf[cur][z], acc[x][z], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // tile j's scales into buffer j % 2 (its epilogue reads them several barriers later)
    auto load_scales = [&](int j) {
        if (raw) return;
        int row0, col0;
        tile_origin(j, row0, col0);
        for (int r = threadIdx.x; r < BM; r += THREADS) scale_rows[j & 1][r] = row0 + r < m ? sa[row0 + r] : 0.0f;
        for (int c = threadIdx.x; c < BN; c += THREADS) scale_cols[j & 1][c] = col0 + c < n ? sb[col0 + c] : 0.0f;
    };
    // Buffer stores: rows past m fall outside the resource's range, columns past
    // n take an offset beyond any range; both are dropped by the hardware.
    auto epilogue = [&](int j) {
        int row0, col0;
        tile_origin(j, row0, col0);
        const __amdgpu_buffer_rsrc_t rsy = __builtin_amdgcn_make_buffer_rsrc(
            (void *)((uint32_t *)y + (size_t)row0 * n), (short)0, min(BM, m - row0) * n * 4, 0x00020000);
        const float *rs = scale_rows[j & 1];
#pragma unroll
        for (int z = 0; z < NB; z++) {
            const int cl = wn * TN + z * 32 + i;
            const uint32_t lane_col = col0 + cl < n ? (uint32_t)((wm * TM + 4 * h) * n + col0 + cl) * 4u : 0x80000000u;
            const float cs = raw ? 0.0f : scale_cols[j & 1][cl];
#pragma unroll
            for (int x = 0; x < MB; x++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int rl = wm * TM + x * 32 + 8 * q + 4 * h;
                    float4 r4 = raw ? float4{} : *(const float4 *)(rs + rl);
                    const float rv[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int32_t d = acc[x][z][4 * q + e];
                        const uint32_t v = raw ? (uint32_t)d
                                               : __builtin_bit_cast(uint32_t, __fmul_rn(__fmul_rn((float)d, rv[e]), cs));
                        const uint32_t soff = __builtin_amdgcn_readfirstlane((uint32_t)((x * 32 + 8 * q + e) * n) * 4u);
                        __builtin_amdgcn_raw_buffer_store_b32(v, rsy, lane_col + soff, 0, 0);
                    }
                }
        }
    };

    load_tile(0);
    load_scales(0);
    // the first NS - 1 steps (NS with the boundary inside the last k-slice, which
    // loads step g + NS rather than g + NS - 1)
#pragma unroll
    for (int j = 0; j < (MID ? NS : NS - 1); j++)
        if (j < stream) {
            if (j > 0 && j % steps == 0) load_tile(j / steps);
            dma(stages + j * STAGE, j % steps, 0, DPW);
        }
    // tiles in the outer loop, so the accumulators restart at zero unconditionally
    // (a conditional restart would keep two copies of them alive)
    if constexpr (!MID) {
        int g = 0, slot = 0;
        for (int j = 0; j < my_tiles; j++) {
            if (j > 0) load_scales(j);
#pragma unroll
            for (int x = 0; x < MB; x++)
#pragma unroll
                for (int z = 0; z < NB; z++) acc[x][z] = int16_t_v{};
            for (int st = 0; st < steps; st++, g++, slot = slot + 1 == NS ? 0 : slot + 1) {
                if (g + NS - 2 < stream)
                    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 2) * DPW) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
                const int nx = g + NS - 1;
                if (nx < stream && nx % steps == 0) load_tile(nx / steps);
                const int nslot = slot == 0 ? NS - 1 : slot - 1;
                compute(stages + slot * STAGE, nx < stream ? stages + nslot * STAGE : nullptr, nx % steps);
            }
            epilogue(j);
        }
    } else {
        // The step boundary sits inside the last k-slice: once this wave's
        // fragment reads of step g and its loads of step g + 1 are done, one
        // barrier frees slot g (its loads of step g + NS go there at once, a
        // whole step ahead) and publishes step g + 1, whose first fragments are
        // read before the last MFMAs of step g issue.
        static_assert(SUBS % 2 == 0, "the first fragments of a step land in buffer 0");
        static_assert((NS - 1) * DPW <= 63, "vmcnt range");
        int4_t af[2][MB], bf[2][NB];
        if (NS - 1 < stream)
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((NS - 1) * DPW) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
        read_frags(stages, 0, af[0], bf[0]);
        int g = 0, slot = 0;
        for (int j = 0; j < my_tiles; j++) {
            if (j > 0) load_scales(j);
#pragma unroll
            for (int x = 0; x < MB; x++)
#pragma unroll
                for (int z = 0; z < NB; z++) acc[x][z] = int16_t_v{};
            for (int st = 0; st < steps; st++, g++, slot = slot + 1 == NS ? 0 : slot + 1) {
                const uint8_t *stage = stages + slot * STAGE;
#pragma unroll
                for (int sub = 0; sub < SUBS; sub++) {
                    const int cur = sub & 1;
                    if (sub + 1 < SUBS) {
                        read_frags(stage, sub + 1, af[cur ^ 1], bf[cur ^ 1]);
                    } else if (g + 1 < stream) {
                        if (g + NS - 1 < stream)
                            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NS - 2) * DPW) : "memory");
                        else
                            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
                        const int nx = g + NS;
                        if (nx < stream) {
                            if (nx % steps == 0) load_tile(nx / steps);
                            dma(stages + slot * STAGE, nx % steps, 0, DPW);
                        }
                        read_frags(stages + (slot + 1 == NS ? 0 : slot + 1) * STAGE, 0, af[cur ^ 1], bf[cur ^ 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int x = 0; x < MB; x++)
#pragma unroll
                        for (int z = 0; z < NB; z++)
                            acc[x][z] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[cur][x], bf[cur][z], acc[x][z], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (steps == 1 && !raw) __syncthreads();  // a one-step tile's scales have no barrier after them
            epilogue(j);
        }
    }
}

// ============================================================================
// pipelined W4A16 GEMM (large M)
// ============================================================================

// unpack_codes without asm: lo/hi masks come in SGPRs and the exponent in a
// VGPR, so each (w & mask) | magic is one v_and_or_b32
__device__ __forceinline__ uint4_t unpack_codes_c(uint32_t w, uint32_t mlo, uint32_t mhi, uint32_t magic) {
    const half2_t bias = {(half_t)-1032.0f, (half_t)-1032.0f};
    const half2_t sixteenth = {(half_t)0.0625f, (half_t)0.0625f};
    const half2_t bias16 = {(half_t)-72.0f, (half_t)-72.0f};
    const uint32_t w8 = w >> 8;
    uint4_t out;
    out[0] = half2_as_word(word_as_half2((w & mlo) | magic) + bias);
    out[1] = half2_as_word(__builtin_elementwise_fma(word_as_half2((w & mhi) | magic), sixteenth, bias16));
    out[2] = half2_as_word(word_as_half2((w8 & mlo) | magic) + bias);
    out[3] = half2_as_word(__builtin_elementwise_fma(word_as_half2((w8 & mhi) | magic), sixteenth, bias16));
    return out;
}

// Block tile BM x BN over WGM x WGN waves; one k-step is one 128-k block, in
// two LDS stages filled by buffer_load ... lds while the other is computed:
//  - activations: BM rows of 256 bytes; chunk c (8 halves) of row r sits at
//    slot c ^ (r & 15), so the 16 rows of a fragment read fall in distinct
//    banks. The byte offset of every load is in the VGPR offset, which the
//    buffer range check covers: rows past m read as zero;
//  - weight codes: the 1 KiB tile16x128 chunk of each 16-column tile, copied
//    as is (its lane order is the MFMA operand order);
//  - scale records go straight to registers, one step ahead.
// The stage loads are issued as asm (dma16) and waited for at the step's
// barrier; the one compute body reads whichever stage is current. Needs
// k % 128 == 0 (the launcher falls back otherwise).
// Codes become f16 exactly as in gemm_w4a16_kernel (exact code times the f16
// scale, rounded once), and each output accumulates one
// v_mfma_f32_16x16x32_f16 per 32-k run in k order, so both kernels give the
// same bits. The MFMA is issued as D[n][m] = W . X^T: lane (q, j) ends with
// four consecutive output columns of one row and stores them as one vector.
// A launch covers the n output columns that codes / scales / out / residual
// point at (a multiple-of-16 slice of the weight); ldo is the row stride of
// out and residual.
// PERSIST: a grid of fewer blocks than tiles, each taking tiles blockIdx.x,
// blockIdx.x + gridDim.x, ... (the same tile order and XCD placement as one
// block per tile) as one stream of k-steps: the last step of a tile loads the
// next tile's first stage, so those loads fly during the epilogue. Each
// tile's arithmetic is unchanged, so both forms give the same bits.
template <int BM, int BN, int WGM, int WGN, bool G32, int EPI, int VALU_PER_MFMA = 2, bool PERSIST = false>
__global__ __launch_bounds__(WGM *WGN * 64) void w4a16_pipe_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, const half_t *__restrict__ x, int m,
    int k, int n, int kbs, void *__restrict__ out, const half_t *__restrict__ residual, int ldo) {
    constexpr int WAVES = WGM * WGN;
    constexpr int TM = BM / WGM, TN = BN / WGN, MB = TM / 16, NT = TN / 16;
    constexpr int XSTAGE = BM * 256, WSTAGE = BN / 16 * 1024;
    constexpr int XPW = BM / 4 / WAVES;   // 4-row activation DMA instructions per wave per step
    constexpr int WPW = (BN / 16 + WAVES - 1) / WAVES;  // code-chunk DMA instructions per wave per step (at most)
    static_assert(XPW * 4 * WAVES == BM && XPW % 4 == 0, "a wave's first DMA row is a multiple of 16");
    static_assert(WPW * 16 * WAVES >= BN && WPW >= 1, "every code chunk has a wave");
    static_assert(MB % 2 == 0, "activation fragments are read in two halves");
    __shared__ __align__(16) uint8_t xs[2 * XSTAGE];
    __shared__ __align__(16) uint8_t ws[2 * WSTAGE];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int wm = wave / WGN, wn = wave % WGN;
    const int q = lane / 16, j = lane % 16;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    const int tiles = (n + 15) / 16;
    const int total = tiles_m * tiles_n;
    // a tile's origin and operand ranges (vb: the block index of the one-block-per-tile form)
    struct Tile {
        int row0, col0;
        int32x4_t rsx, rsw;
        size_t srec[NT];
    };
    auto setup = [&](int vb, Tile &T) {
        int tm, tn;
        xcd_tile(vb, PERSIST ? total : (int)gridDim.x, tiles_m, tiles_n, tm, tn);
        T.row0 = tm * BM;
        T.col0 = tn * BN;
        const int tile0 = T.col0 / 16;
        T.rsx = buffer_rsrc(x + (size_t)T.row0 * k, (uint32_t)(min(BM, m - T.row0) * k * 2));
        T.rsw = buffer_rsrc(codes + (size_t)tile0 * kbs * 1024, (uint32_t)(min(BN / 16, tiles - tile0) * kbs * 1024));
        // scale records of this wave's tiles (clamped to a real tile past n)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) T.srec[nt] = (size_t)min(tile0 + wn * NT + nt, tiles - 1) * kbs * 128;
    };
    int vb = blockIdx.x;
    Tile cur_t;
    setup(vb, cur_t);
    const uint32_t xs_lds = lds_address(xs), ws_lds = lds_address(ws);

    // Activation DMA: lane (q, j) of instruction blk fills slot j of row
    // 4*blk + q, whose source chunk is j ^ (row & 15) = j ^ q ^ 4*(blk & 3).
    const uint32_t xlane = (uint32_t)(q * k * 2);
    const int cx = j ^ q;
    // the next step's loads are spread over the first groups: over two, each
    // load has longer to land than over four (config 5: 1.526-1.529 against
    // 1.540-1.543 ms with f16 output, 1.545-1.556 against 1.572-1.582 with f32;
    // the encoder 6.78-6.83 against 6.86-6.93 ms; all at once: in between)
    constexpr int DMA_GROUPS = 2;
    constexpr int DMA_N = XPW + WPW;
    // loads [DMA_N*part/DMA_GROUPS, DMA_N*(part+1)/DMA_GROUPS) of one stage
    // (k % 128 == 0: every chunk of a step is inside the row)
    auto dma_part = [&](int stage, int kb, int part, int32x4_t rx, int32x4_t rw) {
        const int kk = kb * 128;
#pragma unroll
        for (int p = 0; p < DMA_N; p++) {
            if (p < DMA_N * part / DMA_GROUPS || p >= DMA_N * (part + 1) / DMA_GROUPS) continue;
            if (p < XPW) {
                const int c = cx ^ (4 * (p & 3));
                const int blk = wave * XPW + p;
                const uint32_t voff = xlane + (uint32_t)(blk * 4 * k * 2 + kk * 2) + (uint32_t)(c * 16);
                dma16(__builtin_amdgcn_readfirstlane(xs_lds + stage * XSTAGE + blk * 1024), voff, rx);
            } else {
                const int t = wave * WPW + (p - XPW);  // uniform; past the tile's chunks when BN / 16 is not a multiple of WAVES
                if (BN / 16 % WAVES == 0 || t < BN / 16)
                    dma16(__builtin_amdgcn_readfirstlane(ws_lds + stage * WSTAGE + t * 1024),
                          (uint32_t)((t * kbs + kb) * 1024 + lane * 16), rw);
            }
        }
    };
    // scale records: a uniform tile offset plus the lane's row
    const uint8_t *const srow = scales + j * 8;
    auto load_scales = [&](uint2_t *sc, int kb, const size_t *srec) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) sc[nt] = *(const uint2_t *)(srow + srec[nt] + (size_t)kb * 128);
    };

    float4_t acc[MB][NT];
#pragma unroll
    for (int a = 0; a < MB; a++)
#pragma unroll
        for (int b = 0; b < NT; b++) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    // nibble masks in SGPRs and the f16 exponent in a VGPR (held opaque so
    // they are not folded back into literals, which v_and_or_b32 cannot take)
    uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, magic_v = 0x64006400u;
    asm volatile("" : "+s"(mlo), "+s"(mhi), "+v"(magic_v));
    constexpr int HM = MB / 2;  // activation fragments per group
    // Activation rows of this wave are r = wm*TM + 16*mb + j, so r & 15 = j.
    // Group g = 2s + h covers run s and fragment rows h*HM .. h*HM + HM - 1.
    auto read_x = [&](const uint8_t *xst, int g, half8_t *xf) {
        const int s = g / 2, h = g % 2;
        const uint8_t *base = xst + (wm * TM + h * HM * 16 + j) * 256 + (((4 * s + q) ^ j) * 16);
#pragma unroll
        for (int x2 = 0; x2 < HM; x2++) xf[x2] = *(const half8_t *)(base + x2 * 16 * 256);
    };
    // word s of the code chunks of tiles [t0, t1) -> f16 weight fragments of
    // run s. A lane's 16-byte chunk is read whole at run 0 (lanes 16 bytes
    // apart: no bank conflicts, unlike one 4-byte word per lane).
    uint4_t cw[NT];
    auto dequant_part = [&](const uint8_t *wst, const uint2_t *sc, int s, half8_t *wf, int t0, int t1) {
#pragma unroll
        for (int nt = t0; nt < t1; nt++) {
            if (s == 0) cw[nt] = *(const uint4_t *)(wst + ((wn * NT + nt) * 64 + lane) * 16);
            const uint32_t word = cw[nt][s];
            half_t sh;
            if (G32)
                sh = __builtin_bit_cast(half_t, (unsigned short)((sc[nt][s >> 1] >> (16 * (s & 1))) & 0xffffu));
            else
                sh = (half_t)word_as_float(sc[nt][s >> 1]);
            const half2_t s2 = {sh, sh};
            uint4_t c8 = unpack_codes_c(word, mlo, mhi, magic_v);
#pragma unroll
            for (int e = 0; e < 4; e++) c8[e] = half2_as_word(word_as_half2(c8[e]) * s2);
            wf[nt] = as_half8(c8);
        }
    };
    // Group g = 2s + h: 16 MFMAs of run s on fragment rows h*HM.., interleaved
    // (sched_group_barrier) with the next group's activation reads, half of
    // run s+1's dequantization and, in the first DMA_GROUPS groups, a slice
    // of the next step's stage loads.
    auto compute = [&](const uint8_t *xst, const uint8_t *wst, const uint2_t *sc, int next_stage, int next_kb,
                       int32x4_t rx, int32x4_t rw) {
        half8_t xf[2][HM], wf[2][NT];
        read_x(xst, 0, xf[0]);
        dequant_part(wst, sc, 0, wf[0], 0, NT);
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int s = g / 2, h = g % 2;
            if (g < DMA_GROUPS) dma_part(next_stage, next_kb, g, rx, rw);
            if (g + 1 < 8) read_x(xst, g + 1, xf[(g + 1) & 1]);
            if (s + 1 < 4) dequant_part(wst, sc, s + 1, wf[(s + 1) & 1], h * NT / 2, (h + 1) * NT / 2);
#pragma unroll
            for (int x2 = 0; x2 < HM; x2++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    acc[h * HM + x2][nt] = mfma_f16(wf[s & 1][nt], xf[g & 1][x2], acc[h * HM + x2][nt]);
            // one MFMA, then a share of the reads and VALU work, repeated
#pragma unroll
            for (int i = 0; i < HM * NT; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (i < HM + 1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, VALU_PER_MFMA, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    uint2_t sc[NT], nsc[NT];
#pragma unroll
    for (int part = 0; part < DMA_GROUPS; part++) dma_part(0, 0, part, cur_t.rsx, cur_t.rsw);
    // the last step's "next" loads go to a zero-length buffer: no traffic, no branch
    const int32x4_t none = {cur_t.rsx[0], cur_t.rsx[1], 0, cur_t.rsx[3]};
    load_scales(sc, 0, cur_t.srec);
    int stage = 0;
    const bool vec = (n & 3) == 0 && (ldo & 3) == 0 && ((uintptr_t)out & 15) == 0 &&
                     (EPI != 3 || ((uintptr_t)residual & 7) == 0);
    for (;;) {
        const int nvb = vb + (int)gridDim.x;
        const bool has_next = PERSIST && nvb < total;
        Tile nxt_t;
        if (has_next) setup(nvb, nxt_t);
        for (int kb = 0; kb < kbs; kb++) {
            // this wave's loads of step kb are done; the barrier covers every wave
            // (and every wave has finished reading the stage the next loads overwrite)
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0); the compiler sees it too
            __builtin_amdgcn_s_barrier();
            const bool more = kb + 1 < kbs;
            if (more) load_scales(nsc, kb + 1, cur_t.srec);
            else if (has_next) load_scales(nsc, 0, nxt_t.srec);
            const int32x4_t rx = more ? cur_t.rsx : (has_next ? nxt_t.rsx : none);
            const int32x4_t rw = more ? cur_t.rsw : (has_next ? nxt_t.rsw : none);
            compute(xs + stage * XSTAGE, ws + stage * WSTAGE, sc, stage ^ 1, more ? kb + 1 : 0, rx, rw);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) sc[nt] = nsc[nt];
            stage ^= 1;
        }

        // epilogue: acc[mb][nt][v] = Y[row][col + v]
        const int row0 = cur_t.row0, col0 = cur_t.col0;
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            const int r = row0 + wm * TM + mb * 16 + j;
            if (r >= m) continue;
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int c = col0 + wn * TN + nt * 16 + 4 * q;
                if (c >= n) continue;
                const size_t at = (size_t)r * ldo + c;
                float v[4] = {acc[mb][nt][0], acc[mb][nt][1], acc[mb][nt][2], acc[mb][nt][3]};
                if (EPI == 0) {
                    if (vec) {
                        *(float4_t *)((float *)out + at) = float4_t{v[0], v[1], v[2], v[3]};
                    } else {
                        for (int e = 0; e < 4; e++)
                            if (c + e < n) ((float *)out)[at + e] = v[e];
                    }
                } else {
                    half_t o[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if (EPI == 1) o[e] = (half_t)v[e];
                        else if (EPI == 2) o[e] = (half_t)f32_rounded(gelu_erf(v[e]));
                        else o[e] = (half_t)0.0f;
                    }
                    if (EPI == 3) {
                        if (vec) {
                            const uint2_t rw = *(const uint2_t *)(residual + at);
                            const half2_t r01 = word_as_half2(rw[0]), r23 = word_as_half2(rw[1]);
                            o[0] = (half_t)f32_rounded(v[0] + (float)r01[0]);
                            o[1] = (half_t)f32_rounded(v[1] + (float)r01[1]);
                            o[2] = (half_t)f32_rounded(v[2] + (float)r23[0]);
                            o[3] = (half_t)f32_rounded(v[3] + (float)r23[1]);
                        } else {
                            for (int e = 0; e < 4; e++)
                                if (c + e < n) o[e] = (half_t)f32_rounded(v[e] + (float)residual[at + e]);
                        }
                    }
                    if (vec) {
                        const half2_t o01 = {o[0], o[1]}, o23 = {o[2], o[3]};
                        *(uint2_t *)((half_t *)out + at) = uint2_t{half2_as_word(o01), half2_as_word(o23)};
                    } else {
                        for (int e = 0; e < 4; e++)
                            if (c + e < n) ((half_t *)out)[at + e] = o[e];
                    }
                }
            }
        }
        if (!has_next) break;
#pragma unroll
        for (int a = 0; a < MB; a++)
#pragma unroll
            for (int b = 0; b < NT; b++) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};
        vb = nvb;
        cur_t = nxt_t;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // no LDS write in flight once the block ends
}

// ============================================================================
// pipelined grouped W{4,8}A{8,4} (bit-exact, large M)
// ============================================================================
//
// The reference's fused fold (int8.rs:524-585) with each group's exact int32
// dot taken by v_mfma_i32_16x16x64_i8:
//     acc = fma(f32(dot_g), sw[g][c] * sx[r][g], acc)   for g = 0, 1, ... in order,
// so the outputs equal grouped_kernel's (and the oracle's) bit for bit.
// Block tile BM x BN on WGM x WGN waves; one k-step covers GS 64-groups (2 or
// 4), in two LDS stages filled by buffer_load ... lds while the other is
// computed:
//  - activation codes: BM rows x 64 GS bytes (chunk c of row r at slot
//    c ^ swz(r), swz(r) = (r >> 1) & 7 for 128-byte rows and r & 15 for
//    256-byte rows: conflict-free for the 16 rows of a fragment read);
//  - weight codes: Q4 GS/2 1 KiB tile16x128 chunks per 16-column tile, Q8 GS
//    1 KiB tile16x64 chunks;
//  - weight scales: 64 GS bytes per tile, as [k-step pair][tile][128 B] (Q4:
//    [row][group] f32 pairs, Q8: [group][row]); activation scales: BM rows x
//    GS f32.
// The MFMA takes the weight operand first, so lane (q, j) holds the dots of
// four consecutive output columns of one row: its weight scales are one
// 16-byte LDS read and its activation scale one 4-byte read. The fold (the
// dot as f32, the scale product and the fma per output and group) is VALU
// work and bounds the kernel; the MFMAs take about a third of its time.
// Groups past `groups` (the tail of a k-step) are not folded.
// AFF (fitted affine Q4, int8.rs:566-571): the offsets (the group-64 scale
// layout) and sxq = sx * f32(sum of the row's group codes) are staged like the
// scales, and each group's fold is followed by acc = fma(offset, sxq, acc).
template <int BITS, int BM, int BN, int WGM, int WGN, bool AFF = false, int GS = 2>
__global__ __launch_bounds__(WGM *WGN * 64) void grouped_pipe_kernel(
    const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales, const int8_t *__restrict__ q,
    const float *__restrict__ sx, int m, int n, int groups, int kbs, float *y, const float *res,
    const int *__restrict__ bad, const uint8_t *__restrict__ offsets = nullptr,
    const float *__restrict__ sxq = nullptr) {
    static_assert(!AFF || BITS == 4, "affine offsets are a Q4 form");
    static_assert(GS == 2 || GS == 4, "two or four groups per k-step");
    constexpr int WAVES = WGM * WGN;
    constexpr int TM = BM / WGM, TN = BN / WGN, MB = TM / 16, NT = TN / 16;
    constexpr int TILES = BN / 16;
    constexpr int ROWB = 64 * GS, CH = ROWB / 16, RPI = 1024 / ROWB;  // row bytes, chunks, rows per 1 KiB
    constexpr int KBS = GS / 2;                                         // Q4 k-blocks (and scale pairs) per step
    constexpr int XSTAGE = BM * ROWB;
    constexpr int CSTAGE = TILES * 1024 * (BITS == 4 ? KBS : GS);
    constexpr int SWSTAGE = TILES * 128 * KBS;
    constexpr int SXSTAGE = BM * 4 * GS;
    // 1 KiB loads of a stage, dealt round robin to the waves: XI of RPI
    // activation rows, CI code chunks, SI of 64 activation scales
    constexpr int XI = BM / RPI, CI = CSTAGE / 1024, SI = BM * GS / 64;
    constexpr int XPW = (XI + WAVES - 1) / WAVES, CPW = (CI + WAVES - 1) / WAVES, SPW = (SI + WAVES - 1) / WAVES;
    static_assert(XI * RPI == BM && SI * 64 == BM * GS, "whole 1 KiB activation and 256 B scale loads");
    static_assert(TILES == 8 || TILES == 4, "one 1 KiB (or 512 B) weight-scale load per k-step pair");
    __shared__ __align__(16) uint8_t xs[2 * XSTAGE];
    __shared__ __align__(16) uint8_t cs[2 * CSTAGE];
    __shared__ __align__(16) uint8_t sws[2 * SWSTAGE];
    __shared__ __align__(16) uint8_t sxs[2 * SXSTAGE];
    __shared__ __align__(16) uint8_t ofs[AFF ? 2 * SWSTAGE : 16];
    __shared__ __align__(16) uint8_t sqs[AFF ? 2 * SXSTAGE : 16];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int wm = wave / WGN, wn = wave % WGN;
    const int qd = lane / 16, j = lane % 16;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    const int tiles = (n + 15) / 16, tile0 = col0 / 16, tvalid = min(TILES, tiles - tile0);
    const int rvalid = min(BM, m - row0);
    const uint32_t rowbytes = (uint32_t)groups * 64;
    const int32x4_t rq = buffer_rsrc(q + (size_t)row0 * rowbytes, (uint32_t)rvalid * rowbytes);
    const int32x4_t rc = buffer_rsrc(codes + (size_t)tile0 * kbs * 1024, (uint32_t)(tvalid * kbs * 1024));
    const uint32_t swtile = BITS == 4 ? (uint32_t)kbs * 128 : (uint32_t)groups * 64;  // scale bytes per tile
    const int32x4_t rw = buffer_rsrc(scales + (size_t)tile0 * swtile, (uint32_t)tvalid * swtile);
    const int32x4_t rs = buffer_rsrc(sx + (size_t)row0 * groups, (uint32_t)(rvalid * groups * 4));
    const uint32_t xs_lds = lds_address(xs), cs_lds = lds_address(cs);
    const uint32_t sws_lds = lds_address(sws), sxs_lds = lds_address(sxs);
    int32x4_t ro = rw, rsq = rs;
    uint32_t ofs_lds = 0, sqs_lds = 0;
    if (AFF) {
        ro = buffer_rsrc(offsets + (size_t)tile0 * swtile, (uint32_t)tvalid * swtile);
        rsq = buffer_rsrc(sxq + (size_t)row0 * groups, (uint32_t)(rvalid * groups * 4));
        ofs_lds = lds_address(ofs);
        sqs_lds = lds_address(sqs);
    }
    auto swz = [](int r) { return GS == 2 ? (r >> 1) & 7 : r & 15; };

    // activation loads: lane l of instruction blk fills slot l % CH of row
    // RPI*blk + l/CH; the swizzle depends on blk only through blk % NX
    constexpr int NX = GS == 2 ? 2 : 4;
    const int lrow = lane / CH;
    uint32_t xoff[NX];
#pragma unroll
    for (int u = 0; u < NX; u++)
        xoff[u] = (uint32_t)(lrow * rowbytes + (((lane % CH) ^ swz(lrow + RPI * u)) * 16));
    auto load_stage = [&](int stage, int st, bool live) {
        const int32x4_t nq = live ? rq : int32x4_t{rq[0], rq[1], 0, rq[3]};
        const int32x4_t nc = live ? rc : int32x4_t{rc[0], rc[1], 0, rc[3]};
        const int32x4_t nw = live ? rw : int32x4_t{rw[0], rw[1], 0, rw[3]};
        const int32x4_t ns = live ? rs : int32x4_t{rs[0], rs[1], 0, rs[3]};
        const int32x4_t no = live ? ro : int32x4_t{ro[0], ro[1], 0, ro[3]};
        const int32x4_t nsq = live ? rsq : int32x4_t{rsq[0], rsq[1], 0, rsq[3]};
#pragma unroll
        for (int p = 0; p < XPW; p++) {
            const int blk = wave + p * WAVES;
            if (XI % WAVES == 0 || blk < XI)
                dma16(__builtin_amdgcn_readfirstlane(xs_lds + stage * XSTAGE + blk * 1024),
                      xoff[blk % NX] + (uint32_t)(blk * RPI) * rowbytes + (uint32_t)st * ROWB, nq);
        }
#pragma unroll
        for (int p = 0; p < CPW; p++) {
            // Q4: chunk ci is k-block ci % KBS of the step for tile ci / KBS; Q8: group ci % GS
            const int ci = wave + p * WAVES;
            const int per = BITS == 4 ? KBS : GS;
            const int t = ci / per, kc = st * per + ci % per;
            if (CI % WAVES == 0 || ci < CI)
                dma16(__builtin_amdgcn_readfirstlane(cs_lds + stage * CSTAGE + ci * 1024),
                      (uint32_t)((t * kbs + kc) * 1024 + lane * 16), nc);
        }
        if (wave == WAVES - 1 && (TILES == 8 || lane < TILES * 8)) {
#pragma unroll
            for (int u = 0; u < KBS; u++) {  // one load per pair of groups: lane -> tile l/8, piece l%8
                const int t = lane / 8;
                const uint32_t off = BITS == 4 ? (uint32_t)(t * kbs + st * KBS + u) * 128
                                               : (uint32_t)(t * groups + GS * st + 2 * u) * 64;
                const uint32_t lds = sws_lds + stage * SWSTAGE + u * TILES * 128;
                dma16(__builtin_amdgcn_readfirstlane(lds), off + (uint32_t)(lane % 8) * 16, nw);
                if (AFF)
                    dma16(__builtin_amdgcn_readfirstlane(ofs_lds + stage * SWSTAGE + u * TILES * 128),
                          off + (uint32_t)(lane % 8) * 16, no);
            }
        }
#pragma unroll
        for (int p = 0; p < SPW; p++) {
            const int si = wave + p * WAVES;
            const int r = si * (64 / GS) + lane / GS;
            if (SI % WAVES == 0 || si < SI) {
                dma4(__builtin_amdgcn_readfirstlane(sxs_lds + stage * SXSTAGE + si * 256),
                     (uint32_t)((r * groups + GS * st + lane % GS) * 4), ns);
                if (AFF)
                    dma4(__builtin_amdgcn_readfirstlane(sqs_lds + stage * SXSTAGE + si * 256),
                         (uint32_t)((r * groups + GS * st + lane % GS) * 4), nsq);
            }
        }
    };

    float4_t acc[MB][NT];
#pragma unroll
    for (int a = 0; a < MB; a++)
#pragma unroll
        for (int b = 0; b < NT; b++) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};
    const bool nan_out = bad != nullptr && *bad != 0;
    const int steps = (groups + GS - 1) / GS;

    auto x_frag = [&](const uint8_t *xst, int r, int gp) {
        if (BITS == 4) {
            const int c1 = 4 * gp + qd / 2, c2 = c1 + 2;
            const uint2_t a0 = *(const uint2_t *)(xst + r * ROWB + ((c1 ^ swz(r)) * 16) + 8 * (qd & 1));
            const uint2_t a1 = *(const uint2_t *)(xst + r * ROWB + ((c2 ^ swz(r)) * 16) + 8 * (qd & 1));
            return int4_t{(int)a0[0], (int)a0[1], (int)a1[0], (int)a1[1]};
        }
        const int c = 4 * gp + qd;
        return *(const int4_t *)(xst + r * ROWB + ((c ^ swz(r)) * 16));
    };
    // group gp's weight fragment, scales (and offsets) of tile t
    auto w_frag = [&](const uint8_t *cst, int t, int gp) {
        if (BITS == 4) {
            const uint2_t wds = *(const uint2_t *)(cst + (t * KBS + gp / 2) * 1024 + lane * 16 + (gp % 2) * 8);
            return q4_operand16(wds[0], wds[1]);
        }
        return *(const int4_t *)(cst + (t * GS + gp) * 1024 + lane * 16);
    };
    auto w_scales = [&](const uint8_t *swst, int t, int gp) {
        const uint8_t *rec = swst + (gp / 2) * TILES * 128 + t * 128;
        if (BITS == 4) {
            const float4_t s01 = *(const float4_t *)(rec + qd * 32);       // rows 4qd, 4qd+1
            const float4_t s23 = *(const float4_t *)(rec + qd * 32 + 16);  // rows 4qd+2, 4qd+3
            return gp % 2 ? float4_t{s01[1], s01[3], s23[1], s23[3]} : float4_t{s01[0], s01[2], s23[0], s23[2]};
        }
        return *(const float4_t *)(rec + (gp % 2) * 64 + qd * 16);
    };

    // one group of a stage: weight fragments and scales once, then per row
    // block the activation fragment, its scale, NT MFMAs and the fold
    auto fold_group = [&](const uint8_t *xst, const uint8_t *cst, const uint8_t *swst, const uint8_t *sxst,
                          const uint8_t *ofst, const uint8_t *sqst, int gp) {
        int4_t bfr[NT];
        float4_t swv[NT], ofv[AFF ? NT : 1];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int t = wn * NT + nt;
            bfr[nt] = w_frag(cst, t, gp);
            swv[nt] = w_scales(swst, t, gp);
            if (AFF) ofv[AFF ? nt : 0] = w_scales(ofst, t, gp);
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            const int r = wm * TM + mb * 16 + j;
            const int4_t afr = x_frag(xst, r, gp);
            const float sxv = *(const float *)(sxst + r * 4 * GS + gp * 4);
            const float sqv = AFF ? *(const float *)(sqst + r * 4 * GS + gp * 4) : 0.0f;
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int4_t d = mfma_dot<BITS>(bfr[nt], afr);
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    acc[mb][nt][v] = __builtin_fmaf(dot_of<BITS>(d[v]), __fmul_rn(swv[nt][v], sxv), acc[mb][nt][v]);
                    if (AFF) acc[mb][nt][v] = __builtin_fmaf(ofv[AFF ? nt : 0][v], sqv, acc[mb][nt][v]);
                }
            }
        }
    };

    // Small wave tiles (MB * NT <= 4) take a whole k-step at once: every LDS
    // read of its groups, then every MFMA, then the folds in group order, so
    // a wave waits once per step for its reads and once for its first dots.
    constexpr bool BATCH = MB * NT <= 4;
    auto fold_step = [&](const uint8_t *xst, const uint8_t *cst, const uint8_t *swst, const uint8_t *sxst,
                         const uint8_t *ofst, const uint8_t *sqst, int live_groups) {
        int4_t bfr[GS][NT];
        float4_t swv[GS][NT], ofv[GS][AFF ? NT : 1];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int t = wn * NT + nt;
#pragma unroll
            for (int gp = 0; gp < GS; gp++) {
                bfr[gp][nt] = w_frag(cst, t, gp);
                swv[gp][nt] = w_scales(swst, t, gp);
                if (AFF) ofv[gp][AFF ? nt : 0] = w_scales(ofst, t, gp);
            }
        }
        int4_t afr[GS][MB];
        float sxv[GS][MB], sqv[GS][MB];
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            const int r = wm * TM + mb * 16 + j;
#pragma unroll
            for (int gp = 0; gp < GS; gp++) afr[gp][mb] = x_frag(xst, r, gp);
            if (GS == 2) {
                const uint2_t s2 = *(const uint2_t *)(sxst + r * 8);
                sxv[0][mb] = word_as_float(s2[0]);
                sxv[1][mb] = word_as_float(s2[1]);
            } else {
                const uint4_t s4 = *(const uint4_t *)(sxst + r * 16);
#pragma unroll
                for (int gp = 0; gp < GS; gp++) sxv[gp][mb] = word_as_float(s4[gp]);
            }
            if (AFF) {
#pragma unroll
                for (int gp = 0; gp < GS; gp++) sqv[gp][mb] = *(const float *)(sqst + r * 4 * GS + gp * 4);
            }
        }
        int4_t d[GS][MB][NT];
#pragma unroll
        for (int gp = 0; gp < GS; gp++)
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) d[gp][mb][nt] = mfma_dot<BITS>(bfr[gp][nt], afr[gp][mb]);
#pragma unroll
        for (int gp = 0; gp < GS; gp++) {
            if (gp >= live_groups) break;
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int v = 0; v < 4; v++) {
                        acc[mb][nt][v] = __builtin_fmaf(dot_of<BITS>(d[gp][mb][nt][v]),
                                                        __fmul_rn(swv[gp][nt][v], sxv[gp][mb]), acc[mb][nt][v]);
                        if (AFF)
                            acc[mb][nt][v] = __builtin_fmaf(ofv[gp][AFF ? nt : 0][v], sqv[gp][mb], acc[mb][nt][v]);
                    }
        }
    };

    if (!nan_out) {
        // the step loop unrolled by its two stages, so every LDS address is a
        // per-lane offset fixed for the kernel plus an immediate
        auto run_step = [&](auto stage, int st) {
            constexpr int C = decltype(stage)::value;
            // this wave's loads of step st are done; the barrier covers every wave
            // (and every wave has finished reading the stage the next loads overwrite)
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __builtin_amdgcn_s_barrier();
            load_stage(C ^ 1, st + 1, st + 1 < steps);
            const uint8_t *xst = xs + C * XSTAGE, *cst = cs + C * CSTAGE;
            const uint8_t *swst = sws + C * SWSTAGE, *sxst = sxs + C * SXSTAGE;
            const uint8_t *ofst = ofs + (AFF ? C * SWSTAGE : 0), *sqst = sqs + (AFF ? C * SXSTAGE : 0);
            const int live = min(GS, groups - GS * st);
            if constexpr (BATCH) {
                fold_step(xst, cst, swst, sxst, ofst, sqst, live);
            } else {
#pragma unroll
                for (int gp = 0; gp < GS; gp++)
                    if (gp < live) fold_group(xst, cst, swst, sxst, ofst, sqst, gp);
            }
        };
        load_stage(0, 0, true);
        for (int st = 0; st < steps; st += 2) {
            run_step(std::integral_constant<int, 0>{}, st);
            if (st + 1 < steps) run_step(std::integral_constant<int, 1>{}, st + 1);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // no LDS write in flight once the block ends
    }

    // acc[mb][nt][v] = Y[row][col + v]; with `res` (which may be y itself) the
    // kernel stores res + Y, the same float add as a separate residual pass
    const bool vec = (n & 3) == 0 && ((uintptr_t)y & 15) == 0 && ((uintptr_t)res & 15) == 0;
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int r = row0 + wm * TM + mb * 16 + j;
        if (r >= m) continue;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int c = col0 + wn * TN + nt * 16 + 4 * qd;
            if (c >= n) continue;
            float4_t v = acc[mb][nt];
            if (nan_out) v = float4_t{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
            float *dst = y + (size_t)r * n + c;
            const float *add = res + (size_t)r * n + c;
            if (vec) {
                if (res && !nan_out) {
                    const float4_t h = *(const float4_t *)add;
                    for (int e = 0; e < 4; e++) v[e] = __fadd_rn(h[e], v[e]);
                }
                *(float4_t *)dst = v;
            } else {
                for (int e = 0; e < 4; e++)
                    if (c + e < n) dst[e] = res && !nan_out ? __fadd_rn(add[e], v[e]) : v[e];
            }
        }
    }
}

// Fused MLP on the same pipeline (grouped_q4_mlp.wgsl:1-105, int8.rs fold):
// gate and up products of one BM-row x 64-column block (one requant block),
// silu(g) * u, then the A8 requantization of each row's 64 columns, exactly
// as mlp_requant_kernel computes them. BM/32 waves stacked along M (wave tile
// 32 x 64): a row's 64 columns are held by the four lanes j, j+16, j+32,
// j+48 of one wave, so the row maximum is two shuffles. Q4 weights. BM is
// 256 (8 waves) or 128 (4 waves, half the LDS: two blocks fit a CU). With
// WN = 2 the waves are paired along N instead (wave tile 64 rows x 32 columns
// of each weight): a weight fragment is unpacked once for four row blocks
// rather than two, and the row maximum takes one exchange through LDS between
// the pair.
template <int BM, int WN = 1>
__global__ __launch_bounds__(BM / 32 * 64) void mlp_pipe_kernel(
    const uint8_t *__restrict__ gcodes, const uint8_t *__restrict__ gscales, const uint8_t *__restrict__ ucodes,
    const uint8_t *__restrict__ uscales, const int8_t *__restrict__ q, const float *__restrict__ sx, int m, int n,
    int groups, int kbs, int8_t *__restrict__ qo, float *__restrict__ so, const int *__restrict__ bad) {
    static_assert(BM == 256 || BM == 128, "8 or 4 waves");
    static_assert(WN == 1 || WN == 2, "one or two waves across the 64 columns");
    constexpr int WAVES = BM / 32, MB = 2 * WN, NT = 4 / WN, WR = 32 * WN;
    constexpr int XSTAGE = BM * 128;   // activation codes, 2 groups per step
    constexpr int CSTAGE = 8 * 1024;   // gate tiles 0-3, up tiles 0-3: one tile16x128 chunk each
    constexpr int SWSTAGE = 2 * 512;   // scale records: [weight][4 tiles x 128 B]
    constexpr int SXSTAGE = BM * 8;
    constexpr int XPW = BM / 8 / WAVES;
    __shared__ __align__(16) uint8_t xs[2 * XSTAGE];
    __shared__ __align__(16) uint8_t cs[2 * CSTAGE];
    __shared__ __align__(16) uint8_t sws[2 * SWSTAGE];
    __shared__ __align__(16) uint8_t sxs[2 * SXSTAGE];
    __shared__ float pair_max[WN == 2 ? BM * 2 : 1];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int wm = wave / WN, wn = wave % WN;
    const int qd = lane / 16, j = lane % 16;
    const int tiles_m = (m + BM - 1) / BM, tiles_n = n / 64;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
    const int row0 = tm * BM, col0 = tn * 64, tile0 = col0 / 16;
    const int rvalid = min(BM, m - row0);
    const uint32_t rowbytes = (uint32_t)groups * 64;
    const int32x4_t rq = buffer_rsrc(q + (size_t)row0 * rowbytes, (uint32_t)rvalid * rowbytes);
    const int32x4_t rcg = buffer_rsrc(gcodes + (size_t)tile0 * kbs * 1024, (uint32_t)(4 * kbs * 1024));
    const int32x4_t rcu = buffer_rsrc(ucodes + (size_t)tile0 * kbs * 1024, (uint32_t)(4 * kbs * 1024));
    const int32x4_t rwg = buffer_rsrc(gscales + (size_t)tile0 * kbs * 128, (uint32_t)(4 * kbs * 128));
    const int32x4_t rwu = buffer_rsrc(uscales + (size_t)tile0 * kbs * 128, (uint32_t)(4 * kbs * 128));
    const int32x4_t rs = buffer_rsrc(sx + (size_t)row0 * groups, (uint32_t)(rvalid * groups * 4));
    const uint32_t xs_lds = lds_address(xs), cs_lds = lds_address(cs);
    const uint32_t sws_lds = lds_address(sws), sxs_lds = lds_address(sxs);

    const int lrow = lane / 8;
    const uint32_t xoff[2] = {
        (uint32_t)(lrow * rowbytes + (((lane % 8) ^ ((lrow >> 1) & 7)) * 16)),
        (uint32_t)(lrow * rowbytes + (((lane % 8) ^ (((lrow + 8) >> 1) & 7)) * 16))};
    auto zero_len = [](int32x4_t r) { return int32x4_t{r[0], r[1], 0, r[3]}; };
    auto load_stage = [&](int stage, int st, bool live) {
        const int32x4_t nq = live ? rq : zero_len(rq);
#pragma unroll
        for (int p = 0; p < XPW; p++) {
            const int blk = wave * XPW + p;
            dma16(__builtin_amdgcn_readfirstlane(xs_lds + stage * XSTAGE + blk * 1024),
                  xoff[p & 1] + (uint32_t)(blk * 8) * rowbytes + (uint32_t)st * 128, nq);
        }
#pragma unroll
        for (int ch = wave; ch < 8; ch += WAVES) {  // chunk ch: gate tiles for ch < 4, up tiles for ch >= 4
            const uint32_t lds = __builtin_amdgcn_readfirstlane(cs_lds + stage * CSTAGE + ch * 1024);
            const uint32_t off = (uint32_t)(((ch % 4) * kbs + st) * 1024 + lane * 16);
            if (ch < 4) dma16(lds, off, live ? rcg : zero_len(rcg));
            else dma16(lds, off, live ? rcu : zero_len(rcu));
        }
        if (wave < 2 && lane < 32) {  // wave 0 the gate records, wave 1 the up records: lane l -> tile l / 8, piece l % 8
            const uint32_t lds = __builtin_amdgcn_readfirstlane(sws_lds + stage * SWSTAGE + wave * 512);
            const uint32_t off = (uint32_t)(((lane / 8) * kbs + st) * 128 + (lane % 8) * 16);
            if (wave == 0) dma16(lds, off, live ? rwg : zero_len(rwg));
            else dma16(lds, off, live ? rwu : zero_len(rwu));
        }
        {
            const int r = wave * 32 + lane / 2;
            dma4(__builtin_amdgcn_readfirstlane(sxs_lds + stage * SXSTAGE + wave * 256),
                 (uint32_t)((r * groups + 2 * st + (lane & 1)) * 4), live ? rs : zero_len(rs));
        }
    };

    float4_t ga[MB][NT], ua[MB][NT];
#pragma unroll
    for (int a = 0; a < MB; a++)
#pragma unroll
        for (int b = 0; b < NT; b++) ga[a][b] = ua[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};
    const bool nan_out = bad != nullptr && *bad != 0;
    const int steps = (groups + 1) / 2;

    auto fold_group = [&](const uint8_t *xst, const uint8_t *cst, const uint8_t *swst, const uint8_t *sxst, int gp) {
        int4_t gb[NT], ub[NT];
        float4_t gs[NT], us[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int wgt = 0; wgt < 2; wgt++) {
                const int t = wn * NT + nt;
                const uint2_t wds = *(const uint2_t *)(cst + (wgt * 4 + t) * 1024 + lane * 16 + gp * 8);
                const uint2_t lo = nibbles_to_i8x16(wds[0]), hi = nibbles_to_i8x16(wds[1]);
                const int4_t b = int4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};  // 16 * code
                const float4_t s01 = *(const float4_t *)(swst + wgt * 512 + t * 128 + qd * 32);
                const float4_t s23 = *(const float4_t *)(swst + wgt * 512 + t * 128 + qd * 32 + 16);
                const float4_t sv = gp ? float4_t{s01[1], s01[3], s23[1], s23[3]} : float4_t{s01[0], s01[2], s23[0], s23[2]};
                if (wgt == 0) {
                    gb[nt] = b;
                    gs[nt] = sv;
                } else {
                    ub[nt] = b;
                    us[nt] = sv;
                }
            }
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
            const int r = wm * WR + mb * 16 + j;
            const int c1 = 4 * gp + qd / 2, c2 = c1 + 2;
            const uint2_t a0 = *(const uint2_t *)(xst + r * 128 + ((c1 ^ ((r >> 1) & 7)) * 16) + 8 * (qd & 1));
            const uint2_t a1 = *(const uint2_t *)(xst + r * 128 + ((c2 ^ ((r >> 1) & 7)) * 16) + 8 * (qd & 1));
            const int4_t afr = int4_t{(int)a0[0], (int)a0[1], (int)a1[0], (int)a1[1]};
            const float sxv = *(const float *)(sxst + r * 8 + gp * 4);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const int4_t gd = mfma_i8_biased16(gb[nt], afr);
                const int4_t ud = mfma_i8_biased16(ub[nt], afr);
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    ga[mb][nt][v] = __builtin_fmaf(dot_value16(gd[v]), __fmul_rn(gs[nt][v], sxv), ga[mb][nt][v]);
                    ua[mb][nt][v] = __builtin_fmaf(dot_value16(ud[v]), __fmul_rn(us[nt][v], sxv), ua[mb][nt][v]);
                }
            }
        }
    };

    if (!nan_out) {
        // unrolled by the two stages: every LDS address is a fixed per-lane offset plus an immediate
        auto run_step = [&](auto stage, int st) {
            constexpr int C = decltype(stage)::value;
            __builtin_amdgcn_s_waitcnt(0x0F70);
            __builtin_amdgcn_s_barrier();
            load_stage(C ^ 1, st + 1, st + 1 < steps);
            const uint8_t *xst = xs + C * XSTAGE, *cst = cs + C * CSTAGE;
            const uint8_t *swst = sws + C * SWSTAGE, *sxst = sxs + C * SXSTAGE;
            fold_group(xst, cst, swst, sxst, 0);
            if (2 * st + 1 < groups) fold_group(xst, cst, swst, sxst, 1);
        };
        load_stage(0, 0, true);
        for (int st = 0; st < steps; st += 2) {
            run_step(std::integral_constant<int, 0>{}, st);
            if (st + 1 < steps) run_step(std::integral_constant<int, 1>{}, st + 1);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // no LDS write in flight once the block ends
    }

    // silu(g) * u and the A8 requantization of the row's 64 columns
    const int blocks = n / 64;
    float val[MB][NT][4];
    float rmax[MB];
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        float local = 0.0f;
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float gv = ga[mb][nt][v];
                const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-gv)));
                val[mb][nt][v] = __fmul_rn(__fmul_rn(gv, sig), ua[mb][nt][v]);
                local = fmaxf(local, fabsf(val[mb][nt][v]));
            }
        local = fmaxf(local, __shfl_xor(local, 16));
        local = fmaxf(local, __shfl_xor(local, 32));
        rmax[mb] = local;
    }
    if (WN == 2) {  // the other half of each row's columns is in the paired wave
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
            if (qd == 0) pair_max[(wm * WR + mb * 16 + j) * 2 + wn] = rmax[mb];
        __syncthreads();
#pragma unroll
        for (int mb = 0; mb < MB; mb++) rmax[mb] = fmaxf(rmax[mb], pair_max[(wm * WR + mb * 16 + j) * 2 + (wn ^ 1)]);
    }
#pragma unroll
    for (int mb = 0; mb < MB; mb++) {
        const int r = row0 + wm * WR + mb * 16 + j;
        const float scale = fmaxf(__fdiv_rn(rmax[mb], 127.0f), FLT_MIN);
        const float inverse = __frcp_rn(scale);
        if (r >= m) continue;
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            uint32_t packed = 0;
            if (!nan_out) {
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float c = fminf(fmaxf(__builtin_rintf(__fmul_rn(val[mb][nt][v], inverse)), -127.0f), 127.0f);
                    packed |= ((uint32_t)(uint8_t)(int8_t)(int)c) << (8 * v);
                }
            }
            *(uint32_t *)(qo + (size_t)r * n + col0 + (wn * NT + nt) * 16 + 4 * qd) = packed;
        }
        if (qd == 0 && wn == 0) so[(size_t)r * blocks + tn] = nan_out ? __builtin_nanf("") : scale;
    }
}

inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// ---- variant tables -------------------------------------------------------------

const char *const kGemvNames[] = {"auto", "w16", "w8", "stream8", "stream4", "persist"};
const char *const kGemmNames[] = {"pipe-auto",   "256x256p2w8", "128x128p2w4", "128x256p2w8",
                                   "256x128w2x2", "128x128w2x2", "128x64w2x2", "256x256p2w8-persist",
                                   "256x192p2w8-persist", "256x128p2w8"};
const char *const kI8Names[] = {"256x256p2w8", "256x256p4k64w8", "256x128p3w8", "256x128p3",
                                 "128x128w2x2", "256x128w2x2", "64x64w2x2", "256x256p2w8-stream",
                                 "256x256p2w8-stream-mid", "256x128k64p2-stream2"};
const char *const kGroupedNames[] = {"pipe-auto",    "pipe256x128w8", "wave16x16",   "pipe128x128w4",
                                     "pipe64x128w2", "pipe128x128m8", "pipe128x128n8", "pipe32x128w8",
                                     "pipe64x128w8", "pipe32x128w8g4", "pipe64x128w8g4", "fewrow16",
                                     "pipe32x64w4",  "pipe64x64w8"};
const char *const kMlpNames[] = {"pipe-auto", "pipe256x64w8", "pipe128x64w4", "wave16x64", "pipe256x64n2", "pipe128x64n2"};
const char *const kDeltaNames[] = {"chunked64", "chunked64-c32", "recurrent", "recurrent-rolled", "auto"};
const char *const kNormNames[] = {"fused", "separate"};

template <int W, int MPAD, bool G32, int NP>
void gemv_launch_np(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    using S = GemvShape<MPAD>;
    const size_t lds = (size_t)W * S::SLICE;
    static bool configured[64] = {};  // the LDS limit is a per-device function attribute
    int dev = 0;
    hipGetDevice(&dev);
    if (dev >= 0 && dev < 64 && !configured[dev]) {
        if (hipFuncSetAttribute((const void *)gemv_kernel<W, MPAD, G32, NP>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess)
            configured[dev] = true;
    }
    hipLaunchKernelGGL((gemv_kernel<W, MPAD, G32, NP>), dim3(w.tiles()), dim3(W * 64), lds, s, w.codes, w.scales, x,
                       m, w.cols, w.rows, w.kblocks(), y);
}

// NP: k-block pairs a wave keeps in flight per round, the pairs its chunks
// need up to the staging limit (rounds repeat beyond it).
template <int W, int MPAD, bool G32>
void gemv_launch_one(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    constexpr int NPMAX = GemvShape<MPAD>::NPMAX;
    const int pairs = (cdiv(w.kblocks(), kGemvChunks) + 1) / 2;
    if (pairs <= 1 || NPMAX == 1) gemv_launch_np<W, MPAD, G32, 1>(w, x, m, y, s);
    else if (pairs <= 2 || NPMAX == 2) gemv_launch_np<W, MPAD, G32, (NPMAX < 2 ? NPMAX : 2)>(w, x, m, y, s);
    else if (pairs <= 3) gemv_launch_np<W, MPAD, G32, (NPMAX < 3 ? NPMAX : 3)>(w, x, m, y, s);
    else gemv_launch_np<W, MPAD, G32, NPMAX>(w, x, m, y, s);
}

template <int W, bool G32>
void gemv_launch_m(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    if (m <= 1) gemv_launch_one<W, 1, G32>(w, x, m, y, s);
    else if (m <= 2) gemv_launch_one<W, 2, G32>(w, x, m, y, s);
    else if (m <= 4) gemv_launch_one<W, 4, G32>(w, x, m, y, s);
    else if (m <= 8) gemv_launch_one<W, 8, G32>(w, x, m, y, s);
    else gemv_launch_one<W, 16, G32>(w, x, m, y, s);
}

// The streaming GEMV: one wave per 16-row tile, WAVES tiles per block. False
// (nothing launched) when K is not a multiple of 2048 or the staged rows
// would not leave room for two blocks per compute unit.
template <int WAVES, int MPAD, bool G32, int D>
bool gemv_stream_launch(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    const int kbs = w.kblocks();
    const size_t lds = (size_t)MPAD * ((size_t)kbs * 256 + 16);
    if (kbs % kGemvChunks != 0 || lds > 80 * 1024) return false;
    static bool configured[64] = {};  // the LDS limit is a per-device function attribute
    int dev = 0;
    hipGetDevice(&dev);
    if (dev >= 0 && dev < 64 && !configured[dev]) {
        if (hipFuncSetAttribute((const void *)gemv_stream_kernel<WAVES, MPAD, G32, D>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess)
            configured[dev] = true;
    }
    hipLaunchKernelGGL((gemv_stream_kernel<WAVES, MPAD, G32, D>), dim3(cdiv(w.tiles(), WAVES)), dim3(WAVES * 64),
                       lds, s, w.codes, w.scales, x, m, w.cols, w.rows, kbs, y);
    return true;
}

template <int WAVES, bool G32, int D>
bool gemv_stream_m(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    if (m <= 1) return gemv_stream_launch<WAVES, 1, G32, D>(w, x, m, y, s);
    if (m <= 2) return gemv_stream_launch<WAVES, 2, G32, D>(w, x, m, y, s);
    if (m <= 4) return gemv_stream_launch<WAVES, 4, G32, D>(w, x, m, y, s);
    if (m <= 8) return gemv_stream_launch<WAVES, 8, G32, D>(w, x, m, y, s);
    return false;
}

template <int WAVES, int D>
bool gemv_stream(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    if (w.kind == WeightKind::Q4G32) return gemv_stream_m<WAVES, true, D>(w, x, m, y, s);
    return gemv_stream_m<WAVES, false, D>(w, x, m, y, s);
}

// The persistent GEMV: two blocks per compute unit where its LDS allows, at
// most one per tile. False (nothing launched) where a chunk would hold more
// than one k-block pair (K > 4096) or there are more than 8 rows.
template <int MPAD, bool G32>
bool gemv_persist_launch(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    using S = GemvShape<MPAD>;
    if (w.kblocks() > 2 * kGemvChunks) return false;
    const size_t lds = (size_t)kGemvChunks * S::SLICE + (size_t)2 * kGemvChunks * S::LIVE * 64 * sizeof(float);
    static bool configured[64] = {};  // the LDS limit is a per-device function attribute
    int dev = 0;
    hipGetDevice(&dev);
    if (dev >= 0 && dev < 64 && !configured[dev]) {
        if (hipFuncSetAttribute((const void *)gemv_persist_kernel<MPAD, G32>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess)
            configured[dev] = true;
    }
    const unsigned blocks = std::min((unsigned)w.tiles(), (unsigned)device_cus());
    hipLaunchKernelGGL((gemv_persist_kernel<MPAD, G32>), dim3(blocks), dim3(kGemvChunks * 64), lds, s, w.codes,
                       w.scales, x, m, w.cols, w.rows, w.kblocks(), y);
    return true;
}

template <bool G32>
bool gemv_persist_m(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    if (m <= 1) return gemv_persist_launch<1, G32>(w, x, m, y, s);
    if (m <= 2) return gemv_persist_launch<2, G32>(w, x, m, y, s);
    if (m <= 4) return gemv_persist_launch<4, G32>(w, x, m, y, s);
    if (m <= 8) return gemv_persist_launch<8, G32>(w, x, m, y, s);
    return false;
}

bool gemv_persist(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    return w.kind == WeightKind::Q4G32 ? gemv_persist_m<true>(w, x, m, y, s) : gemv_persist_m<false>(w, x, m, y, s);
}

template <int W>
void gemv_launch(const Weight &w, const half_t *x, int m, float *y, hipStream_t s) {
    if (w.kind == WeightKind::Q4G32)
        gemv_launch_m<W, true>(w, x, m, y, s);
    else
        gemv_launch_m<W, false>(w, x, m, y, s);
}

template <int BM, int BN, int WM, int WN, int EPI>
void gemm_launch(const Weight &w, const half_t *x, int m, void *y, const half_t *res, hipStream_t s) {
    dim3 grid(cdiv(w.rows, BN), cdiv(m, BM));
    size_t lds = BM * 256;
    if (w.kind == WeightKind::Q4G32)
        hipLaunchKernelGGL((gemm_w4a16_kernel<BM, BN, WM, WN, true, EPI>), grid, dim3(WM * WN * 64), lds, s,
                           w.codes, w.scales, x, m, w.cols, w.rows, w.kblocks(), y, res);
    else
        hipLaunchKernelGGL((gemm_w4a16_kernel<BM, BN, WM, WN, false, EPI>), grid, dim3(WM * WN * 64), lds, s,
                           w.codes, w.scales, x, m, w.cols, w.rows, w.kblocks(), y, res);
}

// Columns [c0, c0 + nc) of the product (c0 a multiple of 16) with BM x BN tiles.
template <int BM, int BN, int WGM, int WGN, int EPI, bool PERSIST = false>
bool w4a16_pipe_launch(const Weight &w, const half_t *x, int m, void *y, const half_t *res, hipStream_t s,
                       int c0 = 0, int nc = -1) {
    if (nc < 0) nc = w.rows - c0;
    // whole 128-k steps; byte offsets are 32-bit and relative to the block's first row / tile
    if (w.cols % 128 != 0 || c0 % 16 != 0 || (size_t)BM * w.cols * 2 >= ((size_t)1 << 31) ||
        (size_t)(BN / 16) * w.kblocks() * 1024 >= ((size_t)1 << 31))
        return false;
    if (nc <= 0) return true;
    const size_t t0 = (size_t)(c0 / 16) * w.kblocks();  // first (tile, k-block) of the slice
    const uint8_t *codes = w.codes + t0 * 1024, *scales = w.scales + t0 * 128;
    const size_t esz = EPI == 0 ? 4 : 2;
    void *yo = (uint8_t *)y + (size_t)c0 * esz;
    const half_t *ro = res ? res + c0 : nullptr;
    const unsigned tiles = cdiv(m, BM) * cdiv(nc, BN);
    // persistent: one block per compute unit (a multiple of the 8 XCDs), each taking every gridDim-th tile
    const unsigned blocks = PERSIST ? std::min(tiles, (unsigned)device_cus() / 8 * 8) : tiles;
    if (w.kind == WeightKind::Q4G32)
        hipLaunchKernelGGL((w4a16_pipe_kernel<BM, BN, WGM, WGN, true, EPI, 2, PERSIST>), dim3(blocks),
                           dim3(WGM * WGN * 64), 0, s, codes, scales, x, m, w.cols, nc, w.kblocks(), yo, ro, w.rows);
    else
        hipLaunchKernelGGL((w4a16_pipe_kernel<BM, BN, WGM, WGN, false, EPI, 2, PERSIST>), dim3(blocks),
                           dim3(WGM * WGN * 64), 0, s, codes, scales, x, m, w.cols, nc, w.kblocks(), yo, ro, w.rows);
    return true;
}

// Compute units of the current device (queried once per device).

// Variants 0-3 are the pipelined kernel: "auto", 256x256 tiles on 8 waves
// (one block per CU), 128x128 tiles on 4 waves (two blocks per CU) and
// 128x256 tiles on 8 waves. "auto" runs persistent 256x256 tiles when they
// fill two or more whole waves of compute units, else persistent 256x192
// tiles when those do, else 256x256 tiles over the leading
// columns that fill whole waves of compute units and 128x256 tiles over the
// rest (one launch each), or, below one wave of 256x256 tiles, the largest of
// 256x128, 128x256 and 128x128 that gives at least one tile per unit. 4-6 stage
// through registers. All give the same bits (same f16 dequantization, one MFMA per
// 32-k run in k order); the pipelined ones need k % 128 == 0 and fall back to
// 256x128w2x2 otherwise.
template <int EPI>
void gemm_dispatch(const Weight &w, const half_t *x, int m, void *y, const half_t *res, int variant,
                   hipStream_t s) {
    switch (variant) {
        case 0: {
            const unsigned cus = (unsigned)device_cus();
            const unsigned tm = cdiv(m, 256), tn = cdiv(w.rows, 256);
            const unsigned t192 = w.rows % 192 == 0 ? tm * (unsigned)(w.rows / 192) : 0;
            if (tm * tn >= 2 * cus && (tm * tn) % cus == 0) {
                // whole waves of 256x256 tiles, two or more: one persistent block per compute unit
                if (w4a16_pipe_launch<256, 256, 2, 4, EPI, true>(w, x, m, y, res, s)) return;
            } else if (t192 >= 2 * cus && t192 % cus == 0) {
                // whole waves of 256x192 tiles instead (the encoder's QKV projection: one launch)
                if (w4a16_pipe_launch<256, 192, 2, 4, EPI, true>(w, x, m, y, res, s)) return;
            } else if (tm * tn >= cus) {
                // 256-column blocks that fill whole waves; the rest on 128x256 tiles
                unsigned lead = tn;
                if ((tm * tn) % cus != 0 && tm <= cus && cus % tm == 0) lead = (tm * tn) / cus * (cus / tm);
                const int c1 = (int)std::min<size_t>((size_t)lead * 256, (size_t)w.rows);
                if (w4a16_pipe_launch<256, 256, 2, 4, EPI>(w, x, m, y, res, s, 0, c1) &&
                    w4a16_pipe_launch<128, 256, 2, 4, EPI>(w, x, m, y, res, s, c1, w.rows - c1))
                    return;
            } else if (tm * cdiv(w.rows, 128) >= cus) {
                // 256x128 tiles: per MAC half the dequantization of 128x256 tiles
                // (the encoder's N = 1024 projections: 25 against 27 us at K = 1024, 65 against 73 at 4096)
                if (w4a16_pipe_launch<256, 128, 2, 4, EPI>(w, x, m, y, res, s)) return;
            } else if (cdiv(m, 128) * cdiv(w.rows, 256) >= cus) {
                if (w4a16_pipe_launch<128, 256, 2, 4, EPI>(w, x, m, y, res, s)) return;
            } else {
                if (w4a16_pipe_launch<128, 128, 2, 2, EPI>(w, x, m, y, res, s)) return;
            }
            break;
        }
        case 1: if (w4a16_pipe_launch<256, 256, 2, 4, EPI>(w, x, m, y, res, s)) return; break;
        case 2: if (w4a16_pipe_launch<128, 128, 2, 2, EPI>(w, x, m, y, res, s)) return; break;
        case 3: if (w4a16_pipe_launch<128, 256, 2, 4, EPI>(w, x, m, y, res, s)) return; break;
        case 7: if (w4a16_pipe_launch<256, 256, 2, 4, EPI, true>(w, x, m, y, res, s)) return; break;
        case 8: if (w4a16_pipe_launch<256, 192, 2, 4, EPI, true>(w, x, m, y, res, s)) return; break;
        case 9: if (w4a16_pipe_launch<256, 128, 2, 4, EPI>(w, x, m, y, res, s)) return; break;
        case 5: gemm_launch<128, 128, 2, 2, EPI>(w, x, m, y, res, s); return;
        case 6: gemm_launch<128, 64, 2, 2, EPI>(w, x, m, y, res, s); return;
        default: break;
    }
    gemm_launch<256, 128, 2, 2, EPI>(w, x, m, y, res, s);
}


template <int BITS, int MPAD, int AMODE, bool PROJECT, bool AFF = false>
void gv_launch_one(const Weight &w, const void *a, const float *sa, int m, int abits, float *y,
                   const int *bad_in, int *bad_out, hipStream_t s, const float *res = nullptr) {
    using S = GvShape<MPAD, AFF>;
    static bool configured[64] = {};  // the LDS limit is a per-device function attribute
    int dev = 0;
    hipGetDevice(&dev);
    if (dev >= 0 && dev < 64 && !configured[dev]) {
        if (hipFuncSetAttribute((const void *)grouped_gemv_kernel<BITS, MPAD, AMODE, PROJECT, AFF>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, S::BYTES) == hipSuccess) configured[dev] = true;
    }
    dim3 grid(w.tiles(), cdiv(m, 16));
    hipLaunchKernelGGL((grouped_gemv_kernel<BITS, MPAD, AMODE, PROJECT, AFF>), grid, dim3(kGvWaves * 64), S::BYTES,
                       s, w.codes, w.scales, a, sa, m, w.cols, w.rows, w.groups, w.kblocks(), abits, y, bad_in,
                       bad_out, w.offsets, res);
}

template <int BITS, int AMODE, bool PROJECT, bool AFF = false>
void gv_launch_m(const Weight &w, const void *a, const float *sa, int m, int abits, float *y,
                 const int *bad_in, int *bad_out, hipStream_t s, const float *res = nullptr) {
    if (m <= 1) gv_launch_one<BITS, 1, AMODE, PROJECT, AFF>(w, a, sa, m, abits, y, bad_in, bad_out, s, res);
    else if (m <= 2) gv_launch_one<BITS, 2, AMODE, PROJECT, AFF>(w, a, sa, m, abits, y, bad_in, bad_out, s, res);
    else if (m <= 4) gv_launch_one<BITS, 4, AMODE, PROJECT, AFF>(w, a, sa, m, abits, y, bad_in, bad_out, s, res);
    else if (m <= 8) gv_launch_one<BITS, 8, AMODE, PROJECT, AFF>(w, a, sa, m, abits, y, bad_in, bad_out, s, res);
    else gv_launch_one<BITS, 16, AMODE, PROJECT, AFF>(w, a, sa, m, abits, y, bad_in, bad_out, s, res);
}

template <int AMODE, bool PROJECT>
void gv_launch(const Weight &w, const void *a, const float *sa, int m, int abits, float *y,
               const int *bad_in, int *bad_out, hipStream_t s) {
    if (w.bits == 4)
        gv_launch_m<4, AMODE, PROJECT>(w, a, sa, m, abits, y, bad_in, bad_out, s);
    else
        gv_launch_m<8, AMODE, PROJECT>(w, a, sa, m, abits, y, bad_in, bad_out, s);
}

}  // namespace

int variant_count(const char *family) {
    std::string f(family);
    if (f == "gemv") return 6;
    if (f == "gemm_w4a16") return 10;
    if (f == "i8_gemm") return 10;
    if (f == "grouped") return 14;
    if (f == "mlp") return 6;
    if (f == "delta_scan") return 5;
    if (f == "norm") return 2;
    return 0;
}

int tuned_count(const char *family) {
    // the token scans and "auto" regroup the chunked scan's arithmetic
    if (std::string(family) == "delta_scan") return 2;
    return variant_count(family);
}

const char *variant_name(const char *family, int index) {
    std::string f(family);
    if (index < 0 || index >= variant_count(family)) return nullptr;
    if (f == "gemv") return kGemvNames[index];
    if (f == "gemm_w4a16") return kGemmNames[index];
    if (f == "i8_gemm") return kI8Names[index];
    if (f == "grouped") return kGroupedNames[index];
    if (f == "mlp") return kMlpNames[index];
    if (f == "delta_scan") return kDeltaNames[index];
    if (f == "norm") return kNormNames[index];
    return nullptr;
}

int variant_index(const char *family, const char *name) {
    for (int i = 0; i < variant_count(family); i++)
        if (std::string(variant_name(family, i)) == name) return i;
    return -1;
}

void launch_grouped_small(const Weight &w, const float *x, int m, int abits, float *y, int *bad_out,
                          bool project, hipStream_t s) {
    if (m == 0) return;
    if (w.offsets && !project) {  // fitted affine Q4 (the runtime refuses the other combinations)
        gv_launch_m<4, 0, false, true>(w, x, nullptr, m, abits, y, nullptr, bad_out, s);
        return;
    }
    if (project)
        gv_launch<0, true>(w, x, nullptr, m, abits, y, nullptr, bad_out, s);
    else
        gv_launch<0, false>(w, x, nullptr, m, abits, y, nullptr, bad_out, s);
}

void launch_grouped_codes(const Weight &w, const int8_t *q, const float *sx, int m, float *y,
                          const int *bad_in, bool project, hipStream_t s) {
    if (m == 0) return;
    if (project)
        gv_launch<1, true>(w, q, sx, m, 8, y, bad_in, nullptr, s);
    else
        gv_launch<1, false>(w, q, sx, m, 8, y, bad_in, nullptr, s);
}

void launch_grouped_records(const Weight &w, const uint32_t *records, int m, float *y, hipStream_t s) {
    if (m == 0) return;
    gv_launch<2, false>(w, records, nullptr, m, 8, y, nullptr, nullptr, s);
}

// Variant 1 is grouped_pipe_kernel (256x128 tiles, 8 waves), variant 2 the
// one-wave-per-16x16-tile grouped_kernel, variant 0 ("auto") the first when
// its grid covers at least half the compute units and the second otherwise.
// All fold in the reference order, so all give the same bits.
// The pipelined grouped kernels address a BM-row activation panel and a
// weight tile column with 32-bit byte offsets.
bool grouped_pipe_fits(const Weight &w, int bm) {
    return bm > 0 && (size_t)bm * w.groups * 64 < ((size_t)1 << 31) &&
           (size_t)8 * w.kblocks() * 1024 < ((size_t)1 << 31);
}

template <int BM, int WGM, int WGN, int GS = 2, int BN = 128>
bool grouped_pipe_launch(const Weight &w, const int8_t *q, const float *sx, int m, float *y, const int *bad,
                         hipStream_t s, const float *res, const float *sxq) {
    if (!grouped_pipe_fits(w, BM)) return false;
    const dim3 blocks(cdiv(m, BM) * cdiv(w.rows, BN));
    if (w.offsets)
        hipLaunchKernelGGL((grouped_pipe_kernel<4, BM, BN, WGM, WGN, true, GS>), blocks, dim3(WGM * WGN * 64), 0, s,
                           w.codes, w.scales, q, sx, m, w.rows, w.groups, w.kblocks(), y, res, bad, w.offsets, sxq);
    else if (w.bits == 4)
        hipLaunchKernelGGL((grouped_pipe_kernel<4, BM, BN, WGM, WGN, false, GS>), blocks, dim3(WGM * WGN * 64), 0, s,
                           w.codes, w.scales, q, sx, m, w.rows, w.groups, w.kblocks(), y, res, bad);
    else
        hipLaunchKernelGGL((grouped_pipe_kernel<8, BM, BN, WGM, WGN, false, GS>), blocks, dim3(WGM * WGN * 64), 0, s,
                           w.codes, w.scales, q, sx, m, w.rows, w.groups, w.kblocks(), y, res, bad);
    return true;
}

// Variants: 1 pipelined 256x128 tiles (8 waves), 3 128x128 (4 waves as 2x2),
// 5 128x128 (4 waves side by side, each 128 rows x 32 columns), 6 128x128 (4
// waves stacked, each 32 rows x 128 columns), 4 64x128 (2 waves), 7 32x128 (8
// waves side by side, each 32 rows x 16 columns), 8 64x128 (8 waves as 2x4), 2
// one wave per 16x16 tile; 9 and 10 are 7 and 8 with four groups per k-step
// instead of two; 11 the few-row kernel over the codes (16 rows per block
// row, a block per 16 columns); 12 and 13 are 32x64 tiles on 4 waves (each
// 32 rows x 16 columns, the per-wave work of 7) and 64x64 on 8 waves. Every
// variant folds in group order: all are bitwise equal. "Auto" (0) picks:
//  - the few-row kernel where its grid gives a compute unit at most two
//    blocks (us, A8 codes in: K=9216, N=2560, 17-48 rows: 19.9-21.7 against
//    27.6 pipelined; N=1024, 17-128 rows: 4.8-8.3 against 10.0; N=4096,
//    17-32 rows: 8.1 against 9.8; one block row more and it is slower), not
//    for affine weights, which it does not take;
//  - otherwise, as the fold is VALU work, the tiles whose grid keeps every
//    SIMD busy and every compute unit equally loaded: where a grid's blocks
//    do not divide evenly over the units, those holding one block more end
//    last (640 32x128 blocks at N=2560 put three on half the units and two on
//    the rest; 1280 32x64 blocks put five on each). So 128x128 side by side
//    when their grid gives every unit four blocks, else 64x128 on 8 waves
//    when its grid is two or more whole blocks per unit, else 32x64 on 4
//    waves, and 32x128 with four groups per step when the 32x128 grid gives
//    a unit fewer than two blocks (half the barriers and twice the work
//    between a load and its use; on fuller grids it is 2-5% slower).
// Measured (us at 1024 rows unless stated; 32x128w8 / 32x128w8g4 / 32x64w4 /
// 64x128w8 / 128x128 side by side): N=1024, K=2560 18.0 / 16.3 / 17.1 / 22.0
// / 47.5; N=2560, K=9216 79.0 / 82.7 / 74.6 / 83.9 / 149; N=2560, K=4096
// 39.9 / 41.4 / 37.7 / 43.0 / 72.3; N=4160, K=2560 39.5 / - / 37.6 / 43.0 /
// 56.6; N=8192, K=2560 58.6 / 62.4 / 58.5 / 54.1 / 57.3; 40 rows, N=8192:
// 14.6 / 13.0 / 13.2 / 18.0 / 42.3; 300 rows, N=2560: 15.6 / 14.2 / 14.6 /
// 19.8 / 45.1; 16384 rows, K=4096, N=14336: 2209 / 2354 / 2252 / 2060 / 1813.
int grouped_pick(const Weight &w, int m, int variant) {
    if (variant != 0) return variant;
    const unsigned cus = (unsigned)device_cus(), tn = cdiv(w.rows, 128);
    if (!w.offsets && cdiv(m, 16) * (unsigned)w.tiles() <= 2 * cus) return 11;
    if (cdiv(m, 128) * tn >= 4 * cus) return 5;
    const unsigned b64 = cdiv(m, 64) * tn;
    if (b64 >= 2 * cus && b64 % cus == 0) return 8;
    if (cdiv(m, 32) * tn >= 2 * cus) return 12;
    return 9;
}

// Activation rows per block of a pipelined pick (0: not a pipelined kernel).
int grouped_pipe_rows(int pick) {
    switch (pick) {
        case 1: return 256;
        case 3: case 5: case 6: return 128;
        case 4: case 8: case 10: case 13: return 64;
        case 7: case 9: case 12: return 32;
        default: return 0;
    }
}

// The same predicate decides here and in launch_grouped whether a pipelined
// kernel (the only ones with the residual epilogue) takes the product.
bool grouped_adds_residual(const Weight &w, int m, int variant) {
    if (m <= 16 || w.kind == WeightKind::Q4G32) return false;
    const int pick = grouped_pick(w, m, variant);
    return (pick == 11 && !w.offsets) || grouped_pipe_fits(w, grouped_pipe_rows(pick));
}

bool launch_grouped(const Weight &w, const int8_t *q, const float *sx, int m, float *y,
                    const int *bad, int variant, hipStream_t s, const float *res, const float *sxq) {
    if (m == 0) return true;
    switch (grouped_pick(w, m, variant)) {
        case 1: if (grouped_pipe_launch<256, 2, 4>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 3: if (grouped_pipe_launch<128, 2, 2>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 4: if (grouped_pipe_launch<64, 1, 2>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 5: if (grouped_pipe_launch<128, 1, 4>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 6: if (grouped_pipe_launch<128, 4, 1>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 7: if (grouped_pipe_launch<32, 1, 8>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 8: if (grouped_pipe_launch<64, 2, 4>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 9: if (grouped_pipe_launch<32, 1, 8, 4>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 10: if (grouped_pipe_launch<64, 2, 4, 4>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 12: if (grouped_pipe_launch<32, 1, 4, 2, 64>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 13: if (grouped_pipe_launch<64, 2, 4, 2, 64>(w, q, sx, m, y, bad, s, res, sxq)) return true; break;
        case 11:
            if (w.offsets) break;  // the few-row kernel over codes takes no offsets
            if (w.bits == 4) gv_launch_m<4, 1, false>(w, q, sx, m, 8, y, bad, nullptr, s, res);
            else gv_launch_m<8, 1, false>(w, q, sx, m, 8, y, bad, nullptr, s, res);
            return true;
        default: break;
    }
    if (res) return false;  // only the pipelined kernels add a residual
    dim3 grid(cdiv(w.tiles(), 4), cdiv(m, 16));
    if (w.offsets)
        hipLaunchKernelGGL((grouped_kernel<4, true>), grid, dim3(256), 0, s, w.codes, w.scales, q, sx, m, w.rows,
                           w.groups, w.kblocks(), y, bad, w.offsets, sxq);
    else if (w.bits == 4)
        hipLaunchKernelGGL(grouped_kernel<4>, grid, dim3(256), 0, s, w.codes, w.scales, q, sx, m, w.rows,
                           w.groups, w.kblocks(), y, bad);
    else
        hipLaunchKernelGGL(grouped_kernel<8>, grid, dim3(256), 0, s, w.codes, w.scales, q, sx, m, w.rows,
                           w.groups, w.kblocks(), y, bad);
    return true;
}

// Variants: 1 pipelined 256x64 blocks (8 waves), 2 128x64 blocks (4 waves),
// 4 and 5 the same blocks with the waves paired along N (wave tile 64 x 32), 3
// one wave per 16x64 block. 0 picks the paired 256-row blocks when their grid
// covers half the compute units but not all of them and has fewer blocks than
// the 128-row grid (not at m <= 128, where the 256-row blocks are half empty:
// 54 against 40 us at M = 128, K = 2560, N = 9216), else the paired 128-row
// blocks when theirs covers half, else the one-wave blocks (measured at K=2560,
// N=9216: the paired layouts are 7-16% faster than the stacked ones at every M
// from 229 to 4096, and 128-row blocks beat 256-row blocks from M=1024 up).
// All variants are word-exact with the unfused composition.
void launch_mlp_requant(const Weight &gate, const Weight &up, const int8_t *q, const float *sx,
                        int m, int8_t *qo, float *so, const int *bad, int variant, hipStream_t s) {
    if (m == 0) return;
    const unsigned cus = (unsigned)device_cus(), tn = (unsigned)(gate.rows / 64);
    const bool fits = (size_t)256 * gate.groups * 64 < ((size_t)1 << 31) &&
                      (size_t)4 * gate.kblocks() * 1024 < ((size_t)1 << 31) && ((uintptr_t)qo & 3) == 0 &&
                      gate.rows % 4 == 0;
    int pick = variant;
    if (variant == 0) {
        // 256-row blocks only where they shorten the grid (at m <= 128 both
        // grids have the same blocks, half of each 256-row block empty)
        const unsigned b256 = cdiv(m, 256) * tn, b128 = cdiv(m, 128) * tn;
        if (2 * b256 >= cus && b256 < cus && b256 < b128) pick = 4;
        else if (2 * b128 >= cus) pick = 5;
        else pick = 3;
    }
    if (fits && pick == 1) {
        hipLaunchKernelGGL(mlp_pipe_kernel<256>, dim3(cdiv(m, 256) * tn), dim3(512), 0, s, gate.codes, gate.scales,
                           up.codes, up.scales, q, sx, m, gate.rows, gate.groups, gate.kblocks(), qo, so, bad);
        return;
    }
    if (fits && pick == 2) {
        hipLaunchKernelGGL(mlp_pipe_kernel<128>, dim3(cdiv(m, 128) * tn), dim3(256), 0, s, gate.codes, gate.scales,
                           up.codes, up.scales, q, sx, m, gate.rows, gate.groups, gate.kblocks(), qo, so, bad);
        return;
    }
    if (fits && pick == 4) {
        hipLaunchKernelGGL((mlp_pipe_kernel<256, 2>), dim3(cdiv(m, 256) * tn), dim3(512), 0, s, gate.codes,
                           gate.scales, up.codes, up.scales, q, sx, m, gate.rows, gate.groups, gate.kblocks(), qo,
                           so, bad);
        return;
    }
    if (fits && pick == 5) {
        hipLaunchKernelGGL((mlp_pipe_kernel<128, 2>), dim3(cdiv(m, 128) * tn), dim3(256), 0, s, gate.codes,
                           gate.scales, up.codes, up.scales, q, sx, m, gate.rows, gate.groups, gate.kblocks(), qo,
                           so, bad);
        return;
    }
    dim3 grid(gate.rows / 64, cdiv(m, 16));
    hipLaunchKernelGGL(mlp_requant_kernel, grid, dim3(256), 0, s, gate.codes, gate.scales, up.codes,
                       up.scales, q, sx, m, gate.rows, gate.groups, gate.kblocks(), qo, so, bad);
}

void launch_w4a16(const Weight &w, const half_t *x, int m, float *y, int gemv_variant,
                  int gemm_variant, hipStream_t s) {
    if (m == 0) return;
    if (m <= 16) {
        int v = gemv_variant;
        if (v == 0) {
            // "auto": the persistent kernel for up to 8 rows over four or more tiles
            // per compute unit at K <= 4096 (graph-timed at K = 4096 against the split
            // kernel, M = 1: N = 16384 8.3 against 9.8 us, N = 131072 53.9 against
            // 68.3 us = 0.70 of 8 TB/s; M = 8, N = 131072: 70.4 against 104.9 us, and
            // against 76.6 us for the streaming kernel; at one tile per compute unit,
            // N = 4096, the split kernel is 2-5% faster, and at two, N = 8192 and
            // K = 2560, 4.8-4.9 against 4.9-5.1 us); otherwise the split kernel, or the
            // streaming kernel at 2..8 rows over eight or more tiles per compute unit
            // (K = 4096: M = 4, N = 65536 33 against 39 us)
            const int cus = device_cus();
            if (m <= 8 && w.kblocks() <= 2 * kGemvChunks && w.tiles() >= 4 * cus) v = 5;
            else if (m >= 2 && m <= 8 && w.tiles() >= 8 * cus) v = m > 4 && w.tiles() >= 16 * cus ? 3 : 4;
            else v = 1;
        }
        bool done = false;
        if (v == 3) done = gemv_stream<8, 8>(w, x, m, y, s);
        else if (v == 4) done = gemv_stream<4, 8>(w, x, m, y, s);
        else if (v == 5) done = gemv_persist(w, x, m, y, s);
        if (done) return;
        if (v == 2)
            gemv_launch<8>(w, x, m, y, s);
        else
            gemv_launch<16>(w, x, m, y, s);
    } else {
        gemm_dispatch<0>(w, x, m, y, nullptr, gemm_variant, s);
    }
}

void launch_w4a16_f16(const Weight &w, const half_t *x, int m, half_t *y, int epilogue,
                      const half_t *residual, int variant, hipStream_t s) {
    if (m == 0) return;
    switch (epilogue) {
        case 1: gemm_dispatch<2>(w, x, m, y, residual, variant, s); break;
        case 2: gemm_dispatch<3>(w, x, m, y, residual, variant, s); break;
        default: gemm_dispatch<1>(w, x, m, y, residual, variant, s); break;
    }
}

template <int BM, int BN, int BK, int NS, int WGM = 2, int WGN = 2>
bool i8_pipe_launch(const int8_t *a, const float *sa, int m, const int8_t *b, const float *sb, int n, int k,
                    void *y, int raw, hipStream_t s) {
    if (k % 16 != 0 || (size_t)BM * k >= ((size_t)1 << 31) || (size_t)BN * k >= ((size_t)1 << 31)) return false;
    const unsigned blocks = cdiv(m, BM) * cdiv(n, BN);
    hipLaunchKernelGGL((i8_gemm_pipe_kernel<BM, BN, BK, NS, WGM, WGN>), dim3(blocks), dim3(WGM * WGN * 64), 0, s, a,
                       sa, m, b, sb, n, k, y, raw);
    return true;
}

// BPC blocks per compute unit (what the kernel's LDS and registers allow).
template <int BM, int BN, int BK, int NS, int WGM, int WGN, int BPC, bool MID>
bool i8_stream_launch(const int8_t *a, const float *sa, int m, const int8_t *b, const float *sb, int n, int k,
                      void *y, int raw, hipStream_t s) {
    if (k % 16 != 0 || (size_t)BM * k >= ((size_t)1 << 31) || (size_t)BN * k >= ((size_t)1 << 31) ||
        (size_t)BM * n * 4 >= ((size_t)1 << 31))
        return false;
    const unsigned tiles = cdiv(m, BM) * cdiv(n, BN);
    const unsigned grid = std::min(tiles, (unsigned)(BPC * device_cus() / 8 * 8));
    hipLaunchKernelGGL((i8_gemm_stream_kernel<BM, BN, BK, NS, WGM, WGN, MID>), dim3(grid ? grid : 1), dim3(WGM * WGN * 64), 0, s,
                       a, sa, m, b, sb, n, k, y, raw);
    return true;
}

// Variants 0-3 are the pipelined buffer-to-LDS kernels and 7-9 their
// persistent stream form (int8 B, k % 16 == 0); 4-6 stage through registers
// and take any k and the per-row Q4 B operand.
// Every variant computes exact int32 dots, so all are bitwise equal; when a
// pipelined variant cannot take a shape, the register-staged 128x128 runs.
template <bool Q4B>
void i8_gemm_dispatch(const int8_t *a, const float *sa, int m, const int8_t *b, const float *sb, int n,
                      int k, void *y, int raw, int variant, hipStream_t s) {
    if (!Q4B) {
        switch (variant) {
            case 0: if (i8_pipe_launch<256, 256, 128, 2, 2, 4>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            case 1: if (i8_pipe_launch<256, 256, 64, 4, 2, 4>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            case 2: if (i8_pipe_launch<256, 128, 128, 3, 2, 4>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            case 3: if (i8_pipe_launch<256, 128, 128, 3, 2, 2>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            case 7: if (i8_stream_launch<256, 256, 128, 2, 2, 4, 1, false>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            case 8: if (i8_stream_launch<256, 256, 128, 2, 2, 4, 1, true>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            case 9: if (i8_stream_launch<256, 128, 64, 2, 2, 2, 2, false>(a, sa, m, b, sb, n, k, y, raw, s)) return; break;
            default: break;
        }
    }
    switch (variant) {
        case 5:
            hipLaunchKernelGGL((i8_gemm_kernel<256, 128, 2, 2, Q4B>), dim3(cdiv(n, 128), cdiv(m, 256)), dim3(256), 0,
                               s, a, sa, m, b, sb, n, k, y, raw);
            break;
        case 6:
            hipLaunchKernelGGL((i8_gemm_kernel<64, 64, 2, 2, Q4B>), dim3(cdiv(n, 64), cdiv(m, 64)), dim3(256), 0, s,
                               a, sa, m, b, sb, n, k, y, raw);
            break;
        default:
            hipLaunchKernelGGL((i8_gemm_kernel<128, 128, 2, 2, Q4B>), dim3(cdiv(n, 128), cdiv(m, 128)), dim3(256), 0,
                               s, a, sa, m, b, sb, n, k, y, raw);
            break;
    }
}

void launch_i8_gemm(const int8_t *a, const float *sa, int m, const int8_t *b, const float *sb,
                    int n, int k, void *y, int raw, int variant, hipStream_t s, bool b_q4) {
    if (m == 0 || n == 0) return;
    if (b_q4)
        i8_gemm_dispatch<true>(a, sa, m, b, sb, n, k, y, raw, variant, s);
    else
        i8_gemm_dispatch<false>(a, sa, m, b, sb, n, k, y, raw, variant, s);
}

void launch_i8_gemm_fused(const int8_t *a, const float *sa, int m, const int8_t *wg, const float *sg,
                          const int8_t *wu, const float *su, int n, int k, float *y, hipStream_t s) {
    if (m == 0 || n == 0) return;
    hipLaunchKernelGGL((i8_gemm_kernel<128, 128, 2, 2, false, true>), dim3(cdiv(n, 64), cdiv(m, 128)), dim3(256), 0,
                       s, a, sa, m, wg, sg, n, k, (void *)y, 0, wu, su);
}

int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    hipGetDevice(&dev);
    if (dev < 0 || dev >= 64) return 256;
    if (!cus[dev]) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev] = v;
    }
    return cus[dev];
}

}  // namespace dz
