// epilogue.hip -- layer epilogues and attention for the encoder forward.
//
// Reference behaviour:
//  - LayerNorm with bias:  src/models/decima/cpu.rs:529-540
//  - erf GELU:             src/models/decima/cpu.rs:542-556 (erf by Abramowitz &
//                          Stegun 7.1.26, |error| <= 1.5e-7; the reference calls libm erff)
//  - zero-centred RMSNorm: src/models/pplx_flash/cpu.rs:310-333
//  - SiLU * up:            src/models/pplx_flash/cpu.rs:348-371, 513-518
//  - residual add:         src/models/pplx_flash/cpu.rs:334-347
//  - softmax:              src/models/pplx_flash/cpu.rs:519-529
//  - mean over rows:       src/models/decima/cpu.rs:574-586
//  - attention:            src/models/pplx_flash/backbone.rs:484-615 (softmax
//                          attention over the whole chunk, non-causal)
// Reductions run as wave/block trees, so results match the CPU within float
// tolerance rather than bit for bit.
#include <float.h>

#include <algorithm>
#include <type_traits>

#include "kernels.hpp"

namespace dz {

namespace {

inline unsigned cdiv(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

__device__ __forceinline__ float ld(const void *p, int dtype, size_t i) {
    return dtype == 0 ? ((const float *)p)[i] : (float)((const half_t *)p)[i];
}
__device__ __forceinline__ void st(void *p, int dtype, size_t i, float v) {
    if (dtype == 0)
        ((float *)p)[i] = v;
    else
        ((half_t *)p)[i] = (half_t)v;
}

__device__ __forceinline__ float block_sum(float v, float *sh) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    int w = threadIdx.x / 64;
    __syncthreads();
    if (threadIdx.x % 64 == 0) sh[w] = v;
    __syncthreads();
    float total = 0.0f;
    for (int i = 0; i < (int)blockDim.x / 64; i++) total += sh[i];
    return total;
}

// One 256-thread block per row.
__global__ __launch_bounds__(256) void layernorm_kernel(const void *__restrict__ x,
                                                        void *__restrict__ y, int dtype, int d,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ b, float eps) {
    __shared__ float sh[4];
    size_t base = (size_t)blockIdx.x * d;
    float s = 0.0f;
    for (int i = threadIdx.x; i < d; i += 256) s += ld(x, dtype, base + i);
    float mean = block_sum(s, sh) / (float)d;
    float v = 0.0f;
    for (int i = threadIdx.x; i < d; i += 256) {
        float c = ld(x, dtype, base + i) - mean;
        v += c * c;
    }
    float var = block_sum(v, sh) / (float)d;
    float inv = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < d; i += 256) {
        float c = (ld(x, dtype, base + i) - mean) * inv;
        st(y, dtype, base + i, c * w[i] + b[i]);
    }
}

// f16 rows of d = 512 * C columns. Each wave walks rows wave_id, wave_id +
// total waves, ...: the row sits in registers (C 16-byte chunks per lane:
// columns 512c + 8*lane + 0..7), the gains and biases of the lane's columns
// are loaded once, and the next row's load is issued before the current row
// is normalized. Shuffle-tree sums, the same two-pass mean / variance as
// layernorm_kernel.
template <int C>
__global__ __launch_bounds__(256) void layernorm_f16_rows_kernel(const half_t *__restrict__ x,
                                                                 half_t *__restrict__ y, int rows,
                                                                 const float *__restrict__ w,
                                                                 const float *__restrict__ b, float eps) {
    constexpr int D = 512 * C;
    const int lane = threadIdx.x % 64;
    const int stride = gridDim.x * 4;
    // row-band order per XCD (xcd_unit): a wave normalises rows the same XCD's
    // product blocks wrote, and writes rows the next product reads there
    int row = xcd_unit(blockIdx.x, gridDim.x) * 4 + threadIdx.x / 64;
    if (row >= rows) return;  // whole wave
    float ww[C][8], bb[C][8];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int col = c * 512 + lane * 8;
        const float4_t w0 = *(const float4_t *)(w + col), w1 = *(const float4_t *)(w + col + 4);
        const float4_t b0 = *(const float4_t *)(b + col), b1 = *(const float4_t *)(b + col + 4);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            ww[c][e] = w0[e];
            ww[c][e + 4] = w1[e];
            bb[c][e] = b0[e];
            bb[c][e + 4] = b1[e];
        }
    }
    half8_t h[C];
#pragma unroll
    for (int c = 0; c < C; c++) h[c] = *(const half8_t *)(x + (size_t)row * D + c * 512 + lane * 8);
    for (;;) {
        float v[C][8];
#pragma unroll
        for (int c = 0; c < C; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) v[c][e] = (float)h[c][e];
        const int next = row + stride;
        if (next < rows) {
#pragma unroll
            for (int c = 0; c < C; c++) h[c] = *(const half8_t *)(x + (size_t)next * D + c * 512 + lane * 8);
        }
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < C; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) s += v[c][e];
        s = wave_sum_dpp(s);
        const float mean = s / (float)D;
        float q = 0.0f;
#pragma unroll
        for (int c = 0; c < C; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float d0 = v[c][e] - mean;
                q += d0 * d0;
            }
        q = wave_sum_dpp(q);
        const float inv = 1.0f / sqrtf(q / (float)D + eps);
        half_t *dst = y + (size_t)row * D;
#pragma unroll
        for (int c = 0; c < C; c++) {
            half8_t o;
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = (half_t)((v[c][e] - mean) * inv * ww[c][e] + bb[c][e]);
            *(half8_t *)(dst + c * 512 + lane * 8) = o;
        }
        if (next >= rows) break;
        row = next;
    }
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x,
                                                      float *__restrict__ y, int d,
                                                      const float *__restrict__ w, float eps,
                                                      int zero_centered) {
    __shared__ float sh[4];
    size_t base = (size_t)blockIdx.x * d;
    float s = 0.0f;
    for (int i = threadIdx.x; i < d; i += 256) s += x[base + i] * x[base + i];
    float scale = 1.0f / sqrtf(block_sum(s, sh) / (float)d + eps);
    for (int i = threadIdx.x; i < d; i += 256)
        y[base + i] = (x[base + i] * scale) * (zero_centered ? 1.0f + w[i] : w[i]);
}

// The readout's RMSNorm (pplx_flash/cpu.rs:310-333 rms_from, as applied by
// pplx_flash/mod.rs:149-155): the sum of squares runs in row order, as the
// reference's iterator sum does, so the result is bit-exact with it. One
// 256-thread block per selected row (`rows` picks hidden rows; null takes row
// r): every thread squares its share of the row into LDS (loads in flight
// together), thread 0 adds the squares in row order, and all threads write
// the scaled row.
template <int DT>
__global__ __launch_bounds__(256) void readout_rms_kernel(const void *__restrict__ h,
                                                          const int32_t *__restrict__ rows, int d,
                                                          const float *__restrict__ w, float eps,
                                                          int zero_centered, float *__restrict__ y) {
    extern __shared__ __align__(16) float squares[];
    __shared__ float scale_sh;
    const size_t base = (size_t)(rows ? rows[blockIdx.x] : (int)blockIdx.x) * d;
#pragma unroll 4
    for (int i = threadIdx.x; i < d; i += 256) {
        const float v = ld(h, DT, base + i);
        squares[i] = __fmul_rn(v, v);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        int i = 0;
        for (; i + 8 <= d; i += 8) {
            const float4_t a = *(const float4_t *)(squares + i), b = *(const float4_t *)(squares + i + 4);
            ss = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(ss, a[0]), a[1]), a[2]), a[3]);
            ss = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(ss, b[0]), b[1]), b[2]), b[3]);
        }
        for (; i < d; i++) ss = __fadd_rn(ss, squares[i]);
        // v_sqrt_f32 is not correctly rounded; a float's square root taken in
        // f64 and rounded to f32 is (the exact root is never near enough to a
        // float midpoint for the f64 error to matter)
        const float t = __fadd_rn(__fdiv_rn(ss, (float)d), eps);
        scale_sh = __fdiv_rn(1.0f, __double2float_rn(__dsqrt_rn((double)t)));
    }
    __syncthreads();
    const float scale = scale_sh;
    float *dst = y + (size_t)blockIdx.x * d;
#pragma unroll 4
    for (int i = threadIdx.x; i < d; i += 256) {
        const float g = zero_centered ? __fadd_rn(1.0f, w[i]) : w[i];
        dst[i] = __fmul_rn(__fmul_rn(ld(h, DT, base + i), scale), g);
    }
}

// Sets bit `bit` of *flag when any of the n values is not finite.
__global__ void flag_nonfinite_kernel(const float *__restrict__ y, size_t n, int *flag, int bit) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n && !isfinite(y[i])) atomicOr(flag, bit);
}

__global__ void to_f32_kernel(const void *__restrict__ x, int dtype, size_t n, float *__restrict__ y) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) y[i] = ld(x, dtype, i);
}

// The f16 epilogue of the W4A16 GEMM applied to f32 products (the GEMV
// path): 0 none, 1 erf-GELU, 2 + residual; one rounding to f16 at the end.
__global__ void f16_epilogue_kernel(const float *__restrict__ v, int epi, const half_t *__restrict__ res,
                                    half_t *__restrict__ y, size_t n) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    float t = v[i];
    if (epi == 1) t = gelu_erf(t);
    else if (epi == 2) t = t + (float)res[i];
    y[i] = (half_t)f32_rounded(t);
}

__global__ void gelu_kernel(void *x, int dtype, size_t n) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = ld(x, dtype, i);
    st(x, dtype, i, gelu_erf(v));
}

__global__ void silu_mul_kernel(float *g, const float *u, size_t n) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = g[i];
    float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-v)));  // same ops as the fused MLP epilogue
    g[i] = __fmul_rn(__fmul_rn(v, sig), u[i]);
}

__global__ void add_kernel(void *x, const void *y, int dtype, size_t n) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    st(x, dtype, i, ld(x, dtype, i) + ld(y, dtype, i));
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(float *x, int n) {
    __shared__ float sh[4];
    float *row = x + (size_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, row[i]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    __syncthreads();
    if (threadIdx.x % 64 == 0) sh[threadIdx.x / 64] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        float e = expf(row[i] - mx);
        row[i] = e;
        s += e;
    }
    float total = block_sum(s, sh);
    for (int i = threadIdx.x; i < n; i += 256) row[i] = row[i] / total;
}

// out[b][c] = mean over rows of x[b][r][c]; one thread per (b, c).
// Block (b, column group of 64): thread (g, c) sums rows g, g + 16, ... of
// column 64*blockIdx.x + c, then the 16 partial sums of a column are added
// in g order: a fixed order, so the result does not depend on timing.
__global__ __launch_bounds__(1024) void mean_rows_kernel(const void *__restrict__ x, int dtype, int batch,
                                                         int rows, int d, float *__restrict__ out) {
    __shared__ float part[16][65];
    const int c = threadIdx.x % 64, g = threadIdx.x / 64;
    const int col = blockIdx.x * 64 + c, b = blockIdx.y;
    float s = 0.0f;
    if (col < d)
        for (int r = g; r < rows; r += 16) s += ld(x, dtype, ((size_t)b * rows + r) * d + col);
    part[g][c] = s;
    __syncthreads();
    if (g == 0 && col < d) {
        float t = 0.0f;
        for (int i = 0; i < 16; i++) t += part[i][c];
        out[(size_t)b * d + col] = t / (float)rows;
    }
}

// The f16 form with 16-byte loads: block (b, group of 128 columns); thread
// (g, c8) sums rows g, g + 64, ... of the 8 columns 8*c8 .. 8*c8 + 7, four
// rows in flight at a time; then the 64 partial sums of a column are added in
// g order (a fixed order).
__global__ __launch_bounds__(1024) void mean_rows_f16_kernel(const half_t *__restrict__ x, int rows, int d,
                                                             float *__restrict__ out) {
    __shared__ float part[64][129];
    const int c8 = threadIdx.x % 16, g = threadIdx.x / 16;
    // (column group, sequence) units, a contiguous share per XCD (xcd_unit)
    const int groups = (d + 127) / 128, unit = xcd_unit(blockIdx.x, gridDim.x);
    const int cg = unit % groups, b = unit / groups;
    const int col = cg * 128 + c8 * 8;
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (col < d) {
        const half_t *base = x + (size_t)b * rows * d + col;
        int r = g;
        for (; r + 192 < rows; r += 256) {
            half8_t v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = *(const half8_t *)(base + (size_t)(r + 64 * u) * d);
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int e = 0; e < 8; e++) s[e] += (float)v[u][e];
        }
        for (; r < rows; r += 64) {
            const half8_t v = *(const half8_t *)(base + (size_t)r * d);
#pragma unroll
            for (int e = 0; e < 8; e++) s[e] += (float)v[e];
        }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) part[g][c8 * 8 + e] = s[e];
    __syncthreads();
    if (threadIdx.x < 128 && cg * 128 + (int)threadIdx.x < d) {
        float t = 0.0f;
        for (int i = 0; i < 64; i++) t += part[i][threadIdx.x];
        out[(size_t)b * d + cg * 128 + threadIdx.x] = t / (float)rows;
    }
}

// ---- flash attention, head_dim 64 ----------------------------------------------------
//
// Block = 8 waves x 32 queries of one (batch, head); keys in steps of 64,
// K and V tiles (64 rows x 128 bytes each) double-buffered in LDS by
// buffer_load ... lds, so each K/V row is read from L2 once per 256 queries.
// Scores are computed transposed, S^T = K Q^T (v_mfma_f32_16x16x32_f16, A =
// K rows from LDS, B = Q rows held in registers), so a lane's accumulator
// column is one query: the online-softmax max, sum and rescale are per-lane
// scalars. O^T = V^T P^T: the P^T values a lane holds (keys 16kb + 4q + v of
// query j) are the B operand when the MFMA k-slots of a 32-key block c are
// labelled 8q + e -> key 32c + 16(e / 4) + 4q + e % 4, and the matching V^T
// operand (8 keys of one dh per lane) is read with ds_read_b64_tr_b16, whose
// 16-lane groups give lane 4a + b element b of the 8-byte chunks addressed by
// lanes a, a + 4, a + 8, a + 12.
// LDS swizzles (bank-conflict free for both reads and the loads):
//   K: 16-byte chunk c of row r at slot c ^ ((r >> 1) & 7)
//   V: 8-byte unit u of row r at unit u ^ (4 * ((r >> 1) & 3))
constexpr int kAttnWaves = 8;
constexpr int kAttnQB = 2;                                // 16-query blocks per wave
constexpr int kAttnKeys = 64;                             // per step

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float8_t __attribute__((ext_vector_type(8)));

// max over lanes l, l ^ 16, l ^ 32 and l ^ 48, in registers (permlane swaps)
__device__ __forceinline__ float rows_max4(float v) {
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    v = fmaxf(a, b);
    a = v;
    b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}

template <int W>
__global__ __launch_bounds__(W * 64, 4) void attention_kernel(const half_t *__restrict__ qkv,
                                                                    half_t *__restrict__ out, int seq,
                                                                    int heads, float scale_log2) {
    __shared__ __align__(16) uint8_t ks[2 * kAttnKeys * 128];
    __shared__ __align__(16) uint8_t vs[2 * kAttnKeys * 128];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int q4 = lane / 16, j = lane % 16;
    // blocks in (query block, head, batch) order, a contiguous share per XCD
    // (xcd_unit): the 8 sequences of 1024 tokens of configuration 3 each run on
    // the XCD whose product blocks wrote their qkv rows
    constexpr int QUERIES = W * kAttnQB * 16;  // per block
    constexpr int ROWS = kAttnKeys / W;        // K and V rows each wave copies per step
    const int qblocks = (seq + QUERIES - 1) / QUERIES;
    const int unit = xcd_unit(blockIdx.x, gridDim.x);
    const int qblk = unit % qblocks, h = (unit / qblocks) % heads, b = unit / (qblocks * heads);
    const int width = heads * 64;
    const size_t ld3 = (size_t)3 * width;  // halves per token row of qkv
    const half_t *base = qkv + (size_t)b * seq * ld3;
    const int32x4_t rs = buffer_rsrc(base, (uint32_t)((size_t)seq * ld3 * 2));
    const uint32_t ks_lds = lds_address(ks), vs_lds = lds_address(vs);

    // Q^T fragments: lane (q4, j) holds Q[query j][dh 32ds + 8q4 + e]
    const int q0 = qblk * QUERIES + wave * (kAttnQB * 16);
    half8_t qf[kAttnQB][2];
#pragma unroll
    for (int qb = 0; qb < kAttnQB; qb++) {
        const int query = q0 + qb * 16 + j;
#pragma unroll
        for (int ds = 0; ds < 2; ds++) {
            half8_t v = {};
            if (query < seq) v = *(const half8_t *)(base + (size_t)query * ld3 + h * 64 + ds * 32 + q4 * 8);
            qf[qb][ds] = v;
        }
    }

    // Stage loads: wave w copies K rows and V rows ROWS*w .. ROWS*w + ROWS - 1
    // of a step, 8 rows per instruction (lane l -> row + l/8, 16-byte slot l%8).
    const uint32_t step_bytes = (uint32_t)(kAttnKeys * ld3 * 2);
    auto load_step = [&](int stage, int step) {
#pragma unroll
        for (int i = 0; i < ROWS / 8; i++) {
            const int lrow = wave * ROWS + i * 8 + lane / 8, lslot = lane % 8;
            const uint32_t koff = (uint32_t)(lrow * ld3 * 2 + width * 2 + h * 128 + ((lslot ^ ((lrow >> 1) & 7)) * 16));
            const uint32_t voff =
                (uint32_t)(lrow * ld3 * 2 + 2 * width * 2 + h * 128 + ((lslot ^ (2 * ((lrow >> 1) & 3))) * 16));
            const uint32_t at = (uint32_t)((wave * ROWS + i * 8) * 128);
            dma16(__builtin_amdgcn_readfirstlane(ks_lds + stage * kAttnKeys * 128 + at), koff + step * step_bytes, rs);
            dma16(__builtin_amdgcn_readfirstlane(vs_lds + stage * kAttnKeys * 128 + at), voff + step * step_bytes, rs);
        }
    };

    const float4_t fz = {0.f, 0.f, 0.f, 0.f};
    // the softmax denominators come from the MFMA pipe: an all-ones V^T operand
    // makes every row of lacc the running sum of the f16 P values of query j,
    // the same values the numerator O^T accumulates
    const half8_t ones = {(half_t)1.0f, (half_t)1.0f, (half_t)1.0f, (half_t)1.0f,
                          (half_t)1.0f, (half_t)1.0f, (half_t)1.0f, (half_t)1.0f};
    // The running maximum is raised only when a block's maximum exceeds it by
    // more than tau (8 in the log2 domain), so P stays below 2^8 and most steps
    // skip the rescale; any reference maximum gives the same quotient.
    const float tau = 8.0f / scale_log2;
    float4_t o[kAttnQB][4];  // O^T[dh 16db + 4q4 + v][query j]
    float4_t lacc[kAttnQB];  // every component: sum of P over keys, query j
    float mrow[kAttnQB];
#pragma unroll
    for (int qb = 0; qb < kAttnQB; qb++) {
        mrow[qb] = -INFINITY;
        lacc[qb] = fz;
#pragma unroll
        for (int db = 0; db < 4; db++) o[qb][db] = fz;
    }

    const int steps = (seq + kAttnKeys - 1) / kAttnKeys;
    // one step of 64 keys; MASK (the ragged last step only) sets scores of
    // keys past seq to -inf
    auto step = [&](int st, auto mask_c) {
        constexpr bool MASK = decltype(mask_c)::value;
        const int cur = st & 1;
        // this wave's loads of step st are done; the barrier covers every wave
        // (and every wave has finished reading the stage the next loads overwrite)
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __builtin_amdgcn_s_barrier();
        if (st + 1 < steps) load_step(cur ^ 1, st + 1);
        const uint8_t *kst = ks + cur * kAttnKeys * 128;
        const uint8_t *vst = vs + cur * kAttnKeys * 128;

        // S^T for 64 keys: sc[qb][kb][v] = S^T[key 16kb + 4q4 + v][query j]
        float4_t sc[kAttnQB][4];
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            const int r = kb * 16 + j;
            half8_t kf[2];
#pragma unroll
            for (int ds = 0; ds < 2; ds++) kf[ds] = *(const half8_t *)(kst + r * 128 + (((ds * 4 + q4) ^ ((r >> 1) & 7)) * 16));
#pragma unroll
            for (int qb = 0; qb < kAttnQB; qb++) {
                float4_t acc = mfma_f16(kf[0], qf[qb][0], fz);
                sc[qb][kb] = mfma_f16(kf[1], qf[qb][1], acc);
            }
        }
        half8_t pf[kAttnQB][2];  // P^T operands of the two 32-key blocks
#pragma unroll
        for (int qb = 0; qb < kAttnQB; qb++) {
            // online softmax over this step's keys for query j (lanes j, j+16, j+32, j+48)
            if (MASK) {
#pragma unroll
                for (int kb = 0; kb < 4; kb++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        if (st * kAttnKeys + kb * 16 + q4 * 4 + v >= seq) sc[qb][kb][v] = -INFINITY;
            }
            float bmax = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 4; kb++)
#pragma unroll
                for (int v = 0; v < 4; v++) bmax = fmaxf(bmax, sc[qb][kb][v]);
            bmax = rows_max4(bmax);
            if (__builtin_amdgcn_ballot_w64(bmax > mrow[qb] + tau)) {
                const float mnew = fmaxf(mrow[qb], bmax);
                const float alpha = __builtin_amdgcn_exp2f((mrow[qb] - mnew) * scale_log2);
#pragma unroll
                for (int v = 0; v < 4; v++) lacc[qb][v] *= alpha;
#pragma unroll
                for (int db = 0; db < 4; db++)
#pragma unroll
                    for (int v = 0; v < 4; v++) o[qb][db][v] *= alpha;
                mrow[qb] = mnew;
            }
            const float moff = -mrow[qb] * scale_log2;
            // P^T of the two 32-key blocks, converted two values per instruction
#pragma unroll
            for (int c = 0; c < 2; c++) {
                float8_t e;
#pragma unroll
                for (int i = 0; i < 8; i++)
                    e[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qb][2 * c + i / 4][i % 4], scale_log2, moff));
                pf[qb][c] = __builtin_convertvector(e, half8_t);
            }
        }
        // O^T += V^T P^T over the two 32-key blocks; the V^T operand (8 keys
        // of dh 16db + j) is read just before the MFMAs that use it
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int db = 0; db < 4; db++) {
                short4_t part[2];
#pragma unroll
                for (int r2 = 0; r2 < 2; r2++) {
                    // lane 16g + 4v + a addresses row 32c + 16r2 + 4g + v, unit 4db + a
                    const int row = 32 * c + 16 * r2 + 4 * q4 + (j >> 2);
                    const int unit = (4 * db + (j & 3)) ^ (4 * ((row >> 1) & 3));
                    part[r2] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) short4_t *)(vst + row * 128 + unit * 8));
                }
                const uint2_t lo = __builtin_bit_cast(uint2_t, part[0]), hi = __builtin_bit_cast(uint2_t, part[1]);
                const half8_t vf = as_half8(uint4_t{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
                for (int qb = 0; qb < kAttnQB; qb++) o[qb][db] = mfma_f16(vf, pf[qb][c], o[qb][db]);
            }
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int qb = 0; qb < kAttnQB; qb++) lacc[qb] = mfma_f16(ones, pf[qb][c], lacc[qb]);
    };
    load_step(0, 0);
    const int full = seq / kAttnKeys;  // steps with 64 live keys
    for (int st = 0; st < full; st++) step(st, std::false_type{});
    if (full < steps) step(full, std::true_type{});

    __builtin_amdgcn_s_waitcnt(0x0F70);  // no LDS write in flight once the block ends
#pragma unroll
    for (int qb = 0; qb < kAttnQB; qb++) {
        const float l = lacc[qb][0];
        const int query = q0 + qb * 16 + j;
        if (query >= seq) continue;
        const float inv = 1.0f / l;
        half_t *dst = out + ((size_t)b * seq + query) * width + h * 64;
#pragma unroll
        for (int db = 0; db < 4; db++) {
            const half2_t r01 = {(half_t)(o[qb][db][0] * inv), (half_t)(o[qb][db][1] * inv)};
            const half2_t r23 = {(half_t)(o[qb][db][2] * inv), (half_t)(o[qb][db][3] * inv)};
            *(uint2_t *)(dst + db * 16 + q4 * 4) = uint2_t{half2_as_word(r01), half2_as_word(r23)};
        }
    }
}

// ---- random fill (counter-based hash + Box-Muller) ------------------------------------

__device__ __forceinline__ uint32_t mix32(uint64_t x) {
    x ^= x >> 33;
    x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33;
    x *= 0xc4ceb9fe1a85ec53ull;
    x ^= x >> 33;
    return (uint32_t)x;
}

__global__ void fill_normal_kernel(float *p, size_t n, uint64_t seed, float stddev) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t a = mix32(seed * 0x9e3779b97f4a7c15ull + 2 * i + 1);
    uint32_t b = mix32(seed * 0x9e3779b97f4a7c15ull + 2 * i + 2);
    float u1 = ((a >> 8) + 1) * (1.0f / 16777217.0f);
    float u2 = (b >> 8) * (1.0f / 16777216.0f);
    p[i] = stddev * sqrtf(-2.0f * logf(u1)) * cosf(6.2831853071795864f * u2);
}

__global__ void fill_f32_kernel(float *p, size_t n, float v) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace

void launch_layernorm(const void *x, void *y, int dtype, int rows, int d, const float *w,
                      const float *b, float eps, hipStream_t s) {
    if (!rows) return;
    // one wave per f16 row of 512, 1024 or 2048 columns (16-byte aligned rows and weights)
    const bool fast = dtype == 1 && (d == 512 || d == 1024 || d == 2048) &&
                      (((uintptr_t)x | (uintptr_t)y | (uintptr_t)w | (uintptr_t)b) & 15) == 0;
    if (fast) {
        // 4-wave blocks, two per compute unit (or fewer when rows are few): a
        // wave keeps the gains and biases in registers over its rows and has the
        // next row's load in flight while it normalises the current one
        // one wave per row at a time, the block count rounded to a multiple of
        // the XCD count; past 2 blocks per compute unit waves walk several rows
        const unsigned want = std::min((unsigned)cdiv(rows, 4), (unsigned)(8 * device_cus()));
        const dim3 grid(want >= 64 ? (want + 7) / 8 * 8 : want);
        const half_t *xh = (const half_t *)x;
        half_t *yh = (half_t *)y;
        if (d == 512) hipLaunchKernelGGL(layernorm_f16_rows_kernel<1>, grid, dim3(256), 0, s, xh, yh, rows, w, b, eps);
        else if (d == 1024) hipLaunchKernelGGL(layernorm_f16_rows_kernel<2>, grid, dim3(256), 0, s, xh, yh, rows, w, b, eps);
        else hipLaunchKernelGGL(layernorm_f16_rows_kernel<4>, grid, dim3(256), 0, s, xh, yh, rows, w, b, eps);
        return;
    }
    hipLaunchKernelGGL(layernorm_kernel, dim3(rows), dim3(256), 0, s, x, y, dtype, d, w, b, eps);
}
void launch_rmsnorm(const float *x, float *y, int rows, int d, const float *w, float eps,
                    int zero_centered, hipStream_t s) {
    if (rows)
        hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, y, d, w, eps, zero_centered);
}
void launch_readout_rms(const void *h, int dtype, const int32_t *rows, int n, int d, const float *w,
                        float eps, int zero_centered, float *y, hipStream_t s) {
    if (!n || !d) return;
    const size_t lds = (size_t)d * sizeof(float);
    if (dtype == 1)
        hipLaunchKernelGGL(readout_rms_kernel<1>, dim3(n), dim3(256), lds, s, h, rows, d, w, eps, zero_centered, y);
    else
        hipLaunchKernelGGL(readout_rms_kernel<0>, dim3(n), dim3(256), lds, s, h, rows, d, w, eps, zero_centered, y);
}
void launch_flag_nonfinite(const float *y, size_t n, int *flag, int bit, hipStream_t s) {
    if (n) hipLaunchKernelGGL(flag_nonfinite_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, y, n, flag, bit);
}
void launch_to_f32(const void *x, int dtype, size_t n, float *y, hipStream_t s) {
    if (n) hipLaunchKernelGGL(to_f32_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, x, dtype, n, y);
}
void launch_f16_epilogue(const float *v, int epi, const half_t *res, half_t *y, size_t n, hipStream_t s) {
    if (n) hipLaunchKernelGGL(f16_epilogue_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, v, epi, res, y, n);
}
void launch_gelu(void *x, int dtype, size_t n, hipStream_t s) {
    if (n) hipLaunchKernelGGL(gelu_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, x, dtype, n);
}
void launch_silu_mul(float *g, const float *u, size_t n, hipStream_t s) {
    if (n) hipLaunchKernelGGL(silu_mul_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, g, u, n);
}
void launch_add(void *x, const void *y, int dtype, size_t n, hipStream_t s) {
    if (n) hipLaunchKernelGGL(add_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, x, y, dtype, n);
}
void launch_softmax_rows(float *x, int rows, int n, hipStream_t s) {
    if (rows) hipLaunchKernelGGL(softmax_rows_kernel, dim3(rows), dim3(256), 0, s, x, n);
}
void launch_mean_rows(const void *x, int dtype, int batch, int rows, int d, float *out,
                      hipStream_t s) {
    if (!batch || !d) return;
    if (dtype == 1 && d % 8 == 0 && ((uintptr_t)x & 15) == 0) {
        hipLaunchKernelGGL(mean_rows_f16_kernel, dim3(cdiv(d, 128) * batch), dim3(1024), 0, s, (const half_t *)x, rows,
                           d, out);
        return;
    }
    hipLaunchKernelGGL(mean_rows_kernel, dim3(cdiv(d, 64), batch), dim3(1024), 0, s, x, dtype, batch, rows, d, out);
}
void launch_attention(const half_t *qkv, half_t *out, int batch, int seq, int heads, int dh,
                      float scale, hipStream_t s) {
    (void)dh;
    if (!batch || !seq) return;
    const dim3 grid(cdiv(seq, kAttnWaves * kAttnQB * 16) * heads * batch);
    hipLaunchKernelGGL(attention_kernel<kAttnWaves>, grid, dim3(kAttnWaves * 64), 0, s, qkv, out, seq, heads,
                       scale * 1.4426950408889634f);
}
void launch_fill_normal_f32(float *p, size_t n, uint64_t seed, float stddev, hipStream_t s) {
    if (n) hipLaunchKernelGGL(fill_normal_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, p, n, seed, stddev);
}
void launch_fill_f32(float *p, size_t n, float v, hipStream_t s) {
    if (n) hipLaunchKernelGGL(fill_f32_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, p, n, v);
}

}  // namespace dz
