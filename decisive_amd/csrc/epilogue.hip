// epilogue.hip -- layer epilogues and attention for the encoder forward.
//
// Reference behaviour:
//  - LayerNorm with bias:  src/models/decima/cpu.rs:529-540
//  - erf GELU:             src/models/decima/cpu.rs:542-556
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

// f16 rows of d = 512 * C columns: one wave per row, the row in registers
// (C 16-byte chunks per lane: columns 512c + 8*lane + 0..7), shuffle-tree
// sums, the same two-pass mean / variance as layernorm_kernel.
template <int C>
__global__ __launch_bounds__(256) void layernorm_f16_rows_kernel(const half_t *__restrict__ x,
                                                                 half_t *__restrict__ y, int rows,
                                                                 const float *__restrict__ w,
                                                                 const float *__restrict__ b, float eps) {
    constexpr int D = 512 * C;
    const int row = blockIdx.x * 4 + threadIdx.x / 64, lane = threadIdx.x % 64;
    if (row >= rows) return;  // whole wave
    const half_t *src = x + (size_t)row * D;
    float v[C][8];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const half8_t h = *(const half8_t *)(src + c * 512 + lane * 8);
#pragma unroll
        for (int e = 0; e < 8; e++) v[c][e] = (float)h[e];
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int e = 0; e < 8; e++) s += v[c][e];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    const float mean = s / (float)D;
    float q = 0.0f;
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float d0 = v[c][e] - mean;
            q += d0 * d0;
        }
    for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off);
    const float inv = 1.0f / sqrtf(q / (float)D + eps);
    half_t *dst = y + (size_t)row * D;
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int col = c * 512 + lane * 8;
        const float4_t w0 = *(const float4_t *)(w + col), w1 = *(const float4_t *)(w + col + 4);
        const float4_t b0 = *(const float4_t *)(b + col), b1 = *(const float4_t *)(b + col + 4);
        const float ww[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
        const float bb[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        half8_t o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (half_t)((v[c][e] - mean) * inv * ww[e] + bb[e]);
        *(half8_t *)(dst + col) = o;
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

__global__ void gelu_kernel(void *x, int dtype, size_t n) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= n) return;
    float v = ld(x, dtype, i);
    st(x, dtype, i, 0.5f * v * (1.0f + erff(v * 0.70710678118654752f)));
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
__global__ void mean_rows_kernel(const void *__restrict__ x, int dtype, int batch, int rows, int d,
                                 float *__restrict__ out) {
    size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (id >= (size_t)batch * d) return;
    int c = (int)(id % d), b = (int)(id / d);
    float s = 0.0f;
    for (int r = 0; r < rows; r++) s += ld(x, dtype, ((size_t)b * rows + r) * d + c);
    out[id] = s / (float)rows;
}

// ---- flash attention, head_dim 64 ----------------------------------------------------
//
// Block = 4 waves = 64 queries of one (batch, head). Scores are computed
// transposed, S^T = K Q^T, so a lane's accumulator column is one query: the
// online-softmax rescale is a per-lane scalar and the P^T values a lane holds
// (keys 16*kb + 4*qd + v) are exactly the keys it feeds to O^T = V^T P^T when
// the MFMA k-slots are labelled (kb pair, v). V is staged transposed in LDS.
constexpr int kAttnKeys = 64;
constexpr int kVStride = 72;  // halfs per V^T row (padding against bank conflicts)

__global__ __launch_bounds__(256) void attention_kernel(const half_t *__restrict__ qkv,
                                                        half_t *__restrict__ out, int seq,
                                                        int heads, float scale_log2) {
    __shared__ __align__(16) half_t ks[kAttnKeys * 64];
    __shared__ __align__(16) half_t vt[64 * kVStride];
    const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int qd = lane / 16, j = lane % 16;
    const int qblock = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int width = heads * 64;
    const size_t ld3 = (size_t)3 * width;
    const half_t *base = qkv + (size_t)b * seq * ld3;
    const int query = qblock * 64 + wave * 16 + j;
    const bool qok = query < seq;

    // Q^T fragments: lane (qd, j) holds Q[query j][dh 8qd + e] for dh halves 0/1.
    half8_t qf[2];
    for (int ds = 0; ds < 2; ds++) {
        half8_t v = {};
        if (qok) v = *(const half8_t *)(base + (size_t)query * ld3 + h * 64 + ds * 32 + qd * 8);
        qf[ds] = v;
    }
    const float4_t fz = {0.f, 0.f, 0.f, 0.f};
    float4_t o[4] = {fz, fz, fz, fz};  // O^T[dh 16*db + 4qd + v][query j]
    float mrow = -INFINITY, lsum = 0.0f;

    for (int k0 = 0; k0 < seq; k0 += kAttnKeys) {
        __syncthreads();
        // stage K (row-major, 16-byte chunks swizzled) and V^T
        for (int c = threadIdx.x; c < kAttnKeys * 8; c += 256) {
            int kr = c / 8, ch = c % 8;
            int key = k0 + kr;
            uint4_t kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
            if (key < seq) {
                const half_t *row = base + (size_t)key * ld3 + h * 64 + ch * 8;
                kv = *(const uint4_t *)(row + width);
                vv = *(const uint4_t *)(row + 2 * width);
            }
            *(uint4_t *)(ks + kr * 64 + ((ch ^ (kr & 7)) * 8)) = kv;
            half8_t vh = as_half8(vv);
            for (int e = 0; e < 8; e++) vt[(ch * 8 + e) * kVStride + kr] = vh[e];
        }
        __syncthreads();
        // S^T for 64 keys: 4 key blocks x 2 dh halves
        float4_t sc[4];
        for (int kb = 0; kb < 4; kb++) {
            float4_t acc = fz;
            int kr = kb * 16 + j;  // A row = key (lane%16)
            for (int ds = 0; ds < 2; ds++) {
                int ch = ds * 4 + qd;
                half8_t a = *(const half8_t *)(ks + kr * 64 + ((ch ^ (kr & 7)) * 8));
                acc = mfma_f16(a, qf[ds], acc);
            }
            sc[kb] = acc;  // lane holds S^T[key 16kb + 4qd + v][query j]
        }
        // online softmax over keys for query j (lanes j, j+16, j+32, j+48)
        float bmax = -INFINITY;
        for (int kb = 0; kb < 4; kb++)
            for (int v = 0; v < 4; v++) {
                int key = k0 + kb * 16 + qd * 4 + v;
                float s = key < seq ? sc[kb][v] * scale_log2 : -INFINITY;
                sc[kb][v] = s;
                bmax = fmaxf(bmax, s);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        float mnew = fmaxf(mrow, bmax);
        float alpha = __builtin_amdgcn_exp2f(mrow - mnew);
        mrow = mnew;
        lsum *= alpha;
        for (int db = 0; db < 4; db++)
            for (int v = 0; v < 4; v++) o[db][v] *= alpha;
        half_t p[4][4];
        for (int kb = 0; kb < 4; kb++)
            for (int v = 0; v < 4; v++) {
                float e = __builtin_amdgcn_exp2f(sc[kb][v] - mnew);
                lsum += e;
                p[kb][v] = (half_t)e;
            }
        // O^T += V^T P^T: two 32-slot steps, slots = (kb pair, v)
        for (int c = 0; c < 2; c++) {
            half8_t bfr = {p[2 * c][0], p[2 * c][1], p[2 * c][2], p[2 * c][3],
                           p[2 * c + 1][0], p[2 * c + 1][1], p[2 * c + 1][2], p[2 * c + 1][3]};
            for (int db = 0; db < 4; db++) {
                int dh = db * 16 + j;  // A row = dh (lane%16)
                const half_t *vr = vt + dh * kVStride;
                uint2_t lo = *(const uint2_t *)(vr + (2 * c) * 16 + qd * 4);
                uint2_t hi = *(const uint2_t *)(vr + (2 * c + 1) * 16 + qd * 4);
                uint4_t av = {lo[0], lo[1], hi[0], hi[1]};
                o[db] = mfma_f16(as_half8(av), bfr, o[db]);
            }
        }
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);
    if (!qok) return;
    float inv = 1.0f / lsum;
    half_t *dst = out + ((size_t)b * seq + query) * width + h * 64;
    for (int db = 0; db < 4; db++) {
        half_t r[4];
        for (int v = 0; v < 4; v++) r[v] = (half_t)(o[db][v] * inv);
        *(uint2_t *)(dst + db * 16 + qd * 4) = *(uint2_t *)r;
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
        const dim3 grid(cdiv(rows, 4));
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
    size_t n = (size_t)batch * d;
    if (n) hipLaunchKernelGGL(mean_rows_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, x, dtype, batch, rows, d, out);
}
void launch_attention(const half_t *qkv, half_t *out, int batch, int seq, int heads, int dh,
                      float scale, hipStream_t s) {
    (void)dh;
    if (!batch || !seq) return;
    dim3 grid(cdiv(seq, 64), heads, batch);
    hipLaunchKernelGGL(attention_kernel, grid, dim3(256), 0, s, qkv, out, seq, heads,
                       scale * 1.4426950408889634f);
}
void launch_fill_normal_f32(float *p, size_t n, uint64_t seed, float stddev, hipStream_t s) {
    if (n) hipLaunchKernelGGL(fill_normal_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, p, n, seed, stddev);
}
void launch_fill_f32(float *p, size_t n, float v, hipStream_t s) {
    if (n) hipLaunchKernelGGL(fill_f32_kernel, dim3(cdiv(n, 256)), dim3(256), 0, s, p, n, v);
}

}  // namespace dz
