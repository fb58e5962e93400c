// quant.hip -- weight re-tiling, device quantizers and dequantization.
//
// Reference behaviour (hyperlogue/decisive):
//  - wire layout and its validation: src/models/pplx_flash/packed.rs:3-73
//  - grouped quantizer: int8.rs:305-360 (scale = max(absmax/L, FLT_MIN),
//    code = clamp(rne(v * recip(scale)), +-L)), applied per 64-run at load
//    (int8.rs:51-152) and per (token, 64-run) to activations (int8.rs:178-202)
//  - per-row int8 quantizer: webgpu/int8.rs:107-145
// Divisions and reciprocals use the correctly rounded __fdiv_rn/__frcp_rn and
// products __fmul_rn, so codes and scales equal the CPU's bit for bit.
#include <float.h>

#include "kernels.hpp"

namespace dz {

namespace {

__device__ __forceinline__ uint32_t place_nibble(int e, uint32_t nib) {
    return nib << ((e & 1) * 16 + (e >> 1) * 4);
}

// Offset of lane (q, j) word s of chunk (t, kb) in the Q4 code array.
__device__ __forceinline__ size_t q4_word(int t, int kb, int kbs, int q, int j, int s) {
    return ((((size_t)t * kbs + kb) * 64 + q * 16 + j) * 16) + s * 4;
}

// ---- wire -> native ----------------------------------------------------------

// One thread per (row n, k-block kb, lane q): builds that lane's 16 bytes.
// fitted: the scales of fitted Q4 weights (quantization.rs mse) may be
// negative; any finite nonzero scale is accepted then.
__global__ void upload_q4_kernel(const uint8_t *__restrict__ wire, uint8_t *__restrict__ codes,
                                 uint8_t *__restrict__ scales, int rows, int cols, int np,
                                 int kbs, int g32, int fitted, int *bad) {
    size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    size_t total = (size_t)np * kbs * 4;
    if (id >= total) return;
    int q = (int)(id % 4);
    int kb = (int)((id / 4) % kbs);
    int n = (int)(id / 4 / kbs);
    int t = n / 16, j = n % 16;
    const int run = g32 ? 32 : 64;
    const int gbytes = g32 ? 18 : 36;
    const size_t row_bytes = (size_t)(cols / run) * gbytes;
    uint32_t words[4];
    for (int s = 0; s < 4; s++) {
        uint32_t w = 0;
        for (int e = 0; e < 8; e++) {
            int k = kb * 128 + s * 32 + q * 8 + e;
            uint32_t nib = 8;
            if (n < rows && k < cols) {
                const uint8_t *group = wire + n * row_bytes + (size_t)(k / run) * gbytes;
                int kk = k % run;
                nib = (group[kk / 2] >> (4 * (kk % 2))) & 15u;
            }
            w |= place_nibble(e, nib);
        }
        words[s] = w;
    }
    uint4_t out = {words[0], words[1], words[2], words[3]};
    *(uint4_t *)(codes + q4_word(t, kb, kbs, q, j, 0)) = out;
    if (q != 0) return;
    uint8_t *rec = scales + (((size_t)t * kbs + kb) * 16 + j) * 8;
    if (g32) {
        uint16_t hs[4];
        for (int s = 0; s < 4; s++) {
            int g = kb * 4 + s;
            uint16_t h = 0;
            if (n < rows && g * 32 < cols) {
                const uint8_t *group = wire + n * row_bytes + (size_t)g * 18;
                h = (uint16_t)(group[16] | (group[17] << 8));
                float v = f16_bits_to_float(h);
                if (!(v > 0.0f && v <= 65504.0f)) atomicOr(bad, 1);
            }
            hs[s] = h;
        }
        uint2_t r = {(uint32_t)hs[0] | ((uint32_t)hs[1] << 16), (uint32_t)hs[2] | ((uint32_t)hs[3] << 16)};
        *(uint2_t *)rec = r;
    } else {
        float fs[2];
        for (int h = 0; h < 2; h++) {
            int g = kb * 2 + h;
            float v = 0.0f;
            if (n < rows && g * 64 < cols) {
                const uint8_t *group = wire + n * row_bytes + (size_t)g * 36;
                uint32_t bits = group[32] | (group[33] << 8) | (group[34] << 16) | ((uint32_t)group[35] << 24);
                v = __builtin_bit_cast(float, bits);
                const bool ok = fitted ? (v != 0.0f && fabsf(v) <= FLT_MAX) : (v > 0.0f && v <= FLT_MAX);
                if (!ok) atomicOr(bad, 1);
            }
            fs[h] = v;
        }
        *(float2 *)rec = make_float2(fs[0], fs[1]);
    }
}

__global__ void upload_q8_kernel(const uint8_t *__restrict__ wire, uint8_t *__restrict__ codes,
                                 float *__restrict__ scales, int rows, int cols, int np, int kbs,
                                 int *bad) {
    size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    size_t total = (size_t)np * kbs * 4;
    if (id >= total) return;
    int q = (int)(id % 4);
    int kb = (int)((id / 4) % kbs);
    int n = (int)(id / 4 / kbs);
    int t = n / 16, j = n % 16;
    const size_t row_bytes = (size_t)(cols / 64) * 68;
    uint8_t out[16];
    for (int e = 0; e < 16; e++) {
        int k = kb * 64 + q * 16 + e;
        out[e] = (n < rows && k < cols) ? wire[n * row_bytes + (size_t)kb * 68 + q * 16 + e] : 0;
    }
    uint8_t *dst = codes + ((((size_t)t * kbs + kb) * 64) + q * 16 + j) * 16;
    for (int e = 0; e < 16; e++) dst[e] = out[e];
    if (q == 0) {
        float v = 0.0f;
        if (n < rows && kb * 64 < cols) {
            const uint8_t *g = wire + n * row_bytes + (size_t)kb * 68 + 64;
            v = __builtin_bit_cast(float, (uint32_t)(g[0] | (g[1] << 8) | (g[2] << 16) | ((uint32_t)g[3] << 24)));
            if (!(v > 0.0f && v <= FLT_MAX)) atomicOr(bad, 1);
        }
        scales[((size_t)t * kbs + kb) * 16 + j] = v;
    }
}

// ---- device quantizer ------------------------------------------------------------

__device__ __forceinline__ float load_value(const void *p, int dtype, size_t i) {
    if (dtype == 0) return ((const float *)p)[i];
    if (dtype == 1) return (float)((const half_t *)p)[i];
    uint32_t b = ((const uint16_t *)p)[i];
    return __builtin_bit_cast(float, b << 16);
}

// One thread per (row n, run g) of `run` values (64 or 32).
__global__ void quantize_weight_kernel(const void *__restrict__ values, int dtype,
                                       uint8_t *__restrict__ codes, uint8_t *__restrict__ scales,
                                       int rows, int cols, int kbs, int bits, int run, int *bad) {
    int runs = (cols + run - 1) / run;
    size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (id >= (size_t)rows * runs) return;
    int g = (int)(id % runs);
    int n = (int)(id / runs);
    int t = n / 16, j = n % 16;
    float v[64];
    float maximum = 0.0f;
    bool finite = true;
    for (int i = 0; i < run; i++) {
        int k = g * run + i;
        float x = k < cols ? load_value(values, dtype, (size_t)n * cols + k) : 0.0f;
        finite = finite && __builtin_isfinite(x);
        v[i] = x;
        maximum = fmaxf(maximum, fabsf(x));
    }
    if (!finite) {
        atomicOr(bad, 1);
        return;
    }
    const float limit = bits == 4 ? 7.0f : 127.0f;
    float scale;
    if (run == 32) {  // group-32 / f16 scale: floor at the smallest f16 subnormal
        scale = __fdiv_rn(maximum, 7.0f);
        if (!(scale > 5.9604644775390625e-8f)) scale = 5.9604644775390625e-8f;
    } else {
        scale = fmaxf(__fdiv_rn(maximum, limit), FLT_MIN);
    }
    float inverse = __frcp_rn(scale);
    if (bits == 8) {
        uint8_t *base = codes + (((size_t)t * kbs + g) * 64) * 16;
        for (int q = 0; q < 4; q++) {
            uint8_t *dst = base + (q * 16 + j) * 16;
            for (int e = 0; e < 16; e++) dst[e] = (uint8_t)(int8_t)quantize_code(v[q * 16 + e], inverse, limit);
        }
        ((float *)scales)[((size_t)t * kbs + g) * 16 + j] = scale;
        return;
    }
    // Q4: a 64-run covers sub-blocks 2*(g%2), +1 of k-block g/2; a 32-run one sub-block.
    int kb = run == 64 ? g / 2 : g / 4;
    int s0 = run == 64 ? 2 * (g % 2) : g % 4;
    for (int sub = 0; sub < run / 32; sub++) {
        for (int q = 0; q < 4; q++) {
            uint32_t w = 0;
            for (int e = 0; e < 8; e++) {
                int c = quantize_code(v[sub * 32 + q * 8 + e], inverse, limit);
                w |= place_nibble(e, (uint32_t)(c + 8));
            }
            *(uint32_t *)(codes + q4_word(t, kb, kbs, q, j, s0 + sub)) = w;
        }
    }
    uint8_t *rec = scales + (((size_t)t * kbs + kb) * 16 + j) * 8;
    if (run == 64) {
        ((float *)rec)[g % 2] = scale;
    } else {
        half_t h = (half_t)scale;  // round to nearest even
        ((half_t *)rec)[g % 4] = h;
    }
}

// ---- dequantization ------------------------------------------------------------------

// The NF4 codebook (QLoRA, Dettmers et al. 2023: quantiles of N(0, 1)
// normalized to [-1, 1] with an exact zero), quantization.rs:3-20.
__constant__ float kNf4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

// One thread per (output row r, 8 consecutive k). Fitted Q4 weights decode as
// quantized_rows.rs:89-110 append: value = f32(code) or NF4[code + 8], times
// the scale, then plus the group's offset (affine), each step rounded.
__global__ void dequant_kernel(const uint8_t *__restrict__ codes, const uint8_t *__restrict__ scales,
                               const int32_t *__restrict__ ids, int count, int rows, int cols,
                               int kbs, int bits, int g32, void *__restrict__ y, int dtype,
                               int *bad, const uint8_t *__restrict__ offsets, int nf4) {
    int k8s = (cols + 7) / 8;
    size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (id >= (size_t)count * k8s) return;
    int k0 = (int)(id % k8s) * 8;
    int r = (int)(id / k8s);
    int n = ids ? ids[r] : r;
    int t = n / 16, j = n % 16;
    float out[8];
    if (n < 0 || n >= rows) {  // out-of-range token id: zeros and a flag, never a wild read
        if (bad) atomicOr(bad, 1);
        for (int e = 0; e < 8; e++) out[e] = 0.0f;
    } else if (bits == 4) {
        int kb = k0 / 128, s = (k0 % 128) / 32, q = (k0 % 32) / 8;
        uint32_t w = *(const uint32_t *)(codes + q4_word(t, kb, kbs, q, j, s));
        const uint8_t *rec = scales + (((size_t)t * kbs + kb) * 16 + j) * 8;
        float scale = g32 ? (float)((const half_t *)rec)[s] : ((const float *)rec)[(k0 % 128) / 64];
        for (int e = 0; e < 8; e++) {
            const int nib = (int)((w >> ((e & 1) * 16 + (e >> 1) * 4)) & 15u);
            out[e] = __fmul_rn(nf4 ? kNf4[nib] : (float)(nib - 8), scale);
        }
        if (offsets) {
            const float o = ((const float *)(offsets + (((size_t)t * kbs + kb) * 16 + j) * 8))[(k0 % 128) / 64];
            for (int e = 0; e < 8; e++) out[e] = __fadd_rn(out[e], o);
        }
    } else {
        int kb = k0 / 64, q = (k0 % 64) / 16, off = k0 % 16;
        const int8_t *src = (const int8_t *)(codes + ((((size_t)t * kbs + kb) * 64) + q * 16 + j) * 16 + off);
        float scale = ((const float *)scales)[((size_t)t * kbs + kb) * 16 + j];
        for (int e = 0; e < 8; e++) out[e] = __fmul_rn((float)src[e], scale);
    }
    for (int e = 0; e < 8 && k0 + e < cols; e++) {
        size_t at = (size_t)r * cols + k0 + e;
        if (dtype == 0)
            ((float *)y)[at] = out[e];
        else
            ((half_t *)y)[at] = (half_t)out[e];
    }
}

// ---- activation quantizer (a4) --------------------------------------------------------

// 16 lanes per (row, 64-group); each lane owns 4 consecutive values.
// records != nullptr writes the 17-word records of grouped_q4.rs:3-25 instead:
// words 0..15 the codes (4 per word, element 4l+e in byte e), word 16 the scale.
__global__ void act_quantize_kernel(const float *__restrict__ x, int m, int k, int bits,
                                    int8_t *__restrict__ q, float *__restrict__ sc, int *bad,
                                    uint32_t *__restrict__ records) {
    int groups = (k + 63) / 64;
    size_t gid = (blockIdx.x * (size_t)blockDim.x + threadIdx.x) / 16;
    int l = threadIdx.x % 16;
    bool active = gid < (size_t)m * groups;
    int g = active ? (int)(gid % groups) : 0;
    int r = active ? (int)(gid / groups) : 0;
    float v[4];
    float maximum = 0.0f;
    bool finite = true;
    for (int e = 0; e < 4; e++) {
        int kk = g * 64 + l * 4 + e;
        float val = (active && kk < k) ? x[(size_t)r * k + kk] : 0.0f;
        finite = finite && __builtin_isfinite(val);
        v[e] = val;
        maximum = fmaxf(maximum, fabsf(val));
    }
    for (int off = 8; off > 0; off >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off, 16));
    if (!active) return;
    if (!finite && bad) atomicOr(bad, 1);
    const float limit = bits == 4 ? 7.0f : 127.0f;
    float scale = fmaxf(__fdiv_rn(maximum, limit), FLT_MIN);
    float inverse = __frcp_rn(scale);
    uint32_t word = 0;
    for (int e = 0; e < 4; e++) {
        int kk = g * 64 + l * 4 + e;
        int c = kk < k ? quantize_code(v[e], inverse, limit) : 0;
        word |= ((uint32_t)(uint8_t)(int8_t)c) << (8 * e);
    }
    if (records != nullptr) {
        uint32_t *rec = records + ((size_t)r * groups + g) * 17;
        rec[l] = word;
        if (l == 0) rec[16] = __builtin_bit_cast(uint32_t, scale);
        return;
    }
    *(uint32_t *)(q + ((size_t)r * groups + g) * 64 + l * 4) = word;
    if (l == 0) sc[(size_t)r * groups + g] = scale;
}

// ---- zero-centred RMSNorm fused with the A8 quantizer -------------------------------
//
// Rows of d floats (d % 64 == 0), in two launches:
//  1. rms_row_scale_kernel: lane l of wave 0 owns row 16 * block + l % 16
//     and adds the row's squares in row order, as pplx_flash/cpu.rs:310-333
//     does (the readout norm's arithmetic, bit for bit). Wave 1 streams
//     64-column tiles of the block's 16 rows into 16 LDS stages by
//     buffer_load ... lds, 14 tiles ahead, and squares each tile in place one
//     tile ahead of wave 0, so wave 0's chain of d dependent adds is all it
//     waits for. A tile row's 16-byte chunk c sits at slot c ^ row, so the 16
//     rows' reads of one chunk index hit distinct banks. The row scale
//     1 / sqrt(ss / d + eps) goes to sc[row * groups], the first of the row's
//     group-scale slots.
//  2. rms_apply_quantize_kernel: one block per row takes that scale, then every
//     wave takes 64-column groups: v = (x * scale) * (1 + w) (w when not
//     zero-centred), written to y when y is set, and the group's A8 codes and
//     scale exactly as act_quantize_kernel computes them from v
//     (int8.rs:178-202), so a product of these codes equals the product of y.
//     A non-finite v sets *bad.
constexpr int kRmsRows = 16;    // rows (chains) per block
constexpr int kRmsStages = 16;  // 64-column tiles in LDS

__global__ __launch_bounds__(128) void rms_row_scale_kernel(const float *__restrict__ h, int rows, int d, float eps,
                                                            float *__restrict__ sc) {
    __shared__ __align__(16) float stages[kRmsStages][kRmsRows * 64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int row0 = blockIdx.x * kRmsRows;
    const int nrows = min(kRmsRows, rows - row0), tiles = d / 64;
    constexpr int PER_TILE = kRmsRows / 4;  // DMA instructions per tile
    static_assert((kRmsStages - 2) * PER_TILE <= 63, "vmcnt range");
    if (wave == 1) {
        const int32x4_t rs = buffer_rsrc(h + (size_t)row0 * d, (uint32_t)(nrows * d * 4));
        const uint32_t base = lds_address(&stages[0][0]);
        // DMA instruction i of a tile fills rows 4i..4i+3: lane j -> row 4i + j / 16,
        // slot j % 16, which holds the row's chunk (j % 16) ^ row
        auto dma_tile = [&](int t) {
            const int slot = t % kRmsStages;
#pragma unroll
            for (int i = 0; i < PER_TILE; i++) {
                const int r = 4 * i + lane / 16, c = (lane % 16) ^ r;
                dma16(base + (uint32_t)(slot * kRmsRows * 64 * 4 + i * 1024),
                      (uint32_t)((r * d + t * 64 + 4 * c) * 4), rs);
            }
        };
        auto square_tile = [&](int t) {
            float4_t *p = (float4_t *)stages[t % kRmsStages];
            float4_t v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = p[lane + 64 * i];
#pragma unroll
            for (int i = 0; i < 4; i++)
                p[lane + 64 * i] = float4_t{__fmul_rn(v[i][0], v[i][0]), __fmul_rn(v[i][1], v[i][1]),
                                            __fmul_rn(v[i][2], v[i][2]), __fmul_rn(v[i][3], v[i][3])};
        };
#pragma unroll
        for (int t = 0; t < kRmsStages - 1; t++)
            if (t < tiles) dma_tile(t);
        if (kRmsStages - 2 < tiles)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kRmsStages - 2) * PER_TILE) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        square_tile(0);
        __syncthreads();
        for (int t = 0; t < tiles; t++) {
            if (t + 1 < tiles) {
                // tile t + 1 landed (tiles up to t + NS - 2 are issued)
                if (t + kRmsStages - 2 < tiles)
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kRmsStages - 3) * PER_TILE) : "memory");
                else
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                square_tile(t + 1);
                // wave 0 read tile t - 1 before the last barrier
                if (t + kRmsStages - 1 < tiles) dma_tile(t + kRmsStages - 1);
            }
            __syncthreads();
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no LDS write in flight once the block ends
        return;
    }
    const int r = lane % kRmsRows;
    auto read_half = [&](int t, int half, float4_t *v) {
        const float *row = &stages[t % kRmsStages][r * 64];
#pragma unroll
        for (int c = 0; c < 8; c++) v[c] = *(const float4_t *)(row + 4 * ((8 * half + c) ^ r));
    };
    float ss = 0.0f;
    auto add_half = [&](const float4_t *v) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 8; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) ss = __fadd_rn(ss, v[c][e]);
        __builtin_amdgcn_sched_barrier(0);
    };
    float4_t x0[8], x1[8];
    __syncthreads();  // tile 0 squared
    for (int t = 0; t < tiles; t++) {
        read_half(t, 0, x0);
        read_half(t, 1, x1);
        add_half(x0);
        add_half(x1);
        __syncthreads();  // tile t read; tile t + 1 squared
    }
    if (lane < nrows) {
        // the square root taken in f64 and rounded once (v_sqrt_f32 is not correctly rounded)
        const float q = __fadd_rn(__fdiv_rn(ss, (float)d), eps);
        sc[(size_t)(row0 + lane) * (d / 64)] = __fdiv_rn(1.0f, __double2float_rn(__dsqrt_rn((double)q)));
    }
}

__global__ __launch_bounds__(256) void rms_apply_quantize_kernel(const float *__restrict__ h, int d,
                                                                 const float *__restrict__ w, int zero_centered,
                                                                 float *__restrict__ y, int8_t *__restrict__ q,
                                                                 float *__restrict__ sc, int *bad) {
    const size_t row = blockIdx.x, base = row * (size_t)d;
    const int groups = d / 64;
    const float scale = sc[row * groups];
    __syncthreads();  // every thread has the row scale before group 0's scale replaces it
    // thread t takes columns 4t, 4t + 1, 4t + 2, 4t + 3 of every 1024-column
    // chunk: a 64-column group is 16 consecutive lanes of one wave. Every
    // load of the row is in flight before the first group is computed.
    constexpr int CHUNKS = 4;  // 4096 columns per pass
    const int lane16 = threadIdx.x % 16;
    for (int c0 = 0; c0 < d; c0 += CHUNKS * 1024) {
        float4_t xv[CHUNKS], wv[CHUNKS];
#pragma unroll
        for (int u = 0; u < CHUNKS; u++) {
            const int col = c0 + u * 1024 + 4 * (int)threadIdx.x;
            xv[u] = col < d ? *(const float4_t *)(h + base + col) : float4_t{0.f, 0.f, 0.f, 0.f};
            wv[u] = col < d ? *(const float4_t *)(w + col) : float4_t{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int u = 0; u < CHUNKS; u++) {
            const int col = c0 + u * 1024 + 4 * (int)threadIdx.x;
            if (c0 + u * 1024 >= d) break;  // uniform
            const bool live = col < d;  // the columns of a group are all live or all not
            float4_t v;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float gain = zero_centered ? __fadd_rn(1.0f, wv[u][e]) : wv[u][e];
                v[e] = __fmul_rn(__fmul_rn(xv[u][e], scale), gain);
            }
            float maximum = fabsf(v[0]);
#pragma unroll
            for (int e = 1; e < 4; e++) maximum = fmaxf(maximum, fabsf(v[e]));
            // the group's maximum over its 16 lanes
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off, 16));
            if (!live) continue;
            if (y) *(float4_t *)(y + base + col) = v;
            bool finite = true;
#pragma unroll
            for (int e = 0; e < 4; e++) finite = finite && __builtin_isfinite(v[e]);
            if (!finite && bad) atomicOr(bad, 1);
            const float s = fmaxf(__fdiv_rn(maximum, 127.0f), FLT_MIN);
            const float inverse = __frcp_rn(s);
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) word |= (uint32_t)(uint8_t)(int8_t)quantize_code(v[e], inverse, 127.0f) << (8 * e);
            *(uint32_t *)(q + base + col) = word;
            if (lane16 == 0) sc[row * groups + col / 64] = s;
        }
    }
}

// ---- per-row int8 quantizer (a11) -------------------------------------------------------

__global__ __launch_bounds__(256) void i8_quantize_rows_kernel(const float *__restrict__ x, int k,
                                                                int8_t *__restrict__ q,
                                                                float *__restrict__ scales,
                                                                int32_t *__restrict__ sums) {
    __shared__ float smax[4];
    __shared__ int ssum[4];
    int r = blockIdx.x;
    const float *row = x + (size_t)r * k;
    float maximum = 0.0f;
    for (int i = threadIdx.x; i < k; i += 256) maximum = fmaxf(maximum, fabsf(row[i]));
    for (int off = 32; off > 0; off >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off));
    if (threadIdx.x % 64 == 0) smax[threadIdx.x / 64] = maximum;
    __syncthreads();
    maximum = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    float scale = __fdiv_rn(maximum, 127.0f);
    int total = 0;
    for (int i = threadIdx.x; i < k; i += 256) {
        int v = 0;
        if (scale > 0.0f) {
            v = (int)__builtin_rintf(__fdiv_rn(row[i], scale));
            v = v < -127 ? -127 : (v > 127 ? 127 : v);
        }
        total += v;
        q[(size_t)r * k + i] = (int8_t)v;
    }
    for (int off = 32; off > 0; off >>= 1) total += __shfl_xor(total, off);
    if (threadIdx.x % 64 == 0) ssum[threadIdx.x / 64] = total;
    __syncthreads();
    if (threadIdx.x == 0) {
        scales[r] = scale;
        if (sums) sums[r] = ssum[0] + ssum[1] + ssum[2] + ssum[3];
    }
}

// ---- per-row Q4 (a13) -----------------------------------------------------------------

// webgpu/q4.rs:48-73: one block per row. scale = absmax/7 (f32 division, no
// floor); code = clamp(rne(x/scale), +-7), 0 when scale == 0; word j of the row
// holds element 8j+t as (code + 8) at bits 4t. After the rows*(k/8) code words
// come the rows f32 scales and the rows i32 code sums. Sets *bad on a
// non-finite value.
__global__ __launch_bounds__(256) void q4_quantize_rows_kernel(const void *__restrict__ values, int dtype,
                                                                int rows, int k, uint32_t *__restrict__ out,
                                                                int *bad) {
    __shared__ float smax[4];
    __shared__ int ssum[4];
    const int r = blockIdx.x;
    const size_t base = (size_t)r * k;
    float maximum = 0.0f;
    bool finite = true;
    for (int i = threadIdx.x; i < k; i += 256) {
        float v = load_value(values, dtype, base + i);
        finite = finite && __builtin_isfinite(v);
        maximum = fmaxf(maximum, fabsf(v));
    }
    if (!finite) atomicOr(bad, 1);
    for (int off = 32; off > 0; off >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, off));
    if (threadIdx.x % 64 == 0) smax[threadIdx.x / 64] = maximum;
    __syncthreads();
    maximum = fmaxf(fmaxf(smax[0], smax[1]), fmaxf(smax[2], smax[3]));
    const float scale = __fdiv_rn(maximum, 7.0f);
    const int words = k / 8;
    int total = 0;
    for (int w = threadIdx.x; w < words; w += 256) {
        uint32_t packed = 0;
        for (int t = 0; t < 8; t++) {
            int q = 0;
            if (scale > 0.0f) {
                q = (int)__builtin_rintf(__fdiv_rn(load_value(values, dtype, base + (size_t)w * 8 + t), scale));
                q = q < -7 ? -7 : (q > 7 ? 7 : q);
            }
            total += q;
            packed |= (uint32_t)(q + 8) << (4 * t);
        }
        out[(size_t)r * words + w] = packed;
    }
    for (int off = 32; off > 0; off >>= 1) total += __shfl_xor(total, off);
    if (threadIdx.x % 64 == 0) ssum[threadIdx.x / 64] = total;
    __syncthreads();
    if (threadIdx.x == 0) {
        out[(size_t)rows * words + r] = __builtin_bit_cast(uint32_t, scale);
        out[(size_t)rows * words + rows + r] = (uint32_t)(ssum[0] + ssum[1] + ssum[2] + ssum[3]);
    }
}

// Native Q4 group-64 -> packed.rs wire layout: one thread per (row, 64-run).
__global__ void export_q4g64_kernel(const uint8_t *__restrict__ codes,
                                    const uint8_t *__restrict__ scales, int rows, int cols, int kbs,
                                    uint8_t *__restrict__ wire) {
    int runs = cols / 64;
    size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (id >= (size_t)rows * runs) return;
    int g = (int)(id % runs), n = (int)(id / runs);
    int t = n / 16, j = n % 16, kb = g / 2, s0 = 2 * (g % 2);
    uint8_t *dst = wire + ((size_t)n * runs + g) * 36;
    for (int kk = 0; kk < 64; kk += 2) {
        uint32_t nib[2];
        for (int h = 0; h < 2; h++) {
            int k = kk + h, s = s0 + k / 32, q = (k % 32) / 8, e = k % 8;
            uint32_t w = *(const uint32_t *)(codes + q4_word(t, kb, kbs, q, j, s));
            nib[h] = (w >> ((e & 1) * 16 + (e >> 1) * 4)) & 15u;
        }
        dst[kk / 2] = (uint8_t)(nib[0] | (nib[1] << 4));
    }
    float sc = ((const float *)(scales + (((size_t)t * kbs + kb) * 16 + j) * 8))[g % 2];
    uint32_t b = __builtin_bit_cast(uint32_t, sc);
    for (int i = 0; i < 4; i++) dst[32 + i] = (uint8_t)(b >> (8 * i));
}

__global__ void fill_i32_kernel(int *p, int value, int count) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

inline unsigned blocks_for(size_t n, unsigned per) { return (unsigned)((n + per - 1) / per); }

// int8.rs:191-193 and :568-569: the factor the affine offset term takes per
// (row, 64-group), sx * f32(sum of the group's codes), rounded to f32. One
// thread per (row, group).
__global__ void act_sums_kernel(const int8_t *__restrict__ q, const float *__restrict__ sx, int m, int groups,
                                float *__restrict__ sxq) {
    const size_t id = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (id >= (size_t)m * groups) return;
    const int4_t *p = (const int4_t *)(q + id * 64);
    int sum = 0;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int4_t v = p[u];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t word = (uint32_t)v[w];
#pragma unroll
            for (int b = 0; b < 4; b++) sum += (int)(int8_t)(word >> (8 * b));
        }
    }
    sxq[id] = __fmul_rn(sx[id], (float)sum);
}

}  // namespace

void launch_upload(const Weight &w, const uint8_t *wire, int *bad, hipStream_t s, bool fitted) {
    size_t total = (size_t)w.np * w.kblocks() * 4;
    if (w.kind == WeightKind::Q8G64) {
        hipLaunchKernelGGL(upload_q8_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, wire,
                           w.codes, (float *)w.scales, w.rows, w.cols, w.np, w.kblocks(), bad);
    } else {
        hipLaunchKernelGGL(upload_q4_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, wire,
                           w.codes, w.scales, w.rows, w.cols, w.np, w.kblocks(),
                           w.kind == WeightKind::Q4G32 ? 1 : 0, fitted ? 1 : 0, bad);
    }
}

void launch_quantize_weight(const Weight &w, const void *values, int dtype, int *bad,
                            hipStream_t s) {
    int run = w.kind == WeightKind::Q4G32 ? 32 : 64;
    size_t total = (size_t)w.rows * ((w.cols + run - 1) / run);
    hipLaunchKernelGGL(quantize_weight_kernel, dim3(blocks_for(total, 128)), dim3(128), 0, s,
                       values, dtype, w.codes, w.scales, w.rows, w.cols, w.kblocks(), w.bits, run,
                       bad);
}

void launch_dequant_checked(const Weight &w, const int32_t *ids, int count, void *y, int dtype,
                            int *bad, hipStream_t s) {
    size_t total = (size_t)count * ((w.cols + 7) / 8);
    if (!total) return;
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, w.codes,
                       w.scales, ids, count, w.rows, w.cols, w.kblocks(), w.bits,
                       w.kind == WeightKind::Q4G32 ? 1 : 0, y, dtype, bad, w.offsets, w.nf4 ? 1 : 0);
}

void launch_dequant(const Weight &w, const int32_t *ids, int count, void *y, int dtype,
                    hipStream_t s) {
    launch_dequant_checked(w, ids, count, y, dtype, nullptr, s);
}

void launch_act_quantize(const float *x, int m, int k, int bits, int8_t *q, float *sc, int *bad,
                         hipStream_t s) {
    size_t lanes = (size_t)m * ((k + 63) / 64) * 16;
    if (!lanes) return;
    hipLaunchKernelGGL(act_quantize_kernel, dim3(blocks_for(lanes, 256)), dim3(256), 0, s, x, m, k,
                       bits, q, sc, bad, (uint32_t *)nullptr);
}

void launch_act_sums(const int8_t *q, const float *sx, int m, int groups, float *sxq, hipStream_t s) {
    const size_t n = (size_t)m * groups;
    if (!n) return;
    hipLaunchKernelGGL(act_sums_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, q, sx, m, groups, sxq);
}

void launch_act_quantize_records(const float *x, int m, int k, uint32_t *records, int *bad,
                                 hipStream_t s) {
    size_t lanes = (size_t)m * ((k + 63) / 64) * 16;
    if (!lanes) return;
    hipLaunchKernelGGL(act_quantize_kernel, dim3(blocks_for(lanes, 256)), dim3(256), 0, s, x, m, k,
                       8, (int8_t *)nullptr, (float *)nullptr, bad, records);
}

void launch_rms_quantize(const float *h, int rows, int d, const float *w, float eps, int zero_centered, float *y,
                         int8_t *q, float *sc, int *bad, hipStream_t s) {
    if (!rows) return;
    hipLaunchKernelGGL(rms_row_scale_kernel, dim3((unsigned)((rows + kRmsRows - 1) / kRmsRows)), dim3(128), 0, s, h,
                       rows, d, eps, sc);
    hipLaunchKernelGGL(rms_apply_quantize_kernel, dim3(rows), dim3(256), 0, s, h, d, w, zero_centered, y, q, sc, bad);
}

void launch_i8_quantize_rows(const float *x, int rows, int k, int8_t *q, float *scales,
                             int32_t *sums, hipStream_t s) {
    if (!rows) return;
    hipLaunchKernelGGL(i8_quantize_rows_kernel, dim3(rows), dim3(256), 0, s, x, k, q, scales, sums);
}

void launch_q4_quantize_rows(const void *values, int dtype, int rows, int k, uint32_t *out, int *bad,
                             hipStream_t s) {
    if (!rows) return;
    hipLaunchKernelGGL(q4_quantize_rows_kernel, dim3(rows), dim3(256), 0, s, values, dtype, rows, k, out, bad);
}

void launch_export_q4g64(const Weight &w, uint8_t *wire, hipStream_t s) {
    size_t total = (size_t)w.rows * (w.cols / 64);
    if (!total) return;
    hipLaunchKernelGGL(export_q4g64_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, s, w.codes,
                       w.scales, w.rows, w.cols, w.kblocks(), wire);
}

void launch_fill_i32(int *p, int value, int count, hipStream_t s) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks_for(count, 256)), dim3(256), 0, s, p, value,
                       count);
}

}  // namespace dz
