// probe.hip -- sustained issue rates of the device's units, from register-only
// loops over every compute unit. They are the ceilings the kernels' roofline
// fractions are read against: the published MFMA peaks assume clocks that a
// GEMM on random operands does not hold, and the attention softmax is bound
// by the rate of v_exp_f32 against v_fma_f32. No reference counterpart.
//
//   mfma_f16  v_mfma_f32_16x16x32_f16, 8 independent accumulators per wave,
//             successive instructions on different operand fragments
//   mfma_i8   v_mfma_i32_32x32x32_i8, 4 independent accumulators per wave
//   fma_f32   v_fma_f32, 8 independent chains per wave
//   exp_f32   v_exp_f32, 8 independent chains per wave
//   lds_b128  ds_read_b128 from LDS, 8 loads in flight per wave (bytes per
//             second, not operations)
// Operands are hashed from the thread index (or all zero, for the MFMA kinds
// with zero_operands), so the data toggles as a GEMM's does. One timed launch
// runs for several milliseconds; callers load the device first, since the
// clocks of an idle device ramp up under load.
#include <string.h>

#include <string>

#include "../../include/decisive_rocm.h"
#include "kernels.hpp"

namespace dz {

int32_t ctx_fail(dz_ctx *ctx, int32_t code, const std::string &msg);
int32_t ctx_hip_fail(dz_ctx *ctx, hipError_t e, const char *what);
hipStream_t ctx_stream(dz_ctx *ctx);

namespace {

constexpr int kProbeBlocksPerCu = 8;  // 256-thread blocks: 8 waves per SIMD
constexpr int kProbeThreads = 256;

__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Random f16 in [-1, 1) (or zero) as one 32-bit pair.
__device__ __forceinline__ uint32_t probe_half2(uint32_t h, bool zero) {
    if (zero) return 0;
    const half2_t v = {(half_t)((float)(h & 0xffff) / 32768.0f - 1.0f), (half_t)((float)(h >> 16) / 32768.0f - 1.0f)};
    return half2_as_word(v);
}

// (four waves per SIMD as the register budget: with a larger budget the
// allocator rotated the accumulators through AGPR copies every iteration)
template <bool ZERO>
__global__ __launch_bounds__(kProbeThreads, 4) void probe_mfma_f16_kernel(int iters, float *sink) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    half8_t a[4], b[4];
#pragma unroll
    for (int f = 0; f < 4; f++) {
        uint4_t ua, ub;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            ua[w] = probe_half2(probe_hash(t * 64 + f * 8 + w), ZERO);
            ub[w] = probe_half2(probe_hash(t * 64 + f * 8 + 4 + w + 0x9e37), ZERO);
        }
        a[f] = as_half8(ua);
        b[f] = as_half8(ub);
    }
    float4_t acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = mfma_f16(a[i & 3], b[(i + (i >> 2)) & 3], acc[i]);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) s += acc[i][0] + acc[i][3];
    sink[t] = s;
}

typedef int probe_i32x16 __attribute__((ext_vector_type(16)));

template <bool ZERO>
__global__ __launch_bounds__(kProbeThreads) void probe_mfma_i8_kernel(int iters, float *sink) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    int4_t a[2], b[2];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int w = 0; w < 4; w++) {
            a[f][w] = ZERO ? 0 : (int)probe_hash(t * 64 + f * 8 + w);
            b[f][w] = ZERO ? 0 : (int)probe_hash(t * 64 + f * 8 + 4 + w + 0x9e37);
        }
    probe_i32x16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = probe_i32x16{};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i & 1], b[(i >> 1) & 1], acc[i], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) s += acc[i][e];
    sink[t] = (float)s;
}

// KIND 0: x = fma(x, 0.999, 0.001); KIND 1: x = exp2(-x). Both stay in (0, 1].
template <int KIND>
__global__ __launch_bounds__(kProbeThreads) void probe_valu_kernel(int iters, float *sink) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = (float)(probe_hash(t * 8 + i) & 0xffff) / 65536.0f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (KIND == 0)
                x[i] = __builtin_fmaf(x[i], 0.999f, 0.001f);
            else
                x[i] = __builtin_amdgcn_exp2f(-x[i]);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) s += x[i];
    sink[t] = s;
}

// LDS read bandwidth: every wave reads 8 KB per iteration with ds_read_b128
// (64 lanes x 16 bytes of one 1 KB row per instruction, no bank conflicts).
// Lane l reads element (l + it) % 64 of each row, so the loads stay in the
// loop; two v_xor3 per load keep every byte live.
constexpr int kProbeLdsBytes = 8192;
__global__ __launch_bounds__(kProbeThreads) void probe_lds_kernel(int iters, float *sink) {
    __shared__ __align__(16) uint4_t buf[kProbeLdsBytes / 16];
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    for (int i = threadIdx.x; i < kProbeLdsBytes / 16; i += kProbeThreads) {
        const uint32_t h = probe_hash(blockIdx.x * 4096 + i);
        buf[i] = uint4_t{h, h ^ 0x9e3779b9u, h + 7u, h * 3u};
    }
    __syncthreads();
    const int lane = threadIdx.x % 64;
    uint32_t x0 = 0, x1 = 0;
    for (int it = 0; it < iters; it++) {
        const uint4_t *p = buf + ((lane + it) & 63);
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const uint4_t v = p[u * 64];
            x0 = x0 ^ v[0] ^ v[1];
            x1 = x1 ^ v[2] ^ v[3];
        }
    }
    sink[t] = (float)(x0 ^ x1);
}

}  // namespace

int32_t probe_rate(dz_ctx *ctx, int cus, const char *what, int zero, double *rate) {
    if (!what || !rate) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    const std::string w(what);
    // operations per instruction (FLOP or OP for the MFMA kinds, lane operations for the VALU kinds),
    // instructions per loop iteration per wave, and iterations
    double ops_per_inst = 0;
    int per_iter = 0, iters = 0;
    void (*kernel)(int, float *) = nullptr;
    if (w == "mfma_f16") {
        ops_per_inst = 2.0 * 16 * 16 * 32;
        per_iter = 8;
        iters = 16384;
        kernel = zero ? probe_mfma_f16_kernel<true> : probe_mfma_f16_kernel<false>;
    } else if (w == "mfma_i8") {
        ops_per_inst = 2.0 * 32 * 32 * 32;
        per_iter = 4;
        iters = 16384;
        kernel = zero ? probe_mfma_i8_kernel<true> : probe_mfma_i8_kernel<false>;
    } else if (w == "fma_f32" && !zero) {
        ops_per_inst = 64;
        per_iter = 8;
        iters = 65536;
        kernel = probe_valu_kernel<0>;
    } else if (w == "exp_f32" && !zero) {
        ops_per_inst = 64;
        per_iter = 8;
        iters = 16384;
        kernel = probe_valu_kernel<1>;
    } else if (w == "lds_b128" && !zero) {
        ops_per_inst = 64 * 16;  // bytes
        per_iter = 8;
        iters = 32768;
        kernel = probe_lds_kernel;
    } else {
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS,
                        "probe is mfma_f16, mfma_i8 (zero_operands 0 or 1), fma_f32, exp_f32 or lds_b128 "
                        "(zero_operands 0)");
    }
    const int blocks = cus * kProbeBlocksPerCu;
    hipStream_t s = ctx_stream(ctx);
    float *sink = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&sink, (size_t)blocks * kProbeThreads * sizeof(float));
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    float ms = 0.0f;
    if (e == hipSuccess) {
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kProbeThreads), 0, s, iters / 8, sink);  // warm-up
        hipEventRecord(e0, s);
        hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kProbeThreads), 0, s, iters, sink);
        hipEventRecord(e1, s);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (sink) hipFree(sink);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "rate probe");
    const double waves = (double)blocks * kProbeThreads / 64;
    *rate = waves * iters * per_iter * ops_per_inst / (ms * 1e-3);
    return DZ_OK;
}

}  // namespace dz
