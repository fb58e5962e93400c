// common.hpp -- shared definitions of libdecisive_rocm (gfx950 / CDNA4).
//
// Native HBM layout of a quantized weight [rows x cols] (called N x K below):
//
//   Q4 ("tile16x128"): N is padded to Np = 16*ceil(N/16), K to Kp = 128*ceil(K/128).
//     codes  : [Np/16][Kp/128][64 lanes][16 bytes]       (1 KiB per chunk)
//     scales : [Np/16][Kp/128][16 rows][8 bytes]          (128 B per chunk)
//   Lane l = q*16 + j of a chunk (t, kb) belongs to row n = 16*t + j. Its 16
//   bytes are four 32-bit words; word s holds the 8 codes of
//   k = 128*kb + 32*s + 8*q + e (e = 0..7) as (code + 8) nibbles, e = 2p at bits
//   4p and e = 2p+1 at bits 16 + 4p. With that order
//     ((word >> 4p) & 0x000F000F) | 0x64006400
//   is the f16 pair (1024 + code_2p + 8, 1024 + code_2p+1 + 8), so one packed
//   f16 subtract of 1032 yields the exact codes in k order -- the B fragment of
//   one v_mfma_f32_16x16x32_f16 per word, loaded with a single 128-bit load.
//   The 8-byte scale record of (t, kb, j) is four f16 scales (one per 32-run)
//   for group-32 weights or two f32 scales (one per 64-run) for group-64.
//
//   Q8 ("tile16x64"): Kp = 64*ceil(K/64); codes [Np/16][Kp/64][64 lanes][16 B],
//     lane (q, j) holds int8 codes of k = 64*kb + 16*q + 0..15 in order (the B
//     fragment of v_mfma_i32_16x16x64_i8); scales [Np/16][Kp/64][16] f32.
//
// Padding codes are 0 and padding scales 0, so padded rows/columns contribute
// nothing; kernels never read activations beyond K.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace dz {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef int int4_t __attribute__((ext_vector_type(4)));
typedef unsigned int uint4_t __attribute__((ext_vector_type(4)));
typedef unsigned int uint2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

enum class WeightKind : int { Q4G64 = 0, Q8G64 = 1, Q4G32 = 2 };

struct Weight {
    int rows = 0, cols = 0;       // N x K
    int np = 0, kp = 0;           // padded
    int bits = 4, group = 64;     // code bits and scale run length
    int groups = 0;               // ceil(K/64) for the grouped int8 path
    WeightKind kind = WeightKind::Q4G64;
    uint8_t *codes = nullptr;     // device
    uint8_t *scales = nullptr;    // device
    size_t code_bytes = 0, scale_bytes = 0;
    // Fitted Q4 (quantization.rs): `fitted` for any fitted form; `offsets`,
    // for the affine form, an f32 offset per (row, 64-group) laid out as the
    // group-64 scales ([tile][k-block][16 rows][2 f32], scale_bytes long);
    // `nf4` when the codes index the NF4 codebook.
    uint8_t *offsets = nullptr;
    bool fitted = false, nf4 = false;
    int tiles() const { return np / 16; }
    int kblocks() const { return bits == 4 ? kp / 128 : kp / 64; }
};

// ---- device helpers ---------------------------------------------------------

__device__ __forceinline__ half8_t as_half8(uint4_t v) { return __builtin_bit_cast(half8_t, v); }

// Bit casts of one 32-bit word. Arguments are taken by value: applying
// __builtin_bit_cast to an ext_vector element directly reads element 0.
__device__ __forceinline__ float word_as_float(uint32_t w) { return __builtin_bit_cast(float, w); }
__device__ __forceinline__ half2_t word_as_half2(uint32_t w) { return __builtin_bit_cast(half2_t, w); }
__device__ __forceinline__ uint32_t half2_as_word(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// 8 packed (code+8) nibbles in the tile16x128 order -> 8 exact f16 codes.
__device__ __forceinline__ uint4_t nibbles_to_half8(uint32_t w) {
    const half2_t bias = {(half_t)1032.0f, (half_t)1032.0f};
    uint4_t out;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        uint32_t t = ((w >> (4 * p)) & 0x000F000Fu) | 0x64006400u;
        half2_t h = __builtin_bit_cast(half2_t, t) - bias;
        out[p] = __builtin_bit_cast(uint32_t, h);
    }
    return out;
}

// 8 packed nibbles -> two words of signed int8 codes in k order (e0..e3, e4..e7).
__device__ __forceinline__ uint2_t nibbles_to_i8(uint32_t w) {
    uint32_t lo = w & 0x0F0F0F0Fu;         // bytes: e0 e4 e1 e5
    uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // bytes: e2 e6 e3 e7
    // offset binary -> two's complement per byte without carries
    lo = (lo + 0x78787878u) ^ 0x80808080u;
    hi = (hi + 0x78787878u) ^ 0x80808080u;
    uint2_t out;
    out[0] = __builtin_amdgcn_perm(hi, lo, 0x06040200u);  // e0 e1 e2 e3
    out[1] = __builtin_amdgcn_perm(hi, lo, 0x07050301u);  // e4 e5 e6 e7
    return out;
}

__device__ __forceinline__ float4_t mfma_f16(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int4_t mfma_i8(int4_t a, int4_t b, int4_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// A 64-group dot d (|d| < 2^22: at most 64 * 127 * 127 for W8A8) as an exact
// f32 without v_cvt_f32_i32, which issues at about 60% of an add's rate on
// gfx950: the MFMA accumulates onto kDotBias, the bits of 1.5 * 2^23, where a
// float's ulp is 1, so the int32 result is the bit pattern of 12582912 + d and
// one exact subtraction (dot_value) leaves f32(d), the same bits as the
// conversion.
constexpr int32_t kDotBias = 0x4B400000;
__device__ __forceinline__ int4_t mfma_i8_biased(int4_t a, int4_t b) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, int4_t{kDotBias, kDotBias, kDotBias, kDotBias}, 0, 0, 0);
}
__device__ __forceinline__ float dot_value(int32_t biased) {
    return __fsub_rn(__builtin_bit_cast(float, biased), 12582912.0f);
}

// Q4 weights for the biased MFMA in five VALU operations per 8 codes instead
// of nine: a nibble moved to the top of its byte, with the byte's top bit
// flipped, is the int8 16 * code (offset binary n -> 16 n - 128); the mask and
// the flip are one v_bitop3_b32. The MFMA then sums 16 * d; accumulated onto
// the bits of 1.5 * 2^19, where a float's ulp is 1/16, the int32 result is the
// bit pattern of 786432 + d for |d| < 2^18 (W4A8: at most 64 * 8 * 127), and
// dot_value16 leaves f32(d) exactly, the same bits as dot_value on the plain
// codes.
__device__ __forceinline__ uint2_t nibbles_to_i8x16(uint32_t w) {
    const uint32_t hi = (w & 0xF0F0F0F0u) ^ 0x80808080u;         // bytes: 16 e2, 16 e6, 16 e3, 16 e7
    const uint32_t lo = ((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u;  // bytes: 16 e0, 16 e4, 16 e1, 16 e5
    uint2_t out;
    out[0] = __builtin_amdgcn_perm(hi, lo, 0x06040200u);  // 16 (e0 e1 e2 e3)
    out[1] = __builtin_amdgcn_perm(hi, lo, 0x07050301u);  // 16 (e4 e5 e6 e7)
    return out;
}
constexpr int32_t kDotBias16 = 0x49400000;
__device__ __forceinline__ int4_t mfma_i8_biased16(int4_t a, int4_t b) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, int4_t{kDotBias16, kDotBias16, kDotBias16, kDotBias16}, 0, 0,
                                                 0);
}
__device__ __forceinline__ float dot_value16(int32_t biased) {
    return __fsub_rn(__builtin_bit_cast(float, biased), 786432.0f);
}
// One lane's 16 Q4 codes of a group (two packed words) as the MFMA operand 16 * code.
__device__ __forceinline__ int4_t q4_operand16(uint32_t w0, uint32_t w1) {
    const uint2_t lo = nibbles_to_i8x16(w0), hi = nibbles_to_i8x16(w1);
    return int4_t{(int)lo[0], (int)lo[1], (int)hi[0], (int)hi[1]};
}
// The group dot of weight codes of BITS bits: Q4 operands from q4_operand16,
// Q8 operands as they are; dot_of<BITS> of each result is f32(dot), exactly.
template <int BITS>
__device__ __forceinline__ int4_t mfma_dot(int4_t a, int4_t b) {
    return BITS == 4 ? mfma_i8_biased16(a, b) : mfma_i8_biased(a, b);
}
template <int BITS>
__device__ __forceinline__ float dot_of(int32_t biased) {
    return BITS == 4 ? dot_value16(biased) : dot_value(biased);
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(half_t, (unsigned short)h);
}

// Blocks are dispatched to the 8 XCDs round-robin (block b on XCD b % 8), and
// each XCD has its own L2. A kernel that reads rows another kernel just wrote
// reads them fastest on the XCD that wrote them. The products give XCD x the
// output rows [x M / 8, (x + 1) M / 8) (whole row bands, xcd_tile); this maps
// block b of nblocks to work unit u of nunits so that XCD x takes the units
// [x nunits / 8, (x + 1) nunits / 8) in order, the same share (identity when
// the counts do not divide by 8).
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_unit(int b, int nblocks) {
    return nblocks % kXcds == 0 ? (b % kXcds) * (nblocks / kXcds) + b / kXcds : b;
}

// Sum over the 64 lanes of a wave, left in every lane: four DPP adds inside
// each 16-lane row (xor 1, xor 2, rotate 4, rotate 8), then v_permlane16_swap
// (odd rows of the first operand trade places with even rows of the second)
// and v_permlane32_swap (upper half of the first with the lower half of the
// second) add the rows in pairs. The swaps are issued as asm with nops for
// the VALU-write / permlane-read wait states on either side.
template <int CTRL>
__device__ __forceinline__ float dpp_move_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_move_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_move_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_move_f32<0x124>(v);  // row_ror:4
    v += dpp_move_f32<0x128>(v);  // row_ror:8
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    v = a + b;
    a = v;
    b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}

// Maximum over the 64 lanes of a wave, left in every lane (wave_sum_dpp's
// pattern with fmaxf; the maximum does not depend on the order).
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_move_f32<0xB1>(v));
    v = fmaxf(v, dpp_move_f32<0x4E>(v));
    v = fmaxf(v, dpp_move_f32<0x124>(v));
    v = fmaxf(v, dpp_move_f32<0x128>(v));
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    v = fmaxf(a, b);
    a = v;
    b = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return fmaxf(a, b);
}

// The grouped activation quantizer's code (int8.rs:178-202): rint(v * (1/scale))
// clamped to +-limit, with the correctly rounded reciprocal passed in.
__device__ __forceinline__ int quantize_code(float v, float inverse, float limit) {
    float r = __builtin_rintf(__fmul_rn(v, inverse));
    r = fminf(fmaxf(r, -limit), limit);
    return (int)r;
}

// erf(x) by Abramowitz & Stegun, Handbook of Mathematical Functions (1964),
// formula 7.1.26: erf(x) = 1 - (a1 t + a2 t^2 + a3 t^3 + a4 t^4 + a5 t^5) e^(-x^2)
// with t = 1 / (1 + p x) for x >= 0, |error| <= 1.5e-7, odd extension for x < 0.
// Branch-free (one reciprocal, one exp2); used by the erf-GELU epilogues.
__device__ __forceinline__ float erf_as7126(float x) {
    const float ax = fabsf(x);
    const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, ax, 1.0f));
    float p = 1.061405429f;
    p = __builtin_fmaf(p, t, -1.453152027f);
    p = __builtin_fmaf(p, t, 1.421413741f);
    p = __builtin_fmaf(p, t, -0.284496736f);
    p = __builtin_fmaf(p, t, 0.254829592f);
    p *= t;
    const float e = __builtin_amdgcn_exp2f(-(ax * ax) * 1.4426950408889634f);
    return __builtin_copysignf(__builtin_fmaf(-p, e, 1.0f), x);
}

// v as an f32 value: the compiler cannot fuse the operation that produced it
// into a following f16 conversion (v_fma_mixlo_f16 rounds the exact result
// once, to f16, where f32 code rounds twice), so an f16 epilogue rounds the
// same f32 value that an f32 output holds.
__device__ __forceinline__ float f32_rounded(float v) {
    asm volatile("" : "+v"(v));
    return v;
}

// erf-GELU: 0.5 x (1 + erf(x / sqrt(2)))
__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.0f + erf_as7126(x * 0.70710678118654752f));
}

typedef int int32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resource (stride 0, range-checked offsets) over [p, p + bytes).
__device__ __forceinline__ int32x4_t buffer_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    return int32x4_t{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), (int)bytes, 0x00020000};
}

// 32-bit LDS address of a __shared__ object
__device__ __forceinline__ uint32_t lds_address(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// buffer_load_dwordx4 ... lds: lane l's 16 bytes at rsrc + voff land at
// LDS lds + 16 * l. Issued as asm so that the compiler does not add waits
// for it before LDS reads of other buffers; the caller waits (s_waitcnt
// vmcnt + s_barrier) before reading what it wrote.
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, int32x4_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// buffer_load_dword ... lds: lane l's 4 bytes at rsrc + voff land at LDS
// lds + 4 * l (same contract as dma16).
__device__ __forceinline__ void dma4(uint32_t lds, uint32_t voff, int32x4_t rsrc) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// ---- host helpers ------------------------------------------------------------

struct Status {
    int32_t code = 0;
    std::string message;
};

}  // namespace dz
