// pplx.hip -- the Pplx decider forward on the quantized products: the hybrid
// decoder of hyperlogue/decisive src/models/pplx_flash/backbone.rs (three
// gated-delta layers, then one gated full-attention layer, repeated), the
// final zero-centred RMSNorm and the packed readout (mod.rs:149-185), over
// one sequence of packed embedding rows (native.rs:193-274).
//
// The layer RMSNorms are the readout's bit-exact cpu::rms_from (squares added
// in row order). Every projection is the reference's W4A8 product (dz_linear_pair,
// dz_linear, dz_mlp_requant + dz_linear_q8: the int8.rs group fold, bit-exact
// with the CPU path); the layer ops between them are the kernels below:
//   conv_silu      cpu.rs:372-391 (causal depthwise conv of width 4 + SiLU)
//   delta_prep     backbone.rs:366-379 (q/k unit norms, decay g, beta)
//   delta_scan     backbone.rs:380-407 (the gated delta rule, one state
//                  column per lane group; f32 with fused multiply-adds)
//   delta_gate     backbone.rs:310-326, cpu.rs:392-414
//   head_norm_rope cpu.rs:310-333 per head (zero-centred) + backbone.rs:415-428
//   attention      backbone.rs:509-579 (non-causal softmax attention, GQA)
//   attention_gate cpu.rs:415-429
// Those are tolerance-checked against the oracle's restatement; the
// reference's own orders (sequential sums, unfused products) are kept where
// they cost nothing.
#include <float.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/decisive_rocm.h"
#include "kernels.hpp"

namespace dz {

int32_t ctx_fail(dz_ctx *ctx, int32_t code, const std::string &msg);
int32_t ctx_hip_fail(dz_ctx *ctx, hipError_t e, const char *what);
hipStream_t ctx_stream(dz_ctx *ctx);
int *ctx_flag(dz_ctx *ctx);
const Weight &weight_of(const dz_weight *h);
Weight &weight_mut(dz_weight *h);
int32_t weight_upload(dz_ctx *ctx, const void *packed, size_t bytes, int32_t layout, size_t rows, size_t cols,
                      dz_weight **out);
int32_t weight_upload_fitted(dz_ctx *ctx, const void *packed, size_t bytes, size_t rows, size_t cols, int32_t form,
                             dz_weight **out);
void weight_free(dz_weight *h);
int32_t weight_concat_rows(dz_ctx *ctx, const dz_weight *const *parts, int count, dz_weight **out);
int32_t ctx_readout_rows(dz_ctx *ctx, const Weight &w, const float *norm, const void *hidden, int dtype,
                         const int32_t *select, size_t rows, float eps, float *logits);
int ctx_variant(dz_ctx *ctx, const char *family);
int32_t ctx_product_add(dz_ctx *ctx, const dz_weight *w, const float *x, const int8_t *q, const float *qs,
                        size_t m, float *h, bool *fused, const int *qbad = nullptr);
int32_t ctx_product_flag(dz_ctx *ctx, int **flag);
int32_t ctx_codes_product(dz_ctx *ctx, const dz_weight *w, const int8_t *q, const float *qs, size_t m, float *y,
                          const int *bad);
int32_t ctx_mlp_codes(dz_ctx *ctx, const dz_weight *gate, const dz_weight *up, const int8_t *q, const float *qs,
                      size_t m, int8_t *qo, float *so, const int *bad);

namespace {

constexpr int kLd = 128;   // delta head width (backbone.rs LD)
constexpr int kAd = 256;   // attention head width (backbone.rs AD)
constexpr int kMaxKeys = 8192;

inline unsigned blocks_of(size_t n, unsigned threads) { return (unsigned)((n + threads - 1) / threads); }

__device__ __forceinline__ float sigmoid_ref(float v) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-v))); }
__device__ __forceinline__ float silu_ref(float v) { return __fmul_rn(v, sigmoid_ref(v)); }
__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
// 1/sqrt(t) with the square root correctly rounded (taken in f64)
__device__ __forceinline__ float rsqrt_rn(float t) { return __fdiv_rn(1.0f, __double2float_rn(__dsqrt_rn((double)t))); }

// out[t][c] = silu(sum_tap x[t-3+tap][c] * w[tap][c]); rows before 0 are zero.
// Grid (width / 4 / 256 blocks, n rows): a thread takes four consecutive
// columns of row blockIdx.y (width % 4 == 0, 16-byte aligned rows), so no
// index is divided; each column's arithmetic is the scalar order above.
__global__ void conv_silu_kernel(const float *__restrict__ x, int n, int width, const float *__restrict__ w,
                                 float *__restrict__ out) {
    const int t = blockIdx.y;
    const int c = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (t >= n || c >= width) return;
    float4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int tap = 0; tap < 4; tap++) {
        const int row = t - 3 + tap;
        const float4_t v = row < 0 ? float4_t{0.0f, 0.0f, 0.0f, 0.0f} : *(const float4_t *)(x + (size_t)row * width + c);
        const float4_t k = *(const float4_t *)(w + (size_t)tap * width + c);
#pragma unroll
        for (int e = 0; e < 4; e++) sum[e] = __fadd_rn(sum[e], __fmul_rn(v[e], k[e]));
    }
    float4_t o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = silu_ref(sum[e]);
    *(float4_t *)(out + (size_t)t * width + c) = o;
}

// One block per token, one wave per key head: unit q and k (q also scaled by
// 1/sqrt(ld)) and their dot product; threads below lh compute the decay g and
// beta of head h. Record (t, h) of gb holds {g, beta, k.q of h's key head, log g}.
__global__ void delta_prep_kernel(const float *__restrict__ conv, int lh, int lk, const float *__restrict__ a,
                                  const float *__restrict__ b, int ab_ld, const float *__restrict__ decay,
                                  const float *__restrict__ dt, float *__restrict__ qhat,
                                  float *__restrict__ khat, float *__restrict__ gb) {
    const int t = blockIdx.x, wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const size_t lkv = (size_t)lk * kLd, width = 2 * lkv + (size_t)lh * kLd;
    if (wave < lk) {
        const float *qs = conv + (size_t)t * width + (size_t)wave * kLd;
        const float *ks = qs + lkv;
        const float q0 = qs[lane], q1 = qs[lane + 64], k0 = ks[lane], k1 = ks[lane + 64];
        const float qi = rsqrt_rn(__fadd_rn(wave_sum(q0 * q0 + q1 * q1), 1e-6f));
        const float ki = rsqrt_rn(__fadd_rn(wave_sum(k0 * k0 + k1 * k1), 1e-6f));
        const float root = rsqrt_rn((float)kLd);
        float *qd = qhat + ((size_t)t * lk + wave) * kLd, *kd = khat + ((size_t)t * lk + wave) * kLd;
        const float qa = __fmul_rn(__fmul_rn(q0, qi), root), qb = __fmul_rn(__fmul_rn(q1, qi), root);
        const float ka = __fmul_rn(k0, ki), kb = __fmul_rn(k1, ki);
        qd[lane] = qa;
        qd[lane + 64] = qb;
        kd[lane] = ka;
        kd[lane + 64] = kb;
        const float kq = wave_sum(__builtin_fmaf(ka, qa, kb * qb));
        const int per = lh / lk;
        if (lane < per) gb[((size_t)t * lh + wave * per + lane) * 4 + 2] = kq;
    }
    for (int h = threadIdx.x; h < lh; h += blockDim.x) {
        const float x = __fadd_rn(a[(size_t)t * ab_ld + h], dt[h]);
        const float softplus = x > 20.0f ? x : log1pf(expf(x));
        const float logg = __fmul_rn(-decay[h], softplus);
        gb[((size_t)t * lh + h) * 4] = expf(logg);
        gb[((size_t)t * lh + h) * 4 + 1] = sigmoid_ref(b[(size_t)t * ab_ld + h]);
        gb[((size_t)t * lh + h) * 4 + 3] = logg;
    }
}

// The gated delta rule. A block of 4 waves owns 8 state columns of head h
// (blockIdx.y selects which 8); in each wave, lanes 32c..32c+31 hold column
// 8*blockIdx.y + 2*wave + c, lane r of the half holding state rows 4r..4r+3
// in registers. Per token the reference's steps (S *= g; mem = S^T k;
// delta = (v - mem) beta; S += k delta^T; out = S^T q) are regrouped so that
// both sums read the previous state: mem = g (S^T k), out = g (S^T q) +
// delta (k.q) (k.q from delta_prep), S = g S + k delta^T; the two sums then
// close together and the chain from one token to the next is short. A sum
// over a half closes with four DPP adds inside each 16-lane row (xor 1, xor 2,
// rotate 4, rotate 8) and one row swap (v_permlane16_swap), which leave the
// total in every lane; lane r keeps token t0 + r's output and the wave stores
// a whole chunk at once. Tokens are staged in LDS sixteen at a time, shared
// by the four waves; the next chunk's loads are in flight while this chunk
// computes. 512 blocks cover the 32 heads of the reference model, two waves
// per SIMD.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float half_sum(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x124>(v);  // row_ror:4
    v += dpp_move<0x128>(v);  // row_ror:8
    // rows (0, 1) and (2, 3) exchange (v_permlane16_swap: odd rows of the
    // first operand trade places with even rows of the second), so a + b holds
    // both rows' sums in every lane. Issued as asm: this compiler's builtin
    // for it returns the first result twice. The nops cover the VALU-write /
    // permlane-read wait states on either side.
    float a = v, b = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    return a + b;
}

constexpr int kScanChunk = 16;  // tokens staged in LDS at a time
constexpr int kScanWaves = 4;
constexpr int kScanCols = 2 * kScanWaves;  // state columns per block

// UNROLL: whole 16-token stages run unrolled (constant LDS offsets, no loop
// counter per token; the scan issues its VALU work back to back, so the
// instructions per token set its rate); the arithmetic and its order are the
// same either way, so both forms give the same bits.
template <bool UNROLL>
__global__ __launch_bounds__(kScanWaves * 64) void delta_scan_kernel(const float *__restrict__ qhat,
                                                                     const float *__restrict__ khat,
                                                                     const float *__restrict__ conv,
                                                                     const float *__restrict__ gb, int n, int lh,
                                                                     int lk, float *__restrict__ out) {
    constexpr int T = kScanChunk;
    __shared__ __align__(16) float ks[2][T * kLd], qs[2][T * kLd], vs[2][T * kScanCols], gs[2][T * 4];
    const int h = blockIdx.x, tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const int r = lane % 32, c = lane / 32;
    const int j0 = blockIdx.y * kScanCols, j = j0 + 2 * wave + c;
    const int kh = h / (lh / lk);
    const size_t lkv = (size_t)lk * kLd, width = 2 * lkv + (size_t)lh * kLd;
    constexpr int KQ = T * kLd / 4 / (kScanWaves * 64);  // float4s of k (and of q) per thread
    float S[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // staging registers: KQ float4s of k and of q per thread, v for the first
    // threads, the {g, beta, k.q} records for the first 16
    float4_t rk[KQ], rq[KQ], rv, rg;
    auto load = [&](int t0) {
#pragma unroll
        for (int i = 0; i < KQ; i++) {
            const int id = tid + kScanWaves * 64 * i;
            const int t = min(t0 + id / 32, n - 1);
            const size_t row = ((size_t)t * lk + kh) * kLd + 4 * (id % 32);
            rk[i] = *(const float4_t *)(khat + row);
            rq[i] = *(const float4_t *)(qhat + row);
        }
        if (tid < T * kScanCols / 4) {
            const int tv = min(t0 + tid / (kScanCols / 4), n - 1);
            rv = *(const float4_t *)(conv + (size_t)tv * width + 2 * lkv + (size_t)h * kLd + j0 +
                                     4 * (tid % (kScanCols / 4)));
        }
        if (tid < T) rg = *(const float4_t *)(gb + ((size_t)min(t0 + tid, n - 1) * lh + h) * 4);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < KQ; i++) {
            const int id = tid + kScanWaves * 64 * i;
            *(float4_t *)(&ks[buf][4 * id]) = rk[i];
            *(float4_t *)(&qs[buf][4 * id]) = rq[i];
        }
        if (tid < T * kScanCols / 4) *(float4_t *)(&vs[buf][4 * tid]) = rv;
        if (tid < T) *(float4_t *)(&gs[buf][4 * tid]) = rg;
    };
    if (n > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t0 = 0, buf = 0; t0 < n; t0 += T, buf ^= 1) {
        const bool more = t0 + T < n;
        if (more) load(t0 + T);  // in flight while this chunk computes
        const int count = min(T, n - t0);
        float keep = 0.0f;
        // one token: S^T k and S^T q over the previous state, reduced together;
        // then S = g S + k delta^T with delta = (v - g S^T k) beta and
        // out = g S^T q + delta (k.q)
        auto step = [&](int tt) {
            const float4_t gq = *(const float4_t *)(&gs[buf][tt * 4]);
            const float v = vs[buf][tt * kScanCols + 2 * wave + c];
            const float4_t k4 = *(const float4_t *)(&ks[buf][tt * kLd + 4 * r]);
            const float4_t q4 = *(const float4_t *)(&qs[buf][tt * kLd + 4 * r]);
            const float g = gq[0], beta = gq[1], kq = gq[2];
            float m0 = S[0] * k4[0], m1 = S[1] * k4[1], p0 = S[0] * q4[0], p1 = S[1] * q4[1];
            m0 = __builtin_fmaf(S[2], k4[2], m0);
            m1 = __builtin_fmaf(S[3], k4[3], m1);
            p0 = __builtin_fmaf(S[2], q4[2], p0);
            p1 = __builtin_fmaf(S[3], q4[3], p1);
#pragma unroll
            for (int e = 0; e < 4; e++) S[e] *= g;
            const float sk = half_sum(m0 + m1), sq = half_sum(p0 + p1);
            const float delta = (v - g * sk) * beta;
#pragma unroll
            for (int e = 0; e < 4; e++) S[e] = __builtin_fmaf(k4[e], delta, S[e]);
            const float total = __builtin_fmaf(g, sq, delta * kq);
            keep = r == tt ? total : keep;
        };
        if (UNROLL && count == T) {
            // a whole stage: constant LDS offsets and no loop counter per token
#pragma unroll
            for (int tt = 0; tt < T; tt++) step(tt);
        } else {
            for (int tt = 0; tt < count; tt++) step(tt);
        }
        if (r < count) out[((size_t)h * n + t0 + r) * kLd + j] = keep;
        if (more) store(buf ^ 1);  // the other buffer: last read a whole chunk ago
        __syncthreads();
    }
}

// ---- the gated delta rule by chunks of 64 tokens (f32 MFMA) ----------------
// Over one chunk, with S0 the state before it, gamma_t the decay from the
// chunk start through token t (exp of the running sum of log g) and
// D[t][i] = gamma_t / gamma_i:
//   A = strictly-lower(diag(beta) (K K^T * D)),  (I + A) [Uv | Wk] = [diag(beta) V | diag(beta gamma) K]
//   U = Uv - Wk S0          (the values the chunk's tokens write, u_t = beta_t (v_t - mem_t))
//   O = diag(gamma) Q S0 + lower(Q K^T * D) U
//   S = gamma_last S0 + (diag(gamma_last / gamma) K)^T U
// which is the token-by-token rule regrouped (each u_t is the reference's
// delta). delta_chunk_prep_kernel does everything that does not involve S0,
// for every (head, chunk) at once; delta_chunk_scan_kernel walks the chunks in
// order for 16 state columns per block.
constexpr int kChunk = 64;
constexpr int kChunkWs = 2 * kChunk * kLd + kChunk * kChunk + kLd * kChunk + kChunk;  // floats per (head, chunk)
constexpr int kChunkRow = kLd + 4;    // padded LDS row of K / Q (conflict-free float4 reads across rows)

// One block (4 waves) per (head, chunk). Workspace record (floats):
// Uv [64][128] | Wk [64][128] | P [64][64] | rKT [128][64] (gamma_last/gamma_t K[t][dk]) | gamma [64].
__global__ __launch_bounds__(256) void delta_chunk_prep_kernel(const float *__restrict__ qhat,
                                                               const float *__restrict__ khat,
                                                               const float *__restrict__ conv,
                                                               const float *__restrict__ gb, int n, int lh, int lk,
                                                               float *__restrict__ ws) {
    extern __shared__ __align__(16) float sm[];
    float *ks = sm, *as = ks + kChunk * kChunkRow, *cum = as + kChunk * kChunk, *bet = cum + kChunk,
          *bk = bet + kChunk;
    const int h = blockIdx.x, c = blockIdx.y, tid = threadIdx.x;
    const int wave = tid / 64, lane = tid % 64, col = lane % 16, g = lane / 16;
    const int kh = h / (lh / lk), t0 = c * kChunk;
    const size_t lkv = (size_t)lk * kLd, width = 2 * lkv + (size_t)lh * kLd;
    float *rec = ws + ((size_t)h * gridDim.y + c) * kChunkWs;
    float *uv = rec, *wk = uv + kChunk * kLd, *pm = wk + kChunk * kLd, *rkt = pm + kChunk * kChunk,
          *gam = rkt + kLd * kChunk;
    // stage K rows (zero past n), beta and log g (zero past n); every load of
    // the rows is issued before the first store
    {
        constexpr int KV = kChunk * kLd / 4 / 256;  // float4s per thread
        float4_t kv[KV];
#pragma unroll
        for (int i = 0; i < KV; i++) {
            const int e = tid + 256 * i, t = e / (kLd / 4), u = e % (kLd / 4), tok = t0 + t;
            kv[i] = tok < n ? *(const float4_t *)(khat + ((size_t)tok * lk + kh) * kLd + 4 * u)
                            : float4_t{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int i = 0; i < KV; i++) {
            const int e = tid + 256 * i, t = e / (kLd / 4), u = e % (kLd / 4);
            *(float4_t *)(ks + t * kChunkRow + 4 * u) = kv[i];
        }
    }
    if (tid < kChunk) {
        const int tok = t0 + tid;
        bet[tid] = tok < n ? gb[((size_t)tok * lh + h) * 4 + 1] : 0.0f;
        cum[tid] = tok < n ? gb[((size_t)tok * lh + h) * 4 + 3] : 0.0f;
    }
    // this lane's Q fragment (row 16*wave + col, dims 32g..32g+31) for Q K^T
    float4_t qf[8];
    {
        const int tok = t0 + 16 * wave + col;
#pragma unroll
        for (int i = 0; i < 8; i++)
            qf[i] = tok < n ? *(const float4_t *)(qhat + ((size_t)tok * lk + kh) * kLd + 32 * g + 4 * i)
                            : float4_t{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    if (tid == 0) {  // the running sum of log g in token order, in registers (16-byte LDS reads and writes)
        float4_t c[kChunk / 4];
#pragma unroll
        for (int i = 0; i < kChunk / 4; i++) c[i] = *(const float4_t *)(cum + 4 * i);
        float run = 0.0f;
#pragma unroll
        for (int i = 0; i < kChunk / 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                run += c[i][e];
                c[i][e] = run;
            }
#pragma unroll
        for (int i = 0; i < kChunk / 4; i++) *(float4_t *)(cum + 4 * i) = c[i];
    }
    __syncthreads();
    if (tid < kChunk) bk[tid] = bet[tid] * expf(cum[tid]);
    // K K^T and Q K^T, row block `wave`: lane (col, g) holds rows 16*wave + 4g + i of column block cb
#pragma unroll 1
    for (int cb = 0; cb < 4; cb++) {
        float4_t kk = {0.f, 0.f, 0.f, 0.f}, qk = kk;
        const float *ka = ks + (16 * wave + col) * kChunkRow + 32 * g;
        const float *kb = ks + (16 * cb + col) * kChunkRow + 32 * g;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4_t a4 = *(const float4_t *)(ka + 4 * i), b4 = *(const float4_t *)(kb + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                kk = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[e], b4[e], kk, 0, 0, 0);
                qk = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[i][e], b4[e], qk, 0, 0, 0);
            }
        }
        const int j = 16 * cb + col;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * wave + 4 * g + i;
            const float d = j <= r ? expf(cum[r] - cum[j]) : 0.0f;
            as[r * kChunk + j] = j < r ? bet[r] * d * kk[i] : 0.0f;
            pm[r * kChunk + j] = d * qk[i];
        }
    }
    __syncthreads();
    // (I + A) x = b, one right-hand side per thread: columns of diag(beta) V
    // (waves 0-1), then of diag(beta gamma) K (waves 2-3)
    auto solve = [&](auto vcol_c) {
        constexpr bool VCOL = decltype(vcol_c)::value;
        const int cc = VCOL ? tid : tid - kLd;
        const float *vsrc = conv + 2 * lkv + (size_t)h * kLd + cc;
        float x[kChunk];  // the right-hand side, then the solution in place
#pragma unroll
        for (int i = 0; i < kChunk; i++) {
            if (VCOL) x[i] = t0 + i < n ? bet[i] * vsrc[(size_t)(t0 + i) * width] : 0.0f;
            else x[i] = bk[i] * ks[i * kChunkRow + cc];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 1; i < kChunk; i++) {
            float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
#pragma unroll
            for (int l = 0; l + 3 < i; l += 4) {
                const float4_t a4 = *(const float4_t *)(as + i * kChunk + l);
                s0 = __builtin_fmaf(a4[0], x[l], s0);
                s1 = __builtin_fmaf(a4[1], x[l + 1], s1);
                s2 = __builtin_fmaf(a4[2], x[l + 2], s2);
                s3 = __builtin_fmaf(a4[3], x[l + 3], s3);
            }
#pragma unroll
            for (int l = i & ~3; l < i; l++) s0 = __builtin_fmaf(as[i * kChunk + l], x[l], s0);
            x[i] -= (s0 + s1) + (s2 + s3);
        }
        float *dst = VCOL ? uv : wk;
#pragma unroll
        for (int i = 0; i < kChunk; i++) dst[i * kLd + cc] = x[i];
    };
    if (__builtin_amdgcn_readfirstlane(wave) < 2) solve(std::true_type{});
    else solve(std::false_type{});
    // (gamma_last / gamma_t) K[t][dk], transposed; gamma_t
    {
        const int dk = tid / 2, th = (tid % 2) * 32;
        const float last = cum[kChunk - 1];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            float4_t v4;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = th + 4 * u + e;
                v4[e] = expf(last - cum[t]) * ks[t * kChunkRow + dk];
            }
            *(float4_t *)(rkt + dk * kChunk + th + 4 * u) = v4;
        }
        if (tid < kChunk) gam[tid] = expf(cum[tid]);
    }
}

// One block per (head, CT x 16 state columns), 4 waves per 16 columns; the
// chunks in order. The state S (128 x 16 per column tile) lives in LDS
// transposed (S_T[col][dk]); wave w of a column tile computes rows
// 16w..16w+15 of the chunk's U and O and the state rows 32w..32w+31. Each
// state column's arithmetic is the same for every CT, so CT = 1 and CT = 2
// give the same bits (CT = 2: half the blocks, eight waves each).
template <int CT>
__global__ __launch_bounds__(256 * CT) void delta_chunk_scan_kernel(const float *__restrict__ qhat,
                                                                    const float *__restrict__ ws, int n, int lh,
                                                                    int lk, float *__restrict__ out) {
    constexpr int UROW = kChunk + 4;
    __shared__ __align__(16) float st_all[CT * 16 * kChunkRow];  // S_T [16][128 + 4] per column tile
    __shared__ __align__(16) float ut_all[CT * 16 * UROW];       // U_T [16][64 + 4] per column tile
    const int h = blockIdx.x, tid = threadIdx.x;
    const int ct = tid / 256, wave = (tid / 64) % 4, lane = tid % 64, col = lane % 16, g = lane / 16;
    const int col0 = (blockIdx.y * CT + ct) * 16;  // this column tile's first state column
    float *st = st_all + ct * 16 * kChunkRow, *ut = ut_all + ct * 16 * UROW;
    const int kh = h / (lh / lk);
    const int chunks = (n + kChunk - 1) / kChunk;
    for (int e = tid; e < CT * 16 * kChunkRow; e += 256 * CT) st_all[e] = 0.0f;
    __syncthreads();
    // the global operands of one chunk for this lane; the next chunk's are in
    // flight while the current one computes
    struct Ops {
        float4_t w[8], q[8], p[4], r[2][4];
        float u[4], gm[4], last;
    };
    auto fetch = [&](int c) {
        Ops o;
        const float *rec = ws + ((size_t)h * chunks + c) * kChunkWs;
        const float *uv = rec, *wk = uv + kChunk * kLd, *pm = wk + kChunk * kLd, *rkt = pm + kChunk * kChunk,
                    *gam = rkt + kLd * kChunk;
        const int row = 16 * wave + col, tq = min(c * kChunk + row, n - 1);
        const float *qa = qhat + ((size_t)tq * lk + kh) * kLd + 32 * g;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            o.w[i] = *(const float4_t *)(wk + row * kLd + 32 * g + 4 * i);
            o.q[i] = *(const float4_t *)(qa + 4 * i);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            o.p[i] = *(const float4_t *)(pm + row * kChunk + 16 * g + 4 * i);
#pragma unroll
            for (int d = 0; d < 2; d++) o.r[d][i] = *(const float4_t *)(rkt + (32 * wave + 16 * d + col) * kChunk + 16 * g + 4 * i);
            const int t = 16 * wave + 4 * g + i;
            o.u[i] = uv[t * kLd + col0 + col];
            o.gm[i] = gam[t];
        }
        o.last = gam[kChunk - 1];
        return o;
    };
    // CT = 1 holds the next chunk's operands in registers while this chunk
    // computes; CT = 2 (two waves per SIMD, half the registers each) loads
    // them after the chunk and lets the other wave run meanwhile
    Ops cur = fetch(0);
    for (int c = 0; c < chunks; c++) {
        Ops nxt = cur;
        if (CT == 1 && c + 1 < chunks) nxt = fetch(c + 1);
        const int t0 = c * kChunk;
        // X = Wk S and Q S over the 128 state rows
        float4_t xw = {0.f, 0.f, 0.f, 0.f}, qsv = xw;
        const float *sb = st + col * kChunkRow + 32 * g;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4_t b4 = *(const float4_t *)(sb + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xw = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.w[i][e], b4[e], xw, 0, 0, 0);
                qsv = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.q[i][e], b4[e], qsv, 0, 0, 0);
            }
        }
        // U = Uv - X (rows 16w + 4g + i), into U_T; O starts as gamma Q S
        float4_t u4, o4;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u4[i] = cur.u[i] - xw[i];
            o4[i] = cur.gm[i] * qsv[i];
        }
        *(float4_t *)(ut + col * UROW + 16 * wave + 4 * g) = u4;
        // U complete, every read of the old S done; an LDS-only wait keeps the
        // next chunk's global loads in flight (__syncthreads would drain them)
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        // O += P U and the state update share the U operands
        const float *ub = ut + col * UROW + 16 * g;
        float4_t sn[2];
#pragma unroll
        for (int d = 0; d < 2; d++) {
            const float4_t old = *(const float4_t *)(st + col * kChunkRow + 32 * wave + 16 * d + 4 * g);
            sn[d] = old * cur.last;
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4_t b4 = *(const float4_t *)(ub + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                o4 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.p[i][e], b4[e], o4, 0, 0, 0);
#pragma unroll
                for (int d = 0; d < 2; d++) sn[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.r[d][i][e], b4[e], sn[d], 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = t0 + 16 * wave + 4 * g + i;
            if (t < n) out[((size_t)h * n + t) * kLd + col0 + col] = o4[i];
        }
#pragma unroll
        for (int d = 0; d < 2; d++) *(float4_t *)(st + col * kChunkRow + 32 * wave + 16 * d + 4 * g) = sn[d];
        if (CT == 1)
            cur = nxt;
        else if (c + 1 < chunks)
            cur = fetch(c + 1);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // the new S is complete; U_T is free
        __builtin_amdgcn_s_barrier();
    }
}

// ctx[t][h*ld + i] = ((src*s)*norm[i])*silu(z), s = 1/sqrt(mean(src^2) + 1e-6).
// CODES: instead of ctx, the A8 codes and scales of its two 64-groups per head
// (the activation quantizer's arithmetic, int8.rs:178-202, so they equal
// act_quantize of ctx word for word), with *bad raised on a non-finite value.
template <bool CODES>
__global__ __launch_bounds__(64) void delta_gate_kernel(const float *__restrict__ heads, int n, int lh,
                                                        const float *__restrict__ norm,
                                                        const float *__restrict__ z, int z_ld, float *__restrict__ ctx,
                                                        int8_t *__restrict__ q, float *__restrict__ qs, int *bad) {
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const float *src = heads + ((size_t)h * n + t) * kLd;
    const float s0 = src[lane], s1 = src[lane + 64];
    const float scale = rsqrt_rn(__fadd_rn(wave_sum(s0 * s0 + s1 * s1) / (float)kLd, 1e-6f));
    const size_t at = (size_t)t * lh * kLd + (size_t)h * kLd;
    const float *zr = z + (size_t)t * z_ld + (size_t)h * kLd;
    const float v0 = __fmul_rn(__fmul_rn(__fmul_rn(s0, scale), norm[lane]), silu_ref(zr[lane]));
    const float v1 = __fmul_rn(__fmul_rn(__fmul_rn(s1, scale), norm[lane + 64]), silu_ref(zr[lane + 64]));
    if constexpr (!CODES) {
        ctx[at + lane] = v0;
        ctx[at + lane + 64] = v1;
    } else {
        if ((!__builtin_isfinite(v0) || !__builtin_isfinite(v1)) && bad) atomicOr(bad, 1);
        const float m0 = wave_max_dpp(fabsf(v0)), m1 = wave_max_dpp(fabsf(v1));
        const float c0 = fmaxf(__fdiv_rn(m0, 127.0f), FLT_MIN), c1 = fmaxf(__fdiv_rn(m1, 127.0f), FLT_MIN);
        q[at + lane] = (int8_t)quantize_code(v0, __frcp_rn(c0), 127.0f);
        q[at + lane + 64] = (int8_t)quantize_code(v1, __frcp_rn(c1), 127.0f);
        if (lane == 0) {
            const size_t g = at / 64;
            qs[g] = c0;
            qs[g + 1] = c1;
        }
    }
}

// Per (row, head): zero-centred RMSNorm of the 256 values at src + row*src_row
// + head*src_head, then the rotary embedding of dims [0, 64) at position
// pos[row] (row when pos is null): dims i and i + 32 turn by pos * freq[i].
// src and dst may be the same buffer (each wave reads its values first).
__global__ __launch_bounds__(64) void head_norm_rope_kernel(const float *src, size_t src_row, int src_head,
                                                            int heads, const float *__restrict__ w,
                                                            const int32_t *__restrict__ pos,
                                                            const float *__restrict__ freq, float *dst) {
    const int row = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
    const float4_t x = *(const float4_t *)(src + (size_t)row * src_row + (size_t)head * src_head + lane * 4);
    const float ss = wave_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
    const float scale = rsqrt_rn(__fadd_rn(ss / (float)kAd, 1e-6f));
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; e++) y[e] = __fmul_rn(__fmul_rn(x[e], scale), __fadd_rn(1.0f, w[lane * 4 + e]));
    // lanes 0-7 hold dims 0-31, lanes 8-15 dims 32-63
    const float p = (float)(pos ? pos[row] : row);
    float partner[4];
#pragma unroll
    for (int e = 0; e < 4; e++) partner[e] = __shfl(y[e], lane < 8 ? lane + 8 : lane - 8);
    if (lane < 16) {
        const int base = (lane % 8) * 4;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float sn, cs;
            sincosf(__fmul_rn(p, freq[base + e]), &sn, &cs);
            if (lane < 8) y[e] = __fsub_rn(__fmul_rn(y[e], cs), __fmul_rn(partner[e], sn));
            else y[e] = __fadd_rn(__fmul_rn(y[e], cs), __fmul_rn(partner[e], sn));
        }
    }
    *(float4_t *)(dst + ((size_t)row * heads + head) * kAd + lane * 4) = float4_t{y[0], y[1], y[2], y[3]};
}

// One wave per (head, query): scores over every key (lanes split the keys),
// max-subtracted softmax, then P V with lanes splitting the 256 dims.
// q [nq x ah x 256], k [nk x akv x 256] (normed, rotated), v rows of v_row
// floats with head kh at kh*256; out [ah x nq x 256].
__global__ __launch_bounds__(64) void attention_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                       const float *__restrict__ v, size_t v_row, int nq, int nk,
                                                       int ah, int akv, float scale, float *__restrict__ out) {
    extern __shared__ float sh[];  // q row (256), then the nk scores
    const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
    const int kh = h / (ah / akv);
    float *qs = sh, *ps = sh + kAd;
    *(float4_t *)(qs + lane * 4) = *(const float4_t *)(q + ((size_t)t * ah + h) * kAd + lane * 4);
    __syncthreads();
    float mx = -INFINITY;
    for (int jj = lane; jj < nk; jj += 64) {
        const float4_t *kr = (const float4_t *)(k + ((size_t)jj * akv + kh) * kAd);
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll 8
        for (int u = 0; u < kAd / 4; u += 2) {
            const float4_t a0 = kr[u], a1 = kr[u + 1];
            const float4_t b0 = *(const float4_t *)(qs + 4 * u), b1 = *(const float4_t *)(qs + 4 * u + 4);
#pragma unroll
            for (int e = 0; e < 4; e++) {
                d0 = __builtin_fmaf(a0[e], b0[e], d0);
                d1 = __builtin_fmaf(a1[e], b1[e], d1);
            }
        }
        const float s = (d0 + d1) * scale;
        ps[jj] = s;
        mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int jj = lane; jj < nk; jj += 64) {
        const float p = expf(ps[jj] - mx);
        ps[jj] = p;
        sum += p;
    }
    sum = wave_sum(sum);
    __syncthreads();
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    for (int jj = 0; jj < nk; jj++) {
        const float p = ps[jj];
        const float4_t vv = *(const float4_t *)(v + (size_t)jj * v_row + (size_t)kh * kAd + lane * 4);
#pragma unroll
        for (int e = 0; e < 4; e++) acc[e] = __builtin_fmaf(p, vv[e], acc[e]);
    }
    const float inv = 1.0f / sum;
    *(float4_t *)(out + ((size_t)h * nq + t) * kAd + lane * 4) =
        float4_t{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
}

// Flash attention on f32 MFMA (v_mfma_f32_16x16x4_f32): one workgroup per
// (16 queries, key/value head), one wave per query head of that group (GQA),
// so the K/V blocks staged in LDS serve every head that reads them.
// Per block of 32 keys a wave forms S^T = K Q^T (keys as MFMA rows, queries as
// columns: each lane then holds 8 scores of one query), updates that query's
// running maximum and sum, and adds V^T P^T into its 16 x 256 output tile.
// The contraction index of S^T runs over dims as 64 * (lane / 16) + step, so a
// lane's K operands are 16 consecutive float4s of one key row; K rows are
// padded by 16 bytes so those reads from 16 keys hit distinct banks. Output
// tile (s, u) row r is dim 64s + 4r + u, so one float4 of a V row feeds four
// MFMAs. K/V blocks are double-buffered and loaded straight into LDS; keys
// past the end load the last key's row and score -inf.
constexpr int kAttnKeys = 32;
constexpr int kAttnKRow = kAd * 4 + 16;
constexpr int kAttnVRow = kAd * 4;
constexpr int kAttnBuf = kAttnKeys * (kAttnKRow + kAttnVRow);
constexpr int kAttnLds = 2 * kAttnBuf;
constexpr int kAttnMaxGroup = 8;

__global__ __launch_bounds__(kAttnMaxGroup * 64) void attention_mfma_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, size_t v_row, int nq,
    int nk, int ah, int akv, float scale, float *__restrict__ out) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int group = blockDim.x / 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int kh = blockIdx.y, h = kh * group + wave;
    const int col = lane % 16, g = lane / 16;
    const int t = blockIdx.x * 16 + col;
    float qv[64];
    {
        const float *src = q + ((size_t)(t < nq ? t : 0) * ah + h) * kAd + 64 * g;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float4_t x = t < nq ? *(const float4_t *)(src + 4 * i) : float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++) qv[4 * i + e] = __fmul_rn(x[e], scale);
        }
    }
    const int32x4_t krs = buffer_rsrc(k, (uint32_t)((size_t)nk * akv * kAd * 4));
    const int32x4_t vrs = buffer_rsrc(v, (uint32_t)((size_t)nk * v_row * 4));
    const uint32_t base = lds_address(lds);
    auto issue = [&](int blk, int buf) {
        const uint32_t kb = base + (uint32_t)(buf * kAttnBuf), vb = kb + kAttnKeys * kAttnKRow;
        for (int r = wave; r < 2 * kAttnKeys; r += group) {
            const int key = min(blk * kAttnKeys + r % kAttnKeys, nk - 1);
            if (r < kAttnKeys)
                dma16(kb + r * kAttnKRow, (uint32_t)(((size_t)key * akv + kh) * kAd * 4) + lane * 16, krs);
            else
                dma16(vb + (r - kAttnKeys) * kAttnVRow,
                      (uint32_t)(((size_t)key * v_row + (size_t)kh * kAd) * 4) + lane * 16, vrs);
        }
    };
    float4_t o[16];
#pragma unroll
    for (int i = 0; i < 16; i++) o[i] = float4_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, lsum = 0.0f;
    const int nb = (nk + kAttnKeys - 1) / kAttnKeys;
    issue(0, 0);
    for (int b = 0; b < nb; b++) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's block-b loads have landed
        __syncthreads();                     // every wave's have; block b-1's buffer is free
        if (b + 1 < nb) issue(b + 1, (b + 1) & 1);
        const uint8_t *kt = lds + (b & 1) * kAttnBuf, *vt = kt + kAttnKeys * kAttnKRow;
        float4_t st[2];
#pragma unroll
        for (int T = 0; T < 2; T++) {
            st[T] = float4_t{0.f, 0.f, 0.f, 0.f};
            const uint8_t *kr = kt + (16 * T + col) * kAttnKRow + 256 * g;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4_t kk = *(const float4_t *)(kr + 16 * i);
#pragma unroll
                for (int e = 0; e < 4; e++) st[T] = __builtin_amdgcn_mfma_f32_16x16x4f32(kk[e], qv[4 * i + e], st[T], 0, 0, 0);
            }
        }
        float bm = -INFINITY;
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (b * kAttnKeys + 16 * T + 4 * g + i >= nk) st[T][i] = -INFINITY;
                bm = fmaxf(bm, st[T][i]);
            }
        bm = fmaxf(bm, __shfl_xor(bm, 16));
        bm = fmaxf(bm, __shfl_xor(bm, 32));
        const float mn = fmaxf(m, bm);
        const float alpha = expf(m - mn);
        m = mn;
        lsum = __fmul_rn(lsum, alpha);
#pragma unroll
        for (int i = 0; i < 16; i++) o[i] = o[i] * alpha;
        float pv[2][4];
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pv[T][i] = expf(st[T][i] - m);
                lsum = __fadd_rn(lsum, pv[T][i]);
            }
#pragma unroll
        for (int T = 0; T < 2; T++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint8_t *vr = vt + (16 * T + 4 * g + i) * kAttnVRow + 16 * col;
#pragma unroll
                for (int S = 0; S < 4; S++) {
                    const float4_t vv = *(const float4_t *)(vr + 256 * S);
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        o[4 * S + u] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[u], pv[T][i], o[4 * S + u], 0, 0, 0);
                }
            }
    }
    lsum = __fadd_rn(lsum, __shfl_xor(lsum, 16));
    lsum = __fadd_rn(lsum, __shfl_xor(lsum, 32));
    if (t < nq) {
        const float inv = 1.0f / lsum;
        float *dst = out + ((size_t)h * nq + t) * kAd + 16 * g;
#pragma unroll
        for (int S = 0; S < 4; S++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                *(float4_t *)(dst + 64 * S + 4 * i) =
                    float4_t{o[4 * S][i] * inv, o[4 * S + 1][i] * inv, o[4 * S + 2][i] * inv, o[4 * S + 3][i] * inv};
    }
}

// out[t][h*256 + i] = heads[h][t][i] * sigmoid(z), z at zsrc + t*z_row + h*z_head + i.
// CODES: instead of out, the A8 codes and scales of each 64-group (one wave per
// group; the activation quantizer's arithmetic, int8.rs:178-202), with *bad
// raised on a non-finite value. Grid (ah blocks of 256 threads, n rows):
// block (h, t) takes head h of token t, so no index is divided and a wave
// holds one 64-group.
template <bool CODES>
__global__ void attention_gate_kernel(const float *__restrict__ heads, int n, int ah,
                                      const float *__restrict__ zsrc, size_t z_row, int z_head,
                                      float *__restrict__ out, int8_t *__restrict__ q, float *__restrict__ qs,
                                      int *bad) {
    static_assert(kAd == 256, "one block of 256 threads per head");
    const int t = blockIdx.y, h = blockIdx.x, d = threadIdx.x;
    if (t >= n || h >= ah) return;  // whole block
    const size_t i = ((size_t)t * ah + h) * kAd + d;
    const float z = zsrc[(size_t)t * z_row + (size_t)h * z_head + d];
    const float v = __fmul_rn(heads[((size_t)h * n + t) * kAd + d], sigmoid_ref(z));
    if constexpr (!CODES) {
        out[i] = v;
    } else {
        if (!__builtin_isfinite(v) && bad) atomicOr(bad, 1);
        const float c = fmaxf(__fdiv_rn(wave_max_dpp(fabsf(v)), 127.0f), FLT_MIN);
        q[i] = (int8_t)quantize_code(v, __frcp_rn(c), 127.0f);
        if ((i & 63) == 0) qs[i / 64] = c;
    }
}

// dst[r] = src[idx[r]], rows of `width` floats
__global__ void gather_rows_kernel(const float *__restrict__ src, const int32_t *__restrict__ idx, int rows,
                                   int width, float *__restrict__ dst) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i >= (size_t)rows * width) return;
    const int r = (int)(i / width), c = (int)(i % width);
    dst[i] = src[(size_t)idx[r] * width + c];
}

}  // namespace

// The token-by-token scan alone (the decider's launch and the tuner's): qhat
// and khat [n][lk][128], conv [n][2 lk 128 + lh 128] (v from column
// 2 lk 128 on), gb [n][lh][4] = {g, beta, k.q, -}, out [lh][n][128].
// variant 1 is the rolled loop, any other the unrolled one; the same bits.
void launch_delta_scan_tokens(const float *qhat, const float *khat, const float *conv, const float *gb, int n,
                              int lh, int lk, float *out, bool rolled, hipStream_t s) {
    if (rolled)
        hipLaunchKernelGGL(delta_scan_kernel<false>, dim3(lh, kLd / kScanCols), dim3(64 * kScanWaves), 0, s, qhat,
                           khat, conv, gb, n, lh, lk, out);
    else
        hipLaunchKernelGGL(delta_scan_kernel<true>, dim3(lh, kLd / kScanCols), dim3(64 * kScanWaves), 0, s, qhat,
                           khat, conv, gb, n, lh, lk, out);
}

size_t delta_chunk_ws_bytes(int n, int lh) { return (size_t)lh * ((n + kChunk - 1) / kChunk) * kChunkWs * 4; }

void launch_delta_scan_chunked(const float *qhat, const float *khat, const float *conv, const float *gb, int n,
                               int lh, int lk, float *ws, float *out, int column_tiles, hipStream_t s) {
    if (n <= 0) return;
    constexpr size_t lds = (size_t)(kChunk * kChunkRow + kChunk * kChunk + 3 * kChunk) * 4;
    static bool configured[64] = {};  // the LDS limit is a per-device function attribute
    int dev = 0;
    hipGetDevice(&dev);
    if (dev >= 0 && dev < 64 && !configured[dev]) {
        if (hipFuncSetAttribute((const void *)delta_chunk_prep_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) == hipSuccess)
            configured[dev] = true;
    }
    const unsigned chunks = (unsigned)((n + kChunk - 1) / kChunk);
    hipLaunchKernelGGL(delta_chunk_prep_kernel, dim3(lh, chunks), dim3(256), lds, s, qhat, khat, conv, gb, n, lh, lk,
                       ws);
    if (column_tiles == 2)
        hipLaunchKernelGGL(delta_chunk_scan_kernel<2>, dim3(lh, kLd / 32), dim3(512), 0, s, qhat, ws, n, lh, lk, out);
    else
        hipLaunchKernelGGL(delta_chunk_scan_kernel<1>, dim3(lh, kLd / 16), dim3(256), 0, s, qhat, ws, n, lh, lk, out);
}

}  // namespace dz

struct dz_pplx {
    dz_pplx_config cfg{};
    struct Layer {
        bool attention = false;
        float *input_norm = nullptr, *post_norm = nullptr;
        dz_weight *qkv = nullptr, *z = nullptr, *a = nullptr, *b = nullptr, *out = nullptr;
        float *conv = nullptr, *decay = nullptr, *dt = nullptr, *norm = nullptr;
        dz_weight *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr;
        float *qnorm = nullptr, *knorm = nullptr;
        dz_weight *gate = nullptr, *up = nullptr, *down = nullptr;
        // in_proj_z, in_proj_a and in_proj_b as one weight (rows z, then a, then
        // b), so one product launch covers the three: derived from them, while
        // the weights are resident
        dz_weight *zab = nullptr;
    };
    std::vector<Layer> layers;
    dz_weight *readout = nullptr;
    float *final_norm = nullptr;
    float *freq = nullptr;  // rotary frequencies [32]
    // activations for `capacity` tokens
    size_t capacity = 0;
    std::vector<void *> buffers;
    float *hidden = nullptr, *normed = nullptr, *wide = nullptr, *z = nullptr, *ab = nullptr, *conv_out = nullptr,
          *qhat = nullptr, *khat = nullptr, *gb = nullptr, *heads = nullptr, *ctx = nullptr, *projected = nullptr,
          *key = nullptr, *value = nullptr, *query = nullptr, *picked = nullptr, *gate = nullptr, *up = nullptr,
          *logits = nullptr, *chunk_ws = nullptr;
    int8_t *codes = nullptr;     // the MLP's down_proj input codes
    float *code_scales = nullptr;
    int8_t *ncodes = nullptr;    // the A8 codes of a layer norm's output, shared by its products
    float *nscales = nullptr;
    int32_t *markers = nullptr;
    uint8_t *rows_dev = nullptr;
    dz::Weight rows_weight;
    int32_t rows_form = DZ_ROWS_PACKED;  // how forward_rows decodes the packed embedding rows
    // What the last layer call left in the activation buffers, for
    // dz_pplx_activation: the layer, its kind and row counts, which norm and
    // gate outputs were written in which form, and where z, a and b sit.
    struct Trace {
        int layer = -1;
        bool attention = false;
        size_t n = 0, nq = 0, rows = 0;
        bool mixer = false;  // the mixer half ran (its activations are the layer's)
        bool norm_codes = false, normed = false, gate_codes = false, gate_f32 = false, mlp_codes = false;
        const float *a = nullptr, *b = nullptr;
        int z_ld = 0, ab_ld = 0;
    } trace;
    // Streamed residency (webgpu/streaming.rs:16-369): the layers' projections
    // live in pinned host memory, already in the device layout, and layer i
    // runs from device bank i % 2. The copy stream fills a bank once the layer
    // that used it last has finished (`done`); the compute stream waits for the
    // copy (`copied`). A layer's weight handles point into its bank for good;
    // only the bank's contents change. At most two layers are in flight: one
    // computing, the next one copying.
    struct Streaming {
        bool on = false;
        uint8_t *host = nullptr;            // every layer's projections, layer after layer
        size_t host_bytes = 0;
        std::vector<size_t> offset, bytes;  // per layer, in `host`
        uint8_t *bank[2] = {nullptr, nullptr};
        size_t bank_bytes = 0;
        hipStream_t copy = nullptr;
        hipEvent_t copied[2] = {nullptr, nullptr}, done[2] = {nullptr, nullptr};
        int held[2] = {-1, -1};             // the layer each bank holds (or is receiving)
        uint64_t uploads = 0, reuses = 0, upload_bytes = 0;
    } st;
};

namespace dz {

namespace {

size_t conv_width(const dz_pplx_config &c) { return 2 * (size_t)c.delta_key_heads * kLd + (size_t)c.delta_heads * kLd; }

// The projections of one layer, in the order their bytes sit in host memory
// and in the layer's bank when the weights are streamed.
std::vector<dz_weight *> projections(const dz_pplx::Layer &L) {
    if (L.attention) return {L.q, L.k, L.v, L.o, L.gate, L.up, L.down};
    return {L.qkv, L.z, L.a, L.b, L.out, L.gate, L.up, L.down};
}

int32_t stream_replace(dz_ctx *ctx, dz_pplx *p, int layer, const dz_weight *slot, const dz_weight *w);

// Frees the streamed state's banks, events, copy stream and host copy (the
// caller has synchronized both streams and re-pointed the weight handles).
void streaming_release(dz_pplx *p) {
    auto &st = p->st;
    for (int b = 0; b < 2; b++) {
        if (st.bank[b]) hipFree(st.bank[b]);
        if (st.copied[b]) hipEventDestroy(st.copied[b]);
        if (st.done[b]) hipEventDestroy(st.done[b]);
        st.bank[b] = nullptr;
        st.copied[b] = st.done[b] = nullptr;
        st.held[b] = -1;
    }
    if (st.copy) hipStreamDestroy(st.copy);
    if (st.host) hipHostFree(st.host);
    st.copy = nullptr;
    st.host = nullptr;
    st.host_bytes = st.bank_bytes = 0;
    st.offset.clear();
    st.bytes.clear();
    st.on = false;
}

void free_activations(dz_pplx *p) {
    for (void *b : p->buffers) hipFree(b);
    p->buffers.clear();
    p->capacity = 0;
}

int32_t ensure_capacity(dz_ctx *ctx, dz_pplx *p, size_t n) {
    if (p->capacity >= n) return DZ_OK;
    hipStreamSynchronize(ctx_stream(ctx));
    free_activations(p);
    const dz_pplx_config &c = p->cfg;
    const size_t d = c.hidden, cw = conv_width(c), lv = (size_t)c.delta_heads * kLd;
    const size_t qw = 2 * (size_t)c.attn_heads * kAd, kvw = (size_t)c.attn_kv_heads * kAd;
    const size_t wide = std::max(cw, qw), ctxw = std::max(lv, (size_t)c.attn_heads * kAd);
    hipError_t err = hipSuccess;
    auto get = [&](auto **ptr, size_t bytes) {
        void *q = nullptr;
        if (err == hipSuccess) err = hipMalloc(&q, bytes < 256 ? 256 : bytes);
        if (err == hipSuccess) p->buffers.push_back(q);
        *ptr = (std::remove_reference_t<decltype(**ptr)> *)q;
    };
    get(&p->hidden, n * d * 4);
    get(&p->normed, n * d * 4);
    get(&p->wide, n * wide * 4);
    get(&p->z, n * (lv + 2 * ((size_t)c.delta_heads + 15) / 16 * 16) * 4);  // z, or z | a | b of the joined weight
    get(&p->ab, n * c.delta_heads * 2 * 4);
    get(&p->conv_out, n * cw * 4);
    get(&p->qhat, n * c.delta_key_heads * kLd * 4);
    get(&p->khat, n * c.delta_key_heads * kLd * 4);
    get(&p->gb, n * c.delta_heads * 4 * 4);
    get(&p->chunk_ws, delta_chunk_ws_bytes((int)n, c.delta_heads));
    get(&p->heads, n * std::max(lv, (size_t)c.attn_heads * kAd) * 4);
    get(&p->ctx, n * ctxw * 4);
    get(&p->projected, n * d * 4);
    get(&p->key, n * kvw * 4);
    get(&p->value, n * kvw * 4);
    get(&p->query, n * (size_t)c.attn_heads * kAd * 4);
    get(&p->picked, n * d * 4);
    get(&p->gate, n * (size_t)c.ff * 4);
    get(&p->up, n * (size_t)c.ff * 4);
    get(&p->codes, n * (size_t)c.ff);
    get(&p->code_scales, n * (size_t)(c.ff / 64) * 4);
    get(&p->ncodes, n * d);
    get(&p->nscales, n * (d / 64) * 4);
    get(&p->markers, (size_t)DZ_READOUT_MAX_MARKERS * 4);
    get(&p->logits, (size_t)DZ_READOUT_MAX_MARKERS * DZ_READOUT_CODES * 4);
    get(&p->rows_dev, n * (d / 64) * 36);
    Weight &w = p->rows_weight;
    w.kind = WeightKind::Q4G64;
    w.bits = 4;
    w.group = 64;
    w.rows = (int)n;
    w.cols = (int)d;
    w.groups = (int)(d / 64);
    w.np = (int)((n + 15) / 16 * 16);
    w.kp = (int)((d + 127) / 128 * 128);
    w.code_bytes = (size_t)w.np * w.kp / 2;
    w.scale_bytes = (size_t)w.np * (w.kp / 128) * 8;
    get(&w.codes, w.code_bytes);
    get(&w.scales, w.scale_bytes);
    if (err != hipSuccess) {
        free_activations(p);
        return ctx_hip_fail(ctx, err, "pplx activations");
    }
    p->capacity = n;
    return DZ_OK;
}

int32_t vec_upload(dz_ctx *ctx, float **dst, const float *src, size_t count) {
    if (!*dst) {
        hipError_t e = hipMalloc(dst, count * sizeof(float));
        if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx vector");
    }
    hipError_t e = hipMemcpyAsync(*dst, src, count * sizeof(float), hipMemcpyHostToDevice, ctx_stream(ctx));
    if (e == hipSuccess) e = hipStreamSynchronize(ctx_stream(ctx));
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx vector");
    return DZ_OK;
}

bool starts(const std::string &s, const char *p, std::string *rest) {
    size_t n = strlen(p);
    if (s.compare(0, n, p) != 0) return false;
    *rest = s.substr(n);
    return true;
}

}  // namespace

void pplx_destroy(dz_ctx *ctx, dz_pplx *p) {
    if (!p) return;
    hipStreamSynchronize(ctx_stream(ctx));
    if (p->st.on) {  // the handles point into the banks, which streaming_release frees
        hipStreamSynchronize(p->st.copy);
        for (auto &l : p->layers)
            for (dz_weight *w : projections(l))
                if (w) weight_mut(w).codes = weight_mut(w).scales = nullptr;
    }
    streaming_release(p);
    for (auto &l : p->layers) {
        for (dz_weight *w : {l.qkv, l.z, l.a, l.b, l.out, l.q, l.k, l.v, l.o, l.gate, l.up, l.down, l.zab})
            weight_free(w);
        for (float *f : {l.input_norm, l.post_norm, l.conv, l.decay, l.dt, l.norm, l.qnorm, l.knorm})
            if (f) hipFree(f);
    }
    weight_free(p->readout);
    for (float *f : {p->final_norm, p->freq})
        if (f) hipFree(f);
    free_activations(p);
    delete p;
}

int32_t pplx_create(dz_ctx *ctx, const dz_pplx_config *cfg, dz_pplx **out) {
    if (!cfg || !out) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    *out = nullptr;
    const dz_pplx_config c = *cfg;
    if (c.layers < 1 || c.hidden < 64 || c.hidden % 64 != 0 || c.ff < 64 || c.ff % 64 != 0 ||
        c.delta_head_dim != kLd || c.attn_head_dim != kAd || c.delta_heads < 1 || c.delta_key_heads < 1 ||
        c.delta_heads % c.delta_key_heads != 0 || c.attn_heads < 1 || c.attn_kv_heads < 1 ||
        c.attn_heads % c.attn_kv_heads != 0 || c.delta_key_heads > 16)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS,
                        "pplx config: hidden and ff multiples of 64, delta head dim 128, attention head dim 256, "
                        "heads divisible by their key heads, at most 16 delta key heads");
    dz_pplx *p = new dz_pplx();
    p->cfg = c;
    p->layers.resize(c.layers);
    for (int i = 0; i < c.layers; i++) p->layers[i].attention = i % 4 == 3;  // backbone.rs:132-136
    // backbone.rs:227-229 inv_freq[i] = 1 / 1e7^(2i/64), in f32
    float freq[32];
    for (int i = 0; i < 32; i++) freq[i] = 1.0f / powf(10000000.0f, (float)(2 * i) / 64.0f);
    int32_t rc = vec_upload(ctx, &p->freq, freq, 32);
    if (rc) {
        pplx_destroy(ctx, p);
        return rc;
    }
    *out = p;
    return DZ_OK;
}

// (Re)builds a delta layer's joined z | a | b weight from its three parts,
// while the weights are resident and the parts share one layout; otherwise
// the layer runs the three products. A joining that fails only costs speed.
void join_zab(dz_ctx *ctx, dz_pplx *p, dz_pplx::Layer &L) {
    weight_free(L.zab);
    L.zab = nullptr;
    if (p->st.on || L.attention || !L.z || !L.a || !L.b) return;
    const auto kind = weight_of(L.z).kind;
    if (weight_of(L.a).kind != kind || weight_of(L.b).kind != kind) return;
    const dz_weight *parts[3] = {L.z, L.a, L.b};
    if (weight_concat_rows(ctx, parts, 3, &L.zab) != DZ_OK) L.zab = nullptr;
}

// form: -1 for a packed.rs matrix in `layout`; DZ_FIT_SCALED for a fitted Q4
// (quantization.rs mse) matrix in the DZ_Q4_G64_F32 wire layout.
int32_t pplx_set_weight(dz_ctx *ctx, dz_pplx *p, const char *name, const void *packed, size_t bytes, int32_t layout,
                        size_t rows, size_t cols, int32_t form) {
    if (!p || !name || !packed) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (layout != DZ_Q4_G64_F32 && layout != DZ_Q8_G64_F32)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS, "pplx projections are group-64 packed matrices");
    if (form >= 0 && (form != DZ_FIT_SCALED || layout != DZ_Q4_G64_F32))
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS,
                        "the decider takes fitted Q4 weights in the scaled (MSE) form: its products have no offset "
                        "term and its projections no codebook");
    const dz_pplx_config &c = p->cfg;
    const size_t d = c.hidden, cw = conv_width(c), lv = (size_t)c.delta_heads * kLd;
    std::string s(name), rest;
    dz_weight **slot = nullptr;
    size_t want_r = 0, want_c = 0;
    int layer = -1;
    if (s == "readout") {
        slot = &p->readout;
        want_r = DZ_READOUT_CODES;
        want_c = d;
    } else if (starts(s, "language_model.layers.", &rest)) {
        const size_t dot = rest.find('.');
        const int i = dot == std::string::npos ? -1 : atoi(rest.substr(0, dot).c_str());
        if (i < 0 || i >= c.layers || rest.substr(0, dot) != std::to_string(i))
            return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "layer index out of range: " + s);
        auto &L = p->layers[i];
        const std::string t = rest.substr(dot + 1);
        struct Slot {
            const char *name;
            bool attention;
            dz_weight **w;
            size_t r, c;
        } slots[] = {
            {"linear_attn.in_proj_qkv.weight", false, &L.qkv, cw, d},
            {"linear_attn.in_proj_z.weight", false, &L.z, lv, d},
            {"linear_attn.in_proj_a.weight", false, &L.a, (size_t)c.delta_heads, d},
            {"linear_attn.in_proj_b.weight", false, &L.b, (size_t)c.delta_heads, d},
            {"linear_attn.out_proj.weight", false, &L.out, d, lv},
            {"self_attn.q_proj.weight", true, &L.q, 2 * (size_t)c.attn_heads * kAd, d},
            {"self_attn.k_proj.weight", true, &L.k, (size_t)c.attn_kv_heads * kAd, d},
            {"self_attn.v_proj.weight", true, &L.v, (size_t)c.attn_kv_heads * kAd, d},
            {"self_attn.o_proj.weight", true, &L.o, d, (size_t)c.attn_heads * kAd},
            {"mlp.gate_proj.weight", L.attention, &L.gate, (size_t)c.ff, d},
            {"mlp.up_proj.weight", L.attention, &L.up, (size_t)c.ff, d},
            {"mlp.down_proj.weight", L.attention, &L.down, d, (size_t)c.ff},
        };
        for (const Slot &sl : slots)
            if (t == sl.name) {
                if (sl.attention != L.attention) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "unsupported layer layout: " + s);
                slot = sl.w;
                want_r = sl.r;
                want_c = sl.c;
                layer = i;
            }
    }
    if (!slot) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "unknown pplx tensor: " + s);
    if (rows != want_r || cols != want_c) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "tensor shape mismatch: " + s);
    dz_weight *w = nullptr;
    int32_t rc = form >= 0 ? weight_upload_fitted(ctx, packed, bytes, rows, cols, form, &w)
                           : weight_upload(ctx, packed, bytes, layout, rows, cols, &w);
    if (rc) return rc;
    if (p->st.on && layer >= 0) {  // streamed: the new bytes replace the host copy
        const Weight &a = weight_of(w), &b = weight_of(*slot);
        if (a.kind != b.kind || a.code_bytes != b.code_bytes || a.scale_bytes != b.scale_bytes) {
            weight_free(w);
            return ctx_fail(ctx, DZ_INVALID_REQUEST,
                            "a streamed projection keeps its layout: set resident residency to change it: " + s);
        }
        rc = stream_replace(ctx, p, layer, *slot, w);
        weight_free(w);
        return rc;
    }
    weight_free(*slot);
    *slot = w;
    if (layer >= 0 && (slot == &p->layers[layer].z || slot == &p->layers[layer].a || slot == &p->layers[layer].b))
        join_zab(ctx, p, p->layers[layer]);
    return DZ_OK;
}

int32_t pplx_set_vector(dz_ctx *ctx, dz_pplx *p, const char *name, const float *values, size_t count) {
    if (!p || !name || !values) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    const dz_pplx_config &c = p->cfg;
    const size_t d = c.hidden, cw = conv_width(c);
    std::string s(name), rest;
    if (s == "language_model.norm.weight") {
        if (count != d) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "tensor shape mismatch: " + s);
        return vec_upload(ctx, &p->final_norm, values, count);
    }
    if (!starts(s, "language_model.layers.", &rest)) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "unknown pplx tensor: " + s);
    const size_t dot = rest.find('.');
    const int i = dot == std::string::npos ? -1 : atoi(rest.substr(0, dot).c_str());
    if (i < 0 || i >= c.layers || rest.substr(0, dot) != std::to_string(i))
        return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "layer index out of range: " + s);
    auto &L = p->layers[i];
    const std::string t = rest.substr(dot + 1);
    auto need = [&](bool attention, size_t n) { return L.attention == attention && count == n; };
    if (t == "input_layernorm.weight" && count == d) return vec_upload(ctx, &L.input_norm, values, count);
    if (t == "post_attention_layernorm.weight" && count == d) return vec_upload(ctx, &L.post_norm, values, count);
    if (t == "linear_attn.conv1d.weight" && need(false, cw * 4)) {
        // conv1d.weight [width, 1, 4] -> tap-major [4 x width] (backbone.rs:170-178)
        std::vector<float> packed(4 * cw);
        for (size_t tap = 0; tap < 4; tap++)
            for (size_t ch = 0; ch < cw; ch++) packed[tap * cw + ch] = values[ch * 4 + tap];
        return vec_upload(ctx, &L.conv, packed.data(), packed.size());
    }
    if (t == "linear_attn.A_log" && need(false, (size_t)c.delta_heads)) {
        std::vector<float> decay(values, values + count);
        for (float &v : decay) v = expf(v);  // backbone.rs:179-183
        return vec_upload(ctx, &L.decay, decay.data(), count);
    }
    if (t == "linear_attn.dt_bias" && need(false, (size_t)c.delta_heads)) return vec_upload(ctx, &L.dt, values, count);
    if (t == "linear_attn.norm.weight" && need(false, kLd)) return vec_upload(ctx, &L.norm, values, count);
    if (t == "self_attn.q_norm.weight" && need(true, kAd)) return vec_upload(ctx, &L.qnorm, values, count);
    if (t == "self_attn.k_norm.weight" && need(true, kAd)) return vec_upload(ctx, &L.knorm, values, count);
    return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "unknown pplx tensor or shape: " + s);
}

namespace {

bool complete(const dz_pplx *p, std::string *missing) {
    for (size_t i = 0; i < p->layers.size(); i++) {
        const auto &L = p->layers[i];
        bool ok = L.input_norm && L.post_norm && L.gate && L.up && L.down;
        ok = ok && (L.attention ? (L.q && L.k && L.v && L.o && L.qnorm && L.knorm)
                                : (L.qkv && L.z && L.a && L.b && L.out && L.conv && L.decay && L.dt && L.norm));
        if (!ok) {
            *missing = "layer " + std::to_string(i);
            return false;
        }
    }
    if (!p->readout || !p->final_norm) {
        *missing = "readout or final norm";
        return false;
    }
    return true;
}

// ---- streamed residency (webgpu/streaming.rs:16-369) -------------------------------

// Every part of a layer's bank is 256-byte aligned.
inline size_t bank_align(size_t v) { return (v + 255) / 256 * 256; }

// Bytes of one layer in the bank layout: each projection's codes, then its
// scales, in projections() order.
size_t layer_bank_bytes(const dz_pplx::Layer &L) {
    size_t b = 0;
    for (dz_weight *w : projections(L)) b += bank_align(weight_of(w).code_bytes) + bank_align(weight_of(w).scale_bytes);
    return b;
}

// Offset of projection `w` inside its layer's bank.
size_t bank_offset(const dz_pplx::Layer &L, const dz_weight *w) {
    size_t off = 0;
    for (dz_weight *x : projections(L)) {
        if (x == w) break;
        off += bank_align(weight_of(x).code_bytes) + bank_align(weight_of(x).scale_bytes);
    }
    return off;
}

// Moves every layer projection into pinned host memory (the device layout,
// copied as it is) and points layer i's handles into bank i % 2. The device
// copies are freed only after every byte has reached the host.
int32_t stream_on(dz_ctx *ctx, dz_pplx *p) {
    std::string missing;
    if (!complete(p, &missing)) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "missing pplx weights: " + missing);
    auto &st = p->st;
    const size_t layers = p->layers.size();
    st.offset.assign(layers, 0);
    st.bytes.assign(layers, 0);
    size_t total = 0, bank = 0;
    for (size_t i = 0; i < layers; i++) {
        st.offset[i] = total;
        st.bytes[i] = layer_bank_bytes(p->layers[i]);
        total += st.bytes[i];
        bank = std::max(bank, st.bytes[i]);
    }
    hipStream_t s = ctx_stream(ctx);
    hipError_t e = hipHostMalloc((void **)&st.host, total, hipHostMallocDefault);
    for (int b = 0; b < 2 && e == hipSuccess; b++) e = hipMalloc(&st.bank[b], bank);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&st.copy, hipStreamNonBlocking);
    for (int b = 0; b < 2 && e == hipSuccess; b++) {
        e = hipEventCreateWithFlags(&st.copied[b], hipEventDisableTiming);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&st.done[b], hipEventDisableTiming);
        // recorded once, so that every later wait on them has an event to wait for
        if (e == hipSuccess) e = hipEventRecord(st.copied[b], st.copy);
        if (e == hipSuccess) e = hipEventRecord(st.done[b], s);
    }
    for (size_t i = 0; i < layers && e == hipSuccess; i++) {
        uint8_t *dst = st.host + st.offset[i];
        for (dz_weight *w : projections(p->layers[i])) {
            const Weight &x = weight_of(w);
            e = hipMemcpyAsync(dst, x.codes, x.code_bytes, hipMemcpyDeviceToHost, s);
            dst += bank_align(x.code_bytes);
            if (e == hipSuccess) e = hipMemcpyAsync(dst, x.scales, x.scale_bytes, hipMemcpyDeviceToHost, s);
            dst += bank_align(x.scale_bytes);
            if (e != hipSuccess) break;
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        hipStreamSynchronize(s);
        streaming_release(p);
        return ctx_hip_fail(ctx, e, "streamed residency");
    }
    st.host_bytes = total;
    st.bank_bytes = bank;
    for (size_t i = 0; i < layers; i++) {
        uint8_t *base = st.bank[i % 2];
        for (dz_weight *w : projections(p->layers[i])) {
            Weight &x = weight_mut(w);
            hipFree(x.codes);
            hipFree(x.scales);
            const size_t off = bank_offset(p->layers[i], w);
            x.codes = base + off;
            x.scales = base + off + bank_align(x.code_bytes);
        }
    }
    st.held[0] = st.held[1] = -1;
    st.uploads = st.reuses = st.upload_bytes = 0;
    st.on = true;
    for (auto &L : p->layers) join_zab(ctx, p, L);  // frees the joined copies: the banks hold the parts
    return DZ_OK;
}

// Gives every layer projection its own device memory again, filled from the
// host copy; the streamed state is released only once all of it is there.
int32_t stream_off(dz_ctx *ctx, dz_pplx *p) {
    auto &st = p->st;
    hipStream_t s = ctx_stream(ctx);
    hipError_t e = hipStreamSynchronize(st.copy);
    std::vector<uint8_t *> fresh;
    for (size_t i = 0; i < p->layers.size() && e == hipSuccess; i++) {
        const uint8_t *src = st.host + st.offset[i];
        for (dz_weight *w : projections(p->layers[i])) {
            const Weight &x = weight_of(w);
            uint8_t *c = nullptr, *sc = nullptr;
            e = hipMalloc(&c, x.code_bytes);
            if (e == hipSuccess) fresh.push_back(c);
            if (e == hipSuccess) e = hipMalloc(&sc, x.scale_bytes);
            if (e == hipSuccess) fresh.push_back(sc);
            if (e == hipSuccess) e = hipMemcpyAsync(c, src, x.code_bytes, hipMemcpyHostToDevice, s);
            src += bank_align(x.code_bytes);
            if (e == hipSuccess) e = hipMemcpyAsync(sc, src, x.scale_bytes, hipMemcpyHostToDevice, s);
            src += bank_align(x.scale_bytes);
            if (e != hipSuccess) break;
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
        hipStreamSynchronize(s);
        for (uint8_t *f : fresh) hipFree(f);
        return ctx_hip_fail(ctx, e, "resident weights");
    }
    size_t k = 0;
    for (auto &L : p->layers)
        for (dz_weight *w : projections(L)) {
            Weight &x = weight_mut(w);
            x.codes = fresh[k++];
            x.scales = fresh[k++];
        }
    streaming_release(p);
    for (auto &L : p->layers) join_zab(ctx, p, L);
    return DZ_OK;
}

// Starts the copy of layer i into bank i % 2, after the layer that used the
// bank last has finished, unless the bank already holds layer i.
int32_t stream_in(dz_ctx *ctx, dz_pplx *p, int i) {
    auto &st = p->st;
    const int b = i % 2;
    if (st.held[b] == i) return DZ_OK;
    hipError_t e = hipStreamWaitEvent(st.copy, st.done[b], 0);
    if (e == hipSuccess)
        e = hipMemcpyAsync(st.bank[b], st.host + st.offset[i], st.bytes[i], hipMemcpyHostToDevice, st.copy);
    if (e == hipSuccess) e = hipEventRecord(st.copied[b], st.copy);
    if (e != hipSuccess) {
        st.held[b] = -1;
        return ctx_hip_fail(ctx, e, "layer weight upload");
    }
    if (st.held[b] >= 0) st.reuses++;
    st.held[b] = i;
    st.uploads++;
    st.upload_bytes += st.bytes[i];
    return DZ_OK;
}

// Replaces the host copy of a streamed projection with the device-layout
// bytes of `w` (same shape); the bank is refilled on the layer's next run.
int32_t stream_replace(dz_ctx *ctx, dz_pplx *p, int layer, const dz_weight *slot, const dz_weight *w) {
    auto &st = p->st;
    const Weight &x = weight_of(w);
    uint8_t *dst = st.host + st.offset[layer] + bank_offset(p->layers[layer], slot);
    hipStream_t s = ctx_stream(ctx);
    hipError_t e = hipStreamSynchronize(st.copy);  // no copy is reading the host bytes
    if (e == hipSuccess) e = hipMemcpyAsync(dst, x.codes, x.code_bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dst + bank_align(x.code_bytes), x.scales, x.scale_bytes, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "streamed weight replacement");
    if (st.held[layer % 2] == layer) st.held[layer % 2] = -1;
    return DZ_OK;
}

// dz_linear_pair / dz_linear / the MLP, on the context's stream
int32_t linear(dz_ctx *ctx, const dz_weight *w, const float *x, size_t m, float *y) {
    return dz_linear(ctx, w, x, DZ_F32, m, y, DZ_W4A8);
}

// The residual connection h += W·x (x f32, or A8 codes q with scales qs): in
// the product's epilogue when the pipelined kernel takes the rows, else the
// product into tmp and an add. Both give the same bits.
int32_t product_add(dz_ctx *ctx, const dz_weight *w, const float *x, const int8_t *q, const float *qs, size_t m,
                    float *h, float *tmp, const int *qbad = nullptr) {
    bool fused = false;
    int32_t rc = ctx_product_add(ctx, w, x, q, qs, m, h, &fused, qbad);
    if (rc || fused) return rc;
    rc = x ? linear(ctx, w, x, m, tmp) : dz_linear_q8(ctx, w, q, qs, m, tmp);
    if (rc) return rc;
    launch_add(h, tmp, 0, m * (size_t)weight_of(w).rows, ctx_stream(ctx));
    return DZ_OK;
}

// The zero-centred RMSNorm of the hidden rows (cpu.rs:310-333). With the
// "fused" norm variant and more than 16 rows, one kernel also writes the A8
// codes of the normed rows (p->ncodes / p->nscales, equal to act_quantize of
// them) and every product of the norm's output reads those codes, with one
// non-finite flag (*flag); the normed f32 rows are written only when `need_f32`.
// Otherwise ("separate", or few rows) the normed rows go to p->normed and each
// product quantizes them itself. Both give the same bits.
int32_t layer_norm(dz_ctx *ctx, dz_pplx *p, const float *w, size_t n, bool need_f32, bool *codes, int **flag) {
    const dz_pplx_config &c = p->cfg;
    hipStream_t s = ctx_stream(ctx);
    *codes = false;
    *flag = nullptr;
    if (n <= 16 || ctx_variant(ctx, "norm") != 0 || c.hidden % 64 != 0 || c.hidden > kRmsQuantizeMaxCols) {
        launch_readout_rms(p->hidden, 0, nullptr, (int)n, c.hidden, w, 1e-6f, 1, p->normed, s);
        p->trace.norm_codes = false;
        p->trace.normed = true;
        return DZ_OK;
    }
    int32_t rc = ctx_product_flag(ctx, flag);
    if (rc) return rc;
    launch_rms_quantize(p->hidden, (int)n, c.hidden, w, 1e-6f, 1, need_f32 ? p->normed : nullptr, p->ncodes,
                        p->nscales, *flag, s);
    *codes = true;
    p->trace.norm_codes = true;
    p->trace.normed = need_f32;
    return DZ_OK;
}

// y = W . normed rows: from the norm's codes, or from p->normed (dz_linear)
int32_t normed_product(dz_ctx *ctx, dz_pplx *p, const dz_weight *w, bool codes, const int *flag, size_t n, float *y) {
    return codes ? ctx_codes_product(ctx, w, p->ncodes, p->nscales, n, y, flag) : linear(ctx, w, p->normed, n, y);
}

// backbone.rs:232-250: post-norm MLP with residual, in place on hidden
int32_t mlp(dz_ctx *ctx, dz_pplx *p, const dz_pplx::Layer &L, size_t n) {
    const dz_pplx_config &c = p->cfg;
    hipStream_t s = ctx_stream(ctx);
    bool codes = false;
    int *flag = nullptr;
    int32_t rc = layer_norm(ctx, p, L.post_norm, n, false, &codes, &flag);
    if (rc) return rc;
    if (weight_of(L.gate).kind == WeightKind::Q4G64 && weight_of(L.up).kind == WeightKind::Q4G64) {
        // gate/up, silu(gate)*up and the A8 codes of the down projection in one pass
        if (codes)
            rc = ctx_mlp_codes(ctx, L.gate, L.up, p->ncodes, p->nscales, n, p->codes, p->code_scales, flag);
        else
            rc = dz_mlp_requant(ctx, L.gate, L.up, p->normed, n, p->codes, p->code_scales);
        p->trace.mlp_codes = true;
        p->trace.gate_codes = false;  // the MLP's codes replace the gate's
        if (!rc) rc = product_add(ctx, L.down, nullptr, p->codes, p->code_scales, n, p->hidden, p->projected);
    } else {
        if (codes) {
            rc = normed_product(ctx, p, L.gate, true, flag, n, p->gate);
            if (!rc) rc = normed_product(ctx, p, L.up, true, flag, n, p->up);
        } else {
            rc = dz_linear_pair(ctx, L.gate, L.up, p->normed, n, p->gate, p->up, DZ_W4A8);
        }
        if (!rc) launch_silu_mul(p->gate, p->up, n * (size_t)c.ff, s);
        if (!rc) rc = product_add(ctx, L.down, p->gate, nullptr, nullptr, n, p->hidden, p->projected);
    }
    return rc;
}

// Variants 0 ("chunked64": 16 state columns per block) and 1
// ("chunked64-c32": 32 per block) run the chunked scan, with the same
// arithmetic; 2 ("recurrent", whole stages unrolled) and 3
// ("recurrent-rolled") the token-by-token one, whose order gives other bits;
// 4 ("auto") the token scan below six chunks of tokens and the chunked one
// from there, so its bits depend on the chunk's length. Only 0 and 1 are tuned.
void launch_delta_scan(dz_ctx *ctx, dz_pplx *p, size_t n, hipStream_t s) {
    const dz_pplx_config &c = p->cfg;
    const int v = ctx_variant(ctx, "delta_scan");
    const bool tokens = v == 2 || v == 3 || (v == 4 && n < (size_t)6 * kChunk);
    if (tokens)
        launch_delta_scan_tokens(p->qhat, p->khat, p->conv_out, p->gb, (int)n, c.delta_heads, c.delta_key_heads,
                                 p->heads, v == 3, s);
    else
        launch_delta_scan_chunked(p->qhat, p->khat, p->conv_out, p->gb, (int)n, c.delta_heads, c.delta_key_heads,
                                  p->chunk_ws, p->heads, v == 1 ? 2 : 1, s);
}

int32_t delta_layer(dz_ctx *ctx, dz_pplx *p, const dz_pplx::Layer &L, size_t n) {
    const dz_pplx_config &c = p->cfg;
    hipStream_t s = ctx_stream(ctx);
    const size_t cw = conv_width(c), lh = c.delta_heads;
    bool codes = false;
    int *flag = nullptr;
    int32_t rc = layer_norm(ctx, p, L.input_norm, n, false, &codes, &flag);
    if (rc) return rc;
    // z, a and b: one product of the joined weight when it exists, its output
    // rows z | a | b (each part from a 16-row tile on), else three products
    const float *za = p->z, *aa = p->ab, *ba = p->ab + n * lh;
    int z_ld = (int)(lh * kLd), ab_ld = (int)lh;
    if (L.zab) {
        z_ld = ab_ld = weight_of(L.zab).rows;
        aa = p->z + lh * kLd;
        ba = aa + (lh + 15) / 16 * 16;
    }
    p->trace.a = aa;
    p->trace.b = ba;
    p->trace.z_ld = z_ld;
    p->trace.ab_ld = ab_ld;
    if (codes) {  // the input projections share the norm's codes
        rc = normed_product(ctx, p, L.qkv, true, flag, n, p->wide);
        if (L.zab) {
            if (!rc) rc = normed_product(ctx, p, L.zab, true, flag, n, p->z);
        } else {
            if (!rc) rc = normed_product(ctx, p, L.z, true, flag, n, p->z);
            if (!rc) rc = normed_product(ctx, p, L.a, true, flag, n, p->ab);
            if (!rc) rc = normed_product(ctx, p, L.b, true, flag, n, p->ab + n * lh);
        }
    } else if (L.zab) {
        rc = dz_linear_pair(ctx, L.qkv, L.zab, p->normed, n, p->wide, p->z, DZ_W4A8);
    } else {
        rc = dz_linear_pair(ctx, L.qkv, L.z, p->normed, n, p->wide, p->z, DZ_W4A8);
        if (!rc) rc = dz_linear_pair(ctx, L.a, L.b, p->normed, n, p->ab, p->ab + n * lh, DZ_W4A8);
    }
    if (rc) return rc;
    // cw is a multiple of kLd (128), so of 4; rows of p->wide, L.conv and p->conv_out are 16-byte aligned
    static_assert(kLd % 4 == 0, "whole float4 columns");
    hipLaunchKernelGGL(conv_silu_kernel, dim3(blocks_of(cw / 4, 256), (unsigned)n), dim3(256), 0, s, p->wide, (int)n,
                       (int)cw, L.conv, p->conv_out);
    hipLaunchKernelGGL(delta_prep_kernel, dim3((unsigned)n), dim3(64 * c.delta_key_heads), 0, s, p->conv_out,
                       c.delta_heads, c.delta_key_heads, aa, ba, ab_ld, L.decay, L.dt, p->qhat, p->khat, p->gb);
    launch_delta_scan(ctx, p, n, s);
    // out_proj adds onto the hidden rows in its epilogue; then the gate hands it
    // A8 codes (in the MLP's code buffer, free until the MLP) instead of f32 rows
    if (n > 16 && (size_t)c.ff >= lh * kLd &&
        grouped_adds_residual(weight_of(L.out), (int)n, ctx_variant(ctx, "grouped"))) {
        int *gflag = nullptr;
        rc = ctx_product_flag(ctx, &gflag);
        if (rc) return rc;
        hipLaunchKernelGGL(delta_gate_kernel<true>, dim3((unsigned)n, c.delta_heads), dim3(64), 0, s, p->heads,
                           (int)n, c.delta_heads, L.norm, za, z_ld, nullptr, p->codes, p->code_scales, gflag);
        p->trace.gate_codes = true;
        return product_add(ctx, L.out, nullptr, p->codes, p->code_scales, n, p->hidden, p->projected, gflag);
    }
    hipLaunchKernelGGL(delta_gate_kernel<false>, dim3((unsigned)n, c.delta_heads), dim3(64), 0, s, p->heads, (int)n,
                       c.delta_heads, L.norm, za, z_ld, p->ctx, nullptr, nullptr, nullptr);
    p->trace.gate_f32 = true;
    return product_add(ctx, L.out, p->ctx, nullptr, nullptr, n, p->hidden, p->projected);
}

// The MFMA kernel for query-head groups of up to 8 (the reference's 4) and
// K/V byte offsets within 32 bits; the one-wave-per-query kernel otherwise.
void launch_attention(dz_ctx *ctx, dz_pplx *p, size_t nq, size_t n, hipStream_t s) {
    const dz_pplx_config &c = p->cfg;
    const size_t kvw = (size_t)c.attn_kv_heads * kAd;
    const int group = c.attn_heads / c.attn_kv_heads;
    if (group <= kAttnMaxGroup && n * kvw * sizeof(float) < ((size_t)1 << 31)) {
        static bool configured[64] = {};  // the LDS limit is a per-device function attribute
        int dev = 0;
        hipGetDevice(&dev);
        if (dev >= 0 && dev < 64 && !configured[dev]) {
            if (hipFuncSetAttribute((const void *)attention_mfma_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                kAttnLds) == hipSuccess) configured[dev] = true;
        }
        hipLaunchKernelGGL(attention_mfma_kernel, dim3((unsigned)((nq + 15) / 16), c.attn_kv_heads),
                           dim3(64 * group), kAttnLds, s, p->query, p->key, p->value, kvw, (int)nq, (int)n,
                           c.attn_heads, c.attn_kv_heads, 1.0f / 16.0f, p->heads);
        return;
    }
    (void)ctx;
    const size_t lds = (kAd + n) * sizeof(float);
    hipLaunchKernelGGL(attention_kernel, dim3(c.attn_heads, (unsigned)nq), dim3(64), lds, s, p->query, p->key,
                       p->value, kvw, (int)nq, (int)n, c.attn_heads, c.attn_kv_heads, 1.0f / 16.0f, p->heads);
}

// backbone.rs:471-615; with `markers` (count rows) the queries and the
// hidden rows are cut to the markers (the reference's prune_last).
int32_t attention_layer(dz_ctx *ctx, dz_pplx *p, const dz_pplx::Layer &L, size_t n, const int32_t *markers,
                        size_t count, size_t *rows_out) {
    const dz_pplx_config &c = p->cfg;
    hipStream_t s = ctx_stream(ctx);
    const size_t d = c.hidden, kvw = (size_t)c.attn_kv_heads * kAd, qw = 2 * (size_t)c.attn_heads * kAd;
    bool codes = false;
    int *flag = nullptr;
    int32_t rc = layer_norm(ctx, p, L.input_norm, n, markers != nullptr, &codes, &flag);
    if (rc) return rc;
    if (codes) {
        rc = normed_product(ctx, p, L.k, true, flag, n, p->key);
        if (!rc) rc = normed_product(ctx, p, L.v, true, flag, n, p->value);
    } else {
        rc = dz_linear_pair(ctx, L.k, L.v, p->normed, n, p->key, p->value, DZ_W4A8);
    }
    if (rc) return rc;
    const size_t nq = markers ? count : n;
    if (markers) {  // the marker rows' queries from their normed rows
        hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_of(count * d, 256)), dim3(256), 0, s, p->normed, markers,
                           (int)count, (int)d, p->picked);
        rc = linear(ctx, L.q, p->picked, nq, p->wide);
    } else {
        rc = normed_product(ctx, p, L.q, codes, flag, n, p->wide);
    }
    if (rc) return rc;
    // queries: [q | z] per head; keys in place
    hipLaunchKernelGGL(head_norm_rope_kernel, dim3((unsigned)nq, c.attn_heads), dim3(64), 0, s, p->wide, qw, 2 * kAd,
                       c.attn_heads, L.qnorm, markers, p->freq, p->query);
    hipLaunchKernelGGL(head_norm_rope_kernel, dim3((unsigned)n, c.attn_kv_heads), dim3(64), 0, s, p->key, kvw, kAd,
                       c.attn_kv_heads, L.knorm, nullptr, p->freq, p->key);
    launch_attention(ctx, p, nq, n, s);
    const dim3 gate_blocks((unsigned)c.attn_heads, (unsigned)nq);  // head, token
    if (!markers && n > 16 && (size_t)c.ff >= (size_t)c.attn_heads * kAd &&
        grouped_adds_residual(weight_of(L.o), (int)n, ctx_variant(ctx, "grouped"))) {
        // as in the delta layer: o_proj reads A8 codes from the MLP's code buffer
        int *gflag = nullptr;
        rc = ctx_product_flag(ctx, &gflag);
        if (rc) return rc;
        hipLaunchKernelGGL(attention_gate_kernel<true>, gate_blocks, dim3(kAd), 0, s, p->heads, (int)nq,
                           c.attn_heads, p->wide + kAd, qw, 2 * kAd, nullptr, p->codes, p->code_scales, gflag);
        p->trace.gate_codes = true;
        rc = product_add(ctx, L.o, nullptr, p->codes, p->code_scales, nq, p->hidden, p->projected, gflag);
        if (rc) return rc;
        *rows_out = nq;
        return DZ_OK;
    }
    hipLaunchKernelGGL(attention_gate_kernel<false>, gate_blocks, dim3(kAd), 0, s, p->heads, (int)nq,
                       c.attn_heads, p->wide + kAd, qw, 2 * kAd, p->ctx, nullptr, nullptr, nullptr);
    p->trace.gate_f32 = true;
    if (markers) {  // the residual rows of the markers, before o_proj adds onto them
        hipLaunchKernelGGL(gather_rows_kernel, dim3(blocks_of(count * d, 256)), dim3(256), 0, s, p->hidden, markers,
                           (int)count, (int)d, p->picked);
        hipError_t e = hipMemcpyAsync(p->hidden, p->picked, count * d * sizeof(float), hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx prune");
    }
    rc = product_add(ctx, L.o, p->ctx, nullptr, nullptr, nq, p->hidden, p->projected);
    if (rc) return rc;
    *rows_out = nq;
    return DZ_OK;
}

}  // namespace

// Layer `index` on hidden rows already in p->hidden (tests and the forward).
void trace_reset(dz_pplx *p, int index, bool attention, size_t n) {
    p->trace = dz_pplx::Trace{};
    p->trace.layer = index;
    p->trace.attention = attention;
    p->trace.n = n;
}

int32_t pplx_run_layer(dz_ctx *ctx, dz_pplx *p, int index, size_t n, const int32_t *markers, size_t count,
                       size_t *rows_out, int part = DZ_PPLX_WHOLE) {
    const auto &L = p->layers[index];
    auto &st = p->st;
    int32_t rc;
    if (st.on) {  // the layer's bank, then the next layer's copy behind it
        rc = stream_in(ctx, p, index);
        if (rc) return rc;
        hipError_t e = hipStreamWaitEvent(ctx_stream(ctx), st.copied[index % 2], 0);
        if (e != hipSuccess) return ctx_hip_fail(ctx, e, "layer weight wait");
        if (index + 1 < (int)p->layers.size()) {
            rc = stream_in(ctx, p, index + 1);
            if (rc) return rc;
        }
    }
    size_t rows = n;
    trace_reset(p, index, L.attention, n);
    if (part != DZ_PPLX_MLP) {
        p->trace.mixer = true;
        if (L.attention) {
            rc = attention_layer(ctx, p, L, n, markers, count, &rows);
        } else {
            rc = delta_layer(ctx, p, L, n);
        }
    } else {
        rc = DZ_OK;
    }
    p->trace.nq = rows;
    if (!rc && part != DZ_PPLX_MIXER) rc = mlp(ctx, p, L, rows);
    p->trace.rows = rows;
    if (st.on) {  // the bank is free again once this layer's kernels have run
        hipError_t e = hipEventRecord(st.done[index % 2], ctx_stream(ctx));
        if (!rc && e != hipSuccess) return ctx_hip_fail(ctx, e, "layer weight release");
    }
    if (rc) return rc;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx layer");
    *rows_out = rows;
    return DZ_OK;
}

int32_t pplx_set_rows_form(dz_ctx *ctx, dz_pplx *p, int32_t form) {
    if (!p) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (form != DZ_ROWS_PACKED && form != DZ_FIT_SCALED && form != DZ_FIT_NF4)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS,
                        "embedding rows are packed, scaled (MSE) or NF4 rows: affine rows carry offsets the row bytes "
                        "do not hold");
    p->rows_form = form;
    return DZ_OK;
}

int32_t pplx_set_residency(dz_ctx *ctx, dz_pplx *p, int32_t residency) {
    if (!p) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (residency != DZ_PPLX_RESIDENT && residency != DZ_PPLX_STREAMED)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS, "residency is DZ_PPLX_RESIDENT or DZ_PPLX_STREAMED");
    const bool streamed = residency == DZ_PPLX_STREAMED;
    if (streamed == p->st.on) return DZ_OK;
    hipError_t e = hipStreamSynchronize(ctx_stream(ctx));
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "stream synchronize");
    return streamed ? stream_on(ctx, p) : stream_off(ctx, p);
}

int32_t pplx_residency_info(dz_ctx *ctx, dz_pplx *p, char *json, size_t cap) {
    if (!p) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    const auto &st = p->st;
    size_t resident = 0, joined = 0;
    for (const auto &L : p->layers) {
        for (dz_weight *w : projections(L))
            if (w) resident += weight_of(w).code_bytes + weight_of(w).scale_bytes;
        if (L.zab) joined += weight_of(L.zab).code_bytes + weight_of(L.zab).scale_bytes;
    }
    auto held = [&](int b) { return st.held[b] < 0 ? std::string("null") : std::to_string(st.held[b]); };
    std::string s = "{\"residency\":\"" + std::string(st.on ? "streamed" : "resident") + "\"";
    s += ",\"layer_weight_bytes\":" + std::to_string(resident);
    s += ",\"device_layer_weight_bytes\":" + std::to_string(st.on ? 2 * st.bank_bytes : resident + joined);
    s += ",\"host_layer_weight_bytes\":" + std::to_string(st.host_bytes);
    s += ",\"banks\":" + std::to_string(st.on ? 2 : 0) + ",\"bank_bytes\":" + std::to_string(st.bank_bytes);
    s += ",\"bank_layers\":[" + held(0) + "," + held(1) + "]";
    s += ",\"layer_uploads\":" + std::to_string(st.uploads) + ",\"bank_reuses\":" + std::to_string(st.reuses);
    s += ",\"upload_bytes\":" + std::to_string(st.upload_bytes) + ",\"max_in_flight_layers\":2}";
    if (!json || cap < s.size() + 1) return ctx_fail(ctx, DZ_RESOURCE_LIMIT, "info buffer too small");
    memcpy(json, s.c_str(), s.size() + 1);
    return DZ_OK;
}

int32_t pplx_layer(dz_ctx *ctx, dz_pplx *p, int index, float *hidden, size_t n, const int32_t *markers_host,
                   size_t count, int part) {
    if (!p || !hidden) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (part != DZ_PPLX_WHOLE && part != DZ_PPLX_MIXER && part != DZ_PPLX_MLP)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS, "unknown layer part");
    if (part == DZ_PPLX_MLP && markers_host)
        return ctx_fail(ctx, DZ_INVALID_REQUEST, "markers cut the mixer's rows: the MLP half takes none");
    if (index < 0 || index >= p->cfg.layers) return ctx_fail(ctx, DZ_INVALID_REQUEST, "layer index out of range");
    if (n == 0 || n > (size_t)kMaxKeys) return ctx_fail(ctx, DZ_INPUT_TOO_LONG, "sequence length outside 1..8192");
    std::string missing;
    if (!complete(p, &missing)) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "missing pplx weights: " + missing);
    const auto &L = p->layers[index];
    if (markers_host && !L.attention) return ctx_fail(ctx, DZ_INVALID_REQUEST, "cannot prune a recurrent layer");
    if (markers_host && (count == 0 || count > (size_t)DZ_READOUT_MAX_MARKERS))
        return ctx_fail(ctx, DZ_INVALID_REQUEST, "marker count outside 1..256");
    for (size_t i = 0; markers_host && i < count; i++)
        if (markers_host[i] < 0 || (size_t)markers_host[i] >= n)
            return ctx_fail(ctx, DZ_INVALID_REQUEST, "readout marker outside the sequence");
    int32_t rc = ensure_capacity(ctx, p, n);
    if (rc) return rc;
    hipStream_t s = ctx_stream(ctx);
    const size_t d = p->cfg.hidden;
    hipError_t e = hipMemcpyAsync(p->hidden, hidden, n * d * 4, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess && markers_host)
        e = hipMemcpyAsync(p->markers, markers_host, count * 4, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx layer input");
    size_t rows = n;
    rc = pplx_run_layer(ctx, p, index, n, markers_host ? p->markers : nullptr, count, &rows, part);
    if (rc) return rc;
    e = hipMemcpyAsync(hidden, p->hidden, rows * d * 4, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx layer output");
    return DZ_OK;
}

// A copy of the activation `name` that the last layer call left (rows of
// `width` bytes, `pitch` apart in the model's buffer) into out_dev.
int32_t pplx_activation(dz_ctx *ctx, dz_pplx *p, const char *name, void *out, size_t bytes) {
    if (!p || !name || !out) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    const auto &t = p->trace;
    if (t.layer < 0) return ctx_fail(ctx, DZ_INVALID_REQUEST, "no layer has run");
    const dz_pplx_config &c = p->cfg;
    const size_t d = c.hidden, cw = conv_width(c), lh = c.delta_heads, lv = lh * kLd;
    const size_t ah = c.attn_heads, qw = 2 * ah * kAd, kvw = (size_t)c.attn_kv_heads * kAd;
    const size_t gw = t.attention ? ah * kAd : lv;  // the gate's width
    const std::string nm(name);
    const void *src = nullptr;
    size_t width = 0, pitch = 0, rows = 0;
    bool ok = true;
    auto set = [&](const void *ptr, size_t row_bytes, size_t count, size_t row_pitch, bool valid) {
        src = ptr;
        width = row_bytes;
        rows = count;
        pitch = row_pitch ? row_pitch : row_bytes;
        ok = valid;
    };
    if (nm == "hidden") set(p->hidden, d * 4, t.rows, 0, true);
    else if (nm == "norm_codes") set(p->ncodes, d, t.n, 0, t.norm_codes);
    else if (nm == "norm_scales") set(p->nscales, d / 64 * 4, t.n, 0, t.norm_codes);
    else if (nm == "normed") set(p->normed, d * 4, t.n, 0, t.normed);
    else if (nm == "gate_codes") set(p->codes, gw, t.nq, 0, t.gate_codes);
    else if (nm == "gate_scales") set(p->code_scales, gw / 64 * 4, t.nq, 0, t.gate_codes);
    else if (nm == "gate") set(p->ctx, gw * 4, t.nq, 0, t.gate_f32);
    else if (nm == "mlp_codes") set(p->codes, (size_t)c.ff, t.rows, 0, t.mlp_codes);
    else if (nm == "mlp_scales") set(p->code_scales, (size_t)c.ff / 64 * 4, t.rows, 0, t.mlp_codes);
    else if (!t.attention && nm == "qkv") set(p->wide, cw * 4, t.n, 0, t.mixer);
    else if (!t.attention && nm == "z") set(p->z, lv * 4, t.n, (size_t)t.z_ld * 4, t.mixer && t.z_ld > 0);
    else if (!t.attention && nm == "a") set(t.a, lh * 4, t.n, (size_t)t.ab_ld * 4, t.mixer && t.a != nullptr);
    else if (!t.attention && nm == "b") set(t.b, lh * 4, t.n, (size_t)t.ab_ld * 4, t.mixer && t.b != nullptr);
    else if (!t.attention && nm == "conv") set(p->conv_out, cw * 4, t.n, 0, t.mixer);
    else if (!t.attention && nm == "heads") set(p->heads, kLd * 4, lh * t.n, 0, t.mixer);
    else if (t.attention && nm == "q") set(p->wide, qw * 4, t.nq, 0, t.mixer);
    else if (t.attention && nm == "query") set(p->query, ah * kAd * 4, t.nq, 0, t.mixer);
    else if (t.attention && nm == "key") set(p->key, kvw * 4, t.n, 0, t.mixer);
    else if (t.attention && nm == "value") set(p->value, kvw * 4, t.n, 0, t.mixer);
    else if (t.attention && nm == "heads") set(p->heads, kAd * 4, ah * t.nq, 0, t.mixer);
    else return ctx_fail(ctx, DZ_INVALID_PARAMETERS, "unknown activation for this layer: " + nm);
    if (!ok) return ctx_fail(ctx, DZ_INVALID_REQUEST, "the last layer call did not produce " + nm);
    if (bytes != width * rows)
        return ctx_fail(ctx, DZ_INVALID_PARAMETERS,
                        nm + " holds " + std::to_string(width * rows) + " bytes, not " + std::to_string(bytes));
    hipStream_t s = ctx_stream(ctx);
    hipError_t e = hipMemcpy2DAsync(out, width, src, pitch, width, rows, hipMemcpyDeviceToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx activation copy");
    return DZ_OK;
}

int32_t pplx_forward_rows(dz_ctx *ctx, dz_pplx *p, const void *rows_host, size_t n, const int32_t *markers,
                          size_t count, float *logits_host) {
    if (!p || !rows_host || !markers || !logits_host) return ctx_fail(ctx, DZ_INVALID_REQUEST, "null pointer");
    if (n == 0 || n > (size_t)kMaxKeys) return ctx_fail(ctx, DZ_INPUT_TOO_LONG, "sequence length outside 1..8192");
    if (count == 0 || count > (size_t)DZ_READOUT_MAX_MARKERS)
        return ctx_fail(ctx, DZ_INVALID_REQUEST, "marker count outside 1..256");
    for (size_t i = 0; i < count; i++)
        if (markers[i] < 0 || (size_t)markers[i] >= n)
            return ctx_fail(ctx, DZ_INVALID_REQUEST, "readout marker outside the sequence");
    std::string missing;
    if (!complete(p, &missing)) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "missing pplx weights: " + missing);
    int32_t rc = ensure_capacity(ctx, p, n);
    if (rc) return rc;
    hipStream_t s = ctx_stream(ctx);
    const size_t d = p->cfg.hidden;
    // embedding rows: the packed wire rows, unpacked exactly (packed.rs:59-73)
    hipError_t e = hipMemcpyAsync(p->rows_dev, rows_host, n * (d / 64) * 36, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(p->markers, markers, count * 4, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx input upload");
    p->rows_weight.rows = (int)n;
    p->rows_weight.fitted = p->rows_form != DZ_ROWS_PACKED;
    p->rows_weight.nf4 = p->rows_form == DZ_FIT_NF4;  // quantized_rows.rs:98-102
    int bad = 0;
    launch_fill_i32(ctx_flag(ctx), 0, 1, s);
    launch_upload(p->rows_weight, p->rows_dev, ctx_flag(ctx), s, p->rows_weight.fitted);
    launch_dequant(p->rows_weight, nullptr, (int)n, p->hidden, 0, s);
    e = hipMemcpyAsync(&bad, ctx_flag(ctx), sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx input upload");
    if (bad) return ctx_fail(ctx, DZ_INVALID_CHECKPOINT, "invalid packed scale");
    size_t rows = n;
    const int last = p->cfg.layers - 1;
    const bool prune = p->layers[last].attention;  // mod.rs prune_last (a recurrent last layer is not cut)
    for (int i = 0; i < p->cfg.layers; i++) {
        rc = pplx_run_layer(ctx, p, i, rows, prune && i == last ? p->markers : nullptr, count, &rows);
        if (rc) return rc;
    }
    // backbone.rs:247-249: the hidden state stays finite
    launch_fill_i32(ctx_flag(ctx), 0, 1, s);
    launch_flag_nonfinite(p->hidden, rows * d, ctx_flag(ctx), 1, s);
    e = hipMemcpyAsync(&bad, ctx_flag(ctx), sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "pplx forward");
    if (bad) return ctx_fail(ctx, DZ_INFERENCE_FAILED, "non-finite hidden state");
    // mod.rs:149-185: rows are the markers' (pruned) or selected here
    const int32_t *select = prune ? nullptr : p->markers;
    rc = ctx_readout_rows(ctx, weight_of(p->readout), p->final_norm, p->hidden, 0, select, count, DZ_READOUT_EPS,
                          p->logits);
    if (rc) return rc;
    e = hipMemcpyAsync(logits_host, p->logits, count * (size_t)DZ_READOUT_CODES * 4, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return ctx_hip_fail(ctx, e, "logits readback");
    return DZ_OK;
}

}  // namespace dz
