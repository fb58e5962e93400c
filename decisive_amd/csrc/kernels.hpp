// kernels.hpp -- host-side launchers of the HIP kernels (internal to the library).
#pragma once

#include "common.hpp"

namespace dz {

// ---- quant.hip ----------------------------------------------------------------
// Wire layout -> native layout; sets *bad (device int) when a scale is not
// finite and positive (fitted: not finite and nonzero).
void launch_upload(const Weight &w, const uint8_t *wire, int *bad, hipStream_t s, bool fitted = false);
// Device quantizer from f32/f16/bf16 values (dtype 0/1/2); sets *bad on a
// non-finite weight.
void launch_quantize_weight(const Weight &w, const void *values, int dtype, int *bad,
                            hipStream_t s);
// y [rows x cols] f32 (or f16 when dtype == 1) of rows ids (nullptr = all rows).
void launch_dequant(const Weight &w, const int32_t *ids, int count, void *y, int dtype,
                    hipStream_t s);
// As launch_dequant; ids outside [0, rows) give zero rows and set *bad.
void launch_dequant_checked(const Weight &w, const int32_t *ids, int count, void *y, int dtype,
                            int *bad, hipStream_t s);
// Native Q4 group-64 -> the packed.rs wire layout for every row (device buffer).
void launch_export_q4g64(const Weight &w, uint8_t *wire, hipStream_t s);
// int8.rs:178-202 prepare: q [m x G*64], s [m x G]; sets *bad on non-finite x.
void launch_act_quantize(const float *x, int m, int k, int bits, int8_t *q, float *sc, int *bad,
                         hipStream_t s);
// sxq [m x groups] = sx * f32(sum of each group's 64 codes): the affine offset
// term's activation factor (int8.rs:568-569).
void launch_act_sums(const int8_t *q, const float *sx, int m, int groups, float *sxq, hipStream_t s);
// grouped_q4.rs:3-25: the same codes and scales as 17-word records per group.
void launch_act_quantize_records(const float *x, int m, int k, uint32_t *records, int *bad,
                                 hipStream_t s);
// pplx_flash/cpu.rs:310-333 zero-centred RMSNorm (the readout norm's bits)
// of f32 rows h [rows x d] (d % 64 == 0, d <= kRmsQuantizeMaxCols) into y
// (may be null) and the A8 codes q / scales sc of the normed rows, equal to
// act_quantize of y; sets *bad (may be null) on a non-finite normed value.
constexpr int kRmsQuantizeMaxCols = 8192;
void launch_rms_quantize(const float *h, int rows, int d, const float *w, float eps, int zero_centered, float *y,
                         int8_t *q, float *sc, int *bad, hipStream_t s);
// webgpu/int8.rs:107-145.
void launch_i8_quantize_rows(const float *x, int rows, int k, int8_t *q, float *scales,
                             int32_t *sums, hipStream_t s);
// webgpu/q4.rs:48-73: per-row Q4 into the word buffer [rows*(k/8) | scales | sums].
void launch_q4_quantize_rows(const void *values, int dtype, int rows, int k, uint32_t *out, int *bad,
                             hipStream_t s);
void launch_fill_i32(int *p, int value, int count, hipStream_t s);

// ---- products.hip --------------------------------------------------------------
// Grouped W{4,8}A{8,4}: bit-exact AVX2 order. bad (may be null): NaN outputs.
// With `res` (which may equal y) the product is added onto it in the kernel;
// only for the cases grouped_adds_residual accepts. Returns false when no
// kernel was launched (a residual product that neither a pipelined kernel
// nor the few-row kernel takes).
bool grouped_adds_residual(const Weight &w, int m, int variant);
// Fitted affine weights (w.offsets) take sxq [m x groups] (launch_act_sums).
bool launch_grouped(const Weight &w, const int8_t *q, const float *sx, int m, float *y,
                    const int *bad, int variant, hipStream_t s, const float *res = nullptr,
                    const float *sxq = nullptr);
// Few-row grouped products (any m; one launch, 16 rows per block row):
//  from f32 x quantized in the kernel (m <= 16 keeps the all-NaN semantics of
//  a non-finite x; bad_out, may be null, is set when x holds one);
void launch_grouped_small(const Weight &w, const float *x, int m, int abits, float *y, int *bad_out,
                          bool project, hipStream_t s);
//  from int8 codes + f32 scales (bad_in, may be null: NaN outputs when set);
void launch_grouped_codes(const Weight &w, const int8_t *q, const float *sx, int m, float *y,
                          const int *bad_in, bool project, hipStream_t s);
//  from the 17-word A8 records of grouped_q4.rs:3-25.
void launch_grouped_records(const Weight &w, const uint32_t *records, int m, float *y, hipStream_t s);
// W4A16: y [m x N] f32 from x f16 [m x K].
void launch_w4a16(const Weight &w, const half_t *x, int m, float *y, int gemv_variant,
                  int gemm_variant, hipStream_t s);
// W4A16 with f16 output and optional fused epilogue (0 none, 1 GELU, 2 +residual f16)
void launch_w4a16_f16(const Weight &w, const half_t *x, int m, half_t *y, int epilogue,
                      const half_t *residual, int variant, hipStream_t s);
// Per-row int8 GEMM: raw int32 or f32 epilogue. With b_q4, b is the per-row Q4
// word buffer of launch_q4_quantize_rows (codes expanded to int8 in registers).
void launch_i8_gemm(const int8_t *a, const float *sa, int m, const int8_t *b, const float *sb,
                    int n, int k, void *y, int raw, int variant, hipStream_t s, bool b_q4 = false);
// webgpu/int8.rs:226-230 gemm(fused=true): y = silu(gate) * up of two per-row int8 products sharing a
void launch_i8_gemm_fused(const int8_t *a, const float *sa, int m, const int8_t *wg, const float *sg,
                          const int8_t *wu, const float *su, int n, int k, float *y, hipStream_t s);
// Fused gate/up W4A8 + SiLU + A8 requantization (grouped_q4_mlp.wgsl).
void launch_mlp_requant(const Weight &gate, const Weight &up, const int8_t *q, const float *sx,
                        int m, int8_t *qo, float *so, const int *bad, int variant, hipStream_t s);

// ---- epilogue.hip ----------------------------------------------------------------
void launch_layernorm(const void *x, void *y, int dtype, int rows, int d, const float *w,
                      const float *b, float eps, hipStream_t s);
void launch_rmsnorm(const float *x, float *y, int rows, int d, const float *w, float eps,
                    int zero_centered, hipStream_t s);
// Readout RMSNorm over n selected rows of h (f32 dtype 0 / f16 dtype 1; rows
// null = the first n rows) into y f32 [n x d]; d <= kReadoutMaxCols.
constexpr int kReadoutMaxCols = 16384;
void launch_readout_rms(const void *h, int dtype, const int32_t *rows, int n, int d, const float *w,
                        float eps, int zero_centered, float *y, hipStream_t s);
void launch_flag_nonfinite(const float *y, size_t n, int *flag, int bit, hipStream_t s);
// y f16 [n] = epilogue(v) (0 none, 1 GELU, 2 + res), rounded once
void launch_f16_epilogue(const float *v, int epi, const half_t *res, half_t *y, size_t n, hipStream_t s);
// y f32 [n] = x (f32 dtype 0 / f16 dtype 1), exact
void launch_to_f32(const void *x, int dtype, size_t n, float *y, hipStream_t s);
void launch_gelu(void *x, int dtype, size_t n, hipStream_t s);
void launch_silu_mul(float *g, const float *u, size_t n, hipStream_t s);
void launch_add(void *x, const void *y, int dtype, size_t n, hipStream_t s);
void launch_softmax_rows(float *x, int rows, int n, hipStream_t s);
void launch_mean_rows(const void *x, int dtype, int batch, int rows, int d, float *out,
                      hipStream_t s);
// The attention kernel addresses one sequence of qkv rows with 32-bit byte
// offsets: (seq + 64) * 3 * heads * 64 halves must stay below 2^31 bytes.
inline bool attention_fits(size_t seq, size_t heads) {
    return (seq + 64) * 3 * heads * 64 * 2 < ((size_t)1 << 31);
}
void launch_attention(const half_t *qkv, half_t *out, int batch, int seq, int heads, int dh,
                      float scale, hipStream_t s);
void launch_fill_normal_f32(float *p, size_t n, uint64_t seed, float stddev, hipStream_t s);
void launch_fill_f32(float *p, size_t n, float v, hipStream_t s);

// Compute units of the current device (cached per device).
int device_cus();

// The decider's gated delta scan (pplx.hip): token by token (rolled: the
// 16-token stages as a loop) and by 64-token chunks (column_tiles 1 or 2:
// 16 or 32 state columns per block; ws holds delta_chunk_ws_bytes).
void launch_delta_scan_tokens(const float *qhat, const float *khat, const float *conv, const float *gb, int n,
                              int lh, int lk, float *out, bool rolled, hipStream_t s);
size_t delta_chunk_ws_bytes(int n, int lh);
void launch_delta_scan_chunked(const float *qhat, const float *khat, const float *conv, const float *gb, int n,
                               int lh, int lk, float *ws, float *out, int column_tiles, hipStream_t s);

// ---- variants (tuner) --------------------------------------------------------------
struct VariantFamily {
    const char *family;
    const char *const *names;
    int count;
};
int variant_count(const char *family);
// Variants the tuner may choose among (the first `tuned_count`, all bitwise
// equal to variant 0); the rest are explicit opt-ins.
int tuned_count(const char *family);
const char *variant_name(const char *family, int index);
int variant_index(const char *family, const char *name);

}  // namespace dz
