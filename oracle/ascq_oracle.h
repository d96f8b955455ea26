/*
 * ascq_oracle.h -- CPU restatement of the asc-devkit quantized-inference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is what the tests compare the HIP product
 * path against, and the CPU baseline timed by bench.py.  Only tests/, the smoke check in
 * __graft_entry__.py and bench.py's cpu_baseline leg may load it.  The product
 * library (libascq.so) never links, loads or calls it, and has no CPU fallback.
 *
 * Every function cites the reference file:line whose arithmetic it restates
 * (paths relative to the asc-devkit source tree).  Numeric conventions:
 *   - f16 / bf16 values travel as their raw uint16_t bit patterns;
 *   - "rne" = IEEE round-to-nearest-even, "sat" = clamp to the finite range of
 *     the destination type (NaN is kept as NaN);
 *   - every fp32 operation is a single IEEE fp32 operation (the library is
 *     compiled with -ffp-contract=off so that mul+add never fuses into an fma).
 *
 * Pinning (what checks each function besides the HIP path) is listed in
 * tests/test_oracle.py; a function whose only check is the restatement itself
 * is marked "parity unpinned" below.
 */
#ifndef ASCQ_ORACLE_H
#define ASCQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: identical to ascq_dtype in include/ascq.h */
enum {
    OQ_INT8 = 1, OQ_UINT8 = 2, OQ_INT4 = 3, OQ_INT32 = 4, OQ_F16 = 5, OQ_BF16 = 6,
    OQ_F32 = 7, OQ_U64 = 8, OQ_FP8_E4M3 = 9, OQ_FP8_E5M2 = 10, OQ_FP4_E2M1 = 11, OQ_E8M0 = 12, OQ_INT64 = 13,
    OQ_FP4_E1M2 = 14, OQ_HIF8 = 15
};
/* RoundMode: impl/basic_api/utils/kernel_utils_mode.h:103-118 (CAST_NONE acts as CAST_RINT on lossy casts,
 * docs/zh/api/SIMD-API/basic_api/memory_vector_compute/type_conversion/Cast.md:92) */
enum { OQ_ROUND_NONE = 0, OQ_ROUND_RINT = 1, OQ_ROUND_FLOOR = 2, OQ_ROUND_CEIL = 3, OQ_ROUND_ROUND = 4, OQ_ROUND_TRUNC = 5 };
/* quant / dequant policies: include/adv_api/quantization/ascend_quant_utils.h:74-81 plus the legacy
 * per-tensor / per-channel entry points of ascend_quant.h:64-293 and ascend_dequant.h:59-285 */
enum { OQ_PER_TENSOR = 0, OQ_PER_CHANNEL = 1, OQ_PER_TOKEN = 2, OQ_PER_GROUP = 3 };
/* antiquant arithmetic: fp16 ops (ascend_antiquant_impl.h:63-96, arch 2201) or fp32 ops
 * (ascend_antiquant_c220_impl.h:46-75 bf16 path; ascend_antiquant_3510_impl.h:320-330) */
enum { OQ_ARITH_F16 = 0, OQ_ARITH_F32 = 1, OQ_ARITH_BF16 = 2 };

/* ---------------- scalar codecs ---------------- */
/* HiFloat8: value of a code (NaN for 0x80, +-inf for 0x6F / 0xEF) and the code of x with ties away from zero
 * (CAST_ROUND); sat != 0 maps NaN to 0 and every overflow to +-32768 (0x6E / 0xEE) */
float oq_hif8_decode(uint8_t code);
uint8_t oq_hif8_encode(float x, int sat);
uint16_t oq_f32_to_f16(float x, int sat);
float oq_f16_to_f32(uint16_t h);
uint16_t oq_f32_to_bf16(float x, int sat);
float oq_bf16_to_f32(uint16_t h);
uint16_t oq_f64_to_f16(double d, int sat);
uint16_t oq_f64_to_bf16(double d, int sat);
/* M1 field of a QUANT_PRE word: bits [31:13] read as an fp32 with the low 13 mantissa bits cleared
 * (docs/zh/api/SIMD-API/c_api/cube_datamove/cube_store_key_features/accompanying_quantization.md:79-103;
 * examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_quant/scripts/gen_data.py:35-39 mask 0xFFFFE000) */
float oq_quant_pre_m1(uint64_t word);
uint64_t oq_pack_quant_pre(float m1, int32_t offset9, int32_t sign);
int32_t oq_round_to_int(float v, int mode);
int8_t oq_sat_s8(int32_t v);
float oq_e2m1_decode(uint8_t nibble);
uint8_t oq_e2m1_encode_rne(float x);
float oq_e8m0_decode(uint8_t e);
uint8_t oq_mx_shared_exp(float amax);
float oq_fp8_decode(uint8_t v, int fmt);

/* ---------------- ops ---------------- */
/* int8 x int8 -> int32 (+ int32 bias), two's-complement wrap; A [M,K] (transA: [K,M]), B [K,N] (transB: [N,K]) */
void oq_matmul_i8(const int8_t* A, const int8_t* B, const int32_t* bias, int32_t* C,
                  int64_t M, int64_t N, int64_t K, int transA, int transB);
/* fixpipe dequant epilogue int32 -> f16 (DEQF16/VDEQF16) or bf16 (QS322BF16_PRE/VQS322BF16_PRE);
 * qvec != NULL selects the per-channel (vector) word qvec[n], else qscalar */
void oq_mm_dequant(const int32_t* acc, void* out, int out_type, int64_t M, int64_t N,
                   const uint64_t* qvec, uint64_t qscalar);
/* f32 -> fp8 (rne; e4m3fn saturating to +-448 with NaN -> 0, e5m2 overflowing to inf) */
uint8_t oq_f32_to_fp8(float x, int fmt);
/* REQ8 / QF322B8 after the multiply: clamp [-256, 255], rint, + 9-bit offset, saturate by the sign flag */
uint8_t oq_requant8(float v, uint64_t word);
uint8_t oq_requant4(float v, uint64_t word);
void oq_mm_requant4(const int32_t* acc, uint8_t* out, int64_t M, int64_t N, const uint64_t* qvec, uint64_t qscalar);
void oq_requant4_f32(const float* v, uint8_t* out, int64_t M, int64_t N, const uint64_t* qvec, uint64_t qscalar);
/* (V)REQ8: int32 -> int8 / uint8 with the word's M1, offset and sign flag */
void oq_mm_requant(const int32_t* acc, uint8_t* out, int64_t M, int64_t N, const uint64_t* qvec, uint64_t qscalar);
/* fp8 x fp8 (or hifloat8 x hifloat8) -> fp32 accumulate (exact products, double sum) -> the QF322*_PRE epilogues */
void oq_matmul_fp8(const uint8_t* A, const uint8_t* B, int a_fmt, int b_fmt, const float* bias, void* out,
                   int out_type, int64_t M, int64_t N, int64_t K, int transA, int transB, int use_q,
                   const uint64_t* qvec, uint64_t qscalar, double* exact_out, double* absdot_out,
                   double* blockmax_out);

/* AscendQuant PER_TOKEN (policy API): q = sat_s8(round(f32(x)*scale[row] (+offset[row]))) */
void oq_quant_per_token(int8_t* dst, const void* src, int src_type, const float* scale, const float* offset,
                        int64_t m, int64_t n, int round_mode);
/* dynamic per-token: absmax per row, multiplier 127/absmax, scale_out = absmax/127 */
void oq_quant_dynamic_per_token(int8_t* dst, float* scale_out, const void* src, int src_type,
                                int64_t m, int64_t n, int round_mode);
/* legacy AscendQuant, arch-3510 form: src f16 / bf16 / f32; dst int8 / hifloat8 (half arithmetic) or fp8
 * (fp32 arithmetic); scale / offset srcT tensors of scale_count, or (scale NULL) the float scalars; a scale tensor
 * with offset NULL takes offset_scalar rounded to srcT */
void oq_quant_legacy(void* dst, int dst_type, const void* src, int src_type, const void* scale, const void* offset,
                     float scale_scalar, float offset_scalar, int64_t cal_count, int64_t scale_count);
/* legacy AscendQuant per-tensor / per-channel in fp16 arithmetic */
void oq_quant_legacy_f16(int8_t* dst, const void* src, int src_type, const uint16_t* scale_vec,
                         uint16_t scale_scalar, const uint16_t* offset_vec, uint16_t offset_scalar,
                         int64_t cal_count, int64_t scale_count);
/* int32 -> fp32 rounding half away from zero (the dequant kernels' MrgZRndA cast); exact below 2^24 */
float oq_i32_to_f32_rna(int32_t v);
/* DeQuantMode (impl/basic_api/utils/kernel_utils_mode.h:193-196) */
enum { OQ_DEQUANT_SINGLE_ROW = 0, OQ_DEQUANT_MULTI_ROW = 1 };
/* Legacy AscendDequant, DequantParams{m, n, calCount} (ascend_dequant.h:38-291): the SINGLE_ROW reshape of
 * {1, m*n, n}, dst rows padded to 32 bytes, columns >= calCount not written; per_tensor selects the scalar
 * deqScale.  dst = cast(f32(src) * scale) (rne, sat). */
void oq_dequant_legacy(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                       float scale_scalar, int per_tensor, int mode, int64_t m, int64_t n, int64_t cal_count);
/* Row stride (elements) of the legacy form's dst after the SINGLE_ROW rule; also returns the effective m, n */
int64_t oq_dequant_legacy_shape(int dst_type, int mode, int64_t* m, int64_t* n, int64_t cal_count);
/* AscendDequant policy form (arch 3510): PER_TOKEN / PER_GROUP (kDim 0 / 1) over rows = calCount / n, int32 or
 * fp32 sources, f16 / bf16 / f32 scales; dst [rows, n] */
void oq_dequant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                       int policy, int k_dim, int64_t n, int64_t cal_count, int64_t group);
/* AscendAntiQuant per tensor: dst[i] = (src[i] + offset) * scale with dst-typed scalars (has_offset 0: scale only) */
void oq_antiquant_scalar(void* dst, int dst_type, const void* src, int src_type, uint16_t offset, uint16_t scale,
                         int has_offset, int64_t count);
/* AscendAntiQuant: dst = (src + offset) * scale, per-channel or per-group */
void oq_antiquant(void* dst, int dst_type, const void* src, int src_type, const void* offset, const void* scale,
                  int64_t K, int64_t N, int64_t group_size, int is_transpose, int arith);
/* AscendAntiQuant policy form (arch 3510): PER_TOKEN / PER_GROUP over [m, n]; int8 (scaleT arithmetic), fp8 (fp32
 * arithmetic) or fp4 E2M1 / E1M2 with E8M0 scales (bf16 product) sources */
void oq_antiquant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale, const void* offset,
                         int scale_type, int policy, int64_t m, int64_t n, int64_t group, int k_dim, int is_transpose);
/* E2M1 code of x in round mode `mode`, saturating at +-6, NaN -> 0 */
uint8_t oq_e2m1_encode(double x, int mode);
/* E1M2 (sign | 1-bit exponent, bias 1 | 2-bit mantissa): decode, and the code of x in round mode `mode`,
 * saturating at +-1.75, NaN -> 0 */
float oq_e1m2_decode(uint8_t nibble);
uint8_t oq_e1m2_encode(double x, int mode);
/* f32 -> fp8, rint + saturation (overflow and inf -> +-max finite, NaN -> 0) */
uint8_t oq_f32_to_fp8_sat(float x, int fmt);
/* AscendQuant policy form (arch 3510): PER_TOKEN / PER_GROUP over [m, n] to int8 (scaleT arithmetic), fp8 (fp32
 * arithmetic) or fp4 E2M1 / E1M2 (scaleT product -> bf16 -> fp4, PER_GROUP only); offset tensor, scalar or none.
 * Parity unpinned for two fp4 sub-cases only: the sign kept on a negative value that rounds to zero, and the
 * code 0 for a NaN bf16 product (no reference data covers either). */
void oq_quant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                     const void* offset, int has_offset, float offset_scalar, int policy, int64_t m, int64_t n,
                     int64_t group, int k_dim, int round_mode);
/* Quantize (the newer interface): PER_TENSOR (scalar scale / offset), PER_CHANNEL, PER_TOKEN, PER_GROUP over [m, n]
 * in fp32 arithmetic to int8 / fp8 / hifloat8 / fp4 (fp4 PER_GROUP only, packed [m, n/2]) */
void oq_quantize(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                 const void* offset, int has_offset, float scale_scalar, float offset_scalar, int policy, int64_t m,
                 int64_t n, int64_t group, int k_dim, int round_mode);
/* Dequantize (the newer interface): PER_TENSOR / PER_CHANNEL through the legacy AscendDequant (MULTI_ROW, {m, n, n}),
 * PER_TOKEN / PER_GROUP through the policy form; dst [m, n] */
void oq_dequantize(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                   float scale_scalar, int policy, int64_t m, int64_t n, int64_t group, int k_dim);
/* AntiQuantize (the newer interface): int8 / hifloat8 / fp8 sources in fp32 arithmetic for every policy (PER_TENSOR
 * scalars of the dst type); fp4 sources as the AscendAntiQuant policy form */
void oq_antiquantize(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                     const void* offset, int has_offset, float scale_scalar, float offset_scalar, int policy,
                     int64_t m, int64_t n, int64_t group, int k_dim);
/* weight-only antiquant matmul = AscendAntiQuant (fp16 ops) + fp16 matmul with fp32 accumulation.
 * Exact sum (double) -> f16; also returns the exact sum and sum |x*w| (for the accumulation bound) */
void oq_antiquant_matmul(uint16_t* y, double* y_exact, double* y_absdot, const uint16_t* x, const void* w,
                         int w_type, const uint16_t* scale, const uint16_t* offset, int64_t group_size,
                         int64_t M, int64_t N, int64_t K, int w_transpose);
/* FasterGelu x / (1 + exp(-1.702 x)) as fp32 ops (Muls, Exp, Adds, Div) */
float oq_faster_gelu(float x);
/* QuantGroupMatmul (MoE): per group g rows [s_g, e_g): y = cast(f32(f32(acc)*scale[g,n]) * pts[m]), with
 * act != 0 cast(FasterGelu(...)) */
void oq_group_matmul(void* y, int out_type, const int8_t* x, const float* pts, const int8_t* w, int w_trans,
                     const float* scale, const int64_t* group_list, int list_type, int64_t G, int64_t M,
                     int64_t K, int64_t N, int act);
/* MX block-scaled matmul (E2M1 or fp8 elements; elem_fmt = A format | B format << 8, B defaulting to A's),
 * fp64 dequant-then-matmul (reference golden) -> bf16 (rne) */
void oq_mx_matmul(uint16_t* C, double* C_exact, double* C_absdot, const uint8_t* A, const uint8_t* B,
                  const uint8_t* scaleA, const uint8_t* scaleB, int64_t M, int64_t N, int64_t K, int transB,
                  int scale_a_layout, int scale_b_layout, int elem_fmt, const int64_t* rows, int64_t n_rows,
                  double* C_blockmax, const float* bias);
/* IterateAll enAtomic: C = op(C, v) in C's type (op 1 add, 2 max, 3 min; c_type OQ_INT32 / F32 / F16 / BF16) */
void oq_c_combine(void* c, const void* v, int c_type, int op, int64_t count);
/* MX quantisation of fp32 data along K: one e8m0 per 32 elements, E2M1 elements (used to make inputs) */
void oq_mx_quantize_fp4(uint8_t* packed, uint8_t* scales, const float* x, int64_t R, int64_t K);

#ifdef __cplusplus
}
#endif
/* NZ fractal ([ceil(cols*esize/32)][ceil(rows/16)][16][32 bytes] per matrix) <-> ND, byte by byte */
void oq_nz_to_nd(uint8_t* dst, const uint8_t* src, int esize, int64_t batch, int64_t rows, int64_t cols,
                 int transpose_out);
void oq_nd_to_nz(uint8_t* dst, const uint8_t* src, int esize, int64_t batch, int64_t rows, int64_t cols);

#endif
