/*
 * ascq_oracle.c -- CPU restatement of the asc-devkit quantized-inference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the tests' reference results and bench.py's CPU baseline).  The
 * product library never links or calls this file.  See ascq_oracle.h for the
 * numeric conventions; each function below cites the reference lines it follows.
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off).
 */
#include "ascq_oracle.h"

#include <math.h>

/* Planted-mistake switches for tests/test_oracle_mutants.py, which compiles this file with -DOQ_MUTANT=n and
 * checks that the pinning tests reject every mutant.  0 (the default) is the oracle itself. */
#ifndef OQ_MUTANT
#define OQ_MUTANT 0
#endif
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------ */
/* scalar codecs                                                             */
/* ------------------------------------------------------------------------ */

/* IEEE binary32 -> binary16, round to nearest even.  sat != 0 clamps overflow (and +-inf) to +-65504,
 * the saturating conversion of docs/zh/api/SIMD-API/basic_api/data_structures/precision_conversion.md:30
 * ("overflow is handled in saturation mode by default") and the DEQF16 boundary rule of
 * docs/zh/api/appendix/matrix_compute_move_out_interface_boundary_value_summary.md:104. */
uint16_t oq_f32_to_f16(float x, int sat)
{
    uint32_t u = f2u(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* NaN, quieted */
    if (a >= 0x477ff000u) return (uint16_t)(sign | (sat ? 0x7bffu : 0x7c00u));    /* >= 65520 or inf */
    if (a >= 0x38800000u) {                                                       /* normal result */
        uint32_t r = a + 0xfffu + (OQ_MUTANT == 10 ? 1u : ((a >> 13) & 1u));
        return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
    }
    /* subnormal / zero result: |x| * 2^24 is exact; rint under the default (nearest-even) mode */
    float m = rintf(u2f(a) * 16777216.0f);
    return (uint16_t)(sign | (uint16_t)m); /* m == 1024 becomes the smallest normal, as it should */
}

float oq_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * (1.0f / 16777216.0f); /* exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* binary32 -> bfloat16, round to nearest even (CAST_RINT, ascend_dequant_common_impl.h:196-206) */
uint16_t oq_f32_to_bf16(float x, int sat)
{
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    if ((u & 0x7fffffffu) == 0x7f800000u) return (uint16_t)(sat ? ((u >> 16) & 0x8000u) | 0x7f7fu : (u >> 16));
    uint32_t r = u + 0x7fffu + ((u >> 16) & 1u);
    uint16_t b = (uint16_t)(r >> 16);
    if (sat && (b & 0x7fffu) == 0x7f80u) b = (uint16_t)((b & 0x8000u) | 0x7f7fu);
    return b;
}

float oq_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* binary64 -> binary16 / bfloat16 with one round-to-nearest-even (used where the exact value of a half op
 * or of an exact dot product is held in a double, so that no double rounding through fp32 occurs) */
uint16_t oq_f64_to_f16(double d, int sat)
{
    if (d != d) return 0x7e00u;
    uint16_t sign = signbit(d) ? 0x8000u : 0u;
    double a = fabs(d);
    if (a >= 65520.0) return (uint16_t)(sign | (sat ? 0x7bffu : 0x7c00u));
    int e;
    frexp(a, &e);              /* a in [2^(e-1), 2^e) */
    int q = e - 11;            /* ulp of an 11-bit significand in that binade */
    if (q < -24) q = -24;      /* subnormal spacing */
    double v = ldexp(nearbyint(ldexp(a, -q)), q);
    return (uint16_t)(sign | oq_f32_to_f16((float)v, 0)); /* v is a binary16 value: exact */
}

uint16_t oq_f64_to_bf16(double d, int sat)
{
    if (d != d) return 0x7fc0u;
    uint16_t sign = signbit(d) ? 0x8000u : 0u;
    double a = fabs(d);
    if (a >= ldexp(511.0, 119)) return (uint16_t)(sign | (sat ? 0x7f7fu : 0x7f80u)); /* (2-2^-8)*2^127 */
    int e;
    frexp(a, &e);
    int q = e - 8;
    if (q < -133) q = -133;
    double v = ldexp(nearbyint(ldexp(a, -q)), q);
    return (uint16_t)(sign | oq_f32_to_bf16((float)v, 0));
}

/* QUANT_PRE M1: bits 13..31 hold a (1,8,10) float; the low 13 bits do not take part
 * (accompanying_quantization.md:79-103, table "M1"; gen_data_s322f16.py:38-52 decodes the same field) */
float oq_quant_pre_m1(uint64_t word) { return u2f((uint32_t)(word & (OQ_MUTANT == 1 ? 0xFFFFFFFFu : 0xFFFFE000u))); }

/* host packing used by the reference sample: (uint64)(*(uint32*)&f) (matmul_quant.asc:111-113), plus the
 * 9-bit offset at bits 37..45 and the sign flag at bit 46 (accompanying_quantization.md table 1/2) */
uint64_t oq_pack_quant_pre(float m1, int32_t offset9, int32_t sign)
{
    return (uint64_t)f2u(m1) | ((uint64_t)((uint32_t)offset9 & 0x1ffu) << 37) | ((uint64_t)(sign & 1) << 46);
}

/* RoundMode semantics of Cast.md "RoundMode" table; NaN converts to 0, results clamp to int32 */
int32_t oq_round_to_int(float v, int mode)
{
    if (v != v) return 0;
    float r;
    switch (mode) {
    case OQ_ROUND_FLOOR: r = floorf(v); break;
    case OQ_ROUND_CEIL: r = ceilf(v); break;
    case OQ_ROUND_ROUND: r = roundf(v); break; /* half away from zero */
    case OQ_ROUND_TRUNC: r = truncf(v); break;
    default: r = OQ_MUTANT == 2 ? roundf(v) : rintf(v); break; /* NONE / RINT: half to even */
    }
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)r;
}

int8_t oq_sat_s8(int32_t v) { return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v)); }

/* OCP MX v1.0 E2M1: sign | 2-bit exponent (bias 1) | 1-bit mantissa; exact values
 * {0, .5, 1, 1.5, 2, 3, 4, 6} (precision_conversion.md "fp4x2_e2m1_t -> bfloat16_t": lossless) */
float oq_e2m1_decode(uint8_t nib)
{
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, OQ_MUTANT == 9 ? 2.5f : 3.0f, 4.0f, 6.0f};
    float v = mag[nib & 7u];
    return (nib & 8u) ? -v : v;
}

/* nearest E2M1 code, ties to the even code, saturating at 6 (OCP MX v1.0 section 5.3 conversion) */
uint8_t oq_e2m1_encode_rne(float x)
{
    uint8_t s = (f2u(x) >> 31) ? 8u : 0u;
    float a = fabsf(x);
    if (a != a) return 0;
    /* midpoints between consecutive magnitudes; at a tie pick the code with an even mantissa bit */
    static const float mid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
    uint8_t c = 0;
    while (c < 7 && a > mid[c]) ++c;
    if (c < 7 && a == mid[c] && (c & 1u)) ++c; /* tie: code c is odd -> go to c+1 (even) */
    return (uint8_t)(s | c);
}

/* E8M0: 2^(e-127); 0xFF is NaN (OCP MX v1.0 section 5.4) */
float oq_e8m0_decode(uint8_t e)
{
    if (e == 0xFFu) return u2f(0x7fc00000u);
    if (e == 0) return u2f(0x00400000u); /* 2^-127, a float subnormal */
    return u2f((uint32_t)e << 23);
}

/* shared exponent = floor(log2(amax)) - emax(E2M1)=2, clamped to [0,254]; amax == 0 gives 127 */
uint8_t oq_mx_shared_exp(float amax)
{
    if (!(amax > 0.0f)) return 127u;
    int e = (int)((f2u(amax) >> 23) & 0xffu);
    if (e == 0) return 0u; /* subnormal amax: floor(log2) - 2 is below the e8m0 range */
    int se = e - 2;
    if (se < 0) se = 0;
    if (se > 254) se = 254;
    return (uint8_t)se;
}

/* fp8: fmt OQ_FP8_E4M3 (e4m3fn: bias 7, no inf, 0x7f/0xff NaN) or OQ_FP8_E5M2 (bias 15, IEEE inf/NaN) */
/* HiFloat8 (impl/utils/debug/npu_arch_9201/asc_type_conversion_utils.h:62-149): bit 7 is the sign; a prefix-coded
 * dot field starting at bit 6 gives the exponent width w -- 11: 4, 10: 3, 01: 2, 001: 1, 0001: 0 -- and the
 * mantissa takes the 7 - |dot| - w bits left; a w-bit exponent field stores the exponent's sign in its top bit and
 * its magnitude with that bit replaced by an implicit 1 (so |E| lies in [2^(w-1), 2^w - 1]); value
 * (-1)^S 2^E (1 + M / 2^mw).  Dot 0000 is the subnormal class 2^(M - 23), M = 1..7 (M = 0: zero, or NaN with the
 * sign bit, 0x80); 0x6F / 0xEF (E = +15 with M = 1) are +-inf.  Largest finite 2^15 (0x6E), smallest 2^-22. */
float oq_hif8_decode(uint8_t code)
{
    if (code == 0x00u) return 0.0f;
    if (code == 0x80u) return NAN;
    if (code == 0x6Fu) return INFINITY;
    if (code == 0xEFu) return -INFINITY;
    const int neg = code >> 7;
    double v;
    if ((code & 0x78u) == 0) {
        v = ldexp(1.0, (int)(code & 7u) - 23);
    } else {
        int w, dw;
        if (code & 0x40u) w = (code & 0x20u) ? 4 : 3, dw = 2;
        else if (code & 0x20u) w = 2, dw = 2;
        else if (code & 0x10u) w = 1, dw = 3;
        else w = 0, dw = 4;
        const int mw = 7 - dw - w;
        const int mant = code & ((1 << mw) - 1);
        int e = 0;
        if (w > 0) {
            const int field = (code >> mw) & ((1 << w) - 1);
            const int mag = (field & ((1 << (w - 1)) - 1)) | (1 << (w - 1));
            e = ((field >> (w - 1)) ^ (OQ_MUTANT == 34 && w == 1)) ? -mag : mag;
        }
        v = ldexp(1.0 + (double)mant / (double)(1 << mw), e);
    }
    return (float)(neg ? -v : v);
}

/* x -> HiFloat8 under CAST_ROUND, the rule of docs/zh/api/SIMD-API/basic_api/reg_vector_compute/type_conversion/
 * Cast.md:254-301 (float source; a half source is the same value, :303-348): E = the unbiased exponent; E > 15 and
 * inf overflow, NaN is 0x80, E < -23 gives 0 (0x00, whatever the sign), E = -23 gives the smallest subnormal
 * 2^-22; E in [-22, -16] rounds to 2^E or 2^(E+1) on the first fraction bit; otherwise the mantissa keeps 3 bits
 * for |E| <= 3, 2 for |E| in [4, 7], 1 for |E| in [8, 15] and rounds up on the next bit (ties away), carrying
 * into E.  Saturation (the SatS casts; __half22hif82_rna_sat.md's table: nan -> 0, +-inf and +-65504 -> +-32768,
 * +-0 -> 0) turns every overflow code into +-32768. */
uint8_t oq_hif8_encode(float x, int sat)
{
    const uint32_t u = f2u(x), a = u & 0x7fffffffu;
    const uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    if (a > 0x7f800000u) return sat ? 0x00u : 0x80u;
    const uint8_t over = (uint8_t)(s | (sat ? 0x6Eu : 0x6Fu));
    if (a == 0x7f800000u) return over;
    int e = (int)(a >> 23) - 127;
    const uint32_t f = a & 0x7fffffu;
    if (e > 15) return over;
    if (e < -23) return 0x00u;
    if (e == -23) return (uint8_t)(s | 0x01u);
    int m = 0;
    if (e <= -16) {
        if (f >> 22) ++e;  /* rounds up to the next power of two */
        if (e <= -16) return (uint8_t)(s | (uint8_t)(e + 23));
    } else {
        const int ae = e < 0 ? -e : e;
        const int mw = ae <= 3 ? 3 : (ae <= 7 ? 2 : 1);
        m = (int)(f >> (23 - mw));
        const int tie = (f & ((1u << (22 - mw)) - 1u)) == 0;
        if (((f >> (22 - mw)) & 1u) && !(OQ_MUTANT == 33 && tie)) {
            if (++m >> mw) m = 0, ++e;
        }
    }
    if (e > 15 || (e == 15 && m != 0)) return over;  /* E = 15, M = 1 is the inf code */
    const int ae = e < 0 ? -e : e, ng = e < 0;
    if (OQ_MUTANT == 31 && ae >= 2) return (uint8_t)(s | 0x20u | ((ae & 3) << 3) | m);
    if (ae == 0) return (uint8_t)(s | 0x08u | m);
    if (ae == 1) return (uint8_t)(s | 0x10u | (ng << 3) | m);
    if (ae <= 3) return (uint8_t)(s | 0x20u | (((ng << 1) | (ae & 1)) << 3) | m);
    if (ae <= 7) return (uint8_t)(s | 0x40u | (((ng << 2) | (ae & 3)) << 2) | m);
    return (uint8_t)(s | 0x60u | (((ng << 3) | (ae & 7)) << 1) | m);
}

float oq_fp8_decode(uint8_t v, int fmt)
{
    int s = v >> 7;
    float r;
    if (fmt == OQ_FP8_E4M3) {
        int e = (v >> 3) & 0xf, m = v & 7;
        if (e == 15 && m == 7) return u2f(0x7fc00000u);
        r = e ? ldexpf(1.0f + m / 8.0f, e - 7) : ldexpf(m / 8.0f, -6);
    } else {
        int e = (v >> 2) & 0x1f, m = v & 3;
        if (e == 31) return m ? u2f(0x7fc00000u) : (s ? -INFINITY : INFINITY);
        r = e ? ldexpf(1.0f + m / 4.0f, e - 15) : ldexpf(m / 4.0f, -14);
    }
    return s ? -r : r;
}

/* f32 -> fp8, round to nearest even, by nearest search over the format's finite values (ties: the code with the
 * even mantissa, i.e. the even code).  e4m3fn follows the fixpipe's default saturation mode
 * (docs/zh/api/appendix/matrix_compute_move_out_interface_boundary_value_summary.md:23, 65-67, 87): |x| >= 448
 * and +-inf give +-448, NaN gives 0.  e5m2 is not under that control (same file :28): overflow rounds to +-inf
 * (|x| >= 61440, the midpoint above the largest finite 57344), NaN stays NaN (0x7F). */
uint8_t oq_f32_to_fp8(float x, int fmt)
{
    const int e4 = fmt == OQ_FP8_E4M3;
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    if (isnan(x)) return e4 ? 0x00 : 0x7F;
    float a = fabsf(x);
    const int top = e4 ? 0x7E : 0x7B; /* largest finite magnitude code */
    if (e4 && a >= 448.0f) return (uint8_t)(sign | 0x7E);
    if (!e4 && a >= 61440.0f) return (uint8_t)(sign | 0x7C);
    /* binary search for the largest code whose value is <= a (codes 0..top increase with value) */
    int lo = 0, hi = top;
    while (lo < hi) {
        int mid = (lo + hi + 1) / 2;
        if (oq_fp8_decode((uint8_t)mid, fmt) <= a) lo = mid;
        else hi = mid - 1;
    }
    int c = lo; /* e5m2 between 57344 and 61440 stays at the top code */
    if (c < top) {
        double d0 = (double)a - oq_fp8_decode((uint8_t)c, fmt);
        double d1 = (double)oq_fp8_decode((uint8_t)(c + 1), fmt) - (double)a;
        if (d1 < d0 || (d1 == d0 && ((c & 1) || OQ_MUTANT == 14))) c = c + 1;
    }
    return (uint8_t)(sign | c);
}

/* (V)REQ8 / (V)QF322B8_PRE after the multiply (gen_data_s322s8.py:56-80, gen_data_f322s8.py:56-80 with the
 * ReLU coefficient equal to M1; accompanying_quantization.md:79-103 for the word): NaN -> 0 (boundary-value
 * table :76-79), clamp to [-256, 255], round half to even, add the 9-bit offset (bits 37-45, 0..511,
 * asc_set_l0c_copy_prequant.md:106), saturate to int8 when the sign flag (bit 46) is set, else to uint8.
 * Bits 32-36 (shift N, MCB) are ignored as on arch 3510 (accompanying_quantization.md table 2). */
uint8_t oq_requant8(float v, uint64_t word)
{
    if (isnan(v)) v = 0.0f;
    if (OQ_MUTANT == 13) v += (float)((word >> 37) & 0x1FFu);
    float c = v < -256.0f ? -256.0f : (v > 255.0f ? 255.0f : v);
    int t = (int)rintf(c) + (OQ_MUTANT == 13 ? 0 : (int)((word >> 37) & 0x1FFu));
    if (((word >> 46) & 1u) || OQ_MUTANT == 15) {
        t = t < -128 ? -128 : (t > 127 ? 127 : t);
        return (uint8_t)(int8_t)t;
    }
    t = t < 0 ? 0 : (t > 255 ? 255 : t);
    return (uint8_t)t;
}

/* (V)REQ4 / (V)QF322S4_PRE, int4 output of the fixpipe (docs/zh/api/SIMD-API/c_api/cube_datamove/
 * cube_store_aux_config/asc_set_l0c_copy_prequant.md:37-41 (modes), :106 and :117 (the 9-bit offset applies to
 * REQ4 / QF322S4_PRE, the sign flag does not), docs/zh/api/appendix/
 * matrix_compute_move_out_interface_boundary_value_summary.md:110-111 (saturation to 7 / -8)).  The reference
 * ships no golden for these modes; the 9-bit intermediate (clamp to [-256, 255], rint, + offset) is taken from
 * REQ8's golden (gen_data_s322s8.py:56-80), so only the documented saturation pins this beyond that assumption.
 * Returns the int4 code in the low nibble. */
uint8_t oq_requant4(float v, uint64_t word)
{
    if (isnan(v)) v = 0.0f;
    float c = v < -256.0f ? -256.0f : (v > 255.0f ? 255.0f : v);
    int t = (int)rintf(c) + (OQ_MUTANT == 17 ? 0 : (int)((word >> 37) & 0x1FFu));
    t = t < -8 ? -8 : (t > 7 ? 7 : t);
    return (uint8_t)(t & 0xF);
}

/* int32 accumulators [M, N] -> (V)REQ4 codes packed two per byte ([M, N/2], even column in the low nibble, the
 * int4b_t layout of examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_int4/scripts/gen_data.py);
 * N even */
void oq_mm_requant4(const int32_t* acc, uint8_t* out, int64_t M, int64_t N, const uint64_t* qvec, uint64_t qscalar)
{
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; n += 2) {
            uint8_t q[2];
            for (int h = 0; h < 2; ++h) {
                const uint64_t w = qvec ? qvec[n + h] : qscalar;
                q[h] = oq_requant4((float)acc[m * N + n + h] * oq_quant_pre_m1(w), w);
            }
            out[(m * N + n) / 2] = OQ_MUTANT == 18 ? (uint8_t)(q[1] | (q[0] << 4)) : (uint8_t)(q[0] | (q[1] << 4));
        }
}

/* fp32 L0C values (acc + bias) [M, N] -> (V)QF322S4_PRE codes: requant4(v * M1, word), packed as above */
void oq_requant4_f32(const float* v, uint8_t* out, int64_t M, int64_t N, const uint64_t* qvec, uint64_t qscalar)
{
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; n += 2) {
            uint8_t q[2];
            for (int h = 0; h < 2; ++h) {
                const uint64_t w = qvec ? qvec[n + h] : qscalar;
                q[h] = oq_requant4(v[m * N + n + h] * oq_quant_pre_m1(w), w);
            }
            out[(m * N + n) / 2] = OQ_MUTANT == 18 ? (uint8_t)(q[1] | (q[0] << 4)) : (uint8_t)(q[0] | (q[1] << 4));
        }
}

static inline double round_to(double x, int t) /* one IEEE rounding into scaleT (half / bf16 / fp32), rne */
{
    if (t == OQ_F16) return oq_f16_to_f32(oq_f64_to_f16(x, 0));
    if (t == OQ_BF16) return oq_bf16_to_f32(oq_f64_to_bf16(x, 0));
    return (double)(float)x;
}

static inline float load_as_f32(const void* p, int type, int64_t i)
{
    switch (type) {
    case OQ_F16: return oq_f16_to_f32(((const uint16_t*)p)[i]);
    case OQ_BF16: return oq_bf16_to_f32(((const uint16_t*)p)[i]);
    case OQ_F32: return ((const float*)p)[i];
    case OQ_INT32: return (float)((const int32_t*)p)[i]; /* rne, exact below 2^24 */
    case OQ_INT8: return (float)((const int8_t*)p)[i];
    case OQ_U64: return u2f((uint32_t)(((const uint64_t*)p)[i] & 0xffffffffu)); /* low half of the word */
    default: return 0.0f;
    }
}

static inline void store_from_f32(void* p, int type, int64_t i, float v)
{
    switch (type) {
    case OQ_F16: ((uint16_t*)p)[i] = oq_f32_to_f16(v, 1); break;
    case OQ_BF16: ((uint16_t*)p)[i] = oq_f32_to_bf16(v, 1); break;
    case OQ_F32: ((float*)p)[i] = v; break;
    default: break;
    }
}

/* ------------------------------------------------------------------------ */
/* Matmul int8 x int8 -> int32 (+bias)                                       */
/* ------------------------------------------------------------------------ */

/* acc[m,n] = sum_k A[m,k]*B[k,n] + bias[n] in int32 (MmadCompute with isBias,
 * impl/adv_api/detail/matmul/stage/compute/mmad_compute.h:40-90; L0C type int32 for int8 inputs,
 * impl/adv_api/detail/matmul/utils/matmul_utils.h:134-175).  The sum is formed in int64 and wrapped. */
void oq_matmul_i8(const int8_t* A, const int8_t* B, const int32_t* bias, int32_t* C,
                  int64_t M, int64_t N, int64_t K, int transA, int transB)
{
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        int64_t* row = (int64_t*)calloc((size_t)N, sizeof(int64_t));
        for (int64_t k = 0; k < K; ++k) {
            int64_t a = transA ? A[k * M + m] : A[m * K + k];
            if (!a) continue;
            if (!transB) {
                const int8_t* b = B + k * N;
                for (int64_t n = 0; n < N; ++n) row[n] += a * b[n];
            } else {
                for (int64_t n = 0; n < N; ++n) row[n] += a * B[n * K + k];
            }
        }
        for (int64_t n = 0; n < N; ++n) {
            int64_t v = row[n] + ((bias && OQ_MUTANT != 4) ? bias[n] : 0);
            C[m * N + n] = (int32_t)(uint32_t)(uint64_t)v;
        }
        free(row);
    }
}

/* DEQF16 / VDEQF16 (int32 -> half) and QS322BF16_PRE / VQS322BF16_PRE (int32 -> bf16):
 * out = sat(rne(f32(acc) * M1)), M1 from the QUANT_PRE word; modes chosen in
 * impl/adv_api/detail/matmul/stage/copy_cube_out/quant/quant_processor_fixpipe.h:89-117,209-234.
 * The product is one fp32 multiply (documented choice; the fixpipe's internal width is not public). */
void oq_mm_dequant(const int32_t* acc, void* out, int out_type, int64_t M, int64_t N,
                   const uint64_t* qvec, uint64_t qscalar)
{
    float ms = oq_quant_pre_m1(qscalar);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float m1 = qvec ? oq_quant_pre_m1(qvec[n]) : ms;
            float v = (float)acc[m * N + n] * m1;
            store_from_f32(out, out_type, m * N + n, v);
        }
}

/* (V)REQ8 epilogue of the int8 Matmul with an int8 / uint8 C (quant_processor_fixpipe.h:89-99, 209-214):
 * out = requant8(f32(acc) * M1, word), word = qvec[n] or qscalar; f32(acc) rounds to nearest even. */
void oq_mm_requant(const int32_t* acc, uint8_t* out, int64_t M, int64_t N, const uint64_t* qvec, uint64_t qscalar)
{
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            uint64_t w = qvec ? qvec[n] : qscalar;
            out[m * N + n] = oq_requant8((float)acc[m * N + n] * oq_quant_pre_m1(w), w);
        }
}

/* an operand element of the fp8 / hifloat8 Matmul: fp8 e4m3fn / e5m2, or hifloat8 (the sample's default scenario,
 * matmul_fp8.asc:229) */
static inline double mm8_decode(uint8_t v, int fmt)
{
    if (fmt == OQ_HIF8) return OQ_MUTANT == 39 ? (double)oq_fp8_decode(v, OQ_FP8_E4M3) : (double)oq_hif8_decode(v);
    return (double)oq_fp8_decode(v, fmt);
}

/* fp8 operands: L0C is fp32 (matmul_utils.h:134-175); a float bias seeds L0C before the k loop (MmadCompute
 * with isBias, mmad_compute.h:40-90; the fp8 sample adds a float [1, N] bias, matmul_fp8/scripts/gen_data.py
 * tf_matmul + bias); the epilogue is (V)QF322{F16,BF16,F32}_PRE (quant_processor_fixpipe.h:101-115):
 * out = cast((acc + bias) * M1), or a plain cast (F322F16 / F322BF16 / F32) when no quant word is set
 * (quant_processor_utils.h:39-43).  The product sum is exact in double and rounded once to fp32 here; the
 * device accumulates in fp32 and aligns the products of each 16-element K group to the group's largest one,
 * so this path is compared within a tolerance built from sum |a b| (absdot_out) and the sum over 16-element
 * K groups of the group's largest |a b| (blockmax_out; either output may be NULL).
 * use_q: 1 when SetQuantScalar / SetQuantVector was called.
 * out_type OQ_INT8 / OQ_UINT8: (V)QF322B8_PRE, oq_requant8((acc + bias) * M1, word); OQ_FP8_E4M3 / _E5M2:
 * (V)QF322FP8_PRE (quant_processor_fixpipe.h:101-103, 219-221), oq_f32_to_fp8((acc + bias) * M1); OQ_HIF8:
 * (V)QF322HIF8_PRE (quant_processor_fixpipe.h:106-107, 223-224), ties away with the saturation-mode rules
 * (matrix_compute_move_out_interface_boundary_value_summary.md:68-70, 88-90: +-inf and every |v| >= 32768 ->
 * +-32768, NaN -> 0), oq_hif8_encode((acc + bias) * M1, sat).
 * a_fmt / b_fmt OQ_HIF8 (both, the hifloat8 Matmul): elements decoded by oq_hif8_decode. */
void oq_matmul_fp8(const uint8_t* A, const uint8_t* B, int a_fmt, int b_fmt, const float* bias, void* out,
                   int out_type, int64_t M, int64_t N, int64_t K, int transA, int transB, int use_q,
                   const uint64_t* qvec, uint64_t qscalar, double* exact_out, double* absdot_out,
                   double* blockmax_out)
{
    float ms = oq_quant_pre_m1(qscalar);
    /* B decoded once, [n][k] */
    double* bd = (double*)malloc((size_t)(N * K) * sizeof(double));
    if (!bd) return;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) bd[n * K + k] = mm8_decode(transB ? B[n * K + k] : B[k * N + n], b_fmt);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        double* arow = (double*)malloc((size_t)K * sizeof(double));
        if (!arow) continue;
        for (int64_t k = 0; k < K; ++k) arow[k] = mm8_decode(transA ? A[k * M + m] : A[m * K + k], a_fmt);
        for (int64_t n = 0; n < N; ++n) {
            const double* bn = bd + n * K;
            double s = 0.0, sa = 0.0, sb = 0.0, bmx = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                double p = arow[k] * bn[k];
                s += p;
                sa += fabs(p);
                if (fabs(p) > bmx) bmx = fabs(p);
                if (k % 16 == 15 || k == K - 1) {
                    sb += bmx;
                    bmx = 0.0;
                }
            }
            if (bias) s += (double)bias[n];
            if (exact_out) exact_out[m * N + n] = s;
            if (absdot_out) absdot_out[m * N + n] = sa;
            if (blockmax_out) blockmax_out[m * N + n] = sb;
            float v = (float)s;
            if (use_q) v = v * (qvec ? oq_quant_pre_m1(qvec[n]) : ms);
            if (out_type == OQ_INT8 || out_type == OQ_UINT8)
                ((uint8_t*)out)[m * N + n] = oq_requant8(v, qvec ? qvec[n] : qscalar);
            else if (out_type == OQ_FP8_E4M3 || out_type == OQ_FP8_E5M2)
                ((uint8_t*)out)[m * N + n] = oq_f32_to_fp8(v, out_type);
            else if (out_type == OQ_HIF8) /* QF322HIF8_PRE, saturation mode */
                ((uint8_t*)out)[m * N + n] = oq_hif8_encode(v, 1);
            else
                store_from_f32(out, out_type, m * N + n, v);
        }
        free(arow);
    }
    free(bd);
}

/* ------------------------------------------------------------------------ */
/* AscendQuant                                                               */
/* ------------------------------------------------------------------------ */

/* PER_TOKEN, int8 output, fp32 scale (policy API include/adv_api/quantization/ascend_quant.h:714-777):
 * QuantPerTokenForS8VF (impl/adv_api/detail/quantization/quant/ascend_quant_per_group_3510_impl.h:142-178)
 * casts x to fp32, Mul by the row scale, Add the row offset (fp32), then TransRegForS8
 * (ascend_quant_3510_impl.h:958-968): fp32 -> s16 (round mode, SAT) -> f16 -> s8 (SAT).  The s16 and f16
 * steps are exact for every value that does not saturate to int8, so the result is sat_s8(round(v)). */
void oq_quant_per_token(int8_t* dst, const void* src, int src_type, const float* scale, const float* offset,
                        int64_t m, int64_t n, int round_mode)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        float s = scale[i];
        float o = offset ? offset[i] : 0.0f;
        for (int64_t j = 0; j < n; ++j) {
            float v = load_as_f32(src, src_type, i * n + j) * s;
            if (offset) v = v + o;
            int32_t r = oq_round_to_int(v, round_mode);
            if (r > 32767) r = 32767;
            if (r < -32768) r = -32768;
            dst[i * n + j] = oq_sat_s8(r);
        }
    }
}

/* Dynamic per-token quant (config "AscendQuant per-token dynamic"): the absmax reduction is the caller's
 * job in the reference (no ReduceMax in impl/adv_api/detail/quantization); this restatement defines it as
 * absmax = max |f32(x)| over the row (NaN ignored), multiplier = 127/absmax (one fp32 division, 0 when
 * absmax == 0), scale_out = absmax/127, then the PER_TOKEN quant above with the multiplier as its scale. */
void oq_quant_dynamic_per_token(int8_t* dst, float* scale_out, const void* src, int src_type,
                                int64_t m, int64_t n, int round_mode)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        float amax = 0.0f;
        for (int64_t j = 0; j < n; ++j) {
            float a = fabsf(load_as_f32(src, src_type, i * n + j));
            if (a > amax) amax = a;
        }
        float mult = amax > 0.0f ? (OQ_MUTANT == 8 ? 1.0f / (amax / 127.0f) : 127.0f / amax) : 0.0f;
        scale_out[i] = amax / 127.0f;
        for (int64_t j = 0; j < n; ++j) {
            float v = load_as_f32(src, src_type, i * n + j) * mult;
            dst[i * n + j] = oq_sat_s8(oq_round_to_int(v, round_mode));
        }
    }
}

/* Legacy AscendQuant, arch-3510 form (include/adv_api/quantization/ascend_quant.h:64-293, 360-460; impl
 * impl/adv_api/detail/quantization/quant/ascend_quant_3510_impl.h:35-620).  Element i of cal_count uses channel
 * c = i % scale_count of the srcT scale / offset tensors, or the float scalars when scale is NULL; a scale tensor with
 * offset NULL is the `const T offset` overload (offset_scalar rounded to srcT).
 *  - int8 / hifloat8 out (QuantPertensorForB8 :35-128, QuantPerchannelForB8 :292-483): source, scale and offset
 *    tensors become half with rne and saturation (MrgZRndRSatS / LayoutZMrgZRndRSatS), the float scalars with a
 *    plain rne conversion (static_cast<half>); t = half(x * s); t = half(t + o); int8: rint with saturation
 *    (LayoutZMrgZRndRSatS), NaN -> 0; hifloat8: ties away with saturation (LayoutZMrgZRndASatS).
 *  - fp8 e4m3 / e5m2 out (QuantPertensorForFp8 :144-170, QuantPerchannelForFp8 :207-260, :483-530): source, scale and
 *    offset in fp32 (exact); y = f32(x * s); y = f32(y + o); rint with saturation (NaN -> 0). */
void oq_quant_legacy(void* dst, int dst_type, const void* src, int src_type, const void* scale, const void* offset,
                     float scale_scalar, float offset_scalar, int64_t cal_count, int64_t scale_count)
{
    const int fp8 = (dst_type == OQ_FP8_E4M3 || dst_type == OQ_FP8_E5M2) && OQ_MUTANT != 32;
    /* the `const T offset` overload: a srcT value */
    const float os = scale ? (float)round_to((double)offset_scalar, src_type) : offset_scalar;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < cal_count; ++i) {
        const int64_t c = scale_count > 0 ? i % scale_count : 0;
        const float x = load_as_f32(src, src_type, i);
        const float s = scale ? load_as_f32(scale, src_type, c) : scale_scalar;
        const float o = offset ? load_as_f32(offset, src_type, c) : os;
        if (fp8) {
            float v = (float)((double)x * (double)s); /* one fp32 rounding of the exact product */
            v = (float)((double)v + (double)o);
            ((uint8_t*)dst)[i] = oq_f32_to_fp8_sat(v, dst_type);
            continue;
        }
        const uint16_t xh = src_type == OQ_F16 ? ((const uint16_t*)src)[i] : oq_f32_to_f16(x, 1);
        const uint16_t sh = scale ? (src_type == OQ_F16 ? oq_f32_to_f16(s, 0) : oq_f32_to_f16(s, 1)) : oq_f32_to_f16(s, 0);
        const uint16_t oh = offset ? (src_type == OQ_F16 ? oq_f32_to_f16(o, 0) : oq_f32_to_f16(o, 1)) : oq_f32_to_f16(o, 0);
        uint16_t t = oq_f64_to_f16((double)oq_f16_to_f32(xh) * (double)oq_f16_to_f32(sh), 0);
        t = oq_f64_to_f16((double)oq_f16_to_f32(t) + (double)oq_f16_to_f32(oh), 0);
        const float tv = oq_f16_to_f32(t);
        if (dst_type == OQ_HIF8) ((uint8_t*)dst)[i] = oq_hif8_encode(tv, 1);
        else if (dst_type != OQ_INT8) ((uint8_t*)dst)[i] = oq_f32_to_fp8_sat(tv, dst_type); /* mutant 32 only */
        else ((int8_t*)dst)[i] = oq_sat_s8(oq_round_to_int(tv, OQ_ROUND_RINT));
    }
}

/* Legacy AscendQuant (per-tensor / per-channel) in fp16 arithmetic, arch 2201:
 * AscendQuantPerChannelIntrinsicsImpl (impl/adv_api/detail/quantization/quant/ascend_quant_pre_impl.h:101-164):
 * fp32 input is first Cast to half (CAST_NONE = rint), then Mul (half), Add/Adds offset (half), then
 * Cast<int8_t, half>(CAST_NONE) which rounds half-to-even and saturates (Cast.md:92, precision_conversion.md:30).
 * Element i uses scale[i % scale_count] (scaleCount divides calCount, ascend_quant_common_impl.h:132-188).
 * The half ops are IEEE binary16 with one rounding each; the product of two halves is exact in fp32 and the
 * sum of two halves is exact in fp64, so one rounding to binary16 reproduces each op. */
void oq_quant_legacy_f16(int8_t* dst, const void* src, int src_type, const uint16_t* scale_vec,
                         uint16_t scale_scalar, const uint16_t* offset_vec, uint16_t offset_scalar,
                         int64_t cal_count, int64_t scale_count)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < cal_count; ++i) {
        uint16_t xh = src_type == OQ_F16 ? ((const uint16_t*)src)[i] : oq_f32_to_f16(((const float*)src)[i], 0);
        int64_t c = scale_count > 0 ? i % scale_count : 0;
        uint16_t sh = scale_vec ? scale_vec[c] : scale_scalar;
        uint16_t oh = offset_vec ? offset_vec[c] : offset_scalar;
        uint16_t t = oq_f64_to_f16((double)oq_f16_to_f32(xh) * (double)oq_f16_to_f32(sh), 0);
        uint16_t u = OQ_MUTANT == 11 ? oq_f64_to_f16((double)oq_f16_to_f32(xh) * oq_f16_to_f32(sh) + oq_f16_to_f32(oh), 0)
                                     : oq_f64_to_f16((double)oq_f16_to_f32(t) + (double)oq_f16_to_f32(oh), 0);
        float tv = oq_f16_to_f32(u);
        dst[i] = oq_sat_s8(oq_round_to_int(tv, OQ_ROUND_RINT));
    }
}

/* ------------------------------------------------------------------------ */
/* AscendDequant                                                             */
/* ------------------------------------------------------------------------ */

/* int32 -> fp32 with ties away from zero: the dequant kernels convert their int32 source with
 * Reg::Cast<float, int32_t, MrgZRndA> (impl/adv_api/detail/quantization/dequant/ascend_dequant_3510_impl.h:61, 115,
 * 184, 434, 504), and MrgZRndA carries RoundMode::CAST_ROUND (impl/basic_api/dav_3510/kernel_operator_vec_vconv_impl.h:
 * 56-57), "away-zero" (impl/basic_api/utils/kernel_utils_mode.h:108).  Exact below 2^24; above, the 24-bit
 * significand of |v| is rounded half up on the magnitude. */
float oq_i32_to_f32_rna(int32_t v)
{
    if (OQ_MUTANT == 27) return (float)v; /* mutant: nearest-even */
    uint64_t a = v < 0 ? (uint64_t)(-(int64_t)v) : (uint64_t)v;
    if (a >= (1u << 24)) {
        int bits = 0;
        while ((a >> bits) > 1) ++bits; /* index of the leading one */
        const int s = bits - 23;        /* bits below the 24-bit significand */
        a = ((a + (1ull << (s - 1))) >> s) << s;
    }
    const float f = (float)a; /* exact: at most 24 significant bits */
    return v < 0 ? -f : f;
}

static inline float dq_src_f32(const void* src, int src_type, int64_t i)
{
    if (src_type == OQ_INT32) return oq_i32_to_f32_rna(((const int32_t*)src)[i]);
    if (src_type == OQ_INT8) return (float)((const int8_t*)src)[i]; /* int8 widened to int32: exact */
    return ((const float*)src)[i];
}

/* UpdateDequantParams (impl/adv_api/detail/quantization/dequant/ascend_dequant_common_impl.h:208-223): under
 * DEQUANT_WITH_SINGLE_ROW (the default mode, include/adv_api/quantization/ascend_dequant.h:59, 88, 150) a
 * {1, n, calCount} whose calCount is a whole number of 32-byte dst blocks and divides n is processed as
 * {n / calCount, calCount, calCount} -- e.g. int32 {1, 16, 8} becomes {2, 8, 8} for an f32 dst but stays
 * {1, 16, 8} for a bf16 dst (8 bf16 elements are half a block).  The dst row stride is n rounded up to a whole
 * 32-byte block of dst elements (dstInner, ascend_dequant_3510_impl.h:44, 99 and ascend_dequant_common_impl.h:
 * 376-377); the source row stride stays n. */
int64_t oq_dequant_legacy_shape(int dst_type, int mode, int64_t* m, int64_t* n, int64_t cal_count)
{
    const int64_t blk = dst_type == OQ_F32 ? 8 : 16; /* dst elements per 32-byte block */
    if (mode == OQ_DEQUANT_SINGLE_ROW && *m == 1 && cal_count > 0 && cal_count % blk == 0 && *n % cal_count == 0 &&
        OQ_MUTANT != 28) {
        *m = *n / cal_count;
        *n = cal_count;
    }
    return OQ_MUTANT == 29 ? *n : (*n + blk - 1) / blk * blk;
}

/* Legacy AscendDequant (include/adv_api/quantization/ascend_dequant.h:38-291, DequantParams{m, n, calCount}
 * ascend_dequant_utils.h:26-30), restated after arch 3510 (DequantPerchannelVFImpl / DequantPertensorVFImpl,
 * ascend_dequant_3510_impl.h:37-210): after the SINGLE_ROW rule above, for each of the m rows and each column
 * j < calCount, dst[i * dstInner + j] = cast(f32(src[i * n + j]) * scale), where scale is deqScale[j] (a uint64
 * deqScale contributes its low 32 bits as an fp32, "only half of uint64_t is used", :62-64; bf16 widens exactly)
 * or, per_tensor, the scalar (Muls, :183-187); f32(int32) rounds ties away (oq_i32_to_f32_rna); cast is rne with
 * saturation to f16 / bf16 (LayoutZMrgZRndRSatS, :70, 131) or a plain fp32 store.  Columns j >= calCount of dst
 * and the padding columns are not written (the 2201 form, CalculateByInner of ascend_dequant_common_impl.h:
 * 366-430, instead writes columns >= calCount unscaled). */
void oq_dequant_legacy(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                       float scale_scalar, int per_tensor, int mode, int64_t m, int64_t n, int64_t cal_count)
{
    const int64_t ldd = oq_dequant_legacy_shape(dst_type, mode, &m, &n, cal_count);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < cal_count; ++j) {
            const float s = per_tensor ? scale_scalar : load_as_f32(scale, scale_type, OQ_MUTANT == 12 ? i % cal_count : j);
            store_from_f32(dst, dst_type, i * ldd + j, dq_src_f32(src, src_type, i * n + j) * s);
        }
    }
}

/* AscendDequant policy form, arch 3510 (include/adv_api/quantization/ascend_dequant.h:293-315;
 * AscendDeQuantParam{m, n, calCount, groupSize}, AscendDeQuantConfig{hasOffset, kDim} ascend_dequant_utils.h:
 * 32-44; dispatch ascend_dequant_3510_impl.h:643-690).  rows = calCount / n, src and dst [rows, n]:
 *   PER_TOKEN (DeQuantPerTokenFor{S32,F32}VF, :254-343): dst[r][c] = cast(f32(src[r][c]) * f32(scale[r]));
 *   PER_GROUP kDim 1 (DeQuantPerGroupForCol{S32,F32}VF, :367-504, GetPerGroupScale :345-366): scale[r][c / g]
 *             with [rows][ceil(n / g)] scales;
 *   PER_GROUP kDim 0 (DeQuantPerGroupForRowVF / RowTailBlock, :506-598): scale[r / g][c] with [ceil(rows / g)][n].
 * int32 sources convert with ties away (MrgZRndA), fp32 sources are used as they are; 16-bit scales widen exactly;
 * one fp32 multiply; StoreRes (:237-252) casts rne + saturating to f16 / bf16 or stores fp32.  The config's offset
 * tensor is never read by these kernels. */
void oq_dequant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                       int policy, int k_dim, int64_t n, int64_t cal_count, int64_t group)
{
    const int64_t rows = cal_count / n;
    const int64_t sk = group > 0 ? (n + group - 1) / group : 0;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < n; ++c) {
            int64_t sidx;
            if (policy == OQ_PER_TOKEN) sidx = r;
            else if ((k_dim == 1) ^ (OQ_MUTANT == 30)) sidx = r * sk + c / group;
            else sidx = (r / group) * n + c;
            const float v = dq_src_f32(src, src_type, r * n + c) * load_as_f32(scale, scale_type, sidx);
            store_from_f32(dst, dst_type, r * n + c, v);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* AscendAntiQuant                                                           */
/* ------------------------------------------------------------------------ */

static inline int32_t load_q(const void* src, int src_type, int64_t idx)
{
    if (src_type == OQ_INT8) return ((const int8_t*)src)[idx];
    /* int4b_t packed two per byte, the even element in the low nibble
     * (examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_int4/scripts/gen_data.py packing) */
    uint8_t byte = ((const uint8_t*)src)[idx >> 1];
    int32_t nib = ((idx & 1) ^ (OQ_MUTANT == 3)) ? (byte >> 4) : (byte & 0xf);
    return nib >= 8 ? nib - 16 : nib;
}

/* dst = scale * (src + offset) (include/adv_api/quantization/ascend_antiquant.h:36-46):
 *  - ARITH_F16 (fp16 output, arch 2201): AntiQuantInnerLoop (impl/adv_api/detail/quantization/antiquant/
 *    ascend_antiquant_impl.h:63-96): Cast int->half (exact), Add offset (half), Mul scale (half);
 *  - ARITH_F32: cast to fp32, Add, Mul in fp32, Cast RINT to the output type
 *    (bf16: ascend_antiquant_c220_impl.h:46-75; 3510 scalar path ascend_antiquant_3510_impl.h:320-330).
 * Layout (ascend_antiquant_impl.h:366-411 and the no-transpose path :285-330):
 *  is_transpose == 0: src [K, N], offset/scale [K/group, N] (group == K: per-channel [1, N]);
 *  is_transpose == 1: src [N, K], offset/scale [N, K/group] (AntiQuantShapeInfo, ascend_antiquant_utils.h:26-31).
 * offset == NULL means no offset (the scale-only overloads). */
static inline double aq_src_value(const void* src, int src_type, int64_t idx)
{
    if (src_type == OQ_FP8_E4M3 || src_type == OQ_FP8_E5M2) return oq_fp8_decode(((const uint8_t*)src)[idx], src_type);
    if (src_type == OQ_HIF8) return oq_hif8_decode(((const uint8_t*)src)[idx]);
    return (double)load_q(src, src_type, idx);
}

/* The arithmetic arch 3510 uses for a legacy AscendAntiQuant of an fp8 or hifloat8 source
 * (AntiQuantPerchannelImpl / AntiQuantPertensorImpl, impl/adv_api/detail/quantization/antiquant/
 * ascend_antiquant_3510_impl.h:334-470, 560-770): fp8 always in fp32 (PerTensorProcessForFp8 :307-333,
 * PerchannelNoTransposeForFp8 :440-468, PerchannelTransposeForFp8 :688-735, PerchannelUnalignedForFp8 :515-558);
 * hifloat8 to f16 in half ops (:334-355, :470-495, :630-645); hifloat8 to bf16 in bf16 ops along rows
 * (PerchannelNoTransposeForB8 :470-495, PerchannelUnalignedForB8 :560-593) and in fp32 ops with one rint cast when
 * transposed or per tensor (:646-687, :357-392).  Other sources keep the caller's choice. */
static int aq_arith_for(int src_type, int dst_type, int is_transpose, int per_tensor, int arith)
{
    if (src_type == OQ_FP8_E4M3 || src_type == OQ_FP8_E5M2) return OQ_ARITH_F32;
    if (src_type == OQ_HIF8) {
        if (dst_type == OQ_F16) return OQ_ARITH_F16;
        return (is_transpose || per_tensor) ? OQ_ARITH_F32 : OQ_ARITH_BF16;
    }
    return arith;
}

/* one element: (q + offset) * scale in the chosen arithmetic, written as dst_type */
static inline void aq_element(void* dst, int dst_type, int64_t idx, double q, int has_off, float of, float sc,
                              int arith)
{
    if (arith == OQ_ARITH_F16 && dst_type == OQ_F16) {
        /* half(q) is exact; q + offset and the product are exact in double, rounded once each */
        uint16_t w = oq_f64_to_f16(q, 0);
        if (OQ_MUTANT == 7) {
            w = oq_f64_to_f16(q * (double)sc, 0);
            if (has_off) w = oq_f64_to_f16((double)oq_f16_to_f32(w) + (double)of, 0);
        } else {
            if (has_off) w = oq_f64_to_f16(q + (double)of, 0);
            w = oq_f64_to_f16((double)oq_f16_to_f32(w) * (double)sc, 0);
        }
        ((uint16_t*)dst)[idx] = w;
    } else if (arith == OQ_ARITH_BF16 && dst_type == OQ_BF16) {
        uint16_t w = oq_f64_to_bf16(q, 0);
        if (has_off) w = oq_f64_to_bf16((double)oq_bf16_to_f32(w) + (double)of, 0);
        w = oq_f64_to_bf16((double)oq_bf16_to_f32(w) * (double)sc, 0);
        ((uint16_t*)dst)[idx] = w;
    } else {
        float v = (float)q;
        if (has_off) v = v + of;
        v = v * sc;
        store_from_f32(dst, dst_type, idx, v);
    }
}

void oq_antiquant(void* dst, int dst_type, const void* src, int src_type, const void* offset, const void* scale,
                  int64_t K, int64_t N, int64_t group_size, int is_transpose, int arith)
{
    int64_t G = group_size > 0 ? K / group_size : 1;
    int64_t g = group_size > 0 ? group_size : K;
    const int ar = aq_arith_for(src_type, dst_type, is_transpose, 0, arith);
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) {
            int64_t idx = is_transpose ? n * K + k : k * N + n;
            int64_t sidx = is_transpose ? n * G + k / g : (k / g) * N + n;
            float sc = load_as_f32(scale, dst_type, sidx);
            float of = offset ? load_as_f32(offset, dst_type, sidx) : 0.0f;
            aq_element(dst, dst_type, idx, aq_src_value(src, src_type, idx), offset != NULL, of, sc, ar);
        }
}

/* AscendAntiQuant with scalar offset / scale of the output type (include/adv_api/quantization/ascend_antiquant.h:
 * 136-210; arch 3510 AntiQuantPertensorImpl, ascend_antiquant_3510_impl.h:394-415): int8 and hifloat8 in half ops for
 * f16 and fp32 ops for bf16 (PerTensorProcessForB8 :334-392), fp8 in fp32 ops (PerTensorProcessForFp8 :301-333). */
void oq_antiquant_scalar(void* dst, int dst_type, const void* src, int src_type, uint16_t offset, uint16_t scale,
                         int has_offset, int64_t count)
{
    const float sc = dst_type == OQ_F16 ? oq_f16_to_f32(scale) : oq_bf16_to_f32(scale);
    const float of = dst_type == OQ_F16 ? oq_f16_to_f32(offset) : oq_bf16_to_f32(offset);
    const int ar = aq_arith_for(src_type, dst_type, 0, 1, dst_type == OQ_F16 ? OQ_ARITH_F16 : OQ_ARITH_F32);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i)
        aq_element(dst, dst_type, i, aq_src_value(src, src_type, i), has_offset, of, sc, ar);
}

/* AscendAntiQuant<dstT, srcT, scaleT, config{hasOffset, isTranspose, kDim}, policy>(dst, src, scale, offset,
 * {m, n, calCount, groupSize}) of arch 3510 (include/adv_api/quantization/ascend_antiquant.h:235-259; config and
 * policy impl/adv_api/detail/quantization/antiquant/ascend_antiquant_common.h:46-66; dispatch
 * ascend_antiquant_3510_impl.h:2175-2221) over an [m, n] tensor, element (r, c) at r * n + c:
 *  - scale / offset index: PER_TOKEN one per row (isTranspose: one per column, :1510-1550); PER_GROUP along the
 *    columns ([m][ceil(n/g)], ForCol) when (kDim == 1 && !isTranspose) || (kDim == 0 && isTranspose), else along
 *    the rows ([ceil(m/g)][n], ForRow) (:2205-2212);
 *  - int8 source (ForRow / ForCol / PerToken B8 kernels, :1458-1497, :1670-1711, :1965-2011): ConvertSrc to scaleT
 *    (exact, :1386-1403), + offset and * scale in scaleT, each one rounding (half, bf16 or fp32); a 16-bit scaleT
 *    is stored as is (dstT = scaleT), an fp32 one as fp32 or cast rne + saturating (StoreF32Res, :1363-1373);
 *  - fp8 source (Fp8 kernels, :1563-1599, :1874-1917, :2059-2108): fp32 throughout (fp8, scale and offset converted
 *    exactly), + offset then * scale in fp32, StoreF32Res;
 *  - fp4 E2M1 source with E8M0 scales, PER_GROUP only, no offset (:1724-1781, :1793-1828): bf16(src) (exact) times
 *    the scale as bf16 (e << 7; e = 0 gives 0x0040 = 2^-127, e = 255 gives NaN 0x7FFF), one bf16 rounding, then for
 *    half output a rne + saturating cast.
 * offset == NULL: no offset (config.hasOffset false). */
void oq_antiquant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale, const void* offset,
                         int scale_type, int policy, int64_t m, int64_t n, int64_t group, int k_dim, int is_transpose)
{
    const int col_groups = (k_dim == 1 && !is_transpose) || (k_dim == 0 && is_transpose);
    const int64_t sk = group > 0 ? (n + group - 1) / group : 1;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            const int64_t idx = r * n + c;
            int64_t sidx;
            if (policy == OQ_PER_TOKEN) sidx = is_transpose ? c : r;
            else if (col_groups ^ (OQ_MUTANT == 19)) sidx = r * sk + c / group;
            else sidx = (r / group) * n + c;
            if (src_type == OQ_FP4_E2M1 || src_type == OQ_FP4_E1M2) {
                const uint8_t b = ((const uint8_t*)src)[idx >> 1];
                const uint8_t nib = (idx & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 0xF);
                const double v = src_type == OQ_FP4_E1M2 ? oq_e1m2_decode(nib) : oq_e2m1_decode(nib);
                const uint8_t e = ((const uint8_t*)scale)[sidx];
                const double sc = e == 255 ? NAN : (e == 0 ? ldexp(1.0, -127) : ldexp(1.0, (int)e - 127));
                const double p = round_to(v * sc, OQ_BF16);  /* exact product, one bf16 rounding */
                if (dst_type == OQ_F16) ((uint16_t*)dst)[idx] = oq_f64_to_f16(p, 1);
                else ((uint16_t*)dst)[idx] = oq_f64_to_bf16(p, 0);  /* already a bf16 value */
                continue;
            }
            const double s = load_as_f32(scale, scale_type, sidx);
            const double o = offset ? load_as_f32(offset, scale_type, sidx) : 0.0;
            if (src_type == OQ_FP8_E4M3 || src_type == OQ_FP8_E5M2) {
                const int t = OQ_MUTANT == 20 ? scale_type : OQ_F32;  /* mutant: fp8 in scaleT arithmetic */
                double v = oq_fp8_decode(((const uint8_t*)src)[idx], src_type);
                if (offset) v = round_to(v + o, t);
                v = round_to(v * s, t);
                store_from_f32(dst, dst_type, idx, (float)v);
                continue;
            }
            double v = src_type == OQ_HIF8 ? (double)oq_hif8_decode(((const uint8_t*)src)[idx])
                                           : (double)((const int8_t*)src)[idx]; /* exact in every scaleT */
            if (offset) v = round_to(v + o, scale_type);
            v = round_to(v * s, scale_type);
            if (scale_type == OQ_F16) ((uint16_t*)dst)[idx] = oq_f64_to_f16(v, 0);
            else if (scale_type == OQ_BF16) ((uint16_t*)dst)[idx] = oq_f64_to_bf16(v, 0);
            else store_from_f32(dst, dst_type, idx, (float)v);
        }
}

/* ------------------------------------------------------------------------ */
/* AscendQuant policy form (arch 3510): PER_TOKEN / PER_GROUP                */
/* ------------------------------------------------------------------------ */

/* E2M1 code of x under round mode `mode` with saturation at +-6: Cast<fp4x2_e2m1_t, bfloat16_t> accepts
 * floor / rint / round / ceil / trunc (docs/zh/api/SIMD-API/tensor_api/reg_vector_compute/type_conversion/
 * cast.md:96); TransRegForFp4 sends every other mode to rint (ascend_quant_3510_impl.h:995-1036).  The magnitude
 * is bracketed on the code table; a directed mode picks by the sign of x; a negative value that rounds to zero
 * keeps its sign.  NaN -> 0 (the saturating casts' rule, cast.md:108-109). */
uint8_t oq_e2m1_encode(double x, int mode)
{
    static const double mag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
    if (x != x) return 0;
    const int neg = signbit(x) != 0;
    const uint8_t s = neg ? 8u : 0u;
    const double a = fabs(x);
    if (a >= 6.0) return (uint8_t)(s | 7u);
    int lo = 0;
    while (mag[lo + 1] <= a) ++lo; /* mag[lo] <= a < mag[lo + 1] */
    if (mag[lo] == a) return (uint8_t)(s | lo);
    const int hi = lo + 1;
    const double dl = a - mag[lo], dh = mag[hi] - a;
    int c;
    switch (mode) {
    case OQ_ROUND_TRUNC: c = lo; break;
    case OQ_ROUND_FLOOR: c = (neg && OQ_MUTANT != 25) ? hi : lo; break;
    case OQ_ROUND_CEIL: c = (neg && OQ_MUTANT != 25) ? lo : hi; break;
    case OQ_ROUND_ROUND: c = dl < dh ? lo : hi; break;           /* ties away from zero */
    default: c = dl < dh ? lo : (dh < dl ? hi : ((lo & 1) ? hi : lo)); break; /* ties to the even code */
    }
    return (uint8_t)(s | c);
}

/* fp4x2_e1m2_t: sign | 1-bit exponent (bias 1) | 2-bit mantissa.  Exponent field 0 is subnormal (0.mm x 2^0),
 * field 1 normal (1.mm x 2^0): magnitudes {0, .25, .5, .75, 1, 1.25, 1.5, 1.75}; the largest finite 1.75
 * (docs/zh/api/appendix/mmad_mx_interface_boundary_value_summary.md:11: +inf -> 1.75,
 * -inf -> -1.75, NaN -> 0) and e1m2 -> bf16 lossless (docs/zh/api/SIMD-API/basic_api/
 * data_structures/precision_conversion.md:112-115). */
float oq_e1m2_decode(uint8_t nib)
{
    const int e = (nib >> 2) & 1, mm = nib & 3;
    const float mag = e ? 1.0f + 0.25f * (float)mm : 0.25f * (float)mm;
    return (nib & 8) ? -mag : mag;
}

/* E1M2 code of x in round mode `mode` (bf16 -> fp4x2_e1m2_t, precision_conversion.md:345-354; every other mode
 * rint, TransRegForFp4 ascend_quant_3510_impl.h:995-1036), bracketed on the decoded code table like
 * oq_e2m1_encode: saturating at +-1.75, NaN -> 0, a negative value that rounds to zero keeps its sign. */
uint8_t oq_e1m2_encode(double x, int mode)
{
    if (x != x) return 0;
    const int neg = signbit(x) != 0;
    const uint8_t s = neg ? 8u : 0u;
    const double a = fabs(x);
    if (a >= oq_e1m2_decode(7)) return (uint8_t)(s | 7u);
    int lo = 0;
    while (oq_e1m2_decode((uint8_t)(lo + 1)) <= a) ++lo;
    const double ml = oq_e1m2_decode((uint8_t)lo), mh = oq_e1m2_decode((uint8_t)(lo + 1));
    if (ml == a) return (uint8_t)(s | lo);
    const int hi = lo + 1;
    const double dl = a - ml, dh = mh - a;
    int c;
    switch (mode) {
    case OQ_ROUND_TRUNC: c = lo; break;
    case OQ_ROUND_FLOOR: c = neg ? hi : lo; break;
    case OQ_ROUND_CEIL: c = neg ? lo : hi; break;
    case OQ_ROUND_ROUND: c = dl < dh ? lo : hi; break;
    default: c = dl < dh ? lo : (dh < dl ? hi : ((lo & 1 && OQ_MUTANT != 26) ? hi : lo)); break;
    }
    return (uint8_t)(s | c);
}

/* f32 -> fp8 with rint and saturation (TransRegForFp8, ascend_quant_3510_impl.h:888-896: every round mode but
 * rint maps to LayoutZMrgZRndRSatS, i.e. rint + SAT): finite overflow and +-inf clamp to the largest finite
 * magnitude, NaN -> 0 (cast.md:108-109). */
uint8_t oq_f32_to_fp8_sat(float x, int fmt)
{
    if (x != x) return 0;
    const float mx = fmt == OQ_FP8_E4M3 ? 448.0f : 57344.0f;
    if (fabsf(x) > mx) x = copysignf(mx, x);
    return oq_f32_to_fp8(x, fmt);
}

/* AscendQuant<dstT, srcT, scaleT, false, config{hasOffset, kDim, roundMode}, policy>(dst, src, scale, offset,
 * {m, n, calCount = m * n, groupSize}) (include/adv_api/quantization/ascend_quant.h:714-777; impl
 * ascend_quant_per_group_3510_impl.h:33-79 / 142-346 PER_TOKEN, 347-726 PER_GROUP kDim 1, 727-1340 kDim 0,
 * dispatch 1451-1504).  Scale / offset index of element (r, c): PER_TOKEN scale[r]; PER_GROUP kDim 1
 * scale[r * ceil(n / group) + c / group]; kDim 0 scale[(r / group) * n + c].
 *   int8 dst: y = x * s (+ o), each op rounded in scaleT (a 16-bit src meets an f32 scale as f32), then
 *            clamp(round_mode(y), -128, 127) (TransRegForS8 :934-992; NaN -> 0);
 *   fp8 dst: the same ops in f32 whatever scaleT (:33-79, 393-431), then rint + SAT;
 *   E2M1 dst (PER_GROUP only; offset ignored, :1385): y = x * s in scaleT, a float / half y rounded to bf16 rne
 *            with saturation (NaN -> 0), then the E2M1 cast in round_mode (TransRegForFp4 :995-1036); two codes a
 *            byte, even element in the low nibble.
 * offset: a tensor indexed like scale, or (offset == NULL, has_offset) the scalar offset_scalar rounded to scaleT
 * (the overloads taking `const scaleT offset`, :192-235, 297-333). */
void oq_quant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                     const void* offset, int has_offset, float offset_scalar, int policy, int64_t m, int64_t n,
                     int64_t group, int k_dim, int round_mode)
{
    const int fp8 = dst_type == OQ_FP8_E4M3 || dst_type == OQ_FP8_E5M2;
    const int fp4 = dst_type == OQ_FP4_E2M1 || dst_type == OQ_FP4_E1M2;
    const int t = (fp8 && OQ_MUTANT != 21) ? OQ_F32 : scale_type; /* arithmetic type */
    const int off = has_offset && !fp4;
    const int64_t sk = group > 0 ? (n + group - 1) / group : 1;
    const double os = round_to((double)offset_scalar, scale_type);
    uint8_t* codes = fp4 ? (uint8_t*)malloc((size_t)(m * n) + 1) : NULL;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            const int64_t idx = r * n + c;
            int64_t sidx;
            if (policy == OQ_PER_TOKEN) sidx = r;
            else if ((k_dim == 1) ^ (OQ_MUTANT == 23)) sidx = r * sk + c / group;
            else sidx = (r / group) * n + c;
            const double x = load_as_f32(src, src_type, idx);
            const double s = load_as_f32(scale, scale_type, sidx);
            double v = x * s; /* exact: two 24-bit significands */
            if (!(off && OQ_MUTANT == 24)) v = round_to(v, t);
            if (off) v = round_to(v + (offset ? (double)load_as_f32(offset, scale_type, sidx) : os), t);
            if (fp8) {
                ((uint8_t*)dst)[idx] = oq_f32_to_fp8_sat((float)v, dst_type);
            } else if (dst_type == OQ_HIF8) {
                ((uint8_t*)dst)[idx] = oq_hif8_encode((float)v, 1);
            } else if (fp4) {
                double b = v;
                if (t != OQ_BF16 && OQ_MUTANT != 22) b = v != v ? 0.0 : oq_bf16_to_f32(oq_f64_to_bf16(v, 1));
                codes[idx] = dst_type == OQ_FP4_E1M2 ? oq_e1m2_encode(b, round_mode) : oq_e2m1_encode(b, round_mode);
            } else {
                ((int8_t*)dst)[idx] = oq_sat_s8(oq_round_to_int((float)v, round_mode));
            }
        }
    if (fp4) {
        for (int64_t i = 0; i < m * n; i += 2)
            ((uint8_t*)dst)[i >> 1] = (uint8_t)(codes[i] | ((i + 1 < m * n ? codes[i + 1] : 0u) << 4));
        free(codes);
    }
}

/* ------------------------------------------------------------------------ */
/* Quantize / Dequantize / AntiQuantize (the newer interface, arch 3510)     */
/* ------------------------------------------------------------------------ */

/* scale / offset index of element (r, c) for the four policies of the newer interface; -1 = the scalar */
static inline int64_t policy_index(int policy, int64_t r, int64_t c, int64_t n, int64_t group, int k_dim)
{
    const int64_t sk = group > 0 ? (n + group - 1) / group : 1;
    switch (policy) {
    case OQ_PER_TENSOR: return -1;
    case OQ_PER_CHANNEL: return OQ_MUTANT == 40 ? r : c;
    case OQ_PER_TOKEN: return r;
    default: return k_dim == 1 ? r * sk + c / group : (r / group) * n + c;
    }
}

/* Quantize<config>(dst, src, scale, offset, {m, n, groupSize}) (include/adv_api/quantization/quantize.h:55-94; impl
 * impl/adv_api/detail/quantization/quantize/quantize_impl.h:1006-1066).  Every policy and output type computes in
 * fp32: the source, the scale and the offset are widened exactly (GetPerGroupScaleToFloat :262-278,
 * DuplicateScalarToFloatVector :280-294), y = x * s and then y + o are each one fp32 rounding (:361-364, 758-761,
 * 855-858, 935-938), and CastFp32DstToExpect (:296-312) casts y:
 *   int8: to int16 in round_mode with saturation, to half, to int8 with saturation (TransRegForS8 :128-190), i.e.
 *         clamp(round_mode(y), -128, 127), NaN -> 0 (round modes other than rint / round / floor / ceil / trunc are
 *         rint);
 *   fp8: rint with saturation (TransRegForFp8 :80-90);  hifloat8: ties away from zero (TransRegForHif8 :92-126);
 *   fp4 (PER_GROUP only, no offset: QuantizePerGroupForKColFp4VF :391-432): y to bf16 rne with saturation (NaN -> 0),
 *         then the fp4 code in round_mode (TransRegForFp4 :192-230), two codes a byte, even element low.
 * Scale index: PER_TENSOR the scalar scale_scalar, PER_CHANNEL c, PER_TOKEN r, PER_GROUP kDim 1 r * ceil(n / g) +
 * c / g, kDim 0 (r / g) * n + c; the offset alike, or the scalar offset_scalar when there is no offset tensor.
 * Scalars are scaleT values (rounded rne to scale_type). */
void oq_quantize(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                 const void* offset, int has_offset, float scale_scalar, float offset_scalar, int policy, int64_t m,
                 int64_t n, int64_t group, int k_dim, int round_mode)
{
    const int fp8 = dst_type == OQ_FP8_E4M3 || dst_type == OQ_FP8_E5M2;
    const int fp4 = dst_type == OQ_FP4_E2M1 || dst_type == OQ_FP4_E1M2;
    const int off = has_offset && !fp4;
    const double ss = round_to((double)scale_scalar, scale_type);
    const double os = round_to((double)offset_scalar, scale_type);
    const int t = OQ_MUTANT == 41 ? scale_type : OQ_F32; /* arithmetic type (mutant: AscendQuant's scaleT) */
    uint8_t* codes = fp4 ? (uint8_t*)malloc((size_t)(m * n) + 1) : NULL;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            const int64_t idx = r * n + c, si = policy_index(policy, r, c, n, group, k_dim);
            const double x = load_as_f32(src, src_type, idx);
            const double s = si < 0 ? ss : load_as_f32(scale, scale_type, si);
            double v = round_to(x * s, t); /* x * s exact in double: two 24-bit significands */
            if (off) v = round_to(v + ((offset && si >= 0) ? (double)load_as_f32(offset, scale_type, si) : os), t);
            if (fp8) {
                ((uint8_t*)dst)[idx] = oq_f32_to_fp8_sat((float)v, dst_type);
            } else if (dst_type == OQ_HIF8) {
                ((uint8_t*)dst)[idx] = oq_hif8_encode((float)v, 1);
            } else if (fp4) {
                const double b = v != v ? 0.0 : oq_bf16_to_f32(oq_f64_to_bf16(v, 1));
                codes[idx] = dst_type == OQ_FP4_E1M2 ? oq_e1m2_encode(b, round_mode) : oq_e2m1_encode(b, round_mode);
            } else {
                ((int8_t*)dst)[idx] = oq_sat_s8(oq_round_to_int((float)v, round_mode));
            }
        }
    if (fp4) {
        for (int64_t i = 0; i < m * n; i += 2)
            ((uint8_t*)dst)[i >> 1] = (uint8_t)(codes[i] | ((i + 1 < m * n ? codes[i + 1] : 0u) << 4));
        free(codes);
    }
}

/* Dequantize<config>(dst, src, scale, offset, {m, n, groupSize}) (include/adv_api/quantization/dequantize.h:59-95;
 * impl impl/adv_api/detail/quantization/dequantize/dequantize_impl.h:254-290): PER_TENSOR / PER_CHANNEL are the legacy
 * AscendDequant with params {m, n, n} in DEQUANT_WITH_MULTI_ROW (:94-138), PER_TOKEN / PER_GROUP the policy form with
 * {m, n, m * n, groupSize} and the config's kDim (:140-195); no offset (:102). */
void oq_dequantize(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                   float scale_scalar, int policy, int64_t m, int64_t n, int64_t group, int k_dim)
{
    if (policy == OQ_PER_TENSOR || policy == OQ_PER_CHANNEL) /* the scalar is a scaleT value */
        oq_dequant_legacy(dst, dst_type, src, src_type, scale, scale_type, (float)round_to(scale_scalar, scale_type),
                          policy == OQ_PER_TENSOR, OQ_DEQUANT_MULTI_ROW, m, n, n);
    else
        oq_dequant_policy(dst, dst_type, src, src_type, scale, scale_type, policy, k_dim, n, m * n, group);
}

/* AntiQuantize<config>(dst, src, scale, offset, {m, n, groupSize}) (include/adv_api/quantization/antiquantize.h:
 * 61-98; impl impl/adv_api/detail/quantization/antiquantize/antiquantize_impl.h:284-322, antiquantize_3510_impl.h:
 * 38-396).  int8 / hifloat8 / fp8 sources, every policy: fp32 throughout -- the source widened exactly (int8 and
 * hifloat8 through half, CastAntiQuantizeSrcToFp32 :38-48), + offset then * scale, each one fp32 rounding, and one
 * cast to dstT (rne with saturation; a plain store for fp32: StoreF32Res, PerTensorProcessCommon :266-300,
 * PerChannelNoTransposeCommon :328-367, the per-token and per-group kernels :52-262).  Scale index: PER_TENSOR the
 * scalar (a dstT value), PER_CHANNEL c, PER_TOKEN r, PER_GROUP by kDim (ForCol r * ceil(n / g) + c / g when kDim
 * is 1, ForRow (r / g) * n + c when 0); the offset alike (PER_TENSOR: offset_scalar).  fp4 sources (PER_GROUP, E8M0
 * scales, no offset) are the AscendAntiQuant policy form's fp4 rule (AntiQuantPerGroupForColFp4 / RowFp4,
 * antiquantize_impl.h:201-225). */
void oq_antiquantize(void* dst, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                     const void* offset, int has_offset, float scale_scalar, float offset_scalar, int policy,
                     int64_t m, int64_t n, int64_t group, int k_dim)
{
    if (src_type == OQ_FP4_E2M1 || src_type == OQ_FP4_E1M2) {
        oq_antiquant_policy(dst, dst_type, src, src_type, scale, NULL, OQ_E8M0, OQ_PER_GROUP, m, n, group, k_dim, 0);
        return;
    }
    const double ss = round_to((double)scale_scalar, scale_type);
    const double os = round_to((double)offset_scalar, scale_type);
    const int t = OQ_MUTANT == 42 ? scale_type : OQ_F32; /* arithmetic type (mutant: AscendAntiQuant's scaleT) */
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; ++r)
        for (int64_t c = 0; c < n; ++c) {
            const int64_t idx = r * n + c, si = policy_index(policy, r, c, n, group, k_dim);
            const uint8_t code = ((const uint8_t*)src)[idx];
            double v = src_type == OQ_HIF8 ? (double)oq_hif8_decode(code)
                       : src_type == OQ_INT8 ? (double)(int8_t)code : (double)oq_fp8_decode(code, src_type);
            const double s = si < 0 ? ss : load_as_f32(scale, scale_type, si);
            if (has_offset) v = round_to(v + (si < 0 ? os : (double)load_as_f32(offset, scale_type, si)), t);
            v = round_to(v * s, t);
            store_from_f32(dst, dst_type, idx, (float)v);
        }
}

/* Weight-only antiquant matmul (W8A16 / W4A16): the reference composes AscendAntiQuant (fp16 ops, above) with
 * a half x half Matmul whose L0C type is fp32 (GetMmDstType<half> = float, matmul_utils.h:171-174) and whose
 * fixpipe casts fp32 -> half with rint.  Products of two halves are exact; the restatement sums them in
 * double (exact up to one rounding per add at ~2^-53), keeps that sum, and rounds it to half once.
 * x [M,K] half; w [K,N] (w_transpose: [N,K]); scale/offset [K/group, N] (w_transpose: [N, K/group]). */
void oq_antiquant_matmul(uint16_t* y, double* y_exact, double* y_absdot, const uint16_t* x, const void* w,
                         int w_type, const uint16_t* scale, const uint16_t* offset, int64_t group_size,
                         int64_t M, int64_t N, int64_t K, int w_transpose)
{
    uint16_t* wf = (uint16_t*)malloc((size_t)(K * N) * sizeof(uint16_t));
    oq_antiquant(wf, OQ_F16, w, w_type, offset, scale, K, N, group_size, w_transpose, OQ_ARITH_F16);
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        double* acc = (double*)calloc((size_t)N, sizeof(double));
        double* aab = (double*)calloc((size_t)N, sizeof(double));
        for (int64_t k = 0; k < K; ++k) {
            double xv = oq_f16_to_f32(x[m * K + k]);
            if (xv == 0.0) continue;
            for (int64_t n = 0; n < N; ++n) {
                double p = xv * (double)oq_f16_to_f32(wf[w_transpose ? n * K + k : k * N + n]);
                acc[n] += p;
                aab[n] += fabs(p);
            }
        }
        for (int64_t n = 0; n < N; ++n) {
            if (y_exact) y_exact[m * N + n] = acc[n];
            if (y_absdot) y_absdot[m * N + n] = aab[n];
            if (y) y[m * N + n] = oq_f64_to_f16(acc[n], 1);
        }
        free(acc);
        free(aab);
    }
    free(wf);
}

/* ------------------------------------------------------------------------ */
/* QuantGroupMatmul (MoE)                                                    */
/* ------------------------------------------------------------------------ */

/* FasterGelu of the group-matmul example (quant_group_matmul_custom.asc:442-445), restating the fp32 op
 * sequence of the arch 3510 float path (impl/adv_api/detail/activation/gelu/gelu_3510_impl.h:113-122): Muls by
 * -1.702f, Exp, Adds 1, Div -- each an fp32 result (exp taken in double and rounded once to fp32, so it
 * overflows to inf above ~88.72 and the result is then -0, as on the reference). */
float oq_faster_gelu(float x)
{
    float t = x * (OQ_MUTANT == 16 ? 1.702f : -1.702f);
    float e = (float)exp((double)t);
    float d = e + 1.0f;
    return x / d;
}

/* examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/quant_group_matmul_high_performance/
 * quant_group_matmul_custom.asc: group rows [s_g, s_g+cnt_g) (Process :255-288), int32 accumulate on the
 * cube (MMCompute :296-334), then AscendDequant(acc x scale[g,n]) to fp32 (:433; its int32 -> fp32 conversion
 * rounds ties away from zero, as the dequant kernels do: oq_i32_to_f32_rna), Mul by perTokenScale[m]
 * (:439), act != 0: the sample's FasterGelu (:445, oq_faster_gelu in fp32 ops), and the final Cast (:450;
 * CAST_NONE = rint).
 * list_type 0: group_list holds G+1 int64 prefix offsets (offsets[0] = first row); 1: G int64 counts
 * (the reference's GetValue(groupIdx) counts, :263).  w [G,K,N] ND, or [G,N,K] when w_trans. */
void oq_group_matmul(void* y, int out_type, const int8_t* x, const float* pts, const int8_t* w, int w_trans,
                     const float* scale, const int64_t* group_list, int list_type, int64_t G, int64_t M,
                     int64_t K, int64_t N, int act)
{
    int64_t start = list_type == 0 ? group_list[0] : 0;
    for (int64_t g = 0; g < G; ++g) {
        int64_t cnt = list_type == 0 ? group_list[g + 1] - group_list[g] : group_list[g];
        int64_t s = start;
        start += cnt > 0 ? cnt : 0;
        if (cnt <= 0) continue;
        const int8_t* wg = w + g * K * N;
#pragma omp parallel for schedule(static)
        for (int64_t m = s; m < s + cnt; ++m) {
            if (m < 0 || m >= M) continue;
            for (int64_t n = 0; n < N; ++n) {
                int64_t acc = 0;
                for (int64_t k = 0; k < K; ++k)
                    acc += (int64_t)x[m * K + k] * (int64_t)(w_trans ? wg[n * K + k] : wg[k * N + n]);
                const int32_t a32 = (int32_t)(uint32_t)(uint64_t)acc;
                const float f = OQ_MUTANT == 38 ? (float)a32 : oq_i32_to_f32_rna(a32);
                float v = f * (OQ_MUTANT == 5 ? pts[m] : scale[g * N + n]);
                v = v * (OQ_MUTANT == 5 ? scale[g * N + n] : pts[m]);
                if (act) v = oq_faster_gelu(v);
                store_from_f32(y, out_type, m * N + n, v);
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* MX block-scaled matmul                                                    */
/* ------------------------------------------------------------------------ */

static inline float mx_elem(const uint8_t* p, int64_t idx, int fmt)
{
    if (fmt == OQ_FP4_E2M1 || fmt == OQ_FP4_E1M2) {
        uint8_t b = p[idx >> 1];
        const uint8_t nib = (idx & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 0xf);
        return (fmt == OQ_FP4_E1M2 && OQ_MUTANT != 35) ? oq_e1m2_decode(nib) : oq_e2m1_decode(nib);
    }
    return oq_fp8_decode(p[idx], fmt);
}

/* C[m,n] = sum_k a[m,k] 2^(SA[m,k/32]-127) * b[k,n] 2^(SB[k/32,n]-127), golden computed in fp64 and cast to
 * bf16 (examples/01_simd_cpp_api/05_best_practices/01_matrix_compute/matmul_mxfp4_high_performance/scripts/
 * gen_data.py:47-61; MmadMx include/basic_api/kernel_operator_mm_intf.h:348-352; type
 * impl/adv_api/detail/matmul/utils/matmul_type_def.h:114-131).  Packing: two fp4 per byte along the
 * contiguous axis, the even element in the low nibble (gen_data.py:25-34).
 * A [M,K]; B [K,N] (transB: [N,K]).  sK = ceil(K/64)*2 (gen_data.py:40).
 * scale_a_layout 0: scaleA [M, sK]; 1: [sK/2, M, 2].  scale_b_layout 0: scaleB [sK/2, N, 2] (the sample's
 * layout, gen_data.py:63 and README_en.md:64-66); 1: [N, sK].
 * elem_fmt: element type of A (OQ_FP4_E2M1, OQ_FP4_E1M2 -- the high-performance sample's fp4x2_e1m2_t,
 * matmul_mxfp4_high_performance/matmul_mx.h:117-133 --, OQ_FP8_E4M3, OQ_FP8_E5M2; fp8 elements are one per byte,
 * the MX-FP8 sample matmul_mx/matmul_mx.asc:90-244); B uses elem_fmt >> 8 when that is nonzero, else elem_fmt.
 * rows != NULL restricts the computation to the listed rows (C rows not listed are untouched).
 * C_blockmax (may be NULL): per output, the sum over 16-element K groups of the group's largest |a b|.
 * bias (may be NULL): f32 [N] added to the exact sum (the MX sample's SetBias, matmul_mx.asc:99-116,199-201);
 * its magnitude is counted into C_absdot. */
void oq_mx_matmul(uint16_t* C, double* C_exact, double* C_absdot, const uint8_t* A, const uint8_t* B,
                  const uint8_t* scaleA, const uint8_t* scaleB, int64_t M, int64_t N, int64_t K, int transB,
                  int scale_a_layout, int scale_b_layout, int elem_fmt, const int64_t* rows, int64_t n_rows,
                  double* C_blockmax, const float* bias)
{
    int64_t sK = (K + 63) / 64 * 2;
    int64_t nr = rows ? n_rows : M;
    const int fmt_b = (elem_fmt >> 8) ? (elem_fmt >> 8) : elem_fmt;
    elem_fmt &= 0xff;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < nr; ++r) {
        int64_t m = rows ? rows[r] : r;
        double* arow = (double*)malloc((size_t)K * sizeof(double));
        for (int64_t k = 0; k < K; ++k) {
            int64_t kb = k / 32;
            uint8_t sa = scale_a_layout == 0 ? scaleA[m * sK + kb] : scaleA[(kb / 2) * M * 2 + m * 2 + (kb & 1)];
            arow[k] = (double)mx_elem(A, m * K + k, elem_fmt) * (double)oq_e8m0_decode(sa);
        }
        for (int64_t n = 0; n < N; ++n) {
            double s = 0.0, sa_ = 0.0, sbm = 0.0, bmx = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                int64_t kb = k / 32;
                uint8_t sb = (scale_b_layout == 0 && OQ_MUTANT != 6) ? scaleB[(kb / 2) * N * 2 + n * 2 + (kb & 1)]
                                                                     : scaleB[n * sK + kb];
                double b = (double)mx_elem(B, transB ? n * K + k : k * N + n, fmt_b) * (double)oq_e8m0_decode(sb);
                double p = arow[k] * b;
                s += p;
                sa_ += fabs(p);
                if (fabs(p) > bmx) bmx = fabs(p);
                if (k % 16 == 15 || k == K - 1) {
                    sbm += bmx;
                    bmx = 0.0;
                }
            }
            if (bias && OQ_MUTANT != 36) {
                s += (double)bias[n];
                sa_ += fabs((double)bias[n]);
            }
            if (C_exact) C_exact[m * N + n] = s;
            if (C_absdot) C_absdot[m * N + n] = sa_;
            if (C_blockmax) C_blockmax[m * N + n] = sbm;
            if (C) C[m * N + n] = oq_f64_to_bf16(s, 1);
        }
        free(arow);
    }
}

/* ------------------------------------------------------------------------ */
/* IterateAll enAtomic                                                       */
/* ------------------------------------------------------------------------ */

/* C = op(C, v) element-wise in C's type (IterateAll(gm, enAtomic): ATOMIC_ADD / MAX / MIN = 1 / 2 / 3,
 * impl/adv_api/detail/matmul/utils/matmul_config_utils.h:53-55; the copy-out sets SetAtomicAdd/Max/Min<DstT>,
 * scheduler/base/scheduler_base.h:484-494, and "adds the copied data to what GM holds" --
 * docs/zh/api/SIMD-API/basic_api/atomic_operations/SetAtomicAdd.md).  c_type: OQ_INT32 (add wraps, signed
 * max / min), OQ_F32, OQ_F16, OQ_BF16 (add: the exact sum rounded once to C's type, rne, overflow to inf).
 * max / min keep C unless v compares greater / smaller, so a NaN never replaces and is never replaced and a
 * zero of the other sign does not replace a zero.  Parity unpinned: the saturation of the hardware's half /
 * bf16 accumulation and its NaN handling are not published; this restates the IEEE behaviour. */
static double combine_val(uint32_t bits, int t)
{
    if (t == OQ_F32) { float f; memcpy(&f, &bits, 4); return f; }
    if (t == OQ_F16) return oq_f16_to_f32((uint16_t)bits);
    return oq_bf16_to_f32((uint16_t)bits);
}

void oq_c_combine(void* c, const void* v, int c_type, int op, int64_t count)
{
    const int es = (c_type == OQ_INT32 || c_type == OQ_F32) ? 4 : 2;
    for (int64_t i = 0; i < count; ++i) {
        uint32_t a = 0, b = 0;
        memcpy(&a, (const uint8_t*)c + i * es, es);
        memcpy(&b, (const uint8_t*)v + i * es, es);
        uint32_t r = a;
        if (c_type == OQ_INT32) {
            if (op == 1) r = a + b;
            else if (op == 2) r = (int32_t)b > (int32_t)a ? b : a;
            else r = (int32_t)b < (int32_t)a ? b : a;
        } else {
            const double x = combine_val(a, c_type), y = combine_val(b, c_type);
            if (op == 1) {
                const double s = x + y; /* exact: two f32 / f16 / bf16 values sum exactly in fp64 unless their
                                           exponents differ by more than 29, where the rounding cannot change */
                if (c_type == OQ_F32) {
                    const float f = (float)s;
                    memcpy(&r, &f, 4);
                } else if (c_type == OQ_F16) {
                    r = oq_f64_to_f16(s, 0);
                } else {
                    r = oq_f64_to_bf16(s, 0);
                }
            } else if (op == 2) {
                r = (OQ_MUTANT == 37 ? y < x : y > x) ? b : a;
            } else {
                r = (OQ_MUTANT == 37 ? y > x : y < x) ? b : a;
            }
        }
        memcpy((uint8_t*)c + i * es, &r, es);
    }
}

/* MX quantisation along the contiguous axis (rows of length K): shared exponent per 32 elements from the
 * block absmax (oq_mx_shared_exp), elements = E2M1 rne of x / 2^(e-127).  Output: packed [R, K/2] and
 * scales [R, K/32] row-major.  Used to build MX inputs the way the MX-FP4 workload specifies them. */
void oq_mx_quantize_fp4(uint8_t* packed, uint8_t* scales, const float* x, int64_t R, int64_t K)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < R; ++r)
        for (int64_t kb = 0; kb < K / 32; ++kb) {
            const float* blk = x + r * K + kb * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(blk[i]));
            uint8_t e = oq_mx_shared_exp(amax);
            scales[r * (K / 32) + kb] = e;
            float inv = 1.0f / oq_e8m0_decode(e); /* power of two: exact */
            for (int i = 0; i < 32; i += 2) {
                uint8_t lo = oq_e2m1_encode_rne(blk[i] * inv);
                uint8_t hi = oq_e2m1_encode_rne(blk[i + 1] * inv);
                packed[r * (K / 2) + kb * 16 + i / 2] = (uint8_t)(lo | (hi << 4));
            }
        }
}

/* ------------------------------------------------------------------------ */
/* NZ fractal <-> ND                                                         */
/* ------------------------------------------------------------------------ */

/* CubeFormat::NZ (include/adv_api/matmul/matmul_config.h:23-35), as the group-matmul generator writes its weights
 * (quant_group_matmul_high_performance/scripts/gen_data.py:62: reshape [G, k/16, 16, n/32, 32], transpose
 * (0, 3, 1, 2, 4)): element (r, c) of matrix b at byte
 *   b * nz_mat + ((cb * r16 + r / 16) * 16 + r % 16) * 32 + (c * esize) % 32,   cb = (c * esize) / 32,
 * r16 = ceil(rows / 16), nz_mat = ceil(cols * esize / 32) * r16 * 512.  Element by element, byte by byte. */
static int64_t nz_index(int64_t b, int64_t r, int64_t cbyte, int64_t rows, int64_t cols_b)
{
    int64_t r16 = (rows + 15) / 16, c32 = (cols_b + 31) / 32;
    int64_t cb = cbyte / 32;
    return b * c32 * r16 * 512 + ((cb * r16 + r / 16) * 16 + r % 16) * 32 + cbyte % 32;
}

void oq_nz_to_nd(uint8_t* dst, const uint8_t* src, int esize, int64_t batch, int64_t rows, int64_t cols,
                 int transpose_out)
{
    int64_t cols_b = cols * esize;
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t c = 0; c < cols; ++c)
                for (int e = 0; e < esize; ++e) {
                    uint8_t v = src[nz_index(b, r, c * esize + e, rows, cols_b)];
                    if (transpose_out) dst[(b * cols + c) * rows * esize + r * esize + e] = v;
                    else dst[(b * rows + r) * cols_b + c * esize + e] = v;
                }
}

void oq_nd_to_nz(uint8_t* dst, const uint8_t* src, int esize, int64_t batch, int64_t rows, int64_t cols)
{
    int64_t cols_b = cols * esize, r16 = (rows + 15) / 16, c32 = (cols_b + 31) / 32;
    memset(dst, 0, (size_t)(batch * c32 * r16 * 512));
    for (int64_t b = 0; b < batch; ++b)
        for (int64_t r = 0; r < rows; ++r)
            for (int64_t cb = 0; cb < cols_b; ++cb) dst[nz_index(b, r, cb, rows, cols_b)] = src[(b * rows + r) * cols_b + cb];
}
