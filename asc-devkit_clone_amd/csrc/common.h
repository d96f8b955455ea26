// common.h -- shared device helpers for the gfx950 kernels of libascq.
//
// Numeric conventions (the same as the reference arithmetic restated for this library):
//  * f16 / bf16 travel as uint16_t bit patterns;
//  * conversions to f16 / bf16 round to nearest even and saturate to the finite range
//    (docs/zh/api/SIMD-API/basic_api/data_structures/precision_conversion.md:30), NaN stays NaN;
//  * every fp32 operation is one IEEE operation: the library is built with -ffp-contract=off
//    so a multiply followed by an add never becomes an fma unless written as one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include "launch.h"

namespace ascq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float f2x __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef short s8v __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// dtype / round-mode codes shared with include/ascq.h
enum : int32_t {
    DT_INT8 = 1, DT_UINT8 = 2, DT_INT4 = 3, DT_INT32 = 4, DT_F16 = 5, DT_BF16 = 6, DT_F32 = 7, DT_U64 = 8,
    DT_FP8_E4M3 = 9, DT_FP8_E5M2 = 10, DT_FP4_E2M1 = 11, DT_E8M0 = 12, DT_INT64 = 13, DT_FP4_E1M2 = 14, DT_HIF8 = 15
};
enum : int32_t { RM_NONE = 0, RM_RINT = 1, RM_FLOOR = 2, RM_CEIL = 3, RM_ROUND = 4, RM_TRUNC = 5 };

__device__ __forceinline__ uint16_t h_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }
__device__ __forceinline__ _Float16 bits_h(uint16_t u) { return __builtin_bit_cast(_Float16, u); }

// fp32 -> f16, rne, saturating (|x| > 65504 -> +-65504; NaN kept)
__device__ __forceinline__ uint16_t f32_to_f16_sat(float x)
{
    float c = __builtin_fabsf(x) > 65504.0f ? __builtin_copysignf(65504.0f, x) : x;
    return h_bits((_Float16)c);
}
// fp32 -> f16, rne, IEEE overflow to inf
__device__ __forceinline__ uint16_t f32_to_f16(float x) { return h_bits((_Float16)x); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)bits_h(h); }

// fp32 -> bf16, rne, saturating (overflow and inf -> +-max finite, NaN quieted)
__device__ __forceinline__ uint16_t f32_to_bf16_sat(float x)
{
    // the hardware rne conversion (v_cvt_pk_bf16_f32: equal to the bit-level rne on all 2^32 inputs but NaN,
    // checked exhaustively on gfx950), then selects instead of branches: an overflow to inf saturates to +-max
    // finite (0x7F7F), a NaN keeps its sign and top payload bits, quieted
    const uint32_t u = __float_as_uint(x);
    uint32_t b = __builtin_bit_cast(uint16_t, (__bf16)x);
    b = (b & 0x7fffu) == 0x7f80u ? ((b & 0x8000u) | 0x7f7fu) : b;
    return (u & 0x7fffffffu) > 0x7f800000u ? (uint16_t)((u >> 16) | 0x40u) : (uint16_t)b;
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// fp32 -> bf16 value (kept in an fp32 register): rne, overflow to inf, NaN kept
__device__ __forceinline__ float bf16_round(float x)  // rne to bf16, overflow to inf, NaN kept
{
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    return __uint_as_float(((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16);
}

// QUANT_PRE word -> M1 multiplier: bits [31:13] as fp32, low 13 bits cleared
__device__ __forceinline__ float quant_pre_m1(uint64_t w) { return __uint_as_float((uint32_t)w & 0xFFFFE000u); }

// FasterGelu, x / (1 + exp(-1.702 x)) in fp32 (impl/adv_api/detail/activation/gelu/gelu_3510_impl.h:113-122).
// While -1.702 x < 64 (1 + exp < 2^93, a normal reciprocal) with the hardware exp2 (v_exp_f32 of -1.702 x
// log2(e)) and reciprocal (v_rcp_f32): both accurate to about an fp32 ulp, so the result is within ~|2.5 x| fp32
// ulps of the correctly rounded expression -- far below one f16 / bf16 output ulp -- at a quarter of the cost
// of expf and an IEEE division.  Beyond (x < -37.6, results below ~1e-26 that bf16 still represents, down to
// its subnormals) and for NaN: expf and the IEEE division; for x -> -inf the exp overflows to inf and the
// result is -0, as there.
__device__ __forceinline__ float faster_gelu(float x)
{
    const float t = -1.702f * x;
    if (t < 64.0f) return x * __builtin_amdgcn_rcpf(1.0f + __expf(t));
    return x / (1.0f + expf(t));
}

// (V)REQ8 / (V)QF322B8_PRE after the multiply by M1 (examples/02_simd_c_api/03_c_api/03_matrix_compute/
// asc_copy_l0c2gm/scripts/gen_data_s322s8.py:56-80): NaN -> 0, clamp to [-256, 255], round half to even, add
// the word's 9-bit offset (bits 37-45, 0..511), saturate to int8 when the sign flag (bit 46) is set, else to
// uint8.  Bits 32-36 (shift, mode control) are ignored, as on arch 3510.
__device__ __forceinline__ uint8_t requant8(float v, uint64_t w)
{
    if (v != v) v = 0.0f;  // fmaxf would turn NaN into -256
    const float c = fminf(fmaxf(v, -256.0f), 255.0f);
    const int t = (int)__builtin_rintf(c) + (int)((w >> 37) & 0x1FFu);
    if ((w >> 46) & 1u) return (uint8_t)(int8_t)(t < -128 ? -128 : (t > 127 ? 127 : t));
    return (uint8_t)(t < 0 ? 0 : (t > 255 ? 255 : t));
}

// (V)REQ4 / (V)QF322S4_PRE after the multiply by M1: the same 9-bit intermediate as REQ8 (NaN -> 0, clamp to
// [-256, 255], rint, + the word's offset), then saturation to int4 [-8, 7]
// (docs/zh/api/SIMD-API/c_api/cube_datamove/cube_store_aux_config/asc_set_l0c_copy_prequant.md:37-41, 106;
// docs/zh/api/appendix/matrix_compute_move_out_interface_boundary_value_summary.md:110-111).  Returns the code in
// the low 4 bits.
__device__ __forceinline__ uint32_t requant4(float v, uint64_t w)
{
    if (v != v) v = 0.0f;
    const float c = fminf(fmaxf(v, -256.0f), 255.0f);
    const int t = (int)__builtin_rintf(c) + (int)((w >> 37) & 0x1FFu);
    return (uint32_t)(t < -8 ? -8 : (t > 7 ? 7 : t)) & 0xFu;
}

// f32 -> fp8 with round to nearest even, on the bit pattern.  e4m3fn (fmt 0) saturates as the fixpipe's default
// mode does: |x| >= 448 and +-inf give +-448, NaN gives 0.  e5m2 (fmt 1): overflow (|x| >= 61440) gives +-inf,
// NaN gives 0x7F.  Normal results: add the rounding bias below the kept mantissa bits (half minus one, plus the
// kept LSB for ties to even) and shift; subnormal results: scale to the subnormal step and rint.
__device__ __forceinline__ uint8_t f32_to_fp8(float x, int fmt)
{
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
    if (fmt == 0) {
        if (a > 0x7F800000u) return 0;
        if (a >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);  // 448
        if (a < 0x3C800000u)                                   // below 2^-6: multiples of 2^-9
            return (uint8_t)(sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f));
        const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
        return (uint8_t)(sign | (r - (120u << 3)));
    }
    if (a > 0x7F800000u) return 0x7Fu;
    if (a >= 0x47700000u) return (uint8_t)(sign | 0x7Cu);     // 61440 rounds to inf
    if (a < 0x38800000u)                                       // below 2^-14: multiples of 2^-16
        return (uint8_t)(sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 65536.0f));
    const uint32_t r = (a + 0xFFFFFu + ((a >> 21) & 1u)) >> 21;
    return (uint8_t)(sign | (r - (112u << 2)));
}

// fp8 bits -> fp32 from the OCP format definitions: e4m3fn (bias 7, S.1111.111 = NaN, no inf) or e5m2 (bias 15,
// exponent 31 = inf / NaN); every code is exact in fp32
__device__ __forceinline__ float fp8_bits_to_f32(uint32_t v, bool e5m2)
{
    const uint32_t s = (v & 0x80u) << 24;
    if (!e5m2) {
        const uint32_t e = (v >> 3) & 15u, m = v & 7u;
        if (e == 15u && m == 7u) return __uint_as_float(0x7fc00000u);
        if (e == 0u) return __uint_as_float(s | __float_as_uint((float)m * 0x1p-9f));
        return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
    }
    const uint32_t e = (v >> 2) & 31u, m = v & 3u;
    if (e == 31u) return __uint_as_float(m ? 0x7fc00000u : (s | 0x7f800000u));
    if (e == 0u) return __uint_as_float(s | __float_as_uint((float)m * 0x1p-16f));
    return __uint_as_float(s | ((e + 112u) << 23) | (m << 21));
}

// E2M1 nibble -> fp32 (OCP MX v1.0: S.EE.M, bias 1; magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6)
__device__ __forceinline__ float e2m1_to_f32(uint32_t nib)
{
    const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
    const float mag = e == 0u ? 0.5f * (float)m : (1.0f + 0.5f * (float)m) * (float)(1u << (e - 1u));
    return (nib & 8u) ? -mag : mag;
}

// HiFloat8 (the layout of the reference's decoder, impl/utils/debug/npu_arch_9201/asc_type_conversion_utils.h:62-149):
// bit 7 sign; a prefix-coded dot field from bit 6 selects the exponent width w -- 11: 4, 10: 3, 01: 2, 001: 1,
// 0001: 0 -- and the mantissa gets the 7 - |dot| - w remaining bits; the exponent field holds the exponent's sign in
// its top bit and its magnitude with that bit standing for an implicit 1; dot 0000 is the subnormal class 2^(M - 23)
// (M = 0: zero, or NaN with the sign bit); 0x6F / 0xEF are +-inf.  Every code is exact in f16 and f32.
__device__ __forceinline__ float hif8_to_f32(uint32_t c)
{
    const uint32_t s = (c & 0x80u) << 24, b = c & 0x7fu;
    if (c == 0x80u) return __uint_as_float(0x7fc00000u);
    if (b == 0x6Fu) return __uint_as_float(s | 0x7f800000u);
    if ((b & 0x78u) == 0u) return b == 0u ? 0.0f : __uint_as_float(s | ((b + 104u) << 23));  // 2^(M - 23)
    // exponent width w and mantissa width mw from the dot field
    const uint32_t top = b >> 5;
    const uint32_t w = top == 3u ? 4u : (top == 2u ? 3u : (top == 1u ? 2u : ((b >> 4) & 1u)));
    const uint32_t mw = top >= 2u ? 4u - top : 3u;  // 11: 1, 10: 2, else 3
    const uint32_t field = (b >> mw) & ((1u << w) - 1u);
    const uint32_t mag = w ? ((field & ((1u << (w - 1u)) - 1u)) | (1u << (w - 1u))) : 0u;
    const int32_t e = (w && (field >> (w - 1u))) ? -(int32_t)mag : (int32_t)mag;
    const uint32_t m = b & ((1u << mw) - 1u);
    return __uint_as_float(s | ((uint32_t)(e + 127) << 23) | (m << (23u - mw)));
}

// x -> HiFloat8 with ties away from zero and saturation (Cast<hifloat8_t, half | float> under CAST_ROUND with SatS,
// docs/zh/api/SIMD-API/basic_api/reg_vector_compute/type_conversion/Cast.md:254-348): NaN -> 0; |x| < 2^-23 -> 0
// (whatever the sign); [2^-23, 2^-22) -> the smallest subnormal; the subnormal class rounds between powers of two on
// the first fraction bit; otherwise the mantissa keeps 3 / 2 / 1 bits for |E| <= 3 / <= 7 / <= 15 and rounds up on
// the next bit, carrying into the exponent; every overflow (E > 15, or E = 15 with a mantissa bit, the inf code)
// saturates to +-32768.  Returns the code in the low 8 bits.
__device__ __forceinline__ uint32_t hif8_code_rna_sat(float x)
{
    const uint32_t u = __float_as_uint(x), a = u & 0x7fffffffu, s = (u >> 24) & 0x80u;
    int32_t e = (int32_t)(a >> 23) - 127;
    const uint32_t f = a & 0x7fffffu;
    if (a > 0x7f800000u || e < -23) return 0u;  // NaN, zero, tiny
    if (e == -23) return s | 1u;
    uint32_t m = 0u;
    if (e <= -16) {
        e += (int32_t)(f >> 22);
        if (e <= -16) return s | (uint32_t)(e + 23);
    } else if (e <= 15) {
        const uint32_t ae0 = (uint32_t)(e < 0 ? -e : e);
        const uint32_t mw = ae0 <= 3u ? 3u : (ae0 <= 7u ? 2u : 1u);
        m = (f >> (23u - mw)) + ((f >> (22u - mw)) & 1u);
        if (m >> mw) m = 0u, ++e;
    }
    if (e > 15 || (e == 15 && m)) return s | 0x6Eu;
    const uint32_t ae = (uint32_t)(e < 0 ? -e : e), ng = e < 0 ? 1u : 0u;
    uint32_t c;
    if (ae == 0u) c = 0x08u;
    else if (ae == 1u) c = 0x10u | (ng << 3);
    else if (ae <= 3u) c = 0x20u | (((ng << 1) | (ae & 1u)) << 3);
    else if (ae <= 7u) c = 0x40u | (((ng << 2) | (ae & 3u)) << 2);
    else c = 0x60u | (((ng << 3) | (ae & 7u)) << 1);
    return s | c | m;
}

// E1M2 nibble: sign | 1-bit exponent (bias 1) | 2-bit mantissa, magnitudes {0, .25, .5, .75, 1, 1.25, 1.5, 1.75}
// -- the 3-bit magnitude code times 0.25 (docs/zh/api/appendix/mmad_mx_interface_boundary_value_summary.md:11:
// largest finite 1.75)
__device__ __forceinline__ float e1m2_to_f32(uint32_t nib)
{
    const float mag = (float)(nib & 7u) * 0.25f;
    return (nib & 8u) ? -mag : mag;
}

// RoundMode to integral float
__device__ __forceinline__ float round_mode_f(float v, int mode)
{
    switch (mode) {
    case RM_FLOOR: return __builtin_floorf(v);
    case RM_CEIL: return __builtin_ceilf(v);
    case RM_ROUND: return __builtin_roundf(v);
    case RM_TRUNC: return __builtin_truncf(v);
    default: return __builtin_rintf(v);
    }
}

// integral float -> int8 with saturation; NaN -> 0
__device__ __forceinline__ int32_t sat_s8_from_integral(float r)
{
    if (r != r) return 0;
    r = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
    return (int32_t)r;
}

template <int MODE>
__device__ __forceinline__ int32_t quant_s8(float v)
{
    float r;
    if constexpr (MODE == RM_FLOOR) r = __builtin_floorf(v);
    else if constexpr (MODE == RM_CEIL) r = __builtin_ceilf(v);
    else if constexpr (MODE == RM_ROUND) r = __builtin_roundf(v);
    else if constexpr (MODE == RM_TRUNC) r = __builtin_truncf(v);
    else r = __builtin_rintf(v);
    return sat_s8_from_integral(r);
}

__device__ __forceinline__ uint32_t pack4_s8(int32_t a, int32_t b, int32_t c, int32_t d)
{
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// int32 -> fp32 with ties away from zero (the AscendDequant kernels' Cast<float, int32_t, MrgZRndA>, CAST_ROUND):
// exact below 2^24; above, the magnitude's 24-bit significand is rounded half up (add half of the dropped range,
// truncate) and the result converts exactly
__device__ __forceinline__ float i32_to_f32_rna(int32_t v)
{
    uint32_t a = v < 0 ? 0u - (uint32_t)v : (uint32_t)v;
    const int s = 8 - (int)__builtin_clz(a | 1u);  // bits below the 24-bit significand (<= 0: none)
    if (s > 0) a = ((a + (1u << (s - 1))) >> s) << s;
    const float f = (float)a;
    return v < 0 ? -f : f;
}
// |v| > 2^24: the only values whose nearest-even conversion (float)v can differ from i32_to_f32_rna
__device__ __forceinline__ bool i32_beyond_f32_exact(int32_t v) { return (uint32_t)v + (1u << 24) > (2u << 24); }

// store an fp32 value as dtype (F16 / BF16 / F32), rne + sat
__device__ __forceinline__ void store_cast(void* p, int64_t i, float v, int dtype)
{
    if (dtype == DT_F16) ((uint16_t*)p)[i] = f32_to_f16_sat(v);
    else if (dtype == DT_BF16) ((uint16_t*)p)[i] = f32_to_bf16_sat(v);
    else ((float*)p)[i] = v;
}

__device__ __forceinline__ float load_f32_of(const void* p, int64_t i, int dtype)
{
    switch (dtype) {
    case DT_F16: return f16_to_f32(((const uint16_t*)p)[i]);
    case DT_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
    case DT_F32: return ((const float*)p)[i];
    case DT_INT32: return (float)((const int32_t*)p)[i];
    case DT_INT8: return (float)((const int8_t*)p)[i];
    case DT_U64: return __uint_as_float((uint32_t)((const uint64_t*)p)[i]);
    default: return 0.0f;
    }
}

// Division by a runtime-constant divisor d (1 <= d < 2^31) for dividends below 2^31: n / d = (umulhi(n, m) + n) >> s
// with s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1 (the round-up multiplier method)
struct FastDiv {
    uint32_t m, s;
};
static inline FastDiv fast_div(uint32_t d)
{
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    return FastDiv{(uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1), s};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) { return (__umulhi(n, f.m) + n) >> f.s; }

// wave64 reductions
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// The combined bits of one C element.  int32: wrapping add, signed max / min.  f32: IEEE add (rne).  f16 / bf16:
// the fp32 sum of the two values rounded once to the C type (rne, overflow to inf); an fp32 intermediate
// (24 bits >= 2p + 1 for p = 11 and 8) makes the double rounding innocuous, so this is the correctly rounded
// f16 / bf16 sum.  max / min: the new value replaces the old one only when it compares greater / smaller (a NaN
// never replaces and is never replaced; +0 and -0 compare equal, so the old zero stays).
template <int DT>
__device__ __forceinline__ uint32_t c_combine(uint32_t old, uint32_t v, int op)
{
    if constexpr (DT == DT_INT32) {
        const int32_t a = (int32_t)old, b = (int32_t)v;
        if (op == C_ADD) return old + v;
        return (op == C_MAX ? b > a : b < a) ? v : old;
    } else {
        const float a = DT == DT_F32 ? __uint_as_float(old) : (DT == DT_F16 ? f16_to_f32((uint16_t)old) : bf16_to_f32((uint16_t)old));
        const float b = DT == DT_F32 ? __uint_as_float(v) : (DT == DT_F16 ? f16_to_f32((uint16_t)v) : bf16_to_f32((uint16_t)v));
        if (op == C_ADD) {
            const float s = a + b;
            if constexpr (DT == DT_F32) return __float_as_uint(s);
            else if constexpr (DT == DT_F16) return f32_to_f16(s);
            else return __float_as_uint(bf16_round(s)) >> 16;
        }
        return (op == C_MAX ? b > a : b < a) ? v : old;
    }
}

// C[p] = combine(C[p], v) as one atomic operation: the native int32 atomics, else a compare-and-swap loop on the
// aligned 32-bit word that holds the element (it ends once no other writer changed the word in between).
template <int DT>
__device__ __forceinline__ void c_atomic(uint8_t* p, uint32_t v, int op)
{
    if constexpr (DT == DT_INT32) {
        if (op == C_ADD) atomicAdd((int*)p, (int)v);
        else if (op == C_MAX) atomicMax((int*)p, (int)v);
        else atomicMin((int*)p, (int)v);
    } else {
        constexpr bool W16 = DT != DT_F32;
        unsigned* w = (unsigned*)((uintptr_t)p & ~(uintptr_t)3);
        const uint32_t sh = W16 ? (uint32_t)((uintptr_t)p & 2) * 8u : 0u;
        const uint32_t mask = W16 ? 0xFFFFu << sh : 0xFFFFFFFFu;
        unsigned old = *(volatile unsigned*)w;
        for (;;) {
            const uint32_t cur = W16 ? (old & mask) >> sh : old;
            const uint32_t nv = c_combine<DT>(cur, v, op);
            if (nv == cur) break;
            const unsigned nw = W16 ? (old & ~mask) | (nv << sh) : nv;
            const unsigned prev = atomicCAS(w, old, nw);
            if (prev == old) break;
            old = prev;
        }
    }
}

}  // namespace ascq
