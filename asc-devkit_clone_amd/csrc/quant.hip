// quant.hip -- AscendQuant / AscendDequant / AscendAntiQuant for gfx950.
//
// These ops are HBM-bound streams.  Layout in HBM is the reference's: row-major [m, n] tensors, one
// scale per row (per-token) or per column (per-channel).  Each kernel moves 16-byte vectors per lane so a
// wave issues 1 KiB contiguous requests; the per-token dynamic quant keeps a whole row in registers so
// the input is read from HBM exactly once (absmax pass and quantise pass share the registers).
//
// Reference arithmetic (see include/ascq.h for the entry points):
//  per-token quant   impl/adv_api/detail/quantization/quant/ascend_quant_per_group_3510_impl.h:142-178
//                    + TransRegForS8 ascend_quant_3510_impl.h:958-968 -> sat_s8(round(f32(x)*s (+o)))
//  legacy quant      ascend_quant_pre_impl.h:101-164 (half Mul, half Add, Cast<int8_t,half> rint/sat)
//  dequant           ascend_dequant_3510_impl.h:37-75, 254-287; ascend_dequant_common_impl.h:196-364
//  antiquant         ascend_antiquant_impl.h:63-96 (half ops), ascend_antiquant_c220_impl.h:46-75 (fp32 ops)
#include "common.h"
#include "launch.h"

namespace ascq {

// ---------------------------------------------------------------------------------------------
// Dynamic per-token quant, f16 / bf16 input, row resident in registers.
// One 256-thread workgroup per row; thread t holds 16-byte chunks t, t+256, ... (VEC of them).
// ---------------------------------------------------------------------------------------------
template <bool BF16>
__device__ __forceinline__ float half_bits_to_f32(uint32_t w, int hi)
{
    uint16_t b = (uint16_t)(hi ? (w >> 16) : (w & 0xffffu));
    return BF16 ? bf16_to_f32(b) : f16_to_f32(b);
}

template <int VEC, int MODE, bool BF16>
__global__ __launch_bounds__(256) void quant_dyn_row_kernel(const u32x4* __restrict__ x, u32x2* __restrict__ q,
                                                            float* __restrict__ scale_out, uint32_t chunks)
{
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const u32x4* xr = x + (size_t)row * chunks;
    u32x4 v[VEC];
    float amax = 0.0f;
    h2 hmax = {(_Float16)0.0f, (_Float16)0.0f};
    // every lane loads VEC chunks unconditionally (a chunk past the row end repeats the row's last chunk: the
    // absmax is unchanged and it is not stored), so all VEC loads are in flight before the first wait
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        const uint32_t c = t + j * 256u;
        v[j] = __builtin_nontemporal_load(xr + (c < chunks ? c : chunks - 1u));
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (BF16) {
                amax = __builtin_fmaxf(amax, __builtin_fabsf(half_bits_to_f32<true>(w4[e], 0)));
                amax = __builtin_fmaxf(amax, __builtin_fabsf(half_bits_to_f32<true>(w4[e], 1)));
            } else {
                // |h| via the sign mask, packed f16 maxNum (NaN ignored, like the oracle)
                h2 a = __builtin_bit_cast(h2, w4[e] & 0x7fff7fffu);
                hmax = __builtin_elementwise_max(hmax, a);
            }
        }
    }
    if constexpr (!BF16) amax = __builtin_fmaxf((float)hmax.x, (float)hmax.y);
    amax = wave_max(amax);
    if ((t & 63u) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float mult = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (t == 0) scale_out[row] = amax / 127.0f;
    u32x2* qr = q + (size_t)row * chunks;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        uint32_t c = t + j * 256u;
        if (c >= chunks) break;
        uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
        int32_t r[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            r[2 * e] = quant_s8<MODE>(half_bits_to_f32<BF16>(w4[e], 0) * mult);
            r[2 * e + 1] = quant_s8<MODE>(half_bits_to_f32<BF16>(w4[e], 1) * mult);
        }
        u32x2 o = {pack4_s8(r[0], r[1], r[2], r[3]), pack4_s8(r[4], r[5], r[6], r[7])};
        __builtin_nontemporal_store(o, qr + c);
    }
}

// Generic dynamic per-token quant (any n, f16 / bf16 / f32 input): one workgroup per row, two passes
// over the row (the second pass hits L2).
template <int MODE>
__global__ __launch_bounds__(256) void quant_dyn_generic_kernel(const void* __restrict__ x, int8_t* __restrict__ q,
                                                                float* __restrict__ scale_out, uint32_t n,
                                                                int src_type)
{
    __shared__ float red[4];
    const uint32_t row = blockIdx.x;
    const uint32_t t = threadIdx.x;
    const int64_t base = (int64_t)row * n;
    float amax = 0.0f;
    for (uint32_t j = t; j < n; j += 256u) amax = __builtin_fmaxf(amax, __builtin_fabsf(load_f32_of(x, base + j, src_type)));
    amax = wave_max(amax);
    if ((t & 63u) == 0) red[t >> 6] = amax;
    __syncthreads();
    amax = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    const float mult = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (t == 0) scale_out[row] = amax / 127.0f;
    for (uint32_t j = t; j < n; j += 256u) q[base + j] = (int8_t)quant_s8<MODE>(load_f32_of(x, base + j, src_type) * mult);
}

// ---------------------------------------------------------------------------------------------
// Dequant
// ---------------------------------------------------------------------------------------------
// Fast path: int8 [m, n] x fp32 scale[row] -> f16, n % 8 == 0.  A block owns one row segment of 256 * U
// units of 8 elements; lane t converts units t, t + 256, ... (8-byte loads, 16-byte stores, both contiguous
// across the wave), so every store instruction writes whole cache lines.  The row and its scale are per-block
// scalars: no per-element index division.
template <int U>
__global__ __launch_bounds__(256) void dequant_i8_token_f16_kernel(const u32x2* __restrict__ q,
                                                                   const float* __restrict__ scale,
                                                                   u32x4* __restrict__ y, uint32_t units_per_row,
                                                                   uint32_t segs)
{
    const uint32_t row = blockIdx.x / segs;
    const uint32_t u0 = (blockIdx.x - row * segs) * (256u * U) + threadIdx.x;
    const size_t base = (size_t)row * units_per_row;
    const float s = scale[row];
    u32x2 v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {  // unconditional (past the row end: the row's last unit, not stored)
        const uint32_t u = u0 + k * 256u;
        v[k] = __builtin_nontemporal_load(q + base + (u < units_per_row ? u : units_per_row - 1u));
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t u = u0 + k * 256u;
        if (u >= units_per_row) break;
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int32_t w = (int32_t)v[k][e];
            const float f0 = (float)((w << 24) >> 24) * s;
            const float f1 = (float)((w << 16) >> 24) * s;
            const float f2 = (float)((w << 8) >> 24) * s;
            const float f3 = (float)(w >> 24) * s;
            o[2 * e] = (uint32_t)f32_to_f16_sat(f0) | ((uint32_t)f32_to_f16_sat(f1) << 16);
            o[2 * e + 1] = (uint32_t)f32_to_f16_sat(f2) | ((uint32_t)f32_to_f16_sat(f3) << 16);
        }
        __builtin_nontemporal_store((u32x4){o[0], o[1], o[2], o[3]}, y + base + u);
    }
}

// Scale addressing of the dequant kernels (DequantArgs::smode): one scalar; scale[c] (legacy deqScale tensor);
// scale[r] (PER_TOKEN); scale[r][c / g] over [rows][sk] (PER_GROUP kDim 1); scale[r / g][c] over
// [ceil(rows / g)][n] (PER_GROUP kDim 0).
enum : int { DQ_SCALAR = 0, DQ_COL = 1, DQ_ROW = 2, DQ_GROUP_COL = 3, DQ_GROUP_ROW = 4 };

struct DequantArgs {
    void* y;
    const void* src;
    const void* scale;
    float scale_scalar;
    int scale_type;       // DT_F32 / DT_F16 / DT_BF16 / DT_U64 (low 32 bits as fp32)
    uint32_t rows, cols;  // computed block: rows x cols (cols = calCount of the legacy form, else n)
    uint32_t n, ldd;      // source and destination row strides (elements)
    uint32_t group, sk;   // PER_GROUP group size; scales per row for DQ_GROUP_COL
    uint32_t units, upr;  // vector kernel: work units and units per row band
    FastDiv upr_div, g_div;
};

__device__ __forceinline__ float dq_src_f32(const void* p, int64_t i, int src_type)
{
    if (src_type == DT_INT32) return i32_to_f32_rna(((const int32_t*)p)[i]);
    if (src_type == DT_INT8) return (float)((const int8_t*)p)[i];
    return ((const float*)p)[i];
}

__device__ __forceinline__ float dq_scale_at(const void* s, int64_t i, int type)
{
    switch (type) {
    case DT_F16: return f16_to_f32(((const uint16_t*)s)[i]);
    case DT_BF16: return bf16_to_f32(((const uint16_t*)s)[i]);
    case DT_U64: return __uint_as_float(((const uint32_t*)s)[2 * i]);
    default: return ((const float*)s)[i];
    }
}

// Any shape or alignment: one thread per computed element, 64-bit indices.
__global__ __launch_bounds__(256) void dequant_generic_kernel(DequantArgs a, int dst_type, int src_type, int smode)
{
    const int64_t total = (int64_t)a.rows * a.cols;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        const int64_t i = t / a.cols, j = t % a.cols;
        float s;
        switch (smode) {
        case DQ_COL: s = dq_scale_at(a.scale, j, a.scale_type); break;
        case DQ_ROW: s = dq_scale_at(a.scale, i, a.scale_type); break;
        case DQ_GROUP_COL: s = dq_scale_at(a.scale, i * a.sk + j / a.group, a.scale_type); break;
        case DQ_GROUP_ROW: s = dq_scale_at(a.scale, (i / a.group) * a.n + j, a.scale_type); break;
        default: s = a.scale_scalar; break;
        }
        store_cast(a.y, i * a.ldd + j, dq_src_f32(a.src, i * a.n + j, src_type) * s, dst_type);
    }
}

// ---------------------------------------------------------------------------------------------
// AscendAntiQuant (elementwise): dst = (q + offset) * scale
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int32_t load_q(const void* src, int src_type, int64_t idx)
{
    if (src_type == DT_INT8) return ((const int8_t*)src)[idx];
    uint8_t b = ((const uint8_t*)src)[idx >> 1];
    int32_t nib = (idx & 1) ? (b >> 4) : (b & 0xf);
    return nib >= 8 ? nib - 16 : nib;
}

// one source element's exact value: int8 / int4 (two per byte, even element low) / fp8 / hifloat8
__device__ __forceinline__ float aq_src_value(const void* src, int src_type, int64_t idx)
{
    if (src_type == DT_INT8 || src_type == DT_INT4) return (float)load_q(src, src_type, idx);
    const uint32_t c = ((const uint8_t*)src)[idx];
    if (src_type == DT_HIF8) return hif8_to_f32(c);
    return fp8_bits_to_f32(c, src_type == DT_FP8_E5M2);
}

// The arithmetic of one legacy AscendAntiQuant element (AR: DT_F16 half ops, DT_BF16 bf16 ops, DT_F32 fp32 ops with
// one rne + saturating cast): (q + offset) * scale, written as dst_type
__device__ __forceinline__ void aq_elem(void* dst, int dst_type, int64_t idx, float q, bool has_off, float of, float sc,
                                        int ar)
{
    if (ar == DT_F16 && dst_type == DT_F16) {
        _Float16 w = (_Float16)q;
        if (has_off) w = w + (_Float16)of;
        w = w * (_Float16)sc;
        ((uint16_t*)dst)[idx] = h_bits(w);
    } else if (ar == DT_BF16 && dst_type == DT_BF16) {
        float w = q;  // exact in bf16 (hifloat8 codes)
        if (has_off) w = bf16_round(w + of);
        w = bf16_round(w * sc);
        ((uint16_t*)dst)[idx] = (uint16_t)(__float_as_uint(w) >> 16);
    } else {
        float v = q;
        if (has_off) v = v + of;
        store_cast(dst, idx, v * sc, dst_type);
    }
}

// the arithmetic the reference uses: fp8 in fp32; hifloat8 in half (f16), bf16 along rows, fp32 transposed or per
// tensor; int8 / int4 the caller's choice (bf16 output always fp32)
__host__ __device__ __forceinline__ int aq_arith(int src_type, int dst_type, int is_transpose, int per_tensor, int arith)
{
    if (src_type == DT_FP8_E4M3 || src_type == DT_FP8_E5M2) return DT_F32;
    if (src_type == DT_HIF8) return dst_type == DT_F16 ? DT_F16 : ((is_transpose || per_tensor) ? DT_F32 : DT_BF16);
    return (dst_type == DT_F16 && arith == 0) ? DT_F16 : DT_F32;
}

__global__ __launch_bounds__(256) void antiquant_kernel(void* __restrict__ dst, int dst_type,
                                                        const void* __restrict__ src, int src_type,
                                                        const uint16_t* __restrict__ offset,
                                                        const uint16_t* __restrict__ scale, uint32_t K, uint32_t N,
                                                        uint32_t g, int is_transpose, int arith)
{
    const int64_t total = (int64_t)K * N;
    const uint32_t G = K / g;
    const int ar = aq_arith(src_type, dst_type, is_transpose, 0, arith);
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        // t enumerates dst in memory order
        int64_t k, n;
        if (is_transpose) { n = t / K; k = t % K; }
        else { k = t / N; n = t % N; }
        const int64_t sidx = is_transpose ? n * G + k / g : (k / g) * N + n;
        const float sc = load_f32_of(scale, sidx, dst_type);
        const float of = offset ? load_f32_of(offset, sidx, dst_type) : 0.0f;
        aq_elem(dst, dst_type, t, aq_src_value(src, src_type, t), offset != nullptr, of, sc, ar);
    }
}

// per tensor, any count or alignment
__global__ __launch_bounds__(256) void antiquant_scalar_elem_kernel(void* __restrict__ dst, int dst_type,
                                                                    const void* __restrict__ src, int src_type,
                                                                    float of, float sc, int has_off, int64_t count,
                                                                    int ar)
{
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < count; t += (int64_t)gridDim.x * 256)
        aq_elem(dst, dst_type, t, aq_src_value(src, src_type, t), has_off != 0, of, sc, ar);
}

// ---------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------
static int grid_for(int64_t items, int per_block = 256)
{
    int64_t b = (items + per_block - 1) / per_block;
    int64_t cap = 256 * 8 * 4; // 8192 blocks: enough to fill 256 CUs several times over
    if (b > cap) b = cap;
    return (int)(b < 1 ? 1 : b);
}

template <int MODE>
static hipError_t launch_dyn_row(const void* x, int8_t* q, float* s, uint32_t m, uint32_t chunks, bool bf16,
                                 hipStream_t st)
{
    dim3 grid(m), block(256);
#define ASCQ_DYN(V)                                                                                                   \
    if (chunks <= 256u * V) {                                                                                         \
        if (bf16) launch_k((quant_dyn_row_kernel<V, MODE, true>), grid, block, 0, st, (const u32x4*)x,     \
                                     (u32x2*)q, s, chunks);                                                           \
        else launch_k((quant_dyn_row_kernel<V, MODE, false>), grid, block, 0, st, (const u32x4*)x,         \
                                (u32x2*)q, s, chunks);                                                                \
        return hipGetLastError();                                                                                     \
    }
    ASCQ_DYN(1)
    ASCQ_DYN(2)
    ASCQ_DYN(4)
    ASCQ_DYN(8)
#undef ASCQ_DYN
    return hipErrorInvalidValue;
}

hipError_t launch_quant_dynamic_per_token(int8_t* q, float* scale_out, const void* x, int src_type, uint32_t m,
                                          uint32_t n, int round_mode, hipStream_t st)
{
    const bool half_src = (src_type == DT_F16 || src_type == DT_BF16);
    const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
    if (half_src && aligned && n % 8 == 0 && n <= 256u * 8u * 8u) {
        uint32_t chunks = n / 8;
        bool bf = src_type == DT_BF16;
        switch (round_mode) {
        case RM_FLOOR: return launch_dyn_row<RM_FLOOR>(x, q, scale_out, m, chunks, bf, st);
        case RM_CEIL: return launch_dyn_row<RM_CEIL>(x, q, scale_out, m, chunks, bf, st);
        case RM_ROUND: return launch_dyn_row<RM_ROUND>(x, q, scale_out, m, chunks, bf, st);
        case RM_TRUNC: return launch_dyn_row<RM_TRUNC>(x, q, scale_out, m, chunks, bf, st);
        default: return launch_dyn_row<RM_RINT>(x, q, scale_out, m, chunks, bf, st);
        }
    }
    log_fallback("quant_dyn_generic_kernel", !half_src ? "f32 source" : !aligned ? "x not 16-byte or q not 8-byte aligned"
                                               : n % 8 != 0 ? "n not a multiple of 8" : "n > 16384");
    dim3 grid(m), block(256);
    switch (round_mode) {
#define ASCQ_G(MD) launch_k((quant_dyn_generic_kernel<MD>), grid, block, 0, st, x, q, scale_out, n, src_type); break;
    case RM_FLOOR: ASCQ_G(RM_FLOOR)
    case RM_CEIL: ASCQ_G(RM_CEIL)
    case RM_ROUND: ASCQ_G(RM_ROUND)
    case RM_TRUNC: ASCQ_G(RM_TRUNC)
    default: ASCQ_G(RM_RINT)
#undef ASCQ_G
    }
    return hipGetLastError();
}



// AscendAntiQuant policy form (arch 3510, ascend_antiquant_3510_impl.h:1386-1412, 1458-2110, 2175-2221): one thread
// per element of the [m, n] tensor.  Half and bf16 arithmetic is an fp32 operation rounded once to the 16-bit
// type, which equals the correctly rounded 16-bit operation (fp32 carries more than 2p + 2 bits of either).
// One scaleT multiply / add of two scaleT values, correctly rounded with signed zeros kept: f16 runs as a half
// operation (rounding the exact fp32 product to half gives the same value, but the compiler turns that rounding into
// an fma with a +0 addend, v_fma_mixlo_f16 a, b, 0, which makes a -0 product +0); bf16 rounds the fp32 result on
// its bits (exact products; sums are correctly rounded because fp32 has more than 2p + 2 bits of bf16).
__device__ __forceinline__ float mul_rt(float a, float b, int t)
{
    if (t == DT_F16) return (float)((_Float16)a * (_Float16)b);
    if (t == DT_BF16) return bf16_round(a * b);
    return a * b;
}
__device__ __forceinline__ float add_rt(float a, float b, int t)
{
    if (t == DT_F16) return (float)((_Float16)a + (_Float16)b);
    if (t == DT_BF16) return bf16_round(a + b);
    return a + b;
}
template <int T>
__device__ __forceinline__ float mul_t(float a, float b)
{
    if constexpr (T == DT_F16) return (float)((_Float16)a * (_Float16)b);
    else if constexpr (T == DT_BF16) return bf16_round(a * b);
    else return a * b;
}
template <int T>
__device__ __forceinline__ float add_t(float a, float b)
{
    if constexpr (T == DT_F16) return (float)((_Float16)a + (_Float16)b);
    else if constexpr (T == DT_BF16) return bf16_round(a + b);
    else return a + b;
}
__device__ __forceinline__ float load_scale_t(const void* p, int t, int64_t i)
{
    if (t == DT_F16) return f16_to_f32(((const uint16_t*)p)[i]);
    if (t == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}


// ---------------------------------------------------------------------------------------------
// AscendQuant policy form (arch 3510, ascend_quant_per_group_3510_impl.h:33-1340, dispatch :1451-1504):
// PER_TOKEN / PER_GROUP over [m, n] to int8, fp8 or E2M1.  Each lane takes 8 consecutive elements: one or two
// 16-byte source loads, one scale (PER_TOKEN, or a group along the row -- group sizes are multiples of 32) or
// 8 contiguous scales (groups down the columns), and an 8- (int8 / fp8) or 4-byte (E2M1) store.  Rows whose
// length is not a multiple of 8, or unaligned pointers, take the per-element path of the same kernel.
// ---------------------------------------------------------------------------------------------
enum : int { QD_INT8 = 0, QD_E4M3 = 1, QD_E5M2 = 2, QD_E2M1 = 3, QD_E1M2 = 4, QD_HIF8 = 5 };
constexpr bool qd_nibble(int d) { return d == QD_E2M1 || d == QD_E1M2; }  // two codes a byte
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
enum : int { QL_TOKEN = 0, QL_KCOL = 1, QL_KROW = 2 };

// Unsigned division by a runtime constant d for dividends below 2^31: s = ceil(log2 d),
// m = floor(2^32 (2^s - d) / d) + 1, q = (mulhi(n, m) + n) >> s (Granlund & Montgomery, "Division by invariant
// integers using multiplication", PLDI 1994, section 4).

struct QuantPolicyArgs {
    void* dst;
    const void* src;
    const void* scale;
    const void* offset;  // tensor indexed like scale, or null
    float off_scalar;    // used when has_off and offset is null (already a scaleT value)
    float sc_scalar;     // used when scale is null (PER_TENSOR; already a scaleT value)
    int has_off;         // 0 for E2M1, which takes no offset
    int src_type, scale_type, round_mode, layout;
    int64_t m, n, g, sk;
    uint32_t units, upr;  // vector kernel: units of 8 elements, units per row (n / 8)
    FastDiv upr_div, g_div;
};

// f32 -> fp8 with rint and saturation: NaN -> 0, overflow and inf -> +-max finite (TransRegForFp8,
// ascend_quant_3510_impl.h:888-896; docs/zh/api/SIMD-API/tensor_api/reg_vector_compute/type_conversion/cast.md:109)
__device__ __forceinline__ uint32_t f32_to_fp8_sat(float x, bool e5m2)
{
    if (x != x) return 0u;
    const float mx = e5m2 ? 57344.0f : 448.0f;
    return f32_to_fp8(__builtin_fminf(__builtin_fmaxf(x, -mx), mx), e5m2 ? 1 : 0);
}

// bf16 value -> E2M1 code in round mode MODE, saturating at +-6 (Cast<fp4x2_e2m1_t, bfloat16_t>, cast.md:96); NaN -> 0.
// |v| >= 1: the E2M1 codes from 1.0 (code 2) up are consecutive fp32 patterns rounded to one mantissa bit, so the
// code is (pattern + rounding bias) >> 22 less 252 (1.0 = 0x3F800000 -> 254).  The bias rounds the dropped 22 bits:
// half-to-even, half-away, none (trunc), or all-ones (magnitude up: ceil of a positive, floor of a negative value).
// |v| < 1: codes 0, 1, 2 are |round(2 v)| with the signed value rounded, so the directed modes see the sign.  A
// negative value that rounds to zero keeps its sign bit.
template <int MODE>
__device__ __forceinline__ uint32_t e2m1_code(float v)
{
    const uint32_t u = __float_as_uint(v);
    const uint32_t s = (u >> 28) & 8u;
    const uint32_t a = u & 0x7fffffffu;
    uint32_t bias;
    if constexpr (MODE == RM_TRUNC) bias = 0u;
    else if constexpr (MODE == RM_ROUND) bias = 0x200000u;
    else if constexpr (MODE == RM_FLOOR) bias = s ? 0x3FFFFFu : 0u;
    else if constexpr (MODE == RM_CEIL) bias = s ? 0u : 0x3FFFFFu;
    else bias = 0x1FFFFFu + ((a >> 22) & 1u);
    const uint32_t hi = ((a + bias) >> 22) - 252u;
    const uint32_t lo = (uint32_t)__builtin_fminf(__builtin_fabsf(round_mode_f(2.0f * v, MODE)), 2.0f);
    uint32_t c = a >= 0x3F800000u ? hi : lo;
    c = c > 7u ? 7u : c;
    return v != v ? 0u : (s | c);
}

// bf16 value -> E1M2 code in round mode MODE, saturating at +-1.75 (Cast<fp4x2_e1m2_t, bfloat16_t>); NaN -> 0.
// The E1M2 magnitudes are the multiples of 0.25 up to 1.75, so the code is round(4 v) on the signed value (the
// directed modes see the sign), its magnitude clamped to 7; 4 v is exact (an overflow to inf clamps to 7 too).
// A negative value that rounds to zero keeps its sign bit.
template <int MODE>
__device__ __forceinline__ uint32_t e1m2_code(float v)
{
    const uint32_t s = (__float_as_uint(v) >> 28) & 8u;
    const uint32_t c = (uint32_t)__builtin_fminf(__builtin_fabsf(round_mode_f(4.0f * v, MODE)), 7.0f);
    return v != v ? 0u : (s | c);
}


// the output code of a scaleT result v (after the offset): int8 byte, fp8 byte or E2M1 nibble
template <int DST, int T, int MODE>
__device__ __forceinline__ uint32_t quant_code(float v)
{
    if constexpr (DST == QD_INT8) {
        return (uint32_t)sat_s8_from_integral(round_mode_f(v, MODE)) & 0xffu;
    } else if constexpr (DST == QD_HIF8) {  // TransRegForHif8: every mode but HYBRID is CAST_ROUND (ties away)
        return hif8_code_rna_sat(v);
    } else if constexpr (DST == QD_E4M3 || DST == QD_E5M2) {
        return f32_to_fp8_sat(v, DST == QD_E5M2);
    } else {
        // f16 / f32 results go through bf16 (rne, saturating, NaN -> 0): plain rne here gives the same E2M1 code,
        // as NaN maps to 0 and every overflow to +-6 either way.  The rounding is the gfx950 conversion
        // (v_cvt_pk_bf16_f32), equal to the bit-level rne (bf16_round) on every non-NaN fp32 input; a NaN stays a
        // NaN either way and the code functions map it to 0.
        if constexpr (T != DT_BF16) v = (float)(__bf16)v;
        if constexpr (DST == QD_E1M2) return e1m2_code<MODE>(v);  // bf16 rounding first: E1M2 steps are finer
        else return e2m1_code<MODE>(v);
    }
}

template <int DST, int T>
__device__ __forceinline__ uint32_t quant_code_rt(float v, int mode)
{
    switch (mode) {
    case RM_FLOOR: return quant_code<DST, T, RM_FLOOR>(v);
    case RM_CEIL: return quant_code<DST, T, RM_CEIL>(v);
    case RM_ROUND: return quant_code<DST, T, RM_ROUND>(v);
    case RM_TRUNC: return quant_code<DST, T, RM_TRUNC>(v);
    default: return quant_code<DST, T, RM_RINT>(v);
    }
}

// 8 elements of a 16- or 32-bit float type as raw 32-bit words (f16 / bf16: 4 words, f32: 8) and their values
template <int TY>
struct Raw8 {
    uint32_t w[TY == DT_F32 ? 8 : 4];
};
template <int TY>
__device__ __forceinline__ void load_raw8(const void* p, int64_t unit, Raw8<TY>& r)
{
    const u32x4* q = (const u32x4*)p + (TY == DT_F32 ? 2 * unit : unit);
    const u32x4 a = __builtin_nontemporal_load(q);
    r.w[0] = a.x, r.w[1] = a.y, r.w[2] = a.z, r.w[3] = a.w;
    if constexpr (TY == DT_F32) {
        const u32x4 b = __builtin_nontemporal_load(q + 1);
        r.w[4] = b.x, r.w[5] = b.y, r.w[6] = b.z, r.w[7] = b.w;
    }
}
template <int TY>
__device__ __forceinline__ float raw_to_f32(uint32_t w)  // one element in the low bits (16-bit types) or whole word
{
    if constexpr (TY == DT_F32) return __uint_as_float(w);
    else if constexpr (TY == DT_BF16) return __uint_as_float(w << 16);
    else return f16_to_f32((uint16_t)w);
}
template <int TY>
__device__ __forceinline__ float raw8_at(const Raw8<TY>& r, int j)
{
    if constexpr (TY == DT_F32) return __uint_as_float(r.w[j]);
    else return raw_to_f32<TY>((j & 1) ? (r.w[j >> 1] >> 16) : (r.w[j >> 1] & 0xffffu));
}
template <int TY>
__device__ __forceinline__ uint32_t load_raw1(const void* p, int64_t i)
{
    if constexpr (TY == DT_F32) return ((const uint32_t*)p)[i];
    else return ((const uint16_t*)p)[i];
}

// f32 -> fp8 with rint and saturation through the gfx950 conversion (OCP e4m3fn / e5m2, round to nearest even):
// the input is clamped to the largest finite magnitude first and NaN replaced by 0, so only in-range values reach
// the instruction
template <bool E5M2>
__device__ __forceinline__ uint32_t fp8_sat_hw(float x)
{
    const float mx = E5M2 ? 57344.0f : 448.0f;
    x = x != x ? 0.0f : __builtin_fminf(__builtin_fmaxf(x, -mx), mx);
    if constexpr (E5M2) return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(x, 0.0f, 0, false) & 0xffu;
    else return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false) & 0xffu;
}

// Vector path (n % 8 == 0, 16-byte aligned source and row-group scales, fewer than 2^31 units): a unit is 8
// consecutive elements of one row; each lane takes UNR units and first issues every load they need -- source,
// scale and offset, unconditionally (indices clamped into the tensors, the scale table standing in for a missing
// offset tensor) so that no load waits on another -- then converts them.
//  * scales along the row (PER_GROUP kDim 1; PER_TOKEN is the case sk = 1, g = n): a workgroup takes UNR * 256
//    consecutive units per pass, one scale per unit at r * sk + c / g (group sizes are multiples of 32, so a unit
//    never straddles two groups);
//  * groups down the columns (kDim 0, KROW): a lane takes the same 8 columns of UNR consecutive rows r0 .. r0 + UNR - 1
//    (r0 a multiple of UNR, which divides every group size), so one load of 8 scales (and offsets) serves all UNR
//    units; the lanes of a wave still cover consecutive units of each row.
// Stores: 8 bytes (int8 / fp8) or 4 (E2M1) per unit.
// SC: scale type; the arithmetic type T is SC for int8 / E2M1 and fp32 for fp8.  With T = f16 the product and the
// offset add run as packed half operations (each correctly rounded, which is the scaleT arithmetic itself).
constexpr int QP_UNR = 4;

// two f32 -> E2M1 nearest-even codes into byte Q of w (saturating at +-6) / the two values of byte Q of w (gfx950;
// the byte select is an immediate)
template <int Q>
__device__ __forceinline__ uint32_t fp4_pk_f32(uint32_t w, float a, float b)
{
    return __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(w, a, b, 1.0f, Q);
}
template <int Q>
__device__ __forceinline__ f2x f32_pk_fp4(uint32_t w)
{
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, Q);
}
// the eight E2M1 nearest-even codes of f[0..7], element j at bits 4j .. 4j + 3, each value scaled by s first
__device__ __forceinline__ uint32_t fp4_codes8(const float (&f)[8], float s)
{
    uint32_t w = fp4_pk_f32<0>(0u, f[0] * s, f[1] * s);
    w = fp4_pk_f32<1>(w, f[2] * s, f[3] * s);
    w = fp4_pk_f32<2>(w, f[4] * s, f[5] * s);
    return fp4_pk_f32<3>(w, f[6] * s, f[7] * s);
}

// FA: fp32 arithmetic whatever the scale type (the Quantize form: scale and offset widened exactly, one fp32 multiply
// and one fp32 add); otherwise fp32 for fp8 outputs and the scale type's arithmetic for the others (AscendQuant)
template <int DST, int SRC, int SC, int MODE, bool KROW, bool FA = false>
__device__ __forceinline__ void quant_unit(const QuantPolicyArgs& a, uint32_t u, const Raw8<SRC>& xr,
                                           const Raw8<SC>& sr, Raw8<SC> orw, bool off_tensor, uint32_t osc)
{
    constexpr bool FP8 = DST == QD_E4M3 || DST == QD_E5M2;
    constexpr int T = (FP8 || FA) ? DT_F32 : SC;
    constexpr bool HALF = T == DT_F16;  // then SRC == SC == f16
    if (!off_tensor) {  // scalar offset (or none): broadcast it like a per-unit scale
        if constexpr (KROW) {
#pragma unroll
            for (int q = 0; q < (SC == DT_F32 ? 8 : 4); ++q) orw.w[q] = SC == DT_F32 ? osc : (osc | (osc << 16));
        } else {
            orw.w[0] = osc;
        }
    }
    float v[8];
    if constexpr (HALF) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t sw = KROW ? sr.w[q] : (sr.w[0] | (sr.w[0] << 16));
            h2 p = __builtin_bit_cast(h2, xr.w[q]) * __builtin_bit_cast(h2, sw);
            if (a.has_off) {
                const uint32_t ow = KROW ? orw.w[q] : (orw.w[0] | (orw.w[0] << 16));
                p = p + __builtin_bit_cast(h2, ow);
            }
            v[2 * q] = (float)p.x;
            v[2 * q + 1] = (float)p.y;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sj = KROW ? raw8_at<SC>(sr, j) : raw_to_f32<SC>(sr.w[0]);
            float t = mul_t<T>(raw8_at<SRC>(xr, j), sj);
            if (a.has_off) t = add_t<T>(t, KROW ? raw8_at<SC>(orw, j) : raw_to_f32<SC>(orw.w[0]));
            v[j] = t;
        }
    }
    if constexpr (DST == QD_E2M1 && MODE == RM_RINT) {
        // rint E2M1 through the gfx950 conversions: fp32 -> bf16 (v_cvt_pk_bf16_f32, rne) and bf16 -> E2M1
        // (v_cvt_scalef32_pk_fp4_bf16 with scale 1: nearest even, saturating at +-6), two elements each; both agree
        // with the software rounding (bf16_round, e2m1_code<RM_RINT>) on every non-NaN input, and NaN is replaced
        // by 0 first (its code under the saturating casts)
        bf2 b[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float v0 = v[2 * q] != v[2 * q] ? 0.0f : v[2 * q];
            const float v1 = v[2 * q + 1] != v[2 * q + 1] ? 0.0f : v[2 * q + 1];
            if constexpr (T == DT_BF16)  // already bf16 values
                b[q] = (bf2){__builtin_bit_cast(__bf16, (uint16_t)(__float_as_uint(v0) >> 16)),
                             __builtin_bit_cast(__bf16, (uint16_t)(__float_as_uint(v1) >> 16))};
            else
                b[q] = (bf2){(__bf16)v0, (__bf16)v1};
        }
        uint32_t w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(0u, b[0], 1.0f, 0);  // elements 0, 1 -> byte 0
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, b[1], 1.0f, 1);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, b[2], 1.0f, 2);
        w = __builtin_amdgcn_cvt_scalef32_pk_fp4_bf16(w, b[3], 1.0f, 3);
        __builtin_nontemporal_store(w, (uint32_t*)a.dst + u);
        return;
    }
    if constexpr (DST == QD_E2M1 && MODE != RM_RINT) {
        // The directed modes from the gfx950 conversions.  f = the bf16 value of each result (NaN -> 0, its code),
        // w = the nearest-even codes of f (v_cvt_scalef32_pk_fp4_f32, saturating at +-6).
        //  * FLOOR / CEIL / TRUNC: d = the value of each code (v_cvt_scalef32_pk_f32_fp4); where d lies on the wrong
        //    side of f the code moves one step, magnitude +1 or -1 in its low three bits.  Those steps never pass 0 or
        //    7 (a +1 is skipped at 7, where the mode saturates; a -1 only happens above 0), so the eight nibbles of the
        //    word step together by one add and one subtract.
        //  * ROUND (half away): the nearest-even codes of f * (1 + 2^-10).  The nudge moves an exact tie (a midpoint of
        //    the E2M1 grid is a bf16 value) away from zero and moves no other bf16 value across a midpoint: those
        //    lie at least one bf16 step, 2^-8 of the midpoint, away from it.
        float f[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float f0 = v[2 * q], f1 = v[2 * q + 1];
            if constexpr (T != DT_BF16) {
                const uint32_t bw = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2x){f0, f1}, bf2));
                f0 = __uint_as_float(bw << 16);
                f1 = __uint_as_float(bw & 0xffff0000u);
            }
            f[2 * q] = f0 != f0 ? 0.0f : f0;
            f[2 * q + 1] = f1 != f1 ? 0.0f : f1;
        }
        uint32_t w;
        if constexpr (MODE == RM_ROUND) {
            w = fp4_codes8(f, 1.0f + 0x1p-10f);
        } else {
            w = fp4_codes8(f, 1.0f);
            const f2x dq[4] = {f32_pk_fp4<0>(w), f32_pk_fp4<1>(w), f32_pk_fp4<2>(w), f32_pk_fp4<3>(w)};
            uint32_t inc = 0u, dec = 0u;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f2x d = dq[q];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int j = 2 * q + e;
                    const float dj = e ? d.y : d.x, fj = f[j];
                    const bool neg = (__float_as_uint(fj) >> 31) != 0u, top = ((w >> (4 * j)) & 7u) == 7u;
                    const uint32_t bit = 1u << (4 * j);
                    if constexpr (MODE == RM_FLOOR) {
                        if (dj > fj) {
                            if (!neg) dec |= bit;
                            else if (!top) inc |= bit;
                        }
                    } else if constexpr (MODE == RM_CEIL) {
                        if (dj < fj) {
                            if (neg) dec |= bit;
                            else if (!top) inc |= bit;
                        }
                    } else {  // RM_TRUNC
                        if (__builtin_fabsf(dj) > __builtin_fabsf(fj)) dec |= bit;
                    }
                }
            }
            w = w + inc - dec;
        }
        __builtin_nontemporal_store(w, (uint32_t*)a.dst + u);
        return;
    }
    uint32_t code[8];
    if constexpr (qd_nibble(DST) && T != DT_BF16) {
        // the bf16 step of the fp4 codes two elements per conversion (v_cvt_pk_bf16_f32, rne), then the codes of
        // the bf16 values
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bf2 b = __builtin_convertvector((f2x){v[2 * q], v[2 * q + 1]}, bf2);
            const uint32_t w = __builtin_bit_cast(uint32_t, b);
            code[2 * q] = quant_code<DST, DT_BF16, MODE>(__uint_as_float(w << 16));
            code[2 * q + 1] = quant_code<DST, DT_BF16, MODE>(__uint_as_float(w & 0xffff0000u));
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (FP8) code[j] = fp8_sat_hw<DST == QD_E5M2>(v[j]);
            else code[j] = quant_code<DST, T, MODE>(v[j]);
        }
    }
    if constexpr (qd_nibble(DST)) {
        const uint32_t w = code[0] | (code[1] << 4) | (code[2] << 8) | (code[3] << 12) | (code[4] << 16) |
                           (code[5] << 20) | (code[6] << 24) | (code[7] << 28);
        __builtin_nontemporal_store(w, (uint32_t*)a.dst + u);
    } else {
        const u32x2 w = {code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24),
                         code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24)};
        __builtin_nontemporal_store(w, (u32x2*)a.dst + u);
    }
}

template <int SC>
__device__ __forceinline__ uint32_t offset_scalar_bits(float o)
{
    if constexpr (SC == DT_F32) return __float_as_uint(o);
    else if constexpr (SC == DT_BF16) return __float_as_uint(o) >> 16;  // already a bf16 value
    else return (uint32_t)h_bits((_Float16)o);                          // already a half value
}

// scale == null: the scalar sc_scalar for every element (PER_TENSOR)
template <int DST, int SRC, int SC, int MODE, bool FA = false>
__global__ __launch_bounds__(256) void quant_policy_vec_kernel(QuantPolicyArgs a)  // scales along the row
{
    const bool sc_tensor = a.scale != nullptr;
    const void* scp = sc_tensor ? a.scale : a.src;  // (never read without a scale tensor)
    const void* offp = a.offset ? a.offset : scp;
    const bool off_tensor = a.offset != nullptr;
    const uint32_t osc = offset_scalar_bits<SC>(a.off_scalar), ssc = offset_scalar_bits<SC>(a.sc_scalar);
    for (uint32_t b0 = blockIdx.x * (256u * QP_UNR); b0 < a.units; b0 += gridDim.x * (256u * QP_UNR)) {
        Raw8<SRC> xr[QP_UNR];
        Raw8<SC> sr[QP_UNR], orw[QP_UNR];  // one scale / offset each, in w[0]
#pragma unroll
        for (int k = 0; k < QP_UNR; ++k) {
            uint32_t u = b0 + k * 256u + threadIdx.x;
            u = u < a.units ? u : a.units - 1u;  // past the end: load a valid unit, store nothing
            load_raw8<SRC>(a.src, u, xr[k]);
            const uint32_t r = fdiv(u, a.upr_div), c = (u - r * a.upr) * 8u;
            const int64_t si = (int64_t)r * a.sk + fdiv(c, a.g_div);
            sr[k].w[0] = sc_tensor ? load_raw1<SC>(scp, si) : ssc;
            // without an offset tensor quant_unit takes the scalar offset: no load (the fp4 outputs, which write a
            // quarter of what they read, ran 11-12 % faster for it)
            orw[k].w[0] = off_tensor ? load_raw1<SC>(offp, si) : 0u;
        }
#pragma unroll
        for (int k = 0; k < QP_UNR; ++k) {
            const uint32_t u = b0 + k * 256u + threadIdx.x;
            if (u >= a.units) break;
            quant_unit<DST, SRC, SC, MODE, false, FA>(a, u, xr[k], sr[k], orw[k], off_tensor, osc);
        }
    }
}

template <int DST, int SRC, int SC, int MODE, bool FA = false>
__global__ __launch_bounds__(256) void quant_policy_vec_krow_kernel(QuantPolicyArgs a)  // groups down the columns
{
    const void* offp = a.offset ? a.offset : a.scale;
    const bool off_tensor = a.offset != nullptr;
    const uint32_t osc = offset_scalar_bits<SC>(a.off_scalar);
    const uint32_t rows = (uint32_t)a.m;
    for (uint32_t v = blockIdx.x * 256u + threadIdx.x; v < a.units; v += gridDim.x * 256u) {  // units: row blocks x upr
        const uint32_t rb = fdiv(v, a.upr_div), wu = v - rb * a.upr, r0 = rb * QP_UNR;
        const int64_t su = ((int64_t)fdiv(r0, a.g_div) * a.n) / 8 + wu;
        Raw8<SRC> xr[QP_UNR];
        Raw8<SC> sr, orw = {};
        load_raw8<SC>(a.scale, su, sr);
        if (off_tensor) load_raw8<SC>(offp, su, orw);
#pragma unroll
        for (int k = 0; k < QP_UNR; ++k) {
            const uint32_t r = r0 + k < rows ? r0 + k : rows - 1u;
            load_raw8<SRC>(a.src, (int64_t)r * a.upr + wu, xr[k]);
        }
#pragma unroll
        for (int k = 0; k < QP_UNR; ++k) {
            if (r0 + k >= rows) break;
            quant_unit<DST, SRC, SC, MODE, true, FA>(a, (r0 + k) * a.upr + wu, xr[k], sr, orw, off_tensor, osc);
        }
    }
}

// Legacy AscendQuant, arch-3510 form (include/adv_api/quantization/ascend_quant.h:64-293, 360-460; impl
// ascend_quant_3510_impl.h:35-620).  Element i uses channel i % scale_count of the srcT scale / offset tensors, or
// the scalars.  int8 / hifloat8 outputs run in half arithmetic: the source and the srcT tensors become half with rne
// and saturation, the scalars arrive as half already (the host's static_cast<half>), then t = x * s and t = t + o as
// packed half operations (each correctly rounded), then rint with saturation (int8) or ties away with saturation
// (hifloat8).  fp8 outputs run in fp32: y = x * s, y = y + o (exact conversions of srcT), rint with saturation.
struct QuantLegacyArgs {
    void* q;
    const void* x;
    const void* scale;   // srcT [scale_count], or null for the scalars
    const void* offset;  // srcT [scale_count], or null for the scalar offset
    uint32_t sh, oh;     // the scalars as half bits (half arithmetic)
    float sf, of;        // the scalars in fp32 (fp8 outputs)
    int out;             // QD_INT8 / QD_HIF8 / QD_E4M3 / QD_E5M2
    int src_type;        // element kernel
    uint32_t units, rows, upr, scale_count;
    FastDiv upr_div;
    int64_t total;
};

// elements 2q and 2q + 1 of a unit as packed half bits, rne + saturating
template <int SRC>
__device__ __forceinline__ uint32_t half2_sat(const Raw8<SRC>& r, int q)
{
    if constexpr (SRC == DT_F16) return r.w[q];
    else return (uint32_t)f32_to_f16_sat(raw8_at<SRC>(r, 2 * q)) | ((uint32_t)f32_to_f16_sat(raw8_at<SRC>(r, 2 * q + 1)) << 16);
}

template <int SRC, bool F32A>
__device__ __forceinline__ u32x2 quant_legacy_unit(const QuantLegacyArgs& a, const Raw8<SRC>& xr, const Raw8<SRC>* sr,
                                                   const Raw8<SRC>* orr)
{
    uint32_t code[8];
    if constexpr (F32A) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = raw8_at<SRC>(xr, j) * (sr ? raw8_at<SRC>(*sr, j) : a.sf);
            v = v + (orr ? raw8_at<SRC>(*orr, j) : a.of);
            code[j] = a.out == QD_E5M2 ? fp8_sat_hw<true>(v) : fp8_sat_hw<false>(v);
        }
    } else {
        const uint32_t s2 = a.sh | (a.sh << 16), o2 = a.oh | (a.oh << 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            h2 t = __builtin_bit_cast(h2, half2_sat<SRC>(xr, q)) * __builtin_bit_cast(h2, sr ? half2_sat<SRC>(*sr, q) : s2);
            t = t + __builtin_bit_cast(h2, orr ? half2_sat<SRC>(*orr, q) : o2);
            if (a.out == QD_HIF8) {
                code[2 * q] = hif8_code_rna_sat((float)t.x);
                code[2 * q + 1] = hif8_code_rna_sat((float)t.y);
            } else {
                code[2 * q] = (uint32_t)quant_s8<RM_RINT>((float)t.x) & 0xffu;
                code[2 * q + 1] = (uint32_t)quant_s8<RM_RINT>((float)t.y) & 0xffu;
            }
        }
    }
    return (u32x2){code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24),
                   code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24)};
}

// Vector path (cal_count % 8 == 0 and below 2^31, 16-byte aligned source and tensors, scale_count % 8 == 0): a unit
// is 8 consecutive elements.  With channel tensors the data is rows = cal_count / scale_count rows of scale_count
// channels; a lane takes the same 8 channels of QP_UNR consecutive rows and loads their scales / offsets once.  With
// scalars, QP_UNR consecutive units per workgroup pass.  Each lane issues all loads before converting.
template <int SRC, bool F32A, bool SV>
__global__ __launch_bounds__(256) void quant_legacy_vec_kernel(QuantLegacyArgs a)
{
    u32x2* q = (u32x2*)a.q;
    if constexpr (SV) {  // units: row blocks x upr
        const bool ov = a.offset != nullptr;
        for (uint32_t v = blockIdx.x * 256u + threadIdx.x; v < a.units; v += gridDim.x * 256u) {
            const uint32_t rb = fdiv(v, a.upr_div), w = v - rb * a.upr, r0 = rb * QP_UNR;
            Raw8<SRC> sr, orr, xr[QP_UNR];
            load_raw8<SRC>(a.scale, w, sr);
            load_raw8<SRC>(ov ? a.offset : a.scale, w, orr);
#pragma unroll
            for (int k = 0; k < QP_UNR; ++k) {
                const uint32_t r = r0 + k < a.rows ? r0 + k : a.rows - 1u;  // past the last row: reload it, no store
                load_raw8<SRC>(a.x, r * a.upr + w, xr[k]);
            }
#pragma unroll
            for (int k = 0; k < QP_UNR; ++k) {
                if (r0 + k >= a.rows) break;
                __builtin_nontemporal_store(quant_legacy_unit<SRC, F32A>(a, xr[k], &sr, ov ? &orr : nullptr),
                                            q + (r0 + k) * a.upr + w);
            }
        }
    } else {  // units: cal_count / 8
        for (uint32_t b0 = blockIdx.x * (256u * QP_UNR); b0 < a.units; b0 += gridDim.x * (256u * QP_UNR)) {
            Raw8<SRC> xr[QP_UNR];
#pragma unroll
            for (int k = 0; k < QP_UNR; ++k) {
                const uint32_t u = b0 + k * 256u + threadIdx.x;
                load_raw8<SRC>(a.x, u < a.units ? u : a.units - 1u, xr[k]);
            }
#pragma unroll
            for (int k = 0; k < QP_UNR; ++k) {
                const uint32_t u = b0 + k * 256u + threadIdx.x;
                if (u >= a.units) break;
                __builtin_nontemporal_store(quant_legacy_unit<SRC, F32A>(a, xr[k], nullptr, nullptr), q + u);
            }
        }
    }
}

// Any shape or alignment: one thread per element.
__global__ __launch_bounds__(256) void quant_legacy_elem_kernel(QuantLegacyArgs a)
{
    const bool f32a = a.out == QD_E4M3 || a.out == QD_E5M2;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.total; i += (int64_t)gridDim.x * 256) {
        const int64_t c = a.scale_count ? i % a.scale_count : 0;
        const float x = load_scale_t(a.x, a.src_type, i);
        uint32_t code;
        if (f32a) {
            float v = x * (a.scale ? load_scale_t(a.scale, a.src_type, c) : a.sf);
            v = v + (a.offset ? load_scale_t(a.offset, a.src_type, c) : a.of);
            code = a.out == QD_E5M2 ? fp8_sat_hw<true>(v) : fp8_sat_hw<false>(v);
        } else {
            const _Float16 sh = bits_h(a.scale ? f32_to_f16_sat(load_scale_t(a.scale, a.src_type, c)) : (uint16_t)a.sh);
            const _Float16 oh = bits_h(a.offset ? f32_to_f16_sat(load_scale_t(a.offset, a.src_type, c)) : (uint16_t)a.oh);
            _Float16 t = bits_h(f32_to_f16_sat(x)) * sh;
            t = t + oh;
            code = a.out == QD_HIF8 ? hif8_code_rna_sat((float)t) : ((uint32_t)quant_s8<RM_RINT>((float)t) & 0xffu);
        }
        ((uint8_t*)a.q)[i] = (uint8_t)code;
    }
}

template <int SRC, bool F32A>
static void launch_legacy_vec(const QuantLegacyArgs& a, hipStream_t st)
{
    if (a.scale)
        launch_k(quant_legacy_vec_kernel<SRC, F32A, true>, dim3(grid_for(a.units)), dim3(256), 0, st, a);
    else
        launch_k(quant_legacy_vec_kernel<SRC, F32A, false>, dim3(grid_for((a.units + QP_UNR - 1) / QP_UNR)), dim3(256),
                 0, st, a);
}

template <int SRC>
static void launch_legacy_vec_arith(const QuantLegacyArgs& a, hipStream_t st)
{
    if (a.out == QD_E4M3 || a.out == QD_E5M2) launch_legacy_vec<SRC, true>(a, st);
    else launch_legacy_vec<SRC, false>(a, st);
}

hipError_t launch_quant_legacy(void* q, int dst_type, const void* x, int src_type, const void* scale,
                               const void* offset, float scale_scalar, float offset_scalar, uint32_t cal_count,
                               uint32_t scale_count, hipStream_t st)
{
    (void)hipGetLastError();
    QuantLegacyArgs a{};
    a.q = q;
    a.x = x;
    a.scale = scale;
    a.offset = scale ? offset : nullptr;
    a.out = dst_type == DT_HIF8 ? QD_HIF8 : (dst_type == DT_FP8_E4M3 ? QD_E4M3 : (dst_type == DT_FP8_E5M2 ? QD_E5M2 : QD_INT8));
    a.src_type = src_type;
    // a scale tensor's scalar offset is a srcT value (the `const T offset` overloads)
    float os = offset_scalar;
    if (scale && src_type == DT_F16) {
        os = (float)(_Float16)os;
    } else if (scale && src_type == DT_BF16) {
        uint32_t u = __builtin_bit_cast(uint32_t, os);
        if ((u & 0x7fffffffu) <= 0x7f800000u) u = ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16;
        os = __builtin_bit_cast(float, u);
    }
    a.sf = scale_scalar;
    a.of = os;
    a.sh = __builtin_bit_cast(uint16_t, (_Float16)scale_scalar);  // static_cast<half>: rne, IEEE overflow
    a.oh = __builtin_bit_cast(uint16_t, (_Float16)os);
    a.scale_count = scale ? scale_count : 0u;
    a.total = cal_count;
    const bool vec = cal_count % 8 == 0 && cal_count < (1u << 31) && (uintptr_t)x % 16 == 0 && (uintptr_t)q % 8 == 0 &&
                     (!scale || (scale_count % 8 == 0 && (uintptr_t)scale % 16 == 0 && (uintptr_t)a.offset % 16 == 0));
    if (vec && cal_count > 0) {
        a.upr = scale ? scale_count / 8 : 1u;
        a.rows = scale ? cal_count / scale_count : 0u;
        a.units = scale ? (a.rows + QP_UNR - 1) / QP_UNR * a.upr : cal_count / 8;
        a.upr_div = fast_div(a.upr);
        if (src_type == DT_F16) launch_legacy_vec_arith<DT_F16>(a, st);
        else if (src_type == DT_BF16) launch_legacy_vec_arith<DT_BF16>(a, st);
        else launch_legacy_vec_arith<DT_F32>(a, st);
        return hipGetLastError();
    }
    if (cal_count > 0) log_fallback("quant_legacy_elem_kernel", "count, scale count or pointers not aligned to 8 elements");
    launch_k(quant_legacy_elem_kernel, dim3(grid_for(cal_count)), dim3(256), 0, st, a);
    return hipGetLastError();
}

// AscendDequant, vector path: rows of `cols` computed elements at a source row stride of n and a destination row
// stride of ldd (the legacy form's 32-byte padded rows, or n).  A unit is UE consecutive columns of RB
// consecutive rows: UE = 4 for 4-byte sources (int32 / fp32: one 16-byte load per row), 8 for int8 (one 8-byte
// load), so every load and store instruction of a wave covers contiguous spans.  The UE scales of a unit are
// loaded once for its RB rows (per column, or per column of a row group: the groups are multiples of 32 rows, so
// RB rows never straddle one), and all RB source loads are issued before converting.  An int32 source converts
// with ties away from zero: the plain conversion is exact up to 2^24, so the unit takes the slower exact path only
// when one of its values lies beyond (one wave-uniform branch per unit).  dst = cast(f32(src) * scale), rne +
// saturating (store_cast semantics).
template <int UE>
__device__ __forceinline__ void dq_scale_vec(const void* s, int64_t i0, int type, float (&o)[UE])
{
    // i0 is a multiple of UE and s is 16-byte aligned, so every load below is naturally aligned
    if (type == DT_F32) {
#pragma unroll
        for (int q = 0; q < UE / 4; ++q) {
            const u32x4 a = *((const u32x4*)((const float*)s + i0) + q);
            o[4 * q] = __uint_as_float(a.x), o[4 * q + 1] = __uint_as_float(a.y);
            o[4 * q + 2] = __uint_as_float(a.z), o[4 * q + 3] = __uint_as_float(a.w);
        }
    } else if (type == DT_U64) {
#pragma unroll
        for (int q = 0; q < UE / 2; ++q) {
            const u32x4 a = *((const u32x4*)((const uint64_t*)s + i0) + q);
            o[2 * q] = __uint_as_float(a.x), o[2 * q + 1] = __uint_as_float(a.z);
        }
    } else {
        uint32_t w[UE / 2];
        if constexpr (UE == 4) {
            const u32x2 a = *(const u32x2*)((const uint16_t*)s + i0);
            w[0] = a.x, w[1] = a.y;
        } else {
            const u32x4 a = *(const u32x4*)((const uint16_t*)s + i0);
            w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w;
        }
#pragma unroll
        for (int q = 0; q < UE / 2; ++q) {
            o[2 * q] = type == DT_BF16 ? bf16_to_f32((uint16_t)w[q]) : f16_to_f32((uint16_t)w[q]);
            o[2 * q + 1] = type == DT_BF16 ? bf16_to_f32((uint16_t)(w[q] >> 16)) : f16_to_f32((uint16_t)(w[q] >> 16));
        }
    }
}

template <int SRC, int DST, int SM>
__global__ __launch_bounds__(256) void dequant_vec_kernel(DequantArgs a)
{
    constexpr int UE = SRC == DT_INT8 ? 8 : 4;  // elements per unit row
    constexpr int RB = SRC == DT_INT8 ? 4 : 8;  // rows per unit
    for (uint32_t v = blockIdx.x * 256u + threadIdx.x; v < a.units; v += gridDim.x * 256u) {
        const uint32_t rb = fdiv(v, a.upr_div), w = v - rb * a.upr, r0 = rb * RB, c0 = UE * w;
        float sc[UE];
        if constexpr (SM == DQ_COL) dq_scale_vec<UE>(a.scale, c0, a.scale_type, sc);
        if constexpr (SM == DQ_GROUP_ROW) dq_scale_vec<UE>(a.scale, (int64_t)fdiv(r0, a.g_div) * a.n + c0, a.scale_type, sc);
        uint32_t xw[RB][UE == 4 ? 4 : 2];
        float st[RB];
#pragma unroll
        for (int k = 0; k < RB; ++k) {
            const uint32_t r = r0 + k < a.rows ? r0 + k : a.rows - 1u;  // past the last row: reload it, store nothing
            const int64_t e = (int64_t)r * a.n + c0;
            if constexpr (SRC == DT_INT8) {
                const u32x2 x = __builtin_nontemporal_load((const u32x2*)((const int8_t*)a.src + e));
                xw[k][0] = x.x, xw[k][1] = x.y;
            } else {
                const u32x4 x = __builtin_nontemporal_load((const u32x4*)((const uint32_t*)a.src + e));
                xw[k][0] = x.x, xw[k][1] = x.y, xw[k][2] = x.z, xw[k][3] = x.w;
            }
            if constexpr (SM == DQ_ROW) st[k] = dq_scale_at(a.scale, r, a.scale_type);
            else if constexpr (SM == DQ_GROUP_COL) st[k] = dq_scale_at(a.scale, (int64_t)r * a.sk + fdiv(c0, a.g_div), a.scale_type);
            else st[k] = a.scale_scalar;
        }
        float x[RB][UE];
        bool beyond = false;
#pragma unroll
        for (int k = 0; k < RB; ++k)
#pragma unroll
            for (int j = 0; j < UE; ++j) {
                if constexpr (SRC == DT_INT32) {
                    x[k][j] = (float)(int32_t)xw[k][j];
                    beyond |= i32_beyond_f32_exact((int32_t)xw[k][j]);
                } else if constexpr (SRC == DT_F32) {
                    x[k][j] = __uint_as_float(xw[k][j]);
                } else {
                    x[k][j] = (float)(int8_t)((xw[k][j >> 2] >> (8 * (j & 3))) & 0xffu);
                }
            }
        if constexpr (SRC == DT_INT32) {
            if (beyond) {
#pragma unroll
                for (int k = 0; k < RB; ++k)
#pragma unroll
                    for (int j = 0; j < UE; ++j) x[k][j] = i32_to_f32_rna((int32_t)xw[k][j]);
            }
        }
#pragma unroll
        for (int k = 0; k < RB; ++k) {
            if (r0 + k >= a.rows) break;
            float o[UE];
#pragma unroll
            for (int j = 0; j < UE; ++j) o[j] = x[k][j] * ((SM == DQ_COL || SM == DQ_GROUP_ROW) ? sc[j] : st[k]);
            const int64_t e = (int64_t)(r0 + k) * a.ldd + c0;
            if constexpr (DST == DT_F32) {
#pragma unroll
                for (int q = 0; q < UE / 4; ++q)
                    __builtin_nontemporal_store((u32x4){__float_as_uint(o[4 * q]), __float_as_uint(o[4 * q + 1]),
                                                        __float_as_uint(o[4 * q + 2]), __float_as_uint(o[4 * q + 3])},
                                                (u32x4*)((float*)a.y + e) + q);
            } else {
                uint32_t h[UE / 2];
#pragma unroll
                for (int q = 0; q < UE / 2; ++q) {
                    const uint32_t lo = DST == DT_BF16 ? f32_to_bf16_sat(o[2 * q]) : f32_to_f16_sat(o[2 * q]);
                    const uint32_t hi = DST == DT_BF16 ? f32_to_bf16_sat(o[2 * q + 1]) : f32_to_f16_sat(o[2 * q + 1]);
                    h[q] = lo | (hi << 16);
                }
                if constexpr (UE == 4) __builtin_nontemporal_store((u32x2){h[0], h[1]}, (u32x2*)((uint16_t*)a.y + e));
                else __builtin_nontemporal_store((u32x4){h[0], h[1], h[2], h[3]}, (u32x4*)((uint16_t*)a.y + e));
            }
        }
    }
}

template <int SRC, int DST>
static void launch_dequant_vec(DequantArgs a, int smode, hipStream_t st)
{
    const dim3 grid(grid_for(a.units)), block(256);
    switch (smode) {
    case DQ_COL: launch_k(dequant_vec_kernel<SRC, DST, DQ_COL>, grid, block, 0, st, a); break;
    case DQ_ROW: launch_k(dequant_vec_kernel<SRC, DST, DQ_ROW>, grid, block, 0, st, a); break;
    case DQ_GROUP_COL: launch_k(dequant_vec_kernel<SRC, DST, DQ_GROUP_COL>, grid, block, 0, st, a); break;
    case DQ_GROUP_ROW: launch_k(dequant_vec_kernel<SRC, DST, DQ_GROUP_ROW>, grid, block, 0, st, a); break;
    default: launch_k(dequant_vec_kernel<SRC, DST, DQ_SCALAR>, grid, block, 0, st, a); break;
    }
}

template <int SRC>
static void launch_dequant_vec_dst(DequantArgs a, int dst_type, int smode, hipStream_t st)
{
    if (dst_type == DT_F16) launch_dequant_vec<SRC, DT_F16>(a, smode, st);
    else if (dst_type == DT_BF16) launch_dequant_vec<SRC, DT_BF16>(a, smode, st);
    else launch_dequant_vec<SRC, DT_F32>(a, smode, st);
}

hipError_t launch_dequant(void* y, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                          float scale_scalar, int smode, uint32_t rows, uint32_t cols, uint32_t n, uint32_t ldd,
                          uint32_t group, hipStream_t st)
{
    (void)hipGetLastError();  // clear a stale error so the status below is this launch's
    DequantArgs a{};
    a.y = y, a.src = src, a.scale = scale, a.scale_scalar = scale_scalar, a.scale_type = scale_type;
    a.rows = rows, a.cols = cols, a.n = n, a.ldd = ldd, a.group = group;
    a.sk = group ? (n + group - 1) / group : 0;
    a.g_div = fast_div(group ? group : 1u);
    const bool fast = smode == DQ_ROW && src_type == DT_INT8 && dst_type == DT_F16 && scale_type == DT_F32 &&
                      cols == n && ldd == n && n % 8 == 0 && ((uintptr_t)src % 8 == 0) && ((uintptr_t)y % 16 == 0);
    if (fast) {
        // measured at 8192 x 8192: U = 1 34.9 us, 2 34.1 us, 4 36.1 us (unconditional loads); 16-element units (one
        // 16-byte load, two 16-byte stores per lane) 34.9 us at U = 1 and slower above, as each store instruction
        // then covers every other 16 bytes of its span
        constexpr int U = 2;
        const uint32_t upr = n / 8;
        const uint32_t segs = (upr + 256 * U - 1) / (256 * U);
        const uint64_t blocks = (uint64_t)rows * segs;
        if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
        launch_k(dequant_i8_token_f16_kernel<U>, dim3((unsigned)blocks), dim3(256), 0, st, (const u32x2*)src,
                 (const float*)scale, (u32x4*)y, upr, segs);
        return hipGetLastError();
    }
    const uint32_t ue = src_type == DT_INT8 ? 8 : 4, rb = src_type == DT_INT8 ? 4 : 8;
    const int esz = dst_type == DT_F32 ? 4 : 2;
    const int ssz = scale_type == DT_F32 ? 4 : (scale_type == DT_U64 ? 8 : 2);
    const bool vec_scale = smode == DQ_COL || smode == DQ_GROUP_ROW;
    const bool vec = cols % ue == 0 && n % ue == 0 && ldd % ue == 0 && cols > 0 && rows > 0 &&
                     (uint64_t)rows * n < (1ull << 31) && (uint64_t)rows * ldd < (1ull << 31) &&
                     (uintptr_t)src % (src_type == DT_INT8 ? 8 : 16) == 0 &&
                     (uintptr_t)y % (ue * esz > 16 ? 16 : ue * esz) == 0 &&
                     (!vec_scale || (uintptr_t)scale % 16 == 0) && (group == 0 || group % 32 == 0) && ssz > 0;
    if (vec) {
        a.upr = cols / ue;
        a.units = (rows + rb - 1) / rb * a.upr;
        a.upr_div = fast_div(a.upr);
        if (src_type == DT_INT32) launch_dequant_vec_dst<DT_INT32>(a, dst_type, smode, st);
        else if (src_type == DT_INT8) launch_dequant_vec_dst<DT_INT8>(a, dst_type, smode, st);
        else launch_dequant_vec_dst<DT_F32>(a, dst_type, smode, st);
        return hipGetLastError();
    }
    log_fallback("dequant_generic_kernel", "columns, row pitch or pointers not aligned to the vector unit");
    dim3 grid(grid_for((int64_t)rows * cols)), block(256);
    launch_k(dequant_generic_kernel, grid, block, 0, st, a, dst_type, src_type, smode);
    return hipGetLastError();
}

// Any shape or alignment: one thread per output byte (one element; two for E2M1), 64-bit indices.
template <int DST, int T>
__global__ __launch_bounds__(256) void quant_policy_generic_kernel(QuantPolicyArgs a)
{
    const int64_t total = a.m * a.n;
    const int64_t per = qd_nibble(DST) ? 2 : 1;
    const int64_t bytes = total / per;
    for (int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x; b < bytes; b += (int64_t)gridDim.x * 256) {
        uint32_t w = 0;
        for (int64_t h = 0; h < per; ++h) {
            const int64_t e = b * per + h;
            const int64_t r = e / a.n, c = e - r * a.n;
            const int64_t si = a.layout == QL_TOKEN ? r : (a.layout == QL_KCOL ? r * a.sk + c / a.g
                                                                                : (r / a.g) * a.n + c);
            const float x = load_scale_t(a.src, a.src_type, e);
            const float s = a.scale ? load_scale_t(a.scale, a.scale_type, si) : a.sc_scalar;
            float v = mul_t<T>(x, s);
            if (a.has_off) v = add_t<T>(v, a.offset ? load_scale_t(a.offset, a.scale_type, si) : a.off_scalar);
            w |= quant_code_rt<DST, T>(v, a.round_mode) << (4 * h);
        }
        ((uint8_t*)a.dst)[b] = (uint8_t)w;
    }
}

template <int DST, int SRC, int SC, int MODE, bool FA>
static void launch_qp_layout(const QuantPolicyArgs& a, hipStream_t st)
{
    if (a.layout == QL_KROW)
        launch_k(quant_policy_vec_krow_kernel<DST, SRC, SC, MODE, FA>, dim3(grid_for(a.units)), dim3(256), 0, st, a);
    else
        launch_k(quant_policy_vec_kernel<DST, SRC, SC, MODE, FA>, dim3(grid_for((a.units + QP_UNR - 1) / QP_UNR)),
                 dim3(256), 0, st, a);
}

template <int DST, int SRC, int SC, bool FA = false>
static void launch_qp_vec(const QuantPolicyArgs& a, hipStream_t st)
{
    if constexpr (DST == QD_E4M3 || DST == QD_E5M2 || DST == QD_HIF8) {  // one rounding whatever the mode
        launch_qp_layout<DST, SRC, SC, RM_RINT, FA>(a, st);
        return;
    }
    switch (a.round_mode) {
    case RM_FLOOR: launch_qp_layout<DST, SRC, SC, RM_FLOOR, FA>(a, st); break;
    case RM_CEIL: launch_qp_layout<DST, SRC, SC, RM_CEIL, FA>(a, st); break;
    case RM_ROUND: launch_qp_layout<DST, SRC, SC, RM_ROUND, FA>(a, st); break;
    case RM_TRUNC: launch_qp_layout<DST, SRC, SC, RM_TRUNC, FA>(a, st); break;
    default: launch_qp_layout<DST, SRC, SC, RM_RINT, FA>(a, st); break;
    }
}

template <int DST, int SC>
static void launch_qp_src(const QuantPolicyArgs& a, hipStream_t st)
{
    if (a.src_type == DT_F16) launch_qp_vec<DST, DT_F16, SC>(a, st);
    else if (a.src_type == DT_BF16) launch_qp_vec<DST, DT_BF16, SC>(a, st);
    else launch_qp_vec<DST, DT_F32, SC>(a, st);
}

// T: arithmetic type -- the scale type for int8 / E2M1, which pair it with a source of the same type or an f32
// scale; fp32 for fp8, which takes any source and scale type, and for the Quantize form (a 16-bit scale then meets a
// source of its own type and is widened)
template <int DST, int T>
static void launch_qp(const QuantPolicyArgs& a, bool vec, hipStream_t st)
{
    if (!vec) {
        log_fallback("quant_policy_generic_kernel", "n, group or pointers not aligned to the vector unit");
        const int64_t bytes = qd_nibble(DST) ? a.m * a.n / 2 : a.m * a.n;
        launch_k(quant_policy_generic_kernel<DST, T>, dim3(grid_for(bytes)), dim3(256), 0, st, a);
        return;
    }
    if constexpr (DST == QD_E4M3 || DST == QD_E5M2) {
        if (a.scale_type == DT_F16) launch_qp_src<DST, DT_F16>(a, st);
        else if (a.scale_type == DT_BF16) launch_qp_src<DST, DT_BF16>(a, st);
        else launch_qp_src<DST, DT_F32>(a, st);
    } else if constexpr (T == DT_F16) {
        launch_qp_vec<DST, DT_F16, DT_F16>(a, st);
    } else if constexpr (T == DT_BF16) {
        launch_qp_vec<DST, DT_BF16, DT_BF16>(a, st);
    } else if (a.scale_type == DT_F16) {
        launch_qp_vec<DST, DT_F16, DT_F16, true>(a, st);
    } else if (a.scale_type == DT_BF16) {
        launch_qp_vec<DST, DT_BF16, DT_BF16, true>(a, st);
    } else {
        launch_qp_src<DST, DT_F32>(a, st);
    }
}

hipError_t launch_quant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale,
                               int scale_type, const void* offset, int has_offset, float offset_scalar, int per_token,
                               int64_t m, int64_t n, int64_t g, int k_dim, int round_mode, hipStream_t st,
                               float scale_scalar, int f32_arith)
{
    const int dk = dst_type == DT_INT8 ? QD_INT8
                   : dst_type == DT_HIF8 ? QD_HIF8
                   : dst_type == DT_FP8_E4M3 ? QD_E4M3
                   : dst_type == DT_FP8_E5M2 ? QD_E5M2
                   : dst_type == DT_FP4_E1M2 ? QD_E1M2 : QD_E2M1;
    QuantPolicyArgs a;
    a.dst = dst;
    a.src = src;
    a.scale = scale;
    a.has_off = has_offset && !qd_nibble(dk);
    a.offset = a.has_off ? offset : nullptr;
    // the scalar offset (and a scalar scale) are scaleT values: round them (rne) to the scale type once, here
    auto to_scale_type = [&](float v) {
        if (scale_type == DT_F16) return (float)(_Float16)v;
        if (scale_type == DT_BF16) {
            uint32_t u = __builtin_bit_cast(uint32_t, v);
            if ((u & 0x7fffffffu) <= 0x7f800000u) u = ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16;
            return __builtin_bit_cast(float, u);
        }
        return v;
    };
    a.off_scalar = to_scale_type(offset_scalar);
    a.sc_scalar = to_scale_type(scale_scalar);
    a.src_type = src_type;
    a.scale_type = scale_type;
    a.round_mode = round_mode;
    a.layout = per_token ? QL_TOKEN : (k_dim == 1 ? QL_KCOL : QL_KROW);
    a.m = m;
    a.n = n;
    a.g = g > 0 ? g : 1;
    a.sk = (n + a.g - 1) / a.g;
    // vector kernels: units of 8 elements; for groups down the columns, blocks of QP_UNR rows x (n / 8) units
    const int64_t units = a.layout == QL_KROW ? (m + QP_UNR - 1) / QP_UNR * (n / 8) : m * n / 8;
    const bool al = (uintptr_t)src % 16 == 0 && (uintptr_t)dst % (qd_nibble(dk) ? 4 : 8) == 0 &&
                    (a.layout != QL_KROW || ((uintptr_t)scale % 16 == 0 && (uintptr_t)a.offset % 16 == 0)) &&
                    (scale != nullptr || a.layout == QL_TOKEN);
    const bool vec = n % 8 == 0 && al && m * n / 8 < (1ll << 31) && a.g < (1ll << 31) && n < (1ll << 31);
    a.units = vec ? (uint32_t)units : 0u;
    a.upr = vec ? (uint32_t)(n / 8) : 1u;
    a.upr_div = fast_div(a.upr);
    if (vec && a.layout == QL_TOKEN) {  // the vector kernel reads PER_TOKEN as one group of n per row
        a.sk = 1;
        a.g_div = fast_div((uint32_t)n);
    } else {
        a.g_div = fast_div((uint32_t)(vec ? a.g : 1));
    }
    const int t = (dk == QD_E4M3 || dk == QD_E5M2 || f32_arith) ? DT_F32 : scale_type;  // arithmetic type
    if (dk == QD_E4M3) launch_qp<QD_E4M3, DT_F32>(a, vec, st);
    else if (dk == QD_E5M2) launch_qp<QD_E5M2, DT_F32>(a, vec, st);
    else if (dk == QD_INT8) {
        if (t == DT_F16) launch_qp<QD_INT8, DT_F16>(a, vec, st);
        else if (t == DT_BF16) launch_qp<QD_INT8, DT_BF16>(a, vec, st);
        else launch_qp<QD_INT8, DT_F32>(a, vec, st);
    } else if (dk == QD_HIF8) {  // the int8 path's scaleT arithmetic
        if (t == DT_F16) launch_qp<QD_HIF8, DT_F16>(a, vec, st);
        else if (t == DT_BF16) launch_qp<QD_HIF8, DT_BF16>(a, vec, st);
        else launch_qp<QD_HIF8, DT_F32>(a, vec, st);
    } else if (dk == QD_E1M2) {
        if (t == DT_F16) launch_qp<QD_E1M2, DT_F16>(a, vec, st);
        else if (t == DT_BF16) launch_qp<QD_E1M2, DT_BF16>(a, vec, st);
        else launch_qp<QD_E1M2, DT_F32>(a, vec, st);
    } else {
        if (t == DT_F16) launch_qp<QD_E2M1, DT_F16>(a, vec, st);
        else if (t == DT_BF16) launch_qp<QD_E2M1, DT_BF16>(a, vec, st);
        else launch_qp<QD_E2M1, DT_F32>(a, vec, st);
    }
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void antiquant_policy_kernel(void* __restrict__ dst, int dst_type,
                                                               const void* __restrict__ src, int src_type,
                                                               const void* __restrict__ scale,
                                                               const void* __restrict__ offset, int scale_type,
                                                               int per_token, int64_t m, int64_t n, int64_t g,
                                                               int col_groups, int is_transpose, int f32_arith)
{
    const int64_t total = m * n, sk = g > 0 ? (n + g - 1) / g : 1;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
        const int64_t r = idx / n, c = idx % n;
        const int64_t sidx = per_token ? (is_transpose ? c : r) : (col_groups ? r * sk + c / g : (r / g) * n + c);
        if (src_type == DT_FP4_E2M1 || src_type == DT_FP4_E1M2) {  // E8M0 scale, bf16 product, no offset
            const uint32_t b = ((const uint8_t*)src)[idx >> 1];
            const uint32_t nib = (idx & 1) ? (b >> 4) : (b & 0xFu);
            const float v = src_type == DT_FP4_E1M2 ? e1m2_to_f32(nib) : e2m1_to_f32(nib);
            const uint32_t e = ((const uint8_t*)scale)[sidx];
            const float sc = e == 255u ? __uint_as_float(0x7fffffffu) : (e == 0u ? __uint_as_float(0x00400000u)
                                                                                 : __uint_as_float(e << 23));
            const float p = bf16_round(v * sc);
            if (dst_type == DT_F16) ((uint16_t*)dst)[idx] = f32_to_f16_sat(p);
            else ((uint16_t*)dst)[idx] = (uint16_t)(__float_as_uint(p) >> 16);
            continue;
        }
        const float s = load_scale_t(scale, scale_type, sidx);
        const float o = offset ? load_scale_t(offset, scale_type, sidx) : 0.0f;
        if (src_type == DT_FP8_E4M3 || src_type == DT_FP8_E5M2) {  // fp32 arithmetic
            float v = fp8_bits_to_f32(((const uint8_t*)src)[idx], src_type == DT_FP8_E5M2);
            if (offset) v = v + o;
            v = v * s;
            store_cast(dst, idx, v, dst_type);
            continue;
        }
        const uint32_t code = ((const uint8_t*)src)[idx];
        // arithmetic in the scale type (AscendAntiQuant), or in fp32 whatever the scale type (AntiQuantize)
        const int ar = f32_arith ? DT_F32 : scale_type;
        float v = src_type == DT_HIF8 ? hif8_to_f32(code) : (float)(int8_t)code;
        if (offset) v = add_rt(v, o, ar);
        v = mul_rt(v, s, ar);
        if (ar == DT_F16) ((uint16_t*)dst)[idx] = f32_to_f16(v);
        else if (ar == DT_BF16) ((uint16_t*)dst)[idx] = (uint16_t)(__float_as_uint(v) >> 16);
        else store_cast(dst, idx, v, dst_type);
    }
}

// Vector path of the policy form (n % 8 == 0, aligned pointers, fewer than 2^31 units): a unit is 8 consecutive
// elements of one row; each lane issues all loads of its units -- source (8 bytes; 4 for fp4), scale and offset,
// unconditionally with clamped indices, the scale table standing in for a missing offset -- before converting any.
// Scales: one per unit at r * sk + c / g (groups along the row; PER_TOKEN is sk = 1, g = n) or 8 contiguous at
// (r / g) * n + c (groups down the columns; transposed PER_TOKEN is g = m).  Stores: 16 bytes (f16 / bf16) or 32
// (f32) per unit.
constexpr int AQ_UNR = 4;
struct AntiQuantVecArgs {
    void* dst;
    const void* src;
    const void* scale;
    const void* offset;  // or null
    int64_t n, sk;
    uint32_t rows, units, upr;  // units: m * n / 8 (the row-blocked kernel recomputes its own)
    FastDiv upr_div, g_div;
};

// SRC: DT_INT8, DT_FP8_E4M3, DT_FP8_E5M2, DT_FP4_E2M1 or DT_FP4_E1M2; SC: scale type (E8M0 for fp4); DST: output type.
// One unit: source words xw (8 int8 / fp8 codes in two words, or 8 E2M1 nibbles in xw0), scale / offset bits
// (EIGHT: 8 per unit packed like the table; else one).
template <int SRC, int SC, int DST, bool EIGHT, int AR>
__device__ __forceinline__ void aq_unit(const AntiQuantVecArgs& a, uint32_t u, uint32_t xw0, uint32_t xw1,
                                        const uint32_t* sw, const uint32_t* ow, bool has_off)
{
    constexpr bool FP4 = SRC == DT_FP4_E2M1 || SRC == DT_FP4_E1M2, FP8 = SRC == DT_FP8_E4M3 || SRC == DT_FP8_E5M2;
    constexpr int SB = SC == DT_F32 ? 4 : (SC == DT_E8M0 ? 1 : 2);
    float y[8];
    if constexpr (FP4) {
        // E2M1 codes through the gfx950 decode with scale 1 (exact), then the E8M0 scale in fp32 and one bf16 rounding
        float e[8];
        typedef float f2 __attribute__((ext_vector_type(2)));
        if constexpr (SRC == DT_FP4_E1M2) {  // no E1M2 decode instruction: code * 0.25, exact
#pragma unroll
            for (int j = 0; j < 8; ++j) e[j] = e1m2_to_f32(xw0 >> (4 * j));
        } else {
        const f2 d0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(xw0, 1.0f, 0);
        const f2 d1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(xw0, 1.0f, 1);
        const f2 d2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(xw0, 1.0f, 2);
        const f2 d3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(xw0, 1.0f, 3);
        e[0] = d0.x, e[1] = d0.y, e[2] = d1.x, e[3] = d1.y, e[4] = d2.x, e[5] = d2.y, e[6] = d3.x, e[7] = d3.y;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t sb = EIGHT ? (sw[j >> 2] >> (8 * (j & 3))) & 0xffu : sw[0];
            const float sc = sb == 255u ? __uint_as_float(0x7fffffffu)
                                        : (sb == 0u ? __uint_as_float(0x00400000u) : __uint_as_float(sb << 23));
            y[j] = e[j] * sc;  // exact (a power of two times a 3-bit value) up to overflow to inf
        }
        if constexpr (DST == DT_BF16) {
            // the bf16 rounding two elements per gfx950 conversion (v_cvt_pk_bf16_f32, rne, equal to bf16_round on
            // every non-NaN input); a NaN product (E8M0 scale 0xFF) keeps its payload's top half, as bf16_round does
            uint32_t h[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float p0 = y[2 * q], p1 = y[2 * q + 1];
                const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2x){p0, p1}, bf2));
                const uint32_t lo = p0 != p0 ? __float_as_uint(p0) >> 16 : w & 0xffffu;
                const uint32_t hi = p1 != p1 ? __float_as_uint(p1) & 0xffff0000u : w & 0xffff0000u;
                h[q] = lo | hi;
            }
            __builtin_nontemporal_store((u32x4){h[0], h[1], h[2], h[3]}, (u32x4*)a.dst + u);
            return;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = bf16_round(y[j]);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t sb, ob;
            if constexpr (EIGHT && SB == 4) sb = sw[j], ob = ow[j];
            else if constexpr (EIGHT) sb = (sw[j >> 1] >> (16 * (j & 1))) & 0xffffu, ob = (ow[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            else sb = sw[0], ob = ow[0];
            const float s = raw_to_f32<SC>(sb), o = raw_to_f32<SC>(ob);
            const uint32_t code = ((j < 4 ? xw0 : xw1) >> (8 * (j & 3))) & 0xffu;
            if constexpr (FP8) {  // fp32 arithmetic
                float v = fp8_bits_to_f32(code, SRC == DT_FP8_E5M2);
                if (has_off) v = v + o;
                y[j] = v * s;
            } else {  // int8 / int4 / hifloat8: arithmetic in AR (the scale type, or the legacy form's choice)
                float v = SRC == DT_INT4 ? (float)((int32_t)(xw0 << (28 - 4 * j)) >> 28)
                                         : (SRC == DT_HIF8 ? hif8_to_f32(code) : (float)(int8_t)code);
                if (has_off) v = add_t<AR>(v, o);
                y[j] = mul_t<AR>(v, s);
            }
        }
    }
    if constexpr (DST == DT_F32) {
        u32x4* d = (u32x4*)a.dst + 2 * (int64_t)u;
        __builtin_nontemporal_store((u32x4){__float_as_uint(y[0]), __float_as_uint(y[1]), __float_as_uint(y[2]),
                                            __float_as_uint(y[3])}, d);
        __builtin_nontemporal_store((u32x4){__float_as_uint(y[4]), __float_as_uint(y[5]), __float_as_uint(y[6]),
                                            __float_as_uint(y[7])}, d + 1);
        return;
    }
    uint32_t h[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t lo, hi;
        if constexpr (DST == DT_BF16) {
            if constexpr (FP4 || (!FP8 && AR == DT_BF16))  // already bf16 values
                lo = __float_as_uint(y[2 * q]) >> 16, hi = __float_as_uint(y[2 * q + 1]) >> 16;
            else
                lo = f32_to_bf16_sat(y[2 * q]), hi = f32_to_bf16_sat(y[2 * q + 1]);
        } else {
            if constexpr (!FP4 && !FP8 && AR == DT_F16)  // half arithmetic: already half values (inf kept)
                lo = f32_to_f16(y[2 * q]), hi = f32_to_f16(y[2 * q + 1]);
            else
                lo = f32_to_f16_sat(y[2 * q]), hi = f32_to_f16_sat(y[2 * q + 1]);
        }
        h[q] = lo | (hi << 16);
    }
    __builtin_nontemporal_store((u32x4){h[0], h[1], h[2], h[3]}, (u32x4*)a.dst + u);
}

template <int SRC>
__device__ __forceinline__ void aq_load_src(const void* src, uint32_t u, uint32_t& w0, uint32_t& w1)
{
    if constexpr (SRC == DT_FP4_E2M1 || SRC == DT_FP4_E1M2 || SRC == DT_INT4) {
        w0 = __builtin_nontemporal_load((const uint32_t*)src + u), w1 = 0u;
    } else {
        const u32x2 x = __builtin_nontemporal_load((const u32x2*)src + u);
        w0 = x.x, w1 = x.y;
    }
}

// 8 scale (or offset) entries from element index si (a multiple of 8) into w, packed as in memory
template <int SB>
__device__ __forceinline__ void aq_load8(const void* p, int64_t si, uint32_t* w)
{
    if constexpr (SB == 4) {
        const u32x4* q = (const u32x4*)((const float*)p + si);
        const u32x4 a = q[0], b = q[1];
        w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    } else if constexpr (SB == 2) {
        const u32x4 a = *(const u32x4*)((const uint16_t*)p + si);
        w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w;
    } else {
        const u32x2 a = *(const u32x2*)((const uint8_t*)p + si);
        w[0] = a.x, w[1] = a.y;
    }
}

// one scale per unit (groups along the row; PER_TOKEN by row): AQ_UNR * 256 consecutive units per workgroup pass
template <int SRC, int SC, int DST, int AR = SC>
__global__ __launch_bounds__(256) void antiquant_policy_vec_kernel(AntiQuantVecArgs a)
{
    constexpr int SB = SC == DT_F32 ? 4 : (SC == DT_E8M0 ? 1 : 2);
    const bool has_off = a.offset != nullptr;
    const void* offp = has_off ? a.offset : a.scale;
    for (uint32_t b0 = blockIdx.x * (256u * AQ_UNR); b0 < a.units; b0 += gridDim.x * (256u * AQ_UNR)) {
        uint32_t x0[AQ_UNR], x1[AQ_UNR], sw[AQ_UNR], ow[AQ_UNR];
#pragma unroll
        for (int k = 0; k < AQ_UNR; ++k) {
            uint32_t u = b0 + k * 256u + threadIdx.x;
            u = u < a.units ? u : a.units - 1u;  // past the end: load a valid unit, store nothing
            aq_load_src<SRC>(a.src, u, x0[k], x1[k]);
            const uint32_t r = fdiv(u, a.upr_div), c = (u - r * a.upr) * 8u;
            const int64_t si = (int64_t)r * a.sk + fdiv(c, a.g_div);
            // no offset tensor: aq_unit reads no offset, so none is loaded
            if constexpr (SB == 4) sw[k] = ((const uint32_t*)a.scale)[si], ow[k] = has_off ? ((const uint32_t*)offp)[si] : 0u;
            else if constexpr (SB == 2) sw[k] = ((const uint16_t*)a.scale)[si], ow[k] = has_off ? ((const uint16_t*)offp)[si] : 0u;
            else sw[k] = ((const uint8_t*)a.scale)[si], ow[k] = 0u;
        }
#pragma unroll
        for (int k = 0; k < AQ_UNR; ++k) {
            const uint32_t u = b0 + k * 256u + threadIdx.x;
            if (u >= a.units) break;
            aq_unit<SRC, SC, DST, false, AR>(a, u, x0[k], x1[k], &sw[k], &ow[k], has_off);
        }
    }
}

// 8 scales per unit (groups down the columns; PER_TOKEN by column): a lane takes the same 8 columns of AQ_UNR
// consecutive rows (AQ_UNR divides every group size), so one load of 8 scales and offsets serves all of them;
// units: row blocks x (n / 8)
template <int SRC, int SC, int DST, int AR = SC>
__global__ __launch_bounds__(256) void antiquant_policy_vec_krow_kernel(AntiQuantVecArgs a)
{
    constexpr int SB = SC == DT_F32 ? 4 : (SC == DT_E8M0 ? 1 : 2);
    constexpr int SW = (8 * SB + 3) / 4;
    const bool has_off = a.offset != nullptr;
    const void* offp = has_off ? a.offset : a.scale;
    const uint32_t rows = a.rows;
    for (uint32_t v = blockIdx.x * 256u + threadIdx.x; v < a.units; v += gridDim.x * 256u) {
        const uint32_t rb = fdiv(v, a.upr_div), wu = v - rb * a.upr, r0 = rb * AQ_UNR;
        const int64_t si = (int64_t)fdiv(r0, a.g_div) * a.n + 8 * (int64_t)wu;
        uint32_t sw[SW], ow[SW] = {}, x0[AQ_UNR], x1[AQ_UNR];
        aq_load8<SB>(a.scale, si, sw);
        if (SB != 1 && has_off) aq_load8<SB>(offp, si, ow);
#pragma unroll
        for (int k = 0; k < AQ_UNR; ++k) {
            const uint32_t r = r0 + k < rows ? r0 + k : rows - 1u;
            aq_load_src<SRC>(a.src, r * a.upr + wu, x0[k], x1[k]);
        }
#pragma unroll
        for (int k = 0; k < AQ_UNR; ++k) {
            if (r0 + k >= rows) break;
            aq_unit<SRC, SC, DST, true, AR>(a, (r0 + k) * a.upr + wu, x0[k], x1[k], sw, ow, has_off);
        }
    }
}

template <int SRC, int SC, int DST, int AR = SC>
static void launch_aq_vec(const AntiQuantVecArgs& a, bool eight, hipStream_t st)
{
    if (eight) {
        AntiQuantVecArgs b = a;
        b.units = (a.rows + AQ_UNR - 1) / AQ_UNR * a.upr;
        launch_k(antiquant_policy_vec_krow_kernel<SRC, SC, DST, AR>, dim3(grid_for(b.units)), dim3(256), 0, st, b);
    } else {
        launch_k(antiquant_policy_vec_kernel<SRC, SC, DST, AR>, dim3(grid_for((a.units + AQ_UNR - 1) / AQ_UNR)),
                 dim3(256), 0, st, a);
    }
}

template <int SRC, int SC>
static void launch_aq_dst(const AntiQuantVecArgs& a, int dst_type, bool eight, hipStream_t st)
{
    if (dst_type == DT_F16) launch_aq_vec<SRC, SC, DT_F16>(a, eight, st);
    else if (dst_type == DT_BF16) launch_aq_vec<SRC, SC, DT_BF16>(a, eight, st);
    else if constexpr (SRC != DT_FP4_E2M1 && SRC != DT_FP4_E1M2) launch_aq_vec<SRC, SC, DT_F32>(a, eight, st);
}

// fa: fp32 arithmetic for int8 / hifloat8 sources whatever the scale type (AntiQuantize), else the scale type's
template <int SRC>
static void launch_aq_scale(const AntiQuantVecArgs& a, int dst_type, int scale_type, bool eight, hipStream_t st,
                            bool fa)
{
    if constexpr (SRC == DT_FP4_E2M1 || SRC == DT_FP4_E1M2) {
        launch_aq_dst<SRC, DT_E8M0>(a, dst_type, eight, st);
    } else if constexpr (SRC == DT_INT8 || SRC == DT_HIF8) {  // a 16-bit scale writes its own type
        if (scale_type == DT_F16 && fa) launch_aq_vec<SRC, DT_F16, DT_F16, DT_F32>(a, eight, st);
        else if (scale_type == DT_BF16 && fa) launch_aq_vec<SRC, DT_BF16, DT_BF16, DT_F32>(a, eight, st);
        else if (scale_type == DT_F16) launch_aq_vec<SRC, DT_F16, DT_F16>(a, eight, st);
        else if (scale_type == DT_BF16) launch_aq_vec<SRC, DT_BF16, DT_BF16>(a, eight, st);
        else launch_aq_dst<SRC, DT_F32>(a, dst_type, eight, st);
    } else {
        if (scale_type == DT_F16) launch_aq_dst<SRC, DT_F16>(a, dst_type, eight, st);
        else if (scale_type == DT_BF16) launch_aq_dst<SRC, DT_BF16>(a, dst_type, eight, st);
        else launch_aq_dst<SRC, DT_F32>(a, dst_type, eight, st);
    }
}

hipError_t launch_antiquant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale,
                                   const void* offset, int scale_type, int per_token, int64_t m, int64_t n,
                                   int64_t g, int col_groups, int is_transpose, hipStream_t st, int f32_arith)
{
    // one scale per unit (groups along the row, PER_TOKEN by row) or 8 contiguous (groups down the columns,
    // PER_TOKEN by column); for the vector path the per-token cases become groups of n columns / m rows
    const bool eight = per_token ? is_transpose != 0 : !col_groups;
    const int64_t gv = per_token ? (is_transpose ? m : n) : g;
    const int sbytes = scale_type == DT_F32 ? 4 : (scale_type == DT_E8M0 ? 1 : 2);
    const bool al = (uintptr_t)src % 8 == 0 && (uintptr_t)dst % 16 == 0 &&
                    (!eight || ((uintptr_t)scale % (8 * sbytes) == 0 && (uintptr_t)offset % (8 * sbytes) == 0));
    if (n % 8 == 0 && al && m * n / 8 < (1ll << 31) && gv > 0 && gv < (1ll << 31) && n < (1ll << 31)) {
        AntiQuantVecArgs a;
        a.dst = dst;
        a.src = src;
        a.scale = scale;
        a.offset = offset;
        a.n = n;
        a.sk = per_token ? 1 : (n + g - 1) / g;
        a.rows = (uint32_t)m;
        a.units = (uint32_t)(m * n / 8);
        a.upr = (uint32_t)(n / 8);
        a.upr_div = fast_div(a.upr);
        a.g_div = fast_div((uint32_t)gv);
        const bool fa = f32_arith != 0;
        if (src_type == DT_INT8) launch_aq_scale<DT_INT8>(a, dst_type, scale_type, eight, st, fa);
        else if (src_type == DT_HIF8) launch_aq_scale<DT_HIF8>(a, dst_type, scale_type, eight, st, fa);
        else if (src_type == DT_FP8_E4M3) launch_aq_scale<DT_FP8_E4M3>(a, dst_type, scale_type, eight, st, fa);
        else if (src_type == DT_FP8_E5M2) launch_aq_scale<DT_FP8_E5M2>(a, dst_type, scale_type, eight, st, fa);
        else if (src_type == DT_FP4_E1M2) launch_aq_scale<DT_FP4_E1M2>(a, dst_type, scale_type, eight, st, fa);
        else launch_aq_scale<DT_FP4_E2M1>(a, dst_type, scale_type, eight, st, fa);
        return hipGetLastError();
    }
    log_fallback("antiquant_policy_kernel", "n, group or pointers not aligned to the vector unit");
    dim3 grid(grid_for(m * n)), block(256);
    launch_k(antiquant_policy_kernel, grid, block, 0, st, dst, dst_type, src, src_type, scale, offset, scale_type,
             per_token, m, n, g, col_groups, is_transpose, f32_arith);
    return hipGetLastError();
}

// Legacy AscendAntiQuant through the vector kernels of the policy form: [K, N] with scales [K/g, N] is groups of g
// rows down the columns, the transposed [N, K] with scales [N, K/g] groups of g along each row.  The half path is
// the policy form's int8 arithmetic with half scales; the fp32 path keeps its f16 / bf16 tables but computes in
// fp32 (AR) and casts once.  Needs rows of a multiple of 8 elements, g % 4 == 0 (groups down the columns: four
// rows share a scale load) or g % 8 == 0 (along a row), and aligned pointers.
template <int SRC>
static void launch_antiquant_legacy_vec(const AntiQuantVecArgs& a, int dst_type, int arith, bool eight, hipStream_t st)
{
    if constexpr (SRC == DT_FP8_E4M3 || SRC == DT_FP8_E5M2) {  // fp32 ops, one rne cast, whatever arith
        if (dst_type == DT_BF16) launch_aq_vec<SRC, DT_BF16, DT_BF16, DT_F32>(a, eight, st);
        else launch_aq_vec<SRC, DT_F16, DT_F16, DT_F32>(a, eight, st);
    } else if constexpr (SRC == DT_HIF8) {  // half ops to f16; bf16 ops along rows ([K, N]), fp32 ops transposed
        if (dst_type == DT_F16) launch_aq_vec<SRC, DT_F16, DT_F16, DT_F16>(a, eight, st);
        else if (eight) launch_aq_vec<SRC, DT_BF16, DT_BF16, DT_BF16>(a, eight, st);
        else launch_aq_vec<SRC, DT_BF16, DT_BF16, DT_F32>(a, eight, st);
    } else {
        if (dst_type == DT_BF16) launch_aq_vec<SRC, DT_BF16, DT_BF16, DT_F32>(a, eight, st);
        else if (arith == 0) launch_aq_vec<SRC, DT_F16, DT_F16, DT_F16>(a, eight, st);
        else launch_aq_vec<SRC, DT_F16, DT_F16, DT_F32>(a, eight, st);
    }
}

// AscendAntiQuant per tensor (scalar offset / scale of the output type): a unit is 8 consecutive elements, AQ_UNR
// units per lane, every load issued before converting; the scalars ride in the argument block.
template <int SRC, int DST, int AR>
__global__ __launch_bounds__(256) void antiquant_scalar_vec_kernel(AntiQuantVecArgs a, uint32_t sbits, uint32_t obits,
                                                                   int has_off)
{
    for (uint32_t b0 = blockIdx.x * (256u * AQ_UNR); b0 < a.units; b0 += gridDim.x * (256u * AQ_UNR)) {
        uint32_t x0[AQ_UNR], x1[AQ_UNR];
#pragma unroll
        for (int k = 0; k < AQ_UNR; ++k) {
            const uint32_t u = b0 + k * 256u + threadIdx.x;
            aq_load_src<SRC>(a.src, u < a.units ? u : a.units - 1u, x0[k], x1[k]);
        }
#pragma unroll
        for (int k = 0; k < AQ_UNR; ++k) {
            const uint32_t u = b0 + k * 256u + threadIdx.x;
            if (u >= a.units) break;
            aq_unit<SRC, DST, DST, false, AR>(a, u, x0[k], x1[k], &sbits, &obits, has_off != 0);
        }
    }
}

template <int SRC, int DST>
static void launch_aq_scalar(const AntiQuantVecArgs& a, int ar, uint32_t sb, uint32_t ob, int has_off, hipStream_t st)
{
    const dim3 grid(grid_for((a.units + AQ_UNR - 1) / AQ_UNR)), block(256);
    if (ar == DT_F16) launch_k(antiquant_scalar_vec_kernel<SRC, DST, DT_F16>, grid, block, 0, st, a, sb, ob, has_off);
    else launch_k(antiquant_scalar_vec_kernel<SRC, DST, DT_F32>, grid, block, 0, st, a, sb, ob, has_off);
}

template <int SRC>
static void launch_aq_scalar_dst(const AntiQuantVecArgs& a, int dst_type, int ar, uint32_t sb, uint32_t ob,
                                 int has_off, hipStream_t st)
{
    if (dst_type == DT_F16) launch_aq_scalar<SRC, DT_F16>(a, ar, sb, ob, has_off, st);
    else launch_aq_scalar<SRC, DT_BF16>(a, ar, sb, ob, has_off, st);
}

hipError_t launch_antiquant_scalar(void* dst, int dst_type, const void* src, int src_type, uint16_t offset,
                                   uint16_t scale, int has_offset, int64_t count, hipStream_t st, int f32_arith)
{
    (void)hipGetLastError();
    // AscendAntiQuant's arithmetic, or fp32 with one cast whatever the types (AntiQuantize)
    const int ar = f32_arith ? DT_F32 : aq_arith(src_type, dst_type, 0, 1, dst_type == DT_F16 ? 0 : 1);
    const int64_t sbytes = src_type == DT_INT4 ? 4 : 8;  // source bytes per 8 elements
    if (count % 8 == 0 && count / 8 < (1ll << 31) && (uintptr_t)src % sbytes == 0 && (uintptr_t)dst % 16 == 0) {
        AntiQuantVecArgs a{};
        a.dst = dst;
        a.src = src;
        a.units = (uint32_t)(count / 8);
        if (src_type == DT_INT8) launch_aq_scalar_dst<DT_INT8>(a, dst_type, ar, scale, offset, has_offset, st);
        else if (src_type == DT_INT4) launch_aq_scalar_dst<DT_INT4>(a, dst_type, ar, scale, offset, has_offset, st);
        else if (src_type == DT_HIF8) launch_aq_scalar_dst<DT_HIF8>(a, dst_type, ar, scale, offset, has_offset, st);
        else if (src_type == DT_FP8_E4M3) launch_aq_scalar_dst<DT_FP8_E4M3>(a, dst_type, ar, scale, offset, has_offset, st);
        else launch_aq_scalar_dst<DT_FP8_E5M2>(a, dst_type, ar, scale, offset, has_offset, st);
        return hipGetLastError();
    }
    const float sc = dst_type == DT_F16 ? (float)__builtin_bit_cast(_Float16, scale) : __builtin_bit_cast(float, (uint32_t)scale << 16);
    const float of = dst_type == DT_F16 ? (float)__builtin_bit_cast(_Float16, offset) : __builtin_bit_cast(float, (uint32_t)offset << 16);
    log_fallback("antiquant_scalar_elem_kernel", "count not a multiple of 8 or pointers not aligned");
    launch_k(antiquant_scalar_elem_kernel, dim3(grid_for(count)), dim3(256), 0, st, dst, dst_type, src, src_type, of, sc,
             has_offset, count, ar);
    return hipGetLastError();
}

hipError_t launch_antiquant(void* dst, int dst_type, const void* src, int src_type, const void* offset,
                            const void* scale, uint32_t K, uint32_t N, uint32_t g, int is_transpose, int arith,
                            hipStream_t st)
{
    {
        const bool eight = !is_transpose;
        const int64_t rows = is_transpose ? N : K, n = is_transpose ? K : N;
        const bool al = (uintptr_t)src % 8 == 0 && (uintptr_t)dst % 16 == 0 &&
                        (!eight || ((uintptr_t)scale % 16 == 0 && (uintptr_t)offset % 16 == 0));
        if (n % 8 == 0 && g % (eight ? 4 : 8) == 0 && al && rows * n / 8 < (1ll << 31)) {
            AntiQuantVecArgs a;
            a.dst = dst;
            a.src = src;
            a.scale = scale;
            a.offset = offset;
            a.n = n;
            a.sk = eight ? 1 : K / g;
            a.rows = (uint32_t)rows;
            a.units = (uint32_t)(rows * n / 8);
            a.upr = (uint32_t)(n / 8);
            a.upr_div = fast_div(a.upr);
            a.g_div = fast_div(g);
            if (src_type == DT_INT4) launch_antiquant_legacy_vec<DT_INT4>(a, dst_type, arith, eight, st);
            else if (src_type == DT_HIF8) launch_antiquant_legacy_vec<DT_HIF8>(a, dst_type, arith, eight, st);
            else if (src_type == DT_FP8_E4M3) launch_antiquant_legacy_vec<DT_FP8_E4M3>(a, dst_type, arith, eight, st);
            else if (src_type == DT_FP8_E5M2) launch_antiquant_legacy_vec<DT_FP8_E5M2>(a, dst_type, arith, eight, st);
            else launch_antiquant_legacy_vec<DT_INT8>(a, dst_type, arith, eight, st);
            return hipGetLastError();
        }
    }
    log_fallback("antiquant_kernel", "n, group or pointers not aligned to the vector unit");
    dim3 grid(grid_for((int64_t)K * N)), block(256);
    launch_k(antiquant_kernel, grid, block, 0, st, dst, dst_type, src, src_type, (const uint16_t*)offset,
                       (const uint16_t*)scale, K, N, g, is_transpose, arith);
    return hipGetLastError();
}

}  // namespace ascq
