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
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
        uint32_t c = t + j * 256u;
        if (c < chunks) v[j] = __builtin_nontemporal_load(xr + c);
        else v[j] = (u32x4){0u, 0u, 0u, 0u};
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
// Per-token quant with given fp32 scale / offset (policy API PER_TOKEN).
// ---------------------------------------------------------------------------------------------
template <int MODE, bool HAS_OFFSET>
__global__ __launch_bounds__(256) void quant_per_token_kernel(const void* __restrict__ x, int8_t* __restrict__ q,
                                                              const float* __restrict__ scale,
                                                              const float* __restrict__ offset, int64_t total,
                                                              uint32_t n, int src_type)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        int64_t row = i / n;
        float v = load_f32_of(x, i, src_type) * scale[row];
        if constexpr (HAS_OFFSET) v = v + offset[row];
        q[i] = (int8_t)quant_s8<MODE>(v);
    }
}

// ---------------------------------------------------------------------------------------------
// Legacy AscendQuant: half arithmetic.  t = half(x); t = t*s; t = t+o; q = sat_s8(rint(t)).
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_legacy_f16_kernel(const void* __restrict__ x, int8_t* __restrict__ q,
                                                               const uint16_t* __restrict__ scale,
                                                               const uint16_t* __restrict__ offset,
                                                               uint16_t scale_scalar, uint16_t offset_scalar,
                                                               int64_t total, uint32_t scale_count, int src_type)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        _Float16 xh = src_type == DT_F16 ? bits_h(((const uint16_t*)x)[i]) : (_Float16)(((const float*)x)[i]);
        uint32_t c = scale_count ? (uint32_t)(i % scale_count) : 0u;
        _Float16 s = bits_h(scale ? scale[c] : scale_scalar);
        _Float16 o = bits_h(offset ? offset[c] : offset_scalar);
        _Float16 t = xh * s;
        t = t + o;
        q[i] = (int8_t)quant_s8<RM_RINT>((float)t);
    }
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
    for (int k = 0; k < U; ++k) {
        const uint32_t u = u0 + k * 256u;
        v[k] = u < units_per_row ? __builtin_nontemporal_load(q + base + u) : (u32x2){0u, 0u};
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

// Generic: policy PER_CHANNEL (j < cal_count uses scale[j]), PER_TOKEN (scale[i]), PER_TENSOR (scalar).
__global__ __launch_bounds__(256) void dequant_generic_kernel(void* __restrict__ y, int dst_type,
                                                              const void* __restrict__ src, int src_type,
                                                              const void* __restrict__ scale, int scale_type,
                                                              float scale_scalar, int policy, uint32_t m, uint32_t n,
                                                              uint32_t cols)
{
    const int64_t total = (int64_t)m * cols;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        int64_t i = t / cols, j = t % cols;
        float s = policy == 1 ? load_f32_of(scale, j, scale_type)
                              : (policy == 2 ? load_f32_of(scale, i, scale_type) : scale_scalar);
        int64_t idx = i * n + j;
        float v = load_f32_of(src, idx, src_type) * s;
        store_cast(y, idx, v, dst_type);
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

__global__ __launch_bounds__(256) void antiquant_kernel(void* __restrict__ dst, int dst_type,
                                                        const void* __restrict__ src, int src_type,
                                                        const uint16_t* __restrict__ offset,
                                                        const uint16_t* __restrict__ scale, uint32_t K, uint32_t N,
                                                        uint32_t g, int is_transpose, int arith)
{
    const int64_t total = (int64_t)K * N;
    const uint32_t G = K / g;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total; t += (int64_t)gridDim.x * 256) {
        // t enumerates dst in memory order
        int64_t k, n;
        if (is_transpose) { n = t / K; k = t % K; }
        else { k = t / N; n = t % N; }
        int64_t sidx = is_transpose ? n * G + k / g : (k / g) * N + n;
        int32_t qv = load_q(src, src_type, t);
        if (dst_type == DT_F16 && arith == 0) {
            _Float16 w = (_Float16)(float)qv;
            if (offset) w = w + bits_h(offset[sidx]);
            w = w * bits_h(scale[sidx]);
            ((uint16_t*)dst)[t] = h_bits(w);
        } else {
            float sc = load_f32_of(scale, sidx, dst_type);
            float v = (float)qv;
            if (offset) v = v + load_f32_of(offset, sidx, dst_type);
            v = v * sc;
            store_cast(dst, t, v, dst_type);
        }
    }
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

hipError_t launch_quant_per_token(int8_t* q, const void* x, int src_type, const float* scale, const float* offset,
                                  uint32_t m, uint32_t n, int round_mode, hipStream_t st)
{
    int64_t total = (int64_t)m * n;
    dim3 grid(grid_for(total)), block(256);
#define ASCQ_PT(MD)                                                                                                 \
    if (offset) launch_k((quant_per_token_kernel<MD, true>), grid, block, 0, st, x, q, scale, offset,     \
                                   total, n, src_type);                                                             \
    else launch_k((quant_per_token_kernel<MD, false>), grid, block, 0, st, x, q, scale, offset, total, n, \
                            src_type);                                                                              \
    break;
    switch (round_mode) {
    case RM_FLOOR: ASCQ_PT(RM_FLOOR)
    case RM_CEIL: ASCQ_PT(RM_CEIL)
    case RM_ROUND: ASCQ_PT(RM_ROUND)
    case RM_TRUNC: ASCQ_PT(RM_TRUNC)
    default: ASCQ_PT(RM_RINT)
    }
#undef ASCQ_PT
    return hipGetLastError();
}

hipError_t launch_quant_legacy(int8_t* q, const void* x, int src_type, const uint16_t* scale, const uint16_t* offset,
                               uint16_t scale_scalar, uint16_t offset_scalar, uint32_t cal_count,
                               uint32_t scale_count, hipStream_t st)
{
    dim3 grid(grid_for(cal_count)), block(256);
    launch_k(quant_legacy_f16_kernel, grid, block, 0, st, x, q, scale, offset, scale_scalar, offset_scalar,
                       (int64_t)cal_count, scale_count, src_type);
    return hipGetLastError();
}

hipError_t launch_dequant(void* y, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                          float scale_scalar, int policy, uint32_t m, uint32_t n, uint32_t cal_count, hipStream_t st)
{
    const bool fast = policy == 2 && src_type == DT_INT8 && dst_type == DT_F16 && scale_type == DT_F32 &&
                      n % 8 == 0 && ((uintptr_t)src % 8 == 0) && ((uintptr_t)y % 16 == 0) && m > 0 && n > 0;
    if (fast) {
        constexpr int U = 2;  // measured best at 8192 x 8192 (U = 1: 37.6 us, 2: 33.7 us, 4: 34.6 us)
        const uint32_t upr = n / 8;
        const uint32_t segs = (upr + 256 * U - 1) / (256 * U);
        const uint64_t blocks = (uint64_t)m * segs;
        if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
        launch_k(dequant_i8_token_f16_kernel<U>, dim3((unsigned)blocks), dim3(256), 0, st,
                           (const u32x2*)src, (const float*)scale, (u32x4*)y, upr, segs);
        return hipGetLastError();
    }
    uint32_t cols = policy == 1 ? cal_count : n;
    dim3 grid(grid_for((int64_t)m * cols)), block(256);
    launch_k(dequant_generic_kernel, grid, block, 0, st, y, dst_type, src, src_type, scale, scale_type,
                       scale_scalar, policy, m, n, cols);
    return hipGetLastError();
}

// AscendAntiQuant policy form (arch 3510, ascend_antiquant_3510_impl.h:1386-1412, 1458-2110, 2175-2221): one thread
// per element of the [m, n] tensor.  Half and bf16 arithmetic is an fp32 operation rounded once to the 16-bit
// type, which equals the correctly rounded 16-bit operation (fp32 carries more than 2p + 2 bits of either).
__device__ __forceinline__ float bf16_round(float x)  // rne to bf16, overflow to inf, NaN kept
{
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    return __uint_as_float(((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16);
}
__device__ __forceinline__ float round_scale_t(float x, int t)
{
    if (t == DT_F16) return (float)(_Float16)x;
    if (t == DT_BF16) return bf16_round(x);
    return x;
}
__device__ __forceinline__ float load_scale_t(const void* p, int t, int64_t i)
{
    if (t == DT_F16) return f16_to_f32(((const uint16_t*)p)[i]);
    if (t == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

__global__ __launch_bounds__(256) void antiquant_policy_kernel(void* __restrict__ dst, int dst_type,
                                                               const void* __restrict__ src, int src_type,
                                                               const void* __restrict__ scale,
                                                               const void* __restrict__ offset, int scale_type,
                                                               int per_token, int64_t m, int64_t n, int64_t g,
                                                               int col_groups, int is_transpose)
{
    const int64_t total = m * n, sk = g > 0 ? (n + g - 1) / g : 1;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
        const int64_t r = idx / n, c = idx % n;
        const int64_t sidx = per_token ? (is_transpose ? c : r) : (col_groups ? r * sk + c / g : (r / g) * n + c);
        if (src_type == DT_FP4_E2M1) {  // E8M0 scale, bf16 product, no offset
            const uint32_t b = ((const uint8_t*)src)[idx >> 1];
            const float v = e2m1_to_f32((idx & 1) ? (b >> 4) : (b & 0xFu));
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
        float v = (float)((const int8_t*)src)[idx];  // arithmetic in the scale type
        if (offset) v = round_scale_t(v + o, scale_type);
        v = round_scale_t(v * s, scale_type);
        if (scale_type == DT_F16) ((uint16_t*)dst)[idx] = f32_to_f16(v);
        else if (scale_type == DT_BF16) ((uint16_t*)dst)[idx] = (uint16_t)(__float_as_uint(v) >> 16);
        else store_cast(dst, idx, v, dst_type);
    }
}

hipError_t launch_antiquant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale,
                                   const void* offset, int scale_type, int per_token, int64_t m, int64_t n,
                                   int64_t g, int col_groups, int is_transpose, hipStream_t st)
{
    dim3 grid(grid_for(m * n)), block(256);
    launch_k(antiquant_policy_kernel, grid, block, 0, st, dst, dst_type, src, src_type, scale, offset, scale_type,
             per_token, m, n, g, col_groups, is_transpose);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// AscendQuant policy form (arch 3510, ascend_quant_per_group_3510_impl.h:33-1340, dispatch :1451-1504):
// PER_TOKEN / PER_GROUP over [m, n] to int8, fp8 or E2M1.  Each lane takes 8 consecutive elements: one or two
// 16-byte source loads, one scale (PER_TOKEN, or a group along the row -- group sizes are multiples of 32) or
// 8 contiguous scales (groups down the columns), and an 8- (int8 / fp8) or 4-byte (E2M1) store.  Rows whose
// length is not a multiple of 8, or unaligned pointers, take the per-element path of the same kernel.
// ---------------------------------------------------------------------------------------------
enum : int { QD_INT8 = 0, QD_E4M3 = 1, QD_E5M2 = 2, QD_E2M1 = 3 };
enum : int { QL_TOKEN = 0, QL_KCOL = 1, QL_KROW = 2 };

struct QuantPolicyArgs {
    void* dst;
    const void* src;
    const void* scale;
    const void* offset;  // tensor indexed like scale, or null
    float off_scalar;    // used when has_off and offset is null (already a scaleT value)
    int has_off;
    int src_type, scale_type, round_mode, layout, fast;
    int64_t m, n, g, sk, units;  // units: ceil(m * n / 8)
};

// f32 -> fp8 with rint and saturation: NaN -> 0, overflow and inf -> +-max finite (TransRegForFp8,
// ascend_quant_3510_impl.h:888-896; docs/zh/api/SIMD-API/tensor_api/reg_vector_compute/type_conversion/cast.md:109)
__device__ __forceinline__ uint32_t f32_to_fp8_sat(float x, bool e5m2)
{
    if (x != x) return 0u;
    const float mx = e5m2 ? 57344.0f : 448.0f;
    return f32_to_fp8(__builtin_fminf(__builtin_fmaxf(x, -mx), mx), e5m2 ? 1 : 0);
}

// bf16 value -> E2M1 code in round mode `mode`, saturating at +-6 (Cast<fp4x2_e2m1_t, bfloat16_t>, cast.md:96).
// The code table is three uniform segments -- [0, 2) in steps of 0.5 (codes 0-4), [2, 4) in steps of 1 (4-6),
// [4, 6] in steps of 2 (6-7) -- so the code is the segment base plus the rounded, exactly scaled offset into it;
// every base is even, so ties to even on the offset are ties to an even code.  A directed mode on a negative value
// rounds the magnitude the other way.  NaN -> 0.
__device__ __forceinline__ uint32_t bf16_to_e2m1(float v, int mode)
{
    if (v != v) return 0u;
    const uint32_t s = (__float_as_uint(v) >> 28) & 8u;
    const float a = __builtin_fabsf(v);
    if (a >= 6.0f) return s | 7u;
    int mm = mode;
    if (s) mm = mode == RM_FLOOR ? RM_CEIL : (mode == RM_CEIL ? RM_FLOOR : mode);
    float q;
    uint32_t base;
    if (a < 2.0f) q = a * 2.0f, base = 0u;
    else if (a < 4.0f) q = a - 2.0f, base = 4u;
    else q = (a - 4.0f) * 0.5f, base = 6u;
    return s | (base + (uint32_t)round_mode_f(q, mm));
}

// one scaleT rounding of an fp32 result (exact for products of two 16-bit values; a single correct rounding for
// sums, since fp32 holds more than 2p + 2 bits of half and bf16)
template <int T>
__device__ __forceinline__ float rnd_t(float x)
{
    if constexpr (T == DT_F16) return (float)(_Float16)x;
    else if constexpr (T == DT_BF16) return bf16_round(x);
    else return x;
}

__device__ __forceinline__ void load8_f32(const void* p, int t, int64_t i, float (&o)[8])
{
    if (t == DT_F32) {
        const u32x4 a = __builtin_nontemporal_load((const u32x4*)((const float*)p + i));
        const u32x4 b = __builtin_nontemporal_load((const u32x4*)((const float*)p + i) + 1);
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = __uint_as_float(w[j]);
        return;
    }
    const u32x4 a = __builtin_nontemporal_load((const u32x4*)((const uint16_t*)p + i));
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint16_t lo = (uint16_t)(w[j] & 0xffffu), hi = (uint16_t)(w[j] >> 16);
        o[2 * j] = t == DT_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
        o[2 * j + 1] = t == DT_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
}

template <int DST, int T>
__global__ __launch_bounds__(256) void quant_policy_kernel(QuantPolicyArgs a)
{
    const int64_t total = a.m * a.n;
    for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < a.units; u += (int64_t)gridDim.x * 256) {
        const int64_t e0 = u * 8;
        float x[8], s[8], o[8];
        if (a.fast) {  // n % 8 == 0: the 8 elements share a row; aligned 16-byte loads
            const int64_t r = e0 / a.n, c = e0 - r * a.n;
            load8_f32(a.src, a.src_type, e0, x);
            if (a.layout == QL_KROW) {
                const int64_t si = (r / a.g) * a.n + c;
                load8_f32(a.scale, a.scale_type, si, s);
                if (a.offset) load8_f32(a.offset, a.scale_type, si, o);
            } else {
                const int64_t si = a.layout == QL_TOKEN ? r : r * a.sk + c / a.g;
                const float sv = load_scale_t(a.scale, a.scale_type, si);
                const float ov = a.offset ? load_scale_t(a.offset, a.scale_type, si) : 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) s[j] = sv, o[j] = ov;
            }
            if (!a.offset) {
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = a.off_scalar;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t e = e0 + j < total ? e0 + j : total - 1;  // clamped; lanes past the end are not stored
                const int64_t r = e / a.n, c = e - r * a.n;
                const int64_t si = a.layout == QL_TOKEN ? r : (a.layout == QL_KCOL ? r * a.sk + c / a.g
                                                                                    : (r / a.g) * a.n + c);
                x[j] = load_scale_t(a.src, a.src_type, e);
                s[j] = load_scale_t(a.scale, a.scale_type, si);
                o[j] = a.offset ? load_scale_t(a.offset, a.scale_type, si) : a.off_scalar;
            }
        }
        uint32_t code[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = rnd_t<T>(x[j] * s[j]);
            if (DST != QD_E2M1 && a.has_off) v = rnd_t<T>(v + o[j]);
            if constexpr (DST == QD_INT8) {
                code[j] = (uint32_t)sat_s8_from_integral(round_mode_f(v, a.round_mode)) & 0xffu;
            } else if constexpr (DST == QD_E4M3 || DST == QD_E5M2) {
                code[j] = f32_to_fp8_sat(v, DST == QD_E5M2);
            } else {
                if constexpr (T != DT_BF16) v = v != v ? 0.0f : bf16_to_f32(f32_to_bf16_sat(v));
                code[j] = bf16_to_e2m1(v, a.round_mode);
            }
        }
        if constexpr (DST == QD_E2M1) {
            const uint32_t w = code[0] | (code[1] << 4) | (code[2] << 8) | (code[3] << 12) | (code[4] << 16) |
                               (code[5] << 20) | (code[6] << 24) | (code[7] << 28);
            uint8_t* d = (uint8_t*)a.dst + e0 / 2;
            if (a.fast) {
                __builtin_nontemporal_store(w, (uint32_t*)d);
            } else {
                for (int j = 0; j < 4; ++j)
                    if (e0 + 2 * j < total) d[j] = (uint8_t)(w >> (8 * j));
            }
        } else {
            uint8_t* d = (uint8_t*)a.dst + e0;
            if (a.fast) {
                const u32x2 w = {code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24),
                                 code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24)};
                __builtin_nontemporal_store(w, (u32x2*)d);
            } else {
                for (int j = 0; j < 8; ++j)
                    if (e0 + j < total) d[j] = (uint8_t)code[j];
            }
        }
    }
}

hipError_t launch_quant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale,
                               int scale_type, const void* offset, int has_offset, float offset_scalar, int per_token,
                               int64_t m, int64_t n, int64_t g, int k_dim, int round_mode, hipStream_t st)
{
    QuantPolicyArgs a;
    a.dst = dst;
    a.src = src;
    a.scale = scale;
    a.offset = has_offset ? offset : nullptr;
    // the scalar offset is a scaleT value: round it (rne) to the scale type once, here
    float os = offset_scalar;
    if (scale_type == DT_F16) {
        os = (float)(_Float16)os;
    } else if (scale_type == DT_BF16) {
        uint32_t u = __builtin_bit_cast(uint32_t, os);
        if ((u & 0x7fffffffu) <= 0x7f800000u) u = ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16;
        os = __builtin_bit_cast(float, u);
    }
    a.off_scalar = os;
    a.has_off = has_offset;
    a.src_type = src_type;
    a.scale_type = scale_type;
    a.round_mode = round_mode;
    a.layout = per_token ? QL_TOKEN : (k_dim == 1 ? QL_KCOL : QL_KROW);
    a.m = m;
    a.n = n;
    a.g = g > 0 ? g : 1;
    a.sk = (n + a.g - 1) / a.g;
    a.units = (m * n + 7) / 8;
    const int dk = dst_type == DT_INT8 ? QD_INT8
                   : dst_type == DT_FP8_E4M3 ? QD_E4M3
                   : dst_type == DT_FP8_E5M2 ? QD_E5M2 : QD_E2M1;
    const uintptr_t dal = dk == QD_E2M1 ? 4 : 8;
    const bool al = (uintptr_t)src % 16 == 0 && (uintptr_t)dst % dal == 0 &&
                    (a.layout != QL_KROW || ((uintptr_t)scale % 16 == 0 && (uintptr_t)a.offset % 16 == 0));
    a.fast = n % 8 == 0 && al;
    const int t = (dk == QD_E4M3 || dk == QD_E5M2) ? DT_F32 : scale_type;  // arithmetic type
    dim3 grid(grid_for(a.units)), block(256);
#define QP_LAUNCH(D, T) launch_k(quant_policy_kernel<D, T>, grid, block, 0, st, a)
    if (dk == QD_E4M3) QP_LAUNCH(QD_E4M3, DT_F32);
    else if (dk == QD_E5M2) QP_LAUNCH(QD_E5M2, DT_F32);
    else if (dk == QD_INT8) {
        if (t == DT_F16) QP_LAUNCH(QD_INT8, DT_F16);
        else if (t == DT_BF16) QP_LAUNCH(QD_INT8, DT_BF16);
        else QP_LAUNCH(QD_INT8, DT_F32);
    } else {
        if (t == DT_F16) QP_LAUNCH(QD_E2M1, DT_F16);
        else if (t == DT_BF16) QP_LAUNCH(QD_E2M1, DT_BF16);
        else QP_LAUNCH(QD_E2M1, DT_F32);
    }
#undef QP_LAUNCH
    return hipGetLastError();
}

hipError_t launch_antiquant(void* dst, int dst_type, const void* src, int src_type, const void* offset,
                            const void* scale, uint32_t K, uint32_t N, uint32_t g, int is_transpose, int arith,
                            hipStream_t st)
{
    dim3 grid(grid_for((int64_t)K * N)), block(256);
    launch_k(antiquant_kernel, grid, block, 0, st, dst, dst_type, src, src_type, (const uint16_t*)offset,
                       (const uint16_t*)scale, K, N, g, is_transpose, arith);
    return hipGetLastError();
}

}  // namespace ascq
