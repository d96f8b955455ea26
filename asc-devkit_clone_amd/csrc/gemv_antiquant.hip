// gemv_antiquant.hip -- weight-only antiquant matmul (W4A16 / W8A16) for decode shapes on gfx950.
//
// Reference: AscendAntiQuant per group (include/adv_api/quantization/ascend_antiquant.h:47-62;
// impl/adv_api/detail/quantization/antiquant/ascend_antiquant_impl.h:63-96, 366-411) followed by a half
// Matmul with fp32 L0C (impl/adv_api/detail/matmul/utils/matmul_utils.h:171-174).  Here both run in one
// kernel: the weight is dequantised in registers, bit-exactly as AscendAntiQuant does it
//     w = half( half(q + offset) * scale )        (two IEEE binary16 ops, one rounding each)
// and fed to v_mfma_f32_16x16x32_f16 against the activations; accumulation is fp32, the output is rounded
// once to half (rne, saturating).
//
// Packed weight layout (the MFMA-native counterpart of the reference's ND -> NZ weight conversion):
//  * the logical weight w[k][n] is cut into tiles of 16 columns x 128 k; tile (nb, kb) is stored at
//    index nb * (K/128) + kb, so one 16-column strip is contiguous along K;
//  * inside a tile, lane l (0..63) owns column n = 16 nb + (l % 16) and, for each of the four 32-k MFMA
//    steps j, the eight k values 128 kb + 32 j + 8 (l / 16) + e (e = 0..7) -- exactly the B fragment of
//    v_mfma_f32_16x16x32_f16 for that lane.  Lane l's bytes are contiguous: a wave reads the tile with
//    one 16-byte (int4) or two 16-byte (int8) loads per lane, 1 KiB / 2 KiB contiguous per instruction;
//  * codes are stored offset-binary (q + 8 for int4, q + 128 for int8) so that OR-ing them under the
//    binary16 exponent of 1024 gives 1024 + code exactly; subtracting 1032 / 1152 restores q exactly;
//  * int4: in the 32-bit word of step j, element e sits at bits 4*(e/2) (e even) or 16 + 4*(e/2) (e odd),
//    so (word >> 4i) & 0x000F000F yields the pair (2i, 2i+1) as two half lanes;
//    int8: the 8 codes of step j are bytes 0..7 of an 8-byte chunk, in k order.
//
// Roofline: at decode shapes the kernel streams the packed weight once (K*N/2 or K*N bytes) plus the
// scales/offsets; it is HBM-bound at M = 1 and 16 and near the fp16 MFMA ridge at M = 64.
#include "common.h"
#include "launch.h"

namespace ascq {

constexpr int KT = 128;  // k per packed tile

size_t weight_pack_bytes(int w_type, int64_t K, int64_t N)
{
    return (size_t)K * (size_t)N / (w_type == DT_INT4 ? 2 : 1);
}

// one thread per (tile, lane): gathers 32 elements and writes 16 (int4) or 32 (int8) bytes
__global__ __launch_bounds__(256) void weight_pack_kernel(uint8_t* __restrict__ out, const uint8_t* __restrict__ w,
                                                          int w_type, int64_t K, int64_t N, int is_transpose)
{
    const int64_t KB = K / KT, NB = N / 16;
    const int64_t total = NB * KB * 64;
    for (int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x; id < total; id += (int64_t)gridDim.x * 256) {
        const int lane = (int)(id & 63);
        const int64_t tile = id >> 6, nb = tile / KB, kb = tile % KB;
        const int64_t n = nb * 16 + (lane & 15);
        uint32_t words[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 4; ++j)
            for (int e = 0; e < 8; ++e) {
                const int64_t k = kb * KT + 32 * j + 8 * (lane >> 4) + e;
                const int64_t idx = is_transpose ? n * K + k : k * N + n;
                int32_t q;
                if (w_type == DT_INT8) {
                    q = (int8_t)w[idx];
                    const uint32_t code = (uint32_t)(q + 128) & 0xffu;
                    words[2 * j + (e >> 2)] |= code << (8 * (e & 3));
                } else {
                    const uint8_t b = w[idx >> 1];
                    const int32_t nib = (idx & 1) ? (b >> 4) : (b & 0xf);
                    q = nib >= 8 ? nib - 16 : nib;
                    const uint32_t code = (uint32_t)(q + 8) & 0xfu;
                    const int shift = (e & 1) ? 16 + 4 * (e >> 1) : 4 * (e >> 1);
                    words[j] |= code << shift;
                }
            }
        if (w_type == DT_INT8) {
            u32x4* o = (u32x4*)(out + (tile * 64 + lane) * 32);
            o[0] = (u32x4){words[0], words[1], words[2], words[3]};
            o[1] = (u32x4){words[4], words[5], words[6], words[7]};
        } else {
            *(u32x4*)(out + (tile * 64 + lane) * 16) = (u32x4){words[0], words[1], words[2], words[3]};
        }
    }
}

hipError_t launch_weight_pack(void* packed, const void* w, int w_type, int64_t K, int64_t N, int is_transpose,
                              hipStream_t st)
{
    const int64_t total = (K / KT) * (N / 16) * 64;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(weight_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint8_t*)packed,
                       (const uint8_t*)w, w_type, K, N, is_transpose);
    return hipGetLastError();
}

// dequantise one 8-element B fragment: codes -> half(half(q + off) * scale)
template <bool INT4, bool HAS_OFF>
__device__ __forceinline__ h8 dequant8(uint32_t w0, uint32_t w1, h2 off, h2 sc)
{
    uint32_t d[4];
    if constexpr (INT4) {
        // w0 holds all 8 nibbles of the step; pair i = (w0 >> 4i) & 0x000F000F
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = ((w0 >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
    } else {
        // bytes b0..b3 of w0 and w1 -> halves 0x64bb
        d[0] = __builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u);
        d[1] = __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u);
        d[2] = __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u);
        d[3] = __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u);
    }
    const h2 bias = INT4 ? (h2){(_Float16)1032.0f, (_Float16)1032.0f} : (h2){(_Float16)1152.0f, (_Float16)1152.0f};
    h2 r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2 q = __builtin_bit_cast(h2, d[i]) - bias;  // exact
        if constexpr (HAS_OFF) q = q + off;          // one rounding
        r[i] = q * sc;                               // one rounding
    }
    h8 out;
    out.s01 = r[0];
    out.s23 = r[1];
    out.s45 = r[2];
    out.s67 = r[3];
    return out;
}

// One workgroup = KSPLIT waves over the same NBW 16-column strips, each wave a K/KSPLIT range; partial
// 16x16 tiles are summed through LDS in a fixed order.  MT = number of 16-row m tiles (ceil(M/16)).
// Latency: a wave issues all weight loads (and, when the quant group is a multiple of 128, all scale /
// offset loads) of a KPW-tile chunk before its first MFMA, and prefetches the activations one k tile ahead.
template <int MT, int NBW, int KSPLIT, int KPW, bool INT4, bool HAS_OFF, bool G128>
__global__ __launch_bounds__(KSPLIT * 64) void antiquant_gemm_kernel(uint16_t* __restrict__ y,
                                                                     const uint16_t* __restrict__ x,
                                                                     const uint8_t* __restrict__ wp,
                                                                     const uint16_t* __restrict__ scale,
                                                                     const uint16_t* __restrict__ offset,
                                                                     int64_t M, int64_t N, int64_t K, int64_t g)
{
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048;
    constexpr int LANE_BYTES = INT4 ? 16 : 32;
    constexpr int WV = INT4 ? 1 : 2;
    __shared__ v4f red[KSPLIT > 1 ? KSPLIT - 1 : 1][MT][NBW][64];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t KB = K / KT;
    const int64_t kb_per = (KB + KSPLIT - 1) / KSPLIT;
    const int64_t kb0 = wave * kb_per;
    const int64_t kb1 = kb0 + kb_per < KB ? kb0 + kb_per : KB;
    const int64_t nb0 = (int64_t)blockIdx.x * NBW;
    const int64_t NBT = N / 16;
    const int col_in = lane & 15, kq = lane >> 4;

    v4f acc[MT][NBW];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NBW; ++b) acc[a][b] = (v4f){0.f, 0.f, 0.f, 0.f};

    auto load_x = [&](int64_t kb, h8 (&xf)[MT][4]) {
#pragma unroll
        for (int a = 0; a < MT; ++a) {
            const int64_t m = 16 * a + col_in;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xf[a][j] = (m < M && kb < kb1) ? *(const h8*)(x + m * K + kb * KT + 32 * j + 8 * kq) : (h8){};
        }
    };

    for (int64_t kc = kb0; kc < kb1; kc += KPW) {
        u32x4 wv[KPW][NBW][WV];
        h2 sc[G128 ? KPW : 1][NBW], of[G128 ? KPW : 1][NBW];
#pragma unroll
        for (int i = 0; i < KPW; ++i)
#pragma unroll
            for (int b = 0; b < NBW; ++b) {
                const int64_t kb = kc + i, nb = nb0 + b;
                const bool ok = kb < kb1 && nb < NBT;
                const u32x4* p = (const u32x4*)(wp + (nb * KB + kb) * TILE_BYTES + lane * LANE_BYTES);
#pragma unroll
                for (int v = 0; v < WV; ++v) wv[i][b][v] = ok ? __builtin_nontemporal_load(p + v) : (u32x4){0u, 0u, 0u, 0u};
                if constexpr (G128) {
                    const int64_t idx = ((kb * KT) / g) * N + nb * 16 + col_in;
                    const _Float16 s = ok ? bits_h(scale[idx]) : (_Float16)0.0f;
                    const _Float16 o = (HAS_OFF && ok) ? bits_h(offset[idx]) : (_Float16)0.0f;
                    sc[i][b] = (h2){s, s};
                    of[i][b] = (h2){o, o};
                }
            }
        h8 xa[MT][4];
        load_x(kc, xa);
#pragma unroll
        for (int i = 0; i < KPW; ++i) {
            const int64_t kb = kc + i;
            if (kb >= kb1) break;
            h8 xn[MT][4];
            load_x(kb + 1, xn);  // next k tile (zeros past this wave's range)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int b = 0; b < NBW; ++b) {
                    h2 s2, o2;
                    if constexpr (G128) {
                        s2 = sc[i][b];
                        o2 = of[i][b];
                    } else {
                        const int64_t n = (nb0 + b) * 16 + col_in;
                        const bool ok = (nb0 + b) < NBT;
                        const int64_t idx = ((kb * KT + 32 * j + 8 * kq) / g) * N + n;
                        const _Float16 s = ok ? bits_h(scale[idx]) : (_Float16)0.0f;
                        const _Float16 o = (HAS_OFF && ok) ? bits_h(offset[idx]) : (_Float16)0.0f;
                        s2 = (h2){s, s};
                        o2 = (h2){o, o};
                    }
                    uint32_t w0, w1 = 0;
                    if constexpr (INT4) {
                        w0 = wv[i][b][0][j];
                    } else {
                        w0 = wv[i][b][j >> 1][(j & 1) * 2];
                        w1 = wv[i][b][j >> 1][(j & 1) * 2 + 1];
                    }
                    const h8 bf = dequant8<INT4, HAS_OFF>(w0, w1, o2, s2);
#pragma unroll
                    for (int a = 0; a < MT; ++a)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[a][j], bf, acc[a][b], 0, 0, 0);
                }
            }
#pragma unroll
            for (int a = 0; a < MT; ++a)
#pragma unroll
                for (int j = 0; j < 4; ++j) xa[a][j] = xn[a][j];
        }
    }

    if constexpr (KSPLIT > 1) {
        if (wave > 0) {
#pragma unroll
            for (int a = 0; a < MT; ++a)
#pragma unroll
                for (int b = 0; b < NBW; ++b) red[wave - 1][a][b][lane] = acc[a][b];
        }
        __syncthreads();
        if (wave != 0) return;
#pragma unroll
        for (int w = 0; w < KSPLIT - 1; ++w)
#pragma unroll
            for (int a = 0; a < MT; ++a)
#pragma unroll
                for (int b = 0; b < NBW; ++b) acc[a][b] += red[w][a][b][lane];
    }
    // D layout: lane holds rows 4*(lane>>4)+i, column lane&15
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
            const int64_t n = (nb0 + b) * 16 + col_in;
            if (nb0 + b >= NBT) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t m = 16 * a + 4 * kq + i;
                if (m < M) y[m * N + n] = f32_to_f16_sat(acc[a][b][i]);
            }
        }
}

template <int MT, int NBW, int KSPLIT, int KPW, bool INT4, bool HAS_OFF>
static void launch_aq2(uint16_t* y, const uint16_t* x, const void* wp, const uint16_t* scale, const uint16_t* offset,
                       int64_t g, int64_t M, int64_t N, int64_t K, hipStream_t st)
{
    const unsigned blocks = (unsigned)((N / 16 + NBW - 1) / NBW);
    if (g % KT == 0)
        hipLaunchKernelGGL((antiquant_gemm_kernel<MT, NBW, KSPLIT, KPW, INT4, HAS_OFF, true>), dim3(blocks),
                           dim3(KSPLIT * 64), 0, st, y, x, (const uint8_t*)wp, scale, offset, M, N, K, g);
    else
        hipLaunchKernelGGL((antiquant_gemm_kernel<MT, NBW, KSPLIT, KPW, INT4, HAS_OFF, false>), dim3(blocks),
                           dim3(KSPLIT * 64), 0, st, y, x, (const uint8_t*)wp, scale, offset, M, N, K, g);
}

template <int MT, int NBW, int KSPLIT, int KPW>
static void launch_aq(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                      const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, hipStream_t st)
{
    if (int4) {
        if (offset) launch_aq2<MT, NBW, KSPLIT, KPW, true, true>(y, x, wp, scale, offset, g, M, N, K, st);
        else launch_aq2<MT, NBW, KSPLIT, KPW, true, false>(y, x, wp, scale, offset, g, M, N, K, st);
    } else {
        if (offset) launch_aq2<MT, NBW, KSPLIT, KPW, false, true>(y, x, wp, scale, offset, g, M, N, K, st);
        else launch_aq2<MT, NBW, KSPLIT, KPW, false, false>(y, x, wp, scale, offset, g, M, N, K, st);
    }
}

// M is processed in chunks of 64 rows (4 m tiles); decode shapes are a single launch.
hipError_t launch_antiquant_matmul(uint16_t* y, const uint16_t* x, const void* wp, int w_type, const uint16_t* scale,
                                   const uint16_t* offset, int64_t group, int64_t M, int64_t N, int64_t K,
                                   hipStream_t st)
{
    const int64_t g = group > 0 ? group : K;
    const bool int4 = w_type == DT_INT4;
    for (int64_t m0 = 0; m0 < M; m0 += 64) {
        const int64_t mc = (M - m0) < 64 ? (M - m0) : 64;
        const uint16_t* xc = x + m0 * K;
        uint16_t* yc = y + m0 * N;
        if (mc <= 16) launch_aq<1, 1, 4, 8>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        else if (mc <= 32) launch_aq<2, 2, 4, 4>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        else launch_aq<4, 2, 4, 4>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ascq
