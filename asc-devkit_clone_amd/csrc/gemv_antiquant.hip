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

// 0x64006400 (two binary16 1024.0) held in a VGPR: with both masks as literals the compiler cannot fuse the
// and / or of the int4 unpacking into one v_and_or_b32 (a VOP3 instruction takes no literal operand here)
__device__ __forceinline__ uint32_t half_magic_vgpr()
{
    uint32_t m;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(m));
    return m;
}

// dequantise one 8-element B fragment: codes -> half(half(q + off) * scale)
template <bool INT4, bool HAS_OFF>
__device__ __forceinline__ h8 dequant8(uint32_t w0, uint32_t w1, h2 off, h2 sc, uint32_t magic)
{
    uint32_t d[4];
    if constexpr (INT4) {
        // w0 holds all 8 nibbles of the step; pair i = (w0 >> 4i) & 0x000F000F
#pragma unroll
        for (int i = 0; i < 4; ++i) d[i] = ((w0 >> (4 * i)) & 0x000F000Fu) | magic;
    } else {
        // bytes b0..b3 of w0 and w1 -> halves 0x64bb (selector 5 = byte 1 of magic = 0x64)
        d[0] = __builtin_amdgcn_perm(magic, w0, 0x05010500u);
        d[1] = __builtin_amdgcn_perm(magic, w0, 0x05030502u);
        d[2] = __builtin_amdgcn_perm(magic, w1, 0x05010500u);
        d[3] = __builtin_amdgcn_perm(magic, w1, 0x05030502u);
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

typedef __amdgpu_buffer_rsrc_t aq_rsrc_t;
constexpr uint32_t AQ_OOB = 0x80000000u;  // out-of-range buffer offset: the load returns zeros

__device__ __forceinline__ aq_rsrc_t aq_rsrc(const void* base, uint64_t bytes)
{
    const uint32_t n = bytes >= 0x7FFFFFFFull ? 0x7FFFFFFFu : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)n, 0x00020000);
}

// One workgroup = KSPLIT waves over the same NBW 16-column strips; wave w takes the k tiles
// (r * KSPLIT + w) * TPW + i of round r.  In a round a wave first issues every load it needs -- TPW x NBW
// weight tiles, their scale / offset values, and its activation fragments -- as buffer loads (out-of-range
// offsets read zeros: tiles past K multiply zero activations), then dequantises and multiplies.  Partial 16x16
// tiles of the KSPLIT waves are summed through LDS in a fixed order.  MT = number of 16-row m tiles.
// XLDS (decode batches, M <= 4, MT = 1): the activations x[0:M, 0:K] are staged in LDS once per workgroup
// (loads issued before the weights, so their latency hides under the weight stream) and the MFMA A fragments
// are read from there; rows m >= M read a zeroed 16-byte slot.  This keeps the kernel under 64 VGPRs, so every
// workgroup of a decode launch is resident at once and the weight stream overlaps the dequantisation.
template <int MT, int NBW, int KSPLIT, int TPW, bool INT4, bool HAS_OFF, bool G128, bool XLDS>
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
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // XLDS: x[M][K] halves, then 16 zero bytes
    static_assert(!XLDS || MT == 1, "LDS activations are for one m tile");

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t KB = K / KT;
    const int64_t nb0 = (int64_t)blockIdx.x * NBW;
    const int64_t NBT = N / 16;
    const int col_in = lane & 15, kq = lane >> 4;
    const aq_rsrc_t rw = aq_rsrc(wp, (uint64_t)K * N / (INT4 ? 2 : 1));
    const aq_rsrc_t rx = aq_rsrc(x, (uint64_t)M * K * 2);
    const aq_rsrc_t rs = aq_rsrc(scale, (uint64_t)((K + g - 1) / g) * N * 2);
    const aq_rsrc_t ro = aq_rsrc(HAS_OFF ? offset : scale, (uint64_t)((K + g - 1) / g) * N * 2);

    v4f acc[MT][NBW];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NBW; ++b) acc[a][b] = (v4f){0.f, 0.f, 0.f, 0.f};
    const uint32_t magic = half_magic_vgpr();

    // XLDS: stage x (M * K * 2 bytes, a multiple of 256) -- these loads are the first this wave issues
    constexpr int XL = 4;  // 16-byte chunks per thread per pass
    u32x4 xv[XLDS ? XL : 1];
    const int64_t xchunks = XLDS ? M * K * 2 / 16 : 0;
    const int64_t xpasses = (xchunks + (int64_t)KSPLIT * 64 * XL - 1) / ((int64_t)KSPLIT * 64 * XL);
    auto stage_x = [&](int64_t pass) {
#pragma unroll
        for (int u = 0; u < XL; ++u) {
            const int64_t c = (pass * XL + u) * KSPLIT * 64 + threadIdx.x;
            xv[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, c < xchunks ? (uint32_t)(c * 16) : AQ_OOB, 0, 0);
        }
    };
    auto store_x = [&](int64_t pass) {
#pragma unroll
        for (int u = 0; u < XL; ++u) {
            const int64_t c = (pass * XL + u) * KSPLIT * 64 + threadIdx.x;
            if (c < xchunks) *(u32x4*)(xs + c * 16) = xv[u];
        }
    };
    if constexpr (XLDS) {
        if (threadIdx.x == 0) *(u32x4*)(xs + xchunks * 16) = (u32x4){0u, 0u, 0u, 0u};
        for (int64_t ps = 0; ps + 1 < xpasses; ++ps) {  // shapes beyond one pass (large K) stage serially
            stage_x(ps);
            store_x(ps);
        }
        stage_x(xpasses - 1);  // the last pass stays in flight under the first round's weight loads
    }
    bool x_ready = !XLDS;

    const int64_t rounds = (KB + KSPLIT * TPW - 1) / (KSPLIT * TPW);
    for (int64_t r = 0; r < rounds; ++r) {
        const int64_t t0 = (r * KSPLIT + wave) * TPW;  // first k tile of this wave in this round
        u32x4 wv[TPW][NBW][WV];
        uint32_t sc[G128 ? TPW : 1][NBW], of[G128 ? TPW : 1][NBW];
        h8 xa[XLDS ? 1 : TPW][MT][4];
        // issue order = use order (activations, scales, weights of tile 0, then tile 1, ...): loads retire in
        // order, so tile i can start as soon as its own data has landed while later tiles are still in flight
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int64_t kb = t0 + i;
            if constexpr (!XLDS) {
#pragma unroll
                for (int a = 0; a < MT; ++a) {
                    const int64_t m = 16 * a + col_in;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t xo =
                            (m < M && kb < KB) ? (uint32_t)((m * K + kb * KT + 32 * j + 8 * kq) * 2) : AQ_OOB;
                        xa[i][a][j] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0));
                    }
                }
            }
#pragma unroll
            for (int b = 0; b < NBW; ++b) {
                const int64_t nb = nb0 + b;
                const bool ok = kb < KB && nb < NBT;
                if constexpr (G128) {
                    const uint32_t so = ok ? (uint32_t)((((kb * KT) / g) * N + nb * 16 + col_in) * 2) : AQ_OOB;
                    sc[i][b] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0);
                    of[i][b] = HAS_OFF ? __builtin_amdgcn_raw_buffer_load_b16(ro, so, 0, 0) : 0u;
                }
                const uint32_t off = ok ? (uint32_t)((nb * KB + kb) * TILE_BYTES + lane * LANE_BYTES) : AQ_OOB;
#pragma unroll
                for (int v = 0; v < WV; ++v) wv[i][b][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16 * v, 0, 0);
            }
        }
        // every load of the round is in flight before the first dequantisation (the scheduler would otherwise
        // sink loads next to their MFMAs and pay a memory latency per k tile)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (XLDS) {
            if (!x_ready) {  // first round: the staged x lands (it was issued before any weight), then publish it
                store_x(xpasses - 1);
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_s_barrier();
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                x_ready = true;
            }
        }
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int64_t kb = t0 + i;
            if constexpr (XLDS) {
                const bool xok = col_in < M && kb < KB;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t xo = xok ? (col_in * K + kb * KT + 32 * j + 8 * kq) * 2 : xchunks * 16;
                    xa[0][0][j] = *(const h8*)(xs + xo);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int b = 0; b < NBW; ++b) {
                    h2 s2, o2;
                    if constexpr (G128) {
                        const _Float16 sv = bits_h((uint16_t)sc[i][b]), ov = bits_h((uint16_t)of[i][b]);
                        s2 = (h2){sv, sv};
                        o2 = (h2){ov, ov};
                    } else {
                        const int64_t nb = nb0 + b;
                        const bool ok = kb < KB && nb < NBT;
                        const uint32_t so =
                            ok ? (uint32_t)((((kb * KT + 32 * j + 8 * kq) / g) * N + nb * 16 + col_in) * 2) : AQ_OOB;
                        const _Float16 sv = bits_h((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0));
                        const _Float16 ov =
                            HAS_OFF ? bits_h((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(ro, so, 0, 0)) : (_Float16)0.0f;
                        s2 = (h2){sv, sv};
                        o2 = (h2){ov, ov};
                    }
                    uint32_t w0, w1 = 0;
                    if constexpr (INT4) {
                        w0 = wv[i][b][0][j];
                    } else {
                        w0 = wv[i][b][j >> 1][(j & 1) * 2];
                        w1 = wv[i][b][j >> 1][(j & 1) * 2 + 1];
                    }
                    const h8 bf = dequant8<INT4, HAS_OFF>(w0, w1, o2, s2, magic);
#pragma unroll
                    for (int a = 0; a < MT; ++a)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[XLDS ? 0 : i][a][j], bf, acc[a][b], 0, 0, 0);
                }
            }
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

template <int MT, int NBW, int KSPLIT, int TPW, bool INT4, bool HAS_OFF, bool XLDS>
static void launch_aq2(uint16_t* y, const uint16_t* x, const void* wp, const uint16_t* scale, const uint16_t* offset,
                       int64_t g, int64_t M, int64_t N, int64_t K, hipStream_t st)
{
    const unsigned blocks = (unsigned)((N / 16 + NBW - 1) / NBW);
    const size_t lds = XLDS ? (size_t)(M * K * 2 + 16) : 0;
    if (g % KT == 0)
        launch_k((antiquant_gemm_kernel<MT, NBW, KSPLIT, TPW, INT4, HAS_OFF, true, XLDS>), dim3(blocks),
                           dim3(KSPLIT * 64), lds, st, y, x, (const uint8_t*)wp, scale, offset, M, N, K, g);
    else
        launch_k((antiquant_gemm_kernel<MT, NBW, KSPLIT, TPW, INT4, HAS_OFF, false, XLDS>), dim3(blocks),
                           dim3(KSPLIT * 64), lds, st, y, x, (const uint8_t*)wp, scale, offset, M, N, K, g);
}

template <int MT, int NBW, int KSPLIT, int TPW, bool XLDS = false>
static void launch_aq(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                      const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, hipStream_t st)
{
    if (int4) {
        if (offset) launch_aq2<MT, NBW, KSPLIT, TPW, true, true, XLDS>(y, x, wp, scale, offset, g, M, N, K, st);
        else launch_aq2<MT, NBW, KSPLIT, TPW, true, false, XLDS>(y, x, wp, scale, offset, g, M, N, K, st);
    } else {
        if (offset) launch_aq2<MT, NBW, KSPLIT, TPW, false, true, XLDS>(y, x, wp, scale, offset, g, M, N, K, st);
        else launch_aq2<MT, NBW, KSPLIT, TPW, false, false, XLDS>(y, x, wp, scale, offset, g, M, N, K, st);
    }
}

// M is processed in chunks of 64 rows (4 m tiles); decode shapes are a single launch.  The packed weight,
// x and the scales must each stay below 2^31 bytes (buffer offsets; checked by the caller).
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
        // decode batches: int4 stages x in LDS (4 waves x 8 k tiles measured fastest at K = 4096); int8
        // streams twice the bytes per element and does better with 8 waves x 4 tiles and x in registers
        if (int4 && mc <= 4 && mc * K * 2 + 16 <= 48 * 1024)
            launch_aq<1, 1, 4, 8, true>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        else if (mc <= 16) launch_aq<1, 1, 8, 4>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        else if (mc <= 32) launch_aq<2, 2, 8, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        else launch_aq<4, 2, 8, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, st);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ascq
