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
//    so (word >> 4i) & 0x000F000F yields the pair (2i, 2i+1) as two half lanes (dequant8 masks the odd pairs in
//    place instead and divides by 16 exactly);
//    int8: the 8 codes of step j are bytes 0..7 of an 8-byte chunk, in k order.
//
// Roofline: at decode shapes the kernel streams the packed weight once (K*N/2 or K*N bytes) plus the
// scales/offsets; it is HBM-bound at M = 1 and 16 and near the fp16 MFMA ridge at M = 64.
#include <algorithm>
#include <type_traits>

#include "aq_frag.h"
#include "common.h"
#include "launch.h"

namespace ascq {

// one f16 output element: a store, or IterateAll's enAtomic combine
__device__ __forceinline__ void y_put(uint16_t* p, uint16_t v, int atomic)
{
    if (atomic == C_STORE) *p = v;
    else c_atomic<DT_F16>((uint8_t*)p, v, atomic);
}

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

// s_waitcnt vmcnt(N) with the other counters left alone (vmcnt[3:0] | expcnt << 4 | lgkmcnt << 8 | vmcnt[5:4] << 14)
template <int N>
__device__ __forceinline__ void wait_vmcnt_aq()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
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
// are read from there; rows m >= M read a zeroed 16-byte slot.  This takes the four 16-byte activation loads per
// tile off the vector memory path, which then carries little more than the weight stream.
template <int MT, int NBW, int KSPLIT, int TPW, bool INT4, bool HAS_OFF, bool G128, bool XLDS>
__global__ __launch_bounds__(KSPLIT * 64) void antiquant_gemm_kernel(uint16_t* __restrict__ y,
                                                                     const uint16_t* __restrict__ x,
                                                                     const uint8_t* __restrict__ wp,
                                                                     const uint16_t* __restrict__ scale,
                                                                     const uint16_t* __restrict__ offset,
                                                                     int64_t M, int64_t N, int64_t K, int64_t g,
                                                                     int atomic)
{
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048;
    constexpr int LANE_BYTES = INT4 ? 16 : 32;
    constexpr int WV = INT4 ? 1 : 2;
    __shared__ v4f red[KSPLIT > 1 ? KSPLIT - 1 : 1][MT][NBW][64];
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];  // XLDS: x[M][K] halves, then 16 zero bytes
    static_assert(!XLDS || MT == 1, "LDS activations are for one m tile");
    constexpr bool GSC = G128 && TPW % 4 == 0;

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
        // GSC: the scale / offset rows of 4 consecutive tiles come in one 2-byte load each (lane (kq, c) fetches
        // tile t0 + 4 h + kq, column c) and are handed to the lanes that need them with ds_bpermute, instead of
        // two loads per tile -- measured ~1.3 us faster at M = 1, K = 4096, N = 11008
        uint32_t scl[GSC ? TPW / 4 : 1][NBW], ofl[GSC ? TPW / 4 : 1][NBW];
        if constexpr (GSC) {
#pragma unroll
            for (int h = 0; h < TPW / 4; ++h)
#pragma unroll
                for (int b = 0; b < NBW; ++b) {
                    const int64_t kb = t0 + 4 * h + kq;
                    const bool ok = kb < KB && nb0 + b < NBT;
                    const uint32_t so =
                        ok ? (uint32_t)((((kb * KT) / g) * N + (nb0 + b) * 16 + col_in) * 2) : AQ_OOB;
                    scl[h][b] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0);
                    ofl[h][b] = HAS_OFF ? __builtin_amdgcn_raw_buffer_load_b16(ro, so, 0, 0) : 0u;
                }
        }
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
                if constexpr (G128 && !GSC) {
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
                        uint32_t sci, ofi;
                        if constexpr (GSC) {
                            const uint32_t pk = scl[i >> 2][b] | (ofl[i >> 2][b] << 16);
                            const uint32_t v =
                                (uint32_t)__builtin_amdgcn_ds_bpermute(((i & 3) * 16 + col_in) * 4, (int)pk);
                            sci = v & 0xFFFFu;
                            ofi = v >> 16;
                        } else {
                            sci = sc[i][b];
                            ofi = of[i][b];
                        }
                        const _Float16 sv = bits_h((uint16_t)sci), ov = bits_h((uint16_t)ofi);
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
                if (m < M) y_put(y + m * N + n, f32_to_f16_sat(acc[a][b][i]), atomic);
            }
        }
}

// Small-batch form (4 < M <= 64, group size a multiple of 128).  The activation tile x[0:16 MT, k0:k0 + 128 KSW]
// of each round is copied global -> LDS by buffer loads with an LDS destination (no registers) into a ring of ST
// stages, ST - 1 rounds ahead, and shared by all waves of the workgroup; wave (s, kw) owns 16-column strip s of the
// workgroup's NS strips and k tile (round * KSW + kw), whose weight tile (with its scale / offset) is loaded into a
// register ring DW - 1 rounds ahead (DW a multiple of ST: the weights may run further ahead than the activations, so
// that enough bytes are in flight).  Every wave issues the same number of memory operations per round, so one
// s_waitcnt vmcnt with a constant threshold plus one barrier per round make a stage visible and free the stage read
// in the previous round.  Each 16-byte chunk c of row r is stored at chunk c ^ (r % 16) of its LDS
// row (the swizzle is applied to the global address of the copy), so the 16 rows of an MFMA fragment read hit 16
// distinct bank groups.  The KSW partial 16x16 tiles of a strip are summed through LDS in a fixed order.
template <int MT, int NS, int KSW, int ST, bool INT4, bool HAS_OFF, int DW = ST>
struct AqDma {
    static constexpr int NW = NS * KSW, NT = NW * 64;
    static constexpr int ROWS = 16 * MT;
    static constexpr int ROWB = KSW * KT * 2;           // LDS bytes per staged row (one round)
    static constexpr int CH = ROWB / 16;                 // 16-byte chunks per row
    static constexpr int SLOT = ROWS * ROWB;             // one stage
    static constexpr int CPW = 4 * MT / NS;              // 1 KiB copies per wave per round
    static constexpr int WV = INT4 ? 1 : 2;              // 16-byte weight loads per lane per tile
    static constexpr int WL = WV + (HAS_OFF ? 2 : 1);    // vmem operations per wave per round besides the copies
    // at the top of round r, the copies of round r (issued in round r - ST + 1) must have landed; with DW > ST the
    // weights of round r were issued before them, with DW == ST right after them in the same round
    static constexpr int IN_FLIGHT = (DW > ST ? WL : 0) + (ST - 2) * (CPW + WL);
    static constexpr int RED = (KSW - 1) * NS * MT * 64 * 16;
    static constexpr int LDS = ST * SLOT > RED ? ST * SLOT : RED;
    static_assert((4 * MT) % NS == 0 && CPW >= 1, "copies split evenly over the waves");
    static_assert(CH >= 16 && (CH & (CH - 1)) == 0, "swizzle needs 16+ chunks per row, a power of two");
    static_assert(ST >= 3 && IN_FLIGHT < 64 && LDS <= 160 * 1024 && DW % ST == 0, "stages");
};

template <int MT, int NS, int KSW, int ST, bool INT4, bool HAS_OFF, bool ROT = false, int DW = ST>
__global__ __launch_bounds__(NS * KSW * 64) void aq_dma_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ x,
                                                               const uint8_t* __restrict__ wp,
                                                               const uint16_t* __restrict__ scale,
                                                               const uint16_t* __restrict__ offset, int64_t M,
                                                               int64_t N, int64_t K, int64_t g, int64_t ldx,
                                                               int atomic)
{
    using P = AqDma<MT, NS, KSW, ST, INT4, HAS_OFF, DW>;
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048;
    constexpr int LANE_BYTES = INT4 ? 16 : 32;
    __shared__ __attribute__((aligned(16))) uint8_t smem[P::LDS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = wave / KSW, kw = wave % KSW;
    const int64_t KB = K / KT, NBT = N / 16;
    const int64_t nb = (int64_t)blockIdx.x * NS + s;
    const int col_in = lane & 15, kq = lane >> 4;
    const aq_rsrc_t rw = aq_rsrc(wp, (uint64_t)K * N / (INT4 ? 2 : 1));
    const aq_rsrc_t rx = aq_rsrc(x, (uint64_t)((M - 1) * ldx + K) * 2);
    const aq_rsrc_t rs = aq_rsrc(scale, (uint64_t)((K + g - 1) / g) * N * 2);
    const aq_rsrc_t ro = aq_rsrc(HAS_OFF ? offset : scale, (uint64_t)((K + g - 1) / g) * N * 2);
    const uint32_t magic = half_magic_vgpr();
    const int64_t rounds = (KB + KSW - 1) / KSW;
    const int64_t rot = ROT ? (int64_t)((blockIdx.x * 5u) % (uint32_t)rounds) : 0;
    // round r reads k block (r + rot) mod rounds; rounds past the end read zeros
    auto phys = [&](int64_t r) -> int64_t {
        if (r >= rounds) return KB;  // past every k block
        const int64_t q = r + rot;
        return q >= rounds ? q - rounds : q;
    };

    v4f acc[MT];
#pragma unroll
    for (int a = 0; a < MT; ++a) acc[a] = (v4f){0.f, 0.f, 0.f, 0.f};

    // x copies of round r into stage `slot`: copy j of this wave covers chunks 64 (wave CPW + j) .. + 63
    auto issue_x = [&](int64_t r, int slot) {
#pragma unroll
        for (int j = 0; j < P::CPW; ++j) {
            const int gcopy = wave * P::CPW + j;
            const int q = gcopy * 64 + lane;
            const int row = q / P::CH, p = q % P::CH;
            const int c = p ^ (row & 15);  // logical chunk held at physical chunk p
            const int64_t k = phys(r) * KSW * KT + c * 8;
            const uint32_t off = (row < M && k < K) ? (uint32_t)((row * ldx + k) * 2) : AQ_OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void*)(smem + slot * P::SLOT + gcopy * 1024),
                                                     16, off, 0, 0, 0);
        }
    };
    struct WTile {
        u32x4 w[P::WV];
        uint32_t sc, of;
    };
    auto load_w = [&](int64_t r, WTile& t) {
        const int64_t kb = phys(r) * KSW + kw;
        const bool ok = kb < KB && nb < NBT;
        const uint32_t off = ok ? (uint32_t)((nb * KB + kb) * TILE_BYTES + lane * LANE_BYTES) : AQ_OOB;
#pragma unroll
        for (int v = 0; v < P::WV; ++v) t.w[v] = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16 * v, 0, 0);
        const uint32_t so = ok ? (uint32_t)((((kb * KT) / g) * N + nb * 16 + col_in) * 2) : AQ_OOB;
        t.sc = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0);
        if constexpr (HAS_OFF) t.of = __builtin_amdgcn_raw_buffer_load_b16(ro, so, 0, 0);
        else t.of = 0u;
    };
    auto compute = [&](int slot, const WTile& t) {
        const uint8_t* xb = smem + slot * P::SLOT;
        const _Float16 sv = bits_h((uint16_t)t.sc), ov = bits_h((uint16_t)t.of);
        const h2 s2 = (h2){sv, sv}, o2 = (h2){ov, ov};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w0, w1 = 0;
            if constexpr (INT4) {
                w0 = t.w[0][j];
            } else {
                w0 = t.w[j >> 1][(j & 1) * 2];
                w1 = t.w[j >> 1][(j & 1) * 2 + 1];
            }
            const h8 bf = dequant8<INT4, HAS_OFF>(w0, w1, o2, s2, magic);
            const int c = kw * 16 + 4 * j + kq;  // logical chunk of this lane's 8 k values
#pragma unroll
            for (int a = 0; a < MT; ++a) {
                const int row = 16 * a + col_in;
                const h8 xa = *(const h8*)(xb + row * P::ROWB + (c ^ (row & 15)) * 16);
                acc[a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, bf, acc[a], 0, 0, 0);
            }
        }
    };

    WTile wt[DW];
    // prologue: the DW - 1 rounds before round 0 as the loop would have issued them (activations of rounds
    // 0 .. ST - 2, weights of rounds 0 .. DW - 2)
#pragma unroll
    for (int q = 0; q < DW - 1; ++q) {
        if (q >= DW - ST) issue_x(q - DW + ST, q - DW + ST);
        load_w(q, wt[q]);
    }
    // round r: its stage has landed (this wave's copies: vmcnt; everyone's: the barrier, which also frees the
    // stage read in round r - 1), then round r + ST - 1 is issued into that freed stage and the weights of round
    // r + DW - 1 into the weight slot freed by round r - 1, then round r computes
    for (int64_t r0 = 0; r0 < rounds; r0 += DW) {
#pragma unroll
        for (int u = 0; u < DW; ++u) {
            const int64_t r = r0 + u;
            if (r < rounds) {
                __builtin_amdgcn_sched_barrier(0);
                wait_vmcnt_aq<P::IN_FLIGHT>();
                __builtin_amdgcn_sched_barrier(0);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_s_barrier();
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_sched_barrier(0);
                // the next round's operations are always issued (out-of-range ones read zeros), so every wave
                // keeps the same number in flight and the vmcnt threshold stays exact
                issue_x(r + ST - 1, (u + ST - 1) % ST);
                load_w(r + DW - 1, wt[(u + DW - 1) % DW]);
                __builtin_amdgcn_sched_barrier(0);
                compute(u % ST, wt[u]);
            }
        }
    }
    wait_vmcnt_aq<0>();  // no copy may still target LDS when it is reused below or the wave ends
    __syncthreads();

    if constexpr (KSW > 1) {
        v4f* red = (v4f*)smem;  // [KSW - 1][NS][MT][64]
        if (kw > 0) {
#pragma unroll
            for (int a = 0; a < MT; ++a) red[(((kw - 1) * NS + s) * MT + a) * 64 + lane] = acc[a];
        }
        __syncthreads();
        if (kw != 0) return;
#pragma unroll
        for (int w = 0; w < KSW - 1; ++w)
#pragma unroll
            for (int a = 0; a < MT; ++a) acc[a] += red[((w * NS + s) * MT + a) * 64 + lane];
    }
    if (nb >= NBT) return;
    const int64_t n = nb * 16 + col_in;
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t m = 16 * a + 4 * kq + i;
            if (m < M) y_put(y + m * N + n, f32_to_f16_sat(acc[a][i]), atomic);
        }
}

template <int MT, int NBW, int KSPLIT, int TPW, bool INT4, bool HAS_OFF, bool XLDS>
static void launch_aq2(uint16_t* y, const uint16_t* x, const void* wp, const uint16_t* scale, const uint16_t* offset,
                       int64_t g, int64_t M, int64_t N, int64_t K, int atomic, hipStream_t st)
{
    const unsigned blocks = (unsigned)((N / 16 + NBW - 1) / NBW);
    const size_t lds = XLDS ? (size_t)(M * K * 2 + 16) : 0;
    if (g % KT == 0)
        launch_k((antiquant_gemm_kernel<MT, NBW, KSPLIT, TPW, INT4, HAS_OFF, true, XLDS>), dim3(blocks),
                           dim3(KSPLIT * 64), lds, st, y, x, (const uint8_t*)wp, scale, offset, M, N, K, g, atomic);
    else
        launch_k((antiquant_gemm_kernel<MT, NBW, KSPLIT, TPW, INT4, HAS_OFF, false, XLDS>), dim3(blocks),
                           dim3(KSPLIT * 64), lds, st, y, x, (const uint8_t*)wp, scale, offset, M, N, K, g, atomic);
}

template <int MT, int NBW, int KSPLIT, int TPW, bool XLDS = false>
static void launch_aq(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                      const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int atomic, hipStream_t st)
{
    if (int4) {
        if (offset) launch_aq2<MT, NBW, KSPLIT, TPW, true, true, XLDS>(y, x, wp, scale, offset, g, M, N, K, atomic, st);
        else launch_aq2<MT, NBW, KSPLIT, TPW, true, false, XLDS>(y, x, wp, scale, offset, g, M, N, K, atomic, st);
    } else {
        if (offset) launch_aq2<MT, NBW, KSPLIT, TPW, false, true, XLDS>(y, x, wp, scale, offset, g, M, N, K, atomic, st);
        else launch_aq2<MT, NBW, KSPLIT, TPW, false, false, XLDS>(y, x, wp, scale, offset, g, M, N, K, atomic, st);
    }
}

// Column-block form for small batches (M <= 16, group size 128 << s).  The grid is C column blocks; block c covers
// the 16-column strips [c sq + min(c, sr), ...) -- sq or sq + 1 of them, so any C balances.  The workgroup first
// copies x[0:M, 0:K] into LDS once (16-byte chunk c of row r at chunk c ^ (r % 16) of its LDS row, so the 16 rows of
// an MFMA fragment read hit 16 distinct bank groups; fragment rows m >= M read a zeroed row), as buffer loads with an
// LDS destination and the uniform part of every address in the scalar offset.  Wave (sg, kw) of the SG x KW waves
// owns strips sg NBW .. sg NBW + NBW - 1 of the block and the T = KB / KW k tiles kw, kw + KW, ... (T a multiple of
// D); it copies the
// scale / offset rows of its tiles over its strips into its own LDS area, and its weight tiles stream through a
// register ring: D tiles are in flight, and tile i + D is issued as soon as tile i has been multiplied (tiles past
// the end read zeros, so the count in flight stays constant and one s_waitcnt threshold serves every step).  Each
// activation fragment is read from LDS once for the wave's NBW strips; every LDS address is a per-lane base plus a
// uniform offset.  The KW partial 16 x 16 tiles of a strip are summed through LDS in kw order by the wave kw = 0,
// which writes y.
template <int NBW, int SG, int KW, int D>
struct AqXs {
    static constexpr int NW = SG * KW, NT = NW * 64;
    static constexpr int SMAX = SG * NBW;                 // strips per block at most
    static constexpr int WPT = NBW * 8;                   // 4-byte words of scale row per tile and wave
    static constexpr int TPC = 64 / WPT;                  // tiles per 256-byte scale copy
    static constexpr int RED = (KW - 1) * SG * NBW * 1024;  // k-wave partial tiles
    static_assert(TPC >= 1, "scale row of a tile within one copy");
};

// kernel arguments of aq_xs_kernel / aq_ring_kernel, all index arithmetic in 32 bits (the host checks every byte
// size < 2^31)
struct AqXsArgs {
    uint16_t* y;
    const uint16_t* x;
    const uint8_t* wp;
    const uint16_t* scale;
    const uint16_t* offset;
    uint32_t M, N, K, KB;
    uint32_t sq, sr;  // block c has sq + (c < sr) strips, starting at strip c sq + min(c, sr)
    uint32_t gshift;  // group size = 128 << gshift; 31: one group over all of K (aq_kw_kernel also takes 32 and 64:
                      // gshift 0, its SPG says which)
    uint32_t x_bytes, w_bytes, s_bytes;
    int atomic;
};

template <int NBW, int SG, int KW, int D, bool INT4, bool HAS_OFF>
__global__ __launch_bounds__(SG * KW * 64) void aq_xs_kernel(AqXsArgs A)
{
    using P = AqXs<NBW, SG, KW, D>;
    constexpr int NW = P::NW, NT = P::NT, WPT = P::WPT, TPC = P::TPC;
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048;
    constexpr int LANE_BYTES = INT4 ? 16 : 32;
    constexpr int WV = INT4 ? 1 : 2;
    constexpr int TOPS = NBW * WV;  // vector memory operations per ring tile
    static_assert(D * TOPS < 64, "vmcnt range");
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    typedef __attribute__((address_space(3))) void* lds_ptr;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sg = wave / KW, kw = wave % KW;
    const uint32_t col_in = lane & 15, kq = lane >> 4;
    const uint32_t cb = blockIdx.x;
    const uint32_t M = A.M, N = A.N, KB = A.KB;
    const uint32_t T = KB / KW;  // k tiles per wave (KB % KW == 0)
    const uint32_t s0 = cb * A.sq + (cb < A.sr ? cb : A.sr), s1 = s0 + A.sq + (cb < A.sr ? 1u : 0u);
    const uint32_t sb = s0 + (uint32_t)(sg * NBW);  // first strip of this wave
    const uint32_t RL = KB * 256;                   // LDS activation row bytes
    const uint32_t ncp = (T + TPC - 1) / TPC, wsb = ncp * 256;
    // LDS: M activation rows | zero row | scale rows of each wave [ncp][256 B] | offset rows of each wave
    const uint32_t zrow_at = M * RL, sc_at = zrow_at + RL, of_at = sc_at + NW * wsb;
    const aq_rsrc_t rw = aq_rsrc(A.wp, A.w_bytes);
    const aq_rsrc_t rx = aq_rsrc(A.x, A.x_bytes);
    const aq_rsrc_t rs = aq_rsrc(A.scale, A.s_bytes);
    const aq_rsrc_t ro = aq_rsrc(HAS_OFF ? A.offset : A.scale, A.s_bytes);
    const uint32_t magic = half_magic_vgpr();

    // activation rows: 1 KiB block pb of row r (4 k tiles) lands at r RL + 1024 pb; lane l fills physical chunk
    // 64 pb + l, which holds logical chunk 64 pb + (l ^ r % 16)
    {
        const uint32_t bpr = KB / 4;
        for (uint32_t b = (uint32_t)wave; b < M * bpr; b += NW) {
            const uint32_t r = b / bpr, pb = b - r * bpr;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(xs + r * RL + pb * 1024), 16, (lane ^ (r & 15u)) * 16,
                                                     (int)(r * A.K * 2 + pb * 1024), 0, 0);
        }
    }
    for (uint32_t c = threadIdx.x; c < RL / 16; c += NT) *(u32x4*)(xs + zrow_at + c * 16) = (u32x4){0u, 0u, 0u, 0u};
    // this wave's scale / offset rows, NBW * 16 halves per tile: copy c holds tiles c TPC .. c TPC + TPC - 1, lane l
    // word l % WPT of tile c TPC + l / WPT (lanes past TPC WPT and columns past the block read zeros)
    for (uint32_t c = 0; c < ncp; ++c) {
        const uint32_t i = c * TPC + (uint32_t)lane / WPT, wd = (uint32_t)lane % WPT;
        const uint32_t kt = (uint32_t)kw + i * KW;
        const bool ok = (uint32_t)lane < TPC * WPT && i < T && 2 * wd < (s1 > sb ? (s1 - sb) * 16 : 0u);
        const uint32_t voff = ok ? ((kt >> A.gshift) * N * 2 + wd * 4) : AQ_OOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(xs + sc_at + wave * wsb + c * 256), 4, voff, (int)(sb * 32), 0, 0);
        if constexpr (HAS_OFF)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ro, (lds_ptr)(xs + of_at + wave * wsb + c * 256), 4, voff, (int)(sb * 32), 0, 0);
    }

    // per-lane LDS bases: fragment j of tile i at xa_at[j] + i KW 256, with
    // (4 j + kq) ^ col_in = ((4 j) ^ (col_in & 12)) | (kq ^ (col_in & 3)); the scale of (i, strip b) at
    // s_at + (i / TPC) 256 + (i % TPC) WPT 4 + 32 b
    const uint32_t xo0 = ((col_in & 12u) | (kq ^ (col_in & 3u))) * 16;
    uint32_t xa_at[4];
    {
        const uint32_t rb = (col_in < M ? col_in * RL : zrow_at) + (uint32_t)kw * 256;
#pragma unroll
        for (int j = 0; j < 4; ++j) xa_at[j] = rb + (xo0 ^ (64u * j));
    }
    const uint32_t s_at = (uint32_t)wave * wsb + col_in * 2;
    const int nvalid = (int)s1 - (int)sb < NBW ? (int)s1 - (int)sb : NBW;  // strips of this wave in the block

    v4f acc[NBW];
#pragma unroll
    for (int b = 0; b < NBW; ++b) acc[b] = (v4f){0.f, 0.f, 0.f, 0.f};
    // the pipeline for NV = nvalid strips (a compile-time count, so the loop body has no per-strip branch and the
    // memory-operation counts behind every s_waitcnt are exact)
    auto pipeline = [&](auto nv_tag) {
        constexpr int NV = decltype(nv_tag)::value;
        constexpr int TOPS = NV * WV;  // vector memory operations per ring tile
        static_assert(D * TOPS < 64, "vmcnt range");
        // ring tile i: weight tile kw + i KW of the NV strips; tiles past T read zeros
        u32x4 wv[D][NV > 0 ? NV : 1][WV];
        auto load_t = [&](uint32_t i, int slot) {
            const uint32_t kt = (uint32_t)kw + i * KW;
#pragma unroll
            for (int b = 0; b < NV; ++b) {
                const uint32_t off = i < T ? lane * LANE_BYTES : AQ_OOB;
                const int soff = i < T ? (int)(((sb + b) * KB + kt) * TILE_BYTES) : 0;
#pragma unroll
                for (int v = 0; v < WV; ++v)
                    wv[slot][b][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16 * v, soff, 0);
            }
        };
#pragma unroll
        for (int i = 0; i < D; ++i) load_t((uint32_t)i, i);
        // this wave's copies are older than its ring loads: they have landed once at most D TOPS remain
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt_aq<D * TOPS>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the zero row is written
        __builtin_amdgcn_sched_barrier(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NV > 0) {
            for (uint32_t i0 = 0; i0 < T; i0 += D) {
#pragma unroll
                for (int u = 0; u < D; ++u) {
                    const uint32_t i = i0 + u;
                    // tile i has landed once only the D - 1 tiles issued after it are in flight
                    __builtin_amdgcn_sched_barrier(0);
                    wait_vmcnt_aq<(D - 1) * TOPS>();
                    __builtin_amdgcn_sched_barrier(0);
                    const uint32_t so = s_at + (i / TPC) * 256 + (i % TPC) * WPT * 4;
                    const uint32_t xi = i * KW * 256;
                    h2 s2[NV], o2[NV];
#pragma unroll
                    for (int b = 0; b < NV; ++b) {
                        const _Float16 sv = *(const _Float16*)(xs + sc_at + so + 32 * b);
                        const _Float16 ov = HAS_OFF ? *(const _Float16*)(xs + of_at + so + 32 * b) : (_Float16)0.0f;
                        s2[b] = (h2){sv, sv};
                        o2[b] = (h2){ov, ov};
                    }
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const h8 xa = *(const h8*)(xs + xa_at[j] + xi);
#pragma unroll
                        for (int b = 0; b < NV; ++b) {
                            uint32_t w0, w1 = 0;
                            if constexpr (INT4) {
                                w0 = wv[u][b][0][j];
                            } else {
                                w0 = wv[u][b][j >> 1][(j & 1) * 2];
                                w1 = wv[u][b][j >> 1][(j & 1) * 2 + 1];
                            }
                            const h8 bf = dequant8<INT4, HAS_OFF>(w0, w1, o2[b], s2[b], magic);
                            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, bf, acc[b], 0, 0, 0);
                        }
                    }
                    // the slot of tile i is free again: tile i + D goes into it (past T: zeros, same count)
                    __builtin_amdgcn_sched_barrier(0);
                    load_t(i + D, u);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        wait_vmcnt_aq<0>();
    };
    // a wave holds NBW strips of its block, fewer in the block's last strip group
    static_assert(NBW >= 1 && NBW <= 4, "strips per wave");
    if (nvalid >= NBW) pipeline(std::integral_constant<int, NBW>{});
    else if (NBW > 1 && nvalid == 1) pipeline(std::integral_constant<int, 1>{});
    else if (NBW > 2 && nvalid == 2) pipeline(std::integral_constant<int, (NBW > 2 ? 2 : 1)>{});
    else if (NBW > 3 && nvalid == 3) pipeline(std::integral_constant<int, (NBW > 3 ? 3 : 1)>{});
    else pipeline(std::integral_constant<int, 0>{});

    // KW partial tiles -> wave kw = 0 of each strip group, summed in kw order (the shared rows are dead)
    __syncthreads();
    if constexpr (KW > 1) {
        v4f* red = (v4f*)xs;  // [KW - 1][SG][NBW][64]
        if (kw > 0) {
#pragma unroll
            for (int b = 0; b < NBW; ++b) red[(((kw - 1) * SG + sg) * NBW + b) * 64 + lane] = acc[b];
        }
        __syncthreads();
        if (kw != 0) return;
#pragma unroll
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
            for (int b = 0; b < NBW; ++b) acc[b] += red[((w * SG + sg) * NBW + b) * 64 + lane];
    }
    // D layout: lane holds rows 4 kq + i, column col_in of each 16 x 16 tile
#pragma unroll
    for (int b = 0; b < NBW; ++b) {
        if (b >= nvalid) break;
        uint16_t* yc = A.y + (sb + b) * 16 + col_in;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = 4 * kq + i;
            if (m < M) y_put(yc + (uint64_t)m * N, f32_to_f16_sat(acc[b][i]), A.atomic);
        }
    }
}

// LDS bytes of aq_xs_kernel (0 when the shape does not fit)
template <int NBW, int SG, int KW, int D>
inline int64_t aq_xs_lds(int64_t M, int64_t K, bool has_off)
{
    using P = AqXs<NBW, SG, KW, D>;
    const int64_t KB = K / KT, T = KB / KW, ncp = (T + P::TPC - 1) / P::TPC;
    const int64_t lds = std::max<int64_t>((M + 1) * KB * 256 + (int64_t)P::NW * ncp * 256 * (has_off ? 2 : 1), P::RED);
    return lds <= 160 * 1024 ? lds : 0;
}

// the weight, x and scale buffers of the column-block kernels, each below 2^31 - 2^16 bytes: their 32-bit buffer
// offsets, with bit 31 set for an out-of-range load and a step or immediate of under 2^16 added, never wrap
inline bool aq_cols_fit(int64_t M, int64_t N, int64_t K, int64_t g, bool int4)
{
    const uint64_t w_bytes = (uint64_t)K * N / (int4 ? 2 : 1), s_bytes = (uint64_t)((K + g - 1) / g) * N * 2;
    const uint64_t x_bytes = (uint64_t)M * K * 2, lim = 0x7FFF0000ull;
    return M >= 1 && w_bytes < lim && s_bytes < lim && x_bytes < lim && (uint64_t)N < lim;
}

// checks of the column-block and ring kernels common to both; fills the 32-bit argument block
inline bool aq_cols_args(AqXsArgs& A, uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                         const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int C, int smax, int atomic,
                         bool small_groups = false)
{
    const int64_t NBT = N / 16, KB = K / KT;
    const uint64_t w_bytes = (uint64_t)K * N / (int4 ? 2 : 1), s_bytes = (uint64_t)((K + g - 1) / g) * N * 2;
    const uint64_t x_bytes = (uint64_t)M * K * 2;
    // groups of 128 << s, one group over all of K (per channel), or (the K-split kernel) 32 / 64
    const bool g_ok = (g % KT == 0 && ((g / KT) & (g / KT - 1)) == 0) || (g >= K && K % KT == 0) ||
                      (small_groups && (g == 32 || g == 64));
    if (C < 1 || C > NBT || (NBT + C - 1) / C > smax || !g_ok || !aq_cols_fit(M, N, K, g, int4)) return false;
    A.y = y;
    A.x = x;
    A.wp = (const uint8_t*)wp;
    A.scale = scale;
    A.offset = offset;
    A.M = (uint32_t)M;
    A.N = (uint32_t)N;
    A.K = (uint32_t)K;
    A.KB = (uint32_t)KB;
    A.sq = (uint32_t)(NBT / C);
    A.sr = (uint32_t)(NBT % C);
    A.gshift = g >= K ? 31u : g >= KT ? (uint32_t)__builtin_ctzll((unsigned long long)(g / KT)) : 0u;
    A.x_bytes = (uint32_t)x_bytes;
    A.w_bytes = (uint32_t)w_bytes;
    A.s_bytes = (uint32_t)s_bytes;
    A.atomic = atomic;
    return true;
}

template <int NBW, int SG, int KW, int D>
static hipError_t launch_aq_xs(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                               const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int C, int atomic,
                               hipStream_t st)
{
    using P = AqXs<NBW, SG, KW, D>;
    AqXsArgs A;
    const int64_t lds = aq_xs_lds<NBW, SG, KW, D>(M, K, offset != nullptr);
    if (M > 16 || (K / KT) % 4 != 0 || (K / KT) % (KW * D) != 0 || lds == 0 ||
        !aq_cols_args(A, y, x, wp, int4, scale, offset, g, M, N, K, C, P::SMAX, atomic))
        return hipErrorInvalidValue;
#define AQ_XS_LAUNCH(I4, OF)                                                 \
    do {                                                                     \
        constexpr auto kern = aq_xs_kernel<NBW, SG, KW, D, I4, OF>;           \
        hipError_t e = ensure_dynamic_lds<kern>((int)lds);                   \
        if (e != hipSuccess) return e;                                       \
        launch_k(kern, dim3((unsigned)C), dim3(P::NT), (uint32_t)lds, st, A); \
    } while (0)
    if (int4) {
        if (offset) AQ_XS_LAUNCH(true, true);
        else AQ_XS_LAUNCH(true, false);
    } else {
        if (offset) AQ_XS_LAUNCH(false, true);
        else AQ_XS_LAUNCH(false, false);
    }
#undef AQ_XS_LAUNCH
    return hipGetLastError();
}

// Batch form (M > 16, group size 128 << s): the column blocks of aq_xs_kernel, with the activations streamed; the
// grid's y dimension walks row blocks of 16 MT rows (one for a decode batch).  Block c covers the strips
// [c sq + min(c, sr), ...); wave (sg, kw) of the SG x KW waves owns strips
// sg NBW .. sg NBW + NBW - 1 of the block and, in round r, k tile r KW + kw.  The activation tile x[r0:r0 + 16 MT,
// 128 KW r .. 128 KW (r + 1)) of each round (r0 the row block's first row) is copied into an LDS ring of ST stages
// (buffer loads with an LDS destination, 16-byte chunk c of row r at chunk c ^ (r % 16); rows m >= M read zeros),
// ST - 1 rounds ahead, and
// shared by all waves; every wave reads each activation fragment once for its NBW strips, which is what keeps the
// LDS read traffic of a 64-row batch within bounds.  Weight tiles stream through a register ring DW - 1 rounds
// ahead (DW a multiple of ST); the scale / offset rows of a wave's tiles are copied into LDS once, at the start.
// Every wave issues the same number of memory operations per round, so one s_waitcnt vmcnt with a constant threshold
// plus one barrier per round make a stage visible and free the stage read in the previous round.  The KW partial
// tiles of a strip are summed through LDS in kw order by the wave kw = 0, which writes y.
template <int MT, int NBW, int SG, int KW, int ST, int DW, bool INT4, bool HAS_OFF>
struct AqRing {
    static constexpr int NW = SG * KW, NT = NW * 64;
    static constexpr int ROWS = 16 * MT;
    static constexpr int ROWB = KW * KT * 2;   // LDS bytes per staged row (one round)
    static constexpr int CH = ROWB / 16;        // 16-byte chunks per row
    static constexpr int SLOT = ROWS * ROWB;    // one stage
    static constexpr int CPW = 4 * MT * KW / NW;  // 1 KiB copies per wave per round
    static constexpr int WV = INT4 ? 1 : 2;
    static constexpr int WL = NBW * WV;          // weight loads per wave per round
    static constexpr int IN_FLIGHT = (DW > ST ? WL : 0) + (ST - 2) * (CPW + WL);
    static constexpr int WPT = NBW * 8;          // 4-byte words of scale row per tile and wave
    static constexpr int TPC = 64 / WPT;         // tiles per 256-byte scale copy
    static constexpr int RED = (KW - 1) * SG * MT * NBW * 1024;
    static_assert((4 * MT * KW) % NW == 0 && CPW >= 1, "copies split evenly over the waves");
    static_assert(CH >= 16 && (CH & (CH - 1)) == 0, "swizzle needs 16+ chunks per row, a power of two");
    static_assert(ST >= 2 && DW % ST == 0 && DW > ST - 1 && IN_FLIGHT < 64 && TPC >= 1, "stages");
};

template <int MT, int NBW, int SG, int KW, int ST, int DW, bool INT4, bool HAS_OFF>
__global__ __launch_bounds__(SG * KW * 64) void aq_ring_kernel(AqXsArgs A)
{
    using P = AqRing<MT, NBW, SG, KW, ST, DW, INT4, HAS_OFF>;
    constexpr int NW = P::NW, TPC = P::TPC, WPT = P::WPT;
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048;
    constexpr int LANE_BYTES = INT4 ? 16 : 32;
    constexpr int WV = P::WV;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    typedef __attribute__((address_space(3))) void* lds_ptr;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sg = wave / KW, kw = wave % KW;
    const uint32_t col_in = lane & 15, kq = lane >> 4;
    const uint32_t cb = blockIdx.x;
    const uint32_t M = A.M, N = A.N, KB = A.KB;
    const uint32_t row0 = blockIdx.y * (uint32_t)P::ROWS;  // this block's first row (row blocks of 16 MT rows)
    const uint32_t s0 = cb * A.sq + (cb < A.sr ? cb : A.sr), s1 = s0 + A.sq + (cb < A.sr ? 1u : 0u);
    const uint32_t sb = s0 + (uint32_t)(sg * NBW);  // first strip of this wave
    // rounds of KW k tiles; when KW does not divide KB the last round is partial: its tiles past KB read zeros
    // (weights, activations and scale / offset alike, so they add exact zeros)
    const uint32_t rounds = (KB + KW - 1) / KW;
    const uint32_t ncp = (rounds + TPC - 1) / TPC;  // scale copies per wave
    // LDS: ST activation stages | scale rows of each wave [ncp][256 B] | offset rows of each wave
    const uint32_t sc_at = ST * P::SLOT, wsb = ncp * 256;
    const uint32_t of_at = sc_at + NW * wsb;
    const aq_rsrc_t rw = aq_rsrc(A.wp, A.w_bytes);
    const aq_rsrc_t rx = aq_rsrc(A.x, A.x_bytes);
    const aq_rsrc_t rs = aq_rsrc(A.scale, A.s_bytes);
    const aq_rsrc_t ro = aq_rsrc(HAS_OFF ? A.offset : A.scale, A.s_bytes);
    const uint32_t magic = half_magic_vgpr();

    // this wave's scale / offset rows, NBW * 16 halves per round: copy c holds rounds c TPC .. c TPC + TPC - 1
    for (uint32_t c = 0; c < ncp; ++c) {
        const uint32_t i = c * TPC + (uint32_t)lane / WPT, wd = (uint32_t)lane % WPT;
        const uint32_t kt = i * KW + (uint32_t)kw;
        const bool ok = (uint32_t)lane < TPC * WPT && i < rounds && kt < KB && 2 * wd < (s1 > sb ? (s1 - sb) * 16 : 0u);
        const uint32_t voff = ok ? ((kt >> A.gshift) * N * 2 + wd * 4) : AQ_OOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(smem + sc_at + wave * wsb + c * 256), 4, voff, (int)(sb * 32), 0, 0);
        if constexpr (HAS_OFF)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ro, (lds_ptr)(smem + of_at + wave * wsb + c * 256), 4, voff, (int)(sb * 32), 0, 0);
    }

    // activation copies of round r into stage `slot`: copy j of this wave covers chunks 64 (wave CPW + j) .. + 63
    auto issue_x = [&](uint32_t r, int slot) {
#pragma unroll
        for (int j = 0; j < P::CPW; ++j) {
            const uint32_t gcopy = (uint32_t)(wave * P::CPW + j);
            const uint32_t q = gcopy * 64 + lane;
            const uint32_t row = q / P::CH, p = q % P::CH;
            const uint32_t c = p ^ (row & 15u);  // logical chunk held at physical chunk p
            const uint32_t k = r * KW * KT + c * 8;
            const uint32_t off = row0 + row < M && r < rounds && k < A.K ? ((row0 + row) * A.K + k) * 2 : AQ_OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr)(smem + slot * P::SLOT + gcopy * 1024), 16, off, 0, 0, 0);
        }
    };
    struct WTile {
        u32x4 w[NBW][WV];
    };
    auto load_w = [&](uint32_t r, WTile& t) {
        const uint32_t kt = r * KW + (uint32_t)kw;
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
            const uint32_t s = sb + b;
            const uint32_t off = r < rounds && kt < KB && s < s1 ? (s * KB + kt) * TILE_BYTES + lane * LANE_BYTES : AQ_OOB;
#pragma unroll
            for (int v = 0; v < WV; ++v) t.w[b][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16 * v, 0, 0);
        }
    };
    // per-lane LDS bases: fragment (a, j) of this wave's tile in a stage at xa_at[a][j], with
    // (4 j + kq) ^ col_in = ((4 j) ^ (col_in & 12)) | (kq ^ (col_in & 3)) within the wave's 256-byte k tile
    const uint32_t xo0 = ((col_in & 12u) | (kq ^ (col_in & 3u))) * 16;
    uint32_t xa_at[MT][4];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) xa_at[a][j] = (16 * a + col_in) * P::ROWB + (uint32_t)kw * 256 + (xo0 ^ (64u * j));
    const uint32_t s_at = (uint32_t)wave * wsb + col_in * 2;
    const int nvalid = (int)s1 - (int)sb < NBW ? (int)s1 - (int)sb : NBW;  // strips of this wave in the block

    v4f acc[MT][NBW];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NBW; ++b) acc[a][b] = (v4f){0.f, 0.f, 0.f, 0.f};
    auto compute = [&](uint32_t r, int slot, const WTile& t) {
        const uint8_t* xb = smem + slot * P::SLOT;
        h2 s2[NBW], o2[NBW];
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
            const uint32_t so = s_at + (r / TPC) * 256 + (r % TPC) * WPT * 4 + 32 * b;
            const _Float16 sv = *(const _Float16*)(smem + sc_at + so);
            const _Float16 ov = HAS_OFF ? *(const _Float16*)(smem + of_at + so) : (_Float16)0.0f;
            s2[b] = (h2){sv, sv};
            o2[b] = (h2){ov, ov};
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            h8 xa[MT];
#pragma unroll
            for (int a = 0; a < MT; ++a) xa[a] = *(const h8*)(xb + xa_at[a][j]);
#pragma unroll
            for (int b = 0; b < NBW; ++b) {
                if (b >= nvalid) break;
                uint32_t w0, w1 = 0;
                if constexpr (INT4) {
                    w0 = t.w[b][0][j];
                } else {
                    w0 = t.w[b][j >> 1][(j & 1) * 2];
                    w1 = t.w[b][j >> 1][(j & 1) * 2 + 1];
                }
                const h8 bf = dequant8<INT4, HAS_OFF>(w0, w1, o2[b], s2[b], magic);
#pragma unroll
                for (int a = 0; a < MT; ++a)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[a], bf, acc[a][b], 0, 0, 0);
            }
        }
    };

    WTile wt[DW];
    // prologue: the DW - 1 rounds before round 0 as the loop would have issued them (activations of rounds
    // 0 .. ST - 2, weights of rounds 0 .. DW - 2)
#pragma unroll
    for (int q = 0; q < DW - 1; ++q) {
        if (q >= DW - ST) issue_x((uint32_t)(q - DW + ST), q - DW + ST);
        load_w((uint32_t)q, wt[q]);
    }
    // round r: its stage has landed (this wave's copies: vmcnt; everyone's: the barrier, which also frees the stage
    // read in round r - 1), then round r + ST - 1 is issued into that freed stage and the weights of round r + DW - 1
    // into the slot freed by round r - 1; out-of-range rounds read zeros, so the counts stay exact
    for (uint32_t r0 = 0; r0 < rounds; r0 += DW) {
#pragma unroll
        for (int u = 0; u < DW; ++u) {
            const uint32_t r = r0 + u;
            if (r < rounds) {
                __builtin_amdgcn_sched_barrier(0);
                wait_vmcnt_aq<P::IN_FLIGHT>();
                __builtin_amdgcn_sched_barrier(0);
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_s_barrier();
                __atomic_signal_fence(__ATOMIC_SEQ_CST);
                __builtin_amdgcn_sched_barrier(0);
                issue_x(r + ST - 1, (u + ST - 1) % ST);
                load_w(r + DW - 1, wt[(u + DW - 1) % DW]);
                __builtin_amdgcn_sched_barrier(0);
                compute(r, u % ST, wt[u]);
            }
        }
    }
    wait_vmcnt_aq<0>();  // no copy may still target LDS when it is reused below or the wave ends
    __syncthreads();

    if constexpr (KW > 1) {
        v4f* red = (v4f*)smem;  // [KW - 1][SG][MT][NBW][64]
        if (kw > 0) {
#pragma unroll
            for (int a = 0; a < MT; ++a)
#pragma unroll
                for (int b = 0; b < NBW; ++b) red[((((kw - 1) * SG + sg) * MT + a) * NBW + b) * 64 + lane] = acc[a][b];
        }
        __syncthreads();
        if (kw != 0) return;
#pragma unroll
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
            for (int a = 0; a < MT; ++a)
#pragma unroll
                for (int b = 0; b < NBW; ++b) acc[a][b] += red[(((w * SG + sg) * MT + a) * NBW + b) * 64 + lane];
    }
    // D layout: lane holds rows 4 kq + i, column col_in of each 16 x 16 tile
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NBW; ++b) {
            if (b >= nvalid) break;
            uint16_t* yc = A.y + (sb + b) * 16 + col_in;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = row0 + 16 * a + 4 * kq + i;
                if (m < M) y_put(yc + (uint64_t)m * N, f32_to_f16_sat(acc[a][b][i]), A.atomic);
            }
        }
}

// LDS bytes of aq_ring_kernel (0 when the shape does not fit)
template <int MT, int NBW, int SG, int KW, int ST, int DW>
inline int64_t aq_ring_lds(int64_t K, bool has_off)
{
    using P = AqRing<MT, NBW, SG, KW, ST, DW, true, true>;
    const int64_t rounds = (K / KT + KW - 1) / KW, ncp = (rounds + P::TPC - 1) / P::TPC;
    const int64_t lds = std::max<int64_t>((int64_t)ST * P::SLOT + (int64_t)P::NW * ncp * 256 * (has_off ? 2 : 1), P::RED);
    return lds <= 160 * 1024 ? lds : 0;
}

template <int MT, int NBW, int SG, int KW, int ST, int DW>
static hipError_t launch_aq_ring(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                                 const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int C, int atomic,
                                 hipStream_t st)
{
    using P4 = AqRing<MT, NBW, SG, KW, ST, DW, true, true>;
    AqXsArgs A;
    const int64_t lds = aq_ring_lds<MT, NBW, SG, KW, ST, DW>(K, offset != nullptr);
    if (K % KT != 0 || lds == 0 || !aq_cols_args(A, y, x, wp, int4, scale, offset, g, M, N, K, C, SG * NBW, atomic))
        return hipErrorInvalidValue;
    const unsigned RB = (unsigned)((M + 16 * MT - 1) / (16 * MT));  // row blocks (grid.y)
#define AQ_RING_LAUNCH(I4, OF)                                                     \
    do {                                                                           \
        constexpr auto kern = aq_ring_kernel<MT, NBW, SG, KW, ST, DW, I4, OF>;      \
        hipError_t e = ensure_dynamic_lds<kern>((int)lds);                         \
        if (e != hipSuccess) return e;                                             \
        launch_k(kern, dim3((unsigned)C, RB), dim3(P4::NT), (uint32_t)lds, st, A);  \
    } while (0)
    if (int4) {
        if (offset) AQ_RING_LAUNCH(true, true);
        else AQ_RING_LAUNCH(true, false);
    } else {
        if (offset) AQ_RING_LAUNCH(false, true);
        else AQ_RING_LAUNCH(false, false);
    }
#undef AQ_RING_LAUNCH
    return hipGetLastError();
}

// K-split column-block form for batches M <= 16 MT (group size 128 << s).  The grid is C <= 256 column blocks, one per
// CU; block c covers the strips [c sq + min(c, sr), ...), sq or sq + 1 <= NS of them.  Its KW waves split the k
// tiles -- wave kw takes tiles [kw KB / KW, (kw + 1) KB / KW) -- so every CU reads only its own strips of the weight
// and each wave its own k range of x.  Nothing in the main loop is shared, so it has no LDS and no barrier: a wave
// streams its weight tiles, its activation fragments and its tiles' scale / offset values straight into a
// register ring of D tiles (tiles past the end read zeros and multiply zeros, so every step issues the same loads
// and the compiler's counted waits keep D - 1 tiles in flight), dequantises each weight fragment once and multiplies
// it against all MT row tiles.  The NS strips of a short block (sq < NS) read zeros and are not stored.  At the end
// the waves park their partial tiles in LDS row-major and every thread sums a pair of outputs over the KW waves in kw
// order (deterministic), rounds once to half and stores it.
template <int MT, int NS, int KW>
struct AqKw {
    static constexpr int NT = KW * 64;
    static constexpr int ROW = NS * 16;                 // floats per partial row
    static constexpr int LDS = KW * MT * 16 * ROW * 4;  // partial tiles of all waves
    static_assert(LDS <= 160 * 1024, "partials fit in LDS");
};

// SPG: scale / offset groups per k tile of 128 -- 1 for groups of 128 << s, 2 for 64, 4 for 32 (a lane's eight k
// values of MFMA step j lie in group 4 kb / SPG ... of its tile: step j takes group j * SPG / 4 of the tile's SPG)
template <int MT, int NS, int KW, int D, bool INT4, bool HAS_OFF, int SPG = 1>
__global__ __launch_bounds__(KW * 64) void aq_kw_kernel(AqXsArgs A)
{
    using P = AqKw<MT, NS, KW>;
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048;
    constexpr int LANE_BYTES = INT4 ? 16 : 32;
    constexpr int WV = INT4 ? 1 : 2;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int lane = threadIdx.x & 63;
    const uint32_t kw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t col_in = lane & 15, kq = lane >> 4;
    const uint32_t cb = blockIdx.x;
    const uint32_t M = A.M, N = A.N, K = A.K, KB = A.KB;
    const uint32_t s0 = cb * A.sq + (cb < A.sr ? cb : A.sr), ns = A.sq + (cb < A.sr ? 1u : 0u);
    const uint32_t t0 = kw * KB / KW, T = (kw + 1) * KB / KW - t0;  // this wave's k tiles
    const aq_rsrc_t rw = aq_rsrc(A.wp, A.w_bytes);
    const aq_rsrc_t rx = aq_rsrc(A.x, A.x_bytes);
    const aq_rsrc_t rs = aq_rsrc(A.scale, A.s_bytes);
    const aq_rsrc_t ro = aq_rsrc(HAS_OFF ? A.offset : A.scale, A.s_bytes);
    const uint32_t magic = half_magic_vgpr();

    struct Tile {
        u32x4 w[NS][WV];
        u32x4 x[MT][4];
        uint32_t sc[NS][SPG], of[NS][SPG];  // 16-bit values, held in 32 bits (16-bit fields of a ring slot went to scratch)
    };
    // Lane (kq, col_in) reads the B fragment of column col_in of each strip, the A fragments of rows 16 a + col_in
    // (k 32 j + 8 kq .. + 7 of the tile) and the scale / offset of its column.  The per-lane base offsets of tile 0
    // are fixed here, out of range for the strips past the block and the rows past M; in the loop tile t only adds
    // its uniform step and, past this wave's tiles, sets bit 31 (an out-of-range offset: the loads return zeros).
    // Every condition stays out of the loop, so the compiler has no branch to duplicate loads into.  The host keeps
    // every buffer below 2^31 - 2^16 bytes, so no offset plus its step or immediate wraps past 2^32.
    uint32_t wb[NS], sbo[NS], xb[MT];
#pragma unroll
    for (int b = 0; b < NS; ++b) {
        wb[b] = (uint32_t)b < ns ? ((s0 + b) * KB + t0) * TILE_BYTES + lane * LANE_BYTES : AQ_OOB;
        sbo[b] = (uint32_t)b < ns ? ((s0 + b) * 16 + col_in) * 2 : AQ_OOB;
    }
#pragma unroll
    for (int a = 0; a < MT; ++a) {
        const uint32_t row = 16 * a + col_in;
        xb[a] = row < M ? (row * K + t0 * KT + 8 * kq) * 2 : AQ_OOB;
    }
    const uint32_t n2 = N * 2;
    auto issue = [&](uint32_t t, Tile& r) {
        const uint32_t past = (T - 1 - t) & 0x80000000u;  // t >= T (both below 2^31)
        const uint32_t sg = (SPG == 1 ? (t0 + t) >> A.gshift : (t0 + t) * SPG) * n2;
#pragma unroll
        for (int b = 0; b < NS; ++b) {
            const uint32_t off = (wb[b] + t * TILE_BYTES) | past;
#pragma unroll
            for (int v = 0; v < WV; ++v) r.w[b][v] = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16 * v, 0, 0);
        }
#pragma unroll
        for (int a = 0; a < MT; ++a) {
            const uint32_t off = (xb[a] + t * (KT * 2)) | past;
#pragma unroll
            for (int j = 0; j < 4; ++j) r.x[a][j] = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 64 * j, 0, 0);
        }
#pragma unroll
        for (int b = 0; b < NS; ++b)
#pragma unroll
            for (int q = 0; q < SPG; ++q) {
                const uint32_t off = (sbo[b] + sg + q * n2) | past;
                r.sc[b][q] = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
                if constexpr (HAS_OFF) r.of[b][q] = __builtin_amdgcn_raw_buffer_load_b16(ro, off, 0, 0);
            }
    };

    v4f acc[MT][NS];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NS; ++b) acc[a][b] = (v4f){0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const Tile& r) {
        h2 s2[NS][SPG], o2[NS][SPG];
#pragma unroll
        for (int b = 0; b < NS; ++b)
#pragma unroll
            for (int q = 0; q < SPG; ++q) {
                const _Float16 sv = __builtin_bit_cast(_Float16, (uint16_t)r.sc[b][q]);
                const _Float16 ov = HAS_OFF ? __builtin_bit_cast(_Float16, (uint16_t)r.of[b][q]) : (_Float16)0.0f;
                s2[b][q] = (h2){sv, sv};
                o2[b][q] = (h2){ov, ov};
            }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int b = 0; b < NS; ++b) {
                constexpr int JPG = 4 / SPG;  // MFMA steps per group
                uint32_t w0, w1 = 0;
                if constexpr (INT4) {
                    w0 = r.w[b][0][j];
                } else {
                    w0 = r.w[b][j >> 1][(j & 1) * 2];
                    w1 = r.w[b][j >> 1][(j & 1) * 2 + 1];
                }
                const h8 bf = dequant8<INT4, HAS_OFF>(w0, w1, o2[b][j / JPG], s2[b][j / JPG], magic);
#pragma unroll
                for (int a = 0; a < MT; ++a)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, r.x[a][j]), bf, acc[a][b],
                                                                       0, 0, 0);
            }
    };

    Tile ring[D];
#pragma unroll
    for (int q = 0; q < D - 1; ++q) {
        issue((uint32_t)q, ring[q]);
        __builtin_amdgcn_sched_barrier(0);  // tiles in order, so each wait below leaves the later ones in flight
    }
    // step t issues tile t + D - 1 into the slot step t - 1 consumed, then multiplies tile t; the steps are rounded up
    // to a multiple of D (tiles past T read and multiply zeros).  The scheduling barrier keeps each step's loads
    // ahead of its arithmetic (left alone, the scheduler sinks them below it and the ring runs a tile short).
    for (uint32_t r0 = 0; r0 < T; r0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            issue(r0 + u + D - 1, ring[(u + D - 1) % D]);
            __builtin_amdgcn_sched_barrier(0);
            compute(ring[u]);
        }
    }

    // partial tiles row-major in LDS: wave kw's value of output (row, col) at red[(kw * 16 MT + row) * ROW + col]
    float* red = (float*)smem;
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int b = 0; b < NS; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                red[(kw * 16 * MT + 16 * a + 4 * kq + i) * P::ROW + 16 * b + col_in] = acc[a][b][i];
    __syncthreads();
    constexpr int PAIRS = MT * 16 * NS * 8;
    for (int p = threadIdx.x; p < PAIRS; p += P::NT) {
        const uint32_t row = (uint32_t)p / (NS * 8), c = 2 * ((uint32_t)p % (NS * 8));
        if (row >= M || c / 16 >= ns) continue;
        f2x s = *(const f2x*)(red + row * P::ROW + c);
#pragma unroll
        for (int w = 1; w < KW; ++w) s += *(const f2x*)(red + (w * 16 * MT + row) * P::ROW + c);
        uint16_t* yp = A.y + (uint64_t)row * N + s0 * 16 + c;
        y_put(yp, f32_to_f16_sat(s.x), A.atomic);
        y_put(yp + 1, f32_to_f16_sat(s.y), A.atomic);
    }
}

template <int MT, int NS, int KW, int D, int SPG>
static hipError_t launch_aq_kw(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                               const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int C, int atomic,
                               hipStream_t st)
{
    using P = AqKw<MT, NS, KW>;
    AqXsArgs A;
    if (M > 16 * MT || (SPG == 1 ? g < KT : g != KT / SPG) ||
        !aq_cols_args(A, y, x, wp, int4, scale, offset, g, M, N, K, C, NS, atomic, SPG > 1))
        return hipErrorInvalidValue;
#define AQ_KW_LAUNCH(I4, OF)                                                    \
    do {                                                                        \
        constexpr auto kern = aq_kw_kernel<MT, NS, KW, D, I4, OF, SPG>;          \
        hipError_t e = ensure_dynamic_lds<kern>(P::LDS);                        \
        if (e != hipSuccess) return e;                                          \
        launch_k(kern, dim3((unsigned)C), dim3(P::NT), (uint32_t)P::LDS, st, A); \
    } while (0)
    if (int4) {
        if (offset) AQ_KW_LAUNCH(true, true);
        else AQ_KW_LAUNCH(true, false);
    } else {
        if (offset) AQ_KW_LAUNCH(false, true);
        else AQ_KW_LAUNCH(false, false);
    }
#undef AQ_KW_LAUNCH
    return hipGetLastError();
}

// column blocks for a grid of about `target` workgroups whose blocks hold at most smax strips
inline int aq_blocks(int64_t NBT, int smax, int target)
{
    int64_t C = NBT < target ? NBT : target;
    if ((NBT + C - 1) / C > smax) C = (NBT + smax - 1) / smax;
    return (int)C;
}

// aq_kw_kernel for M <= 32 over C = aq_blocks(strips, 4, 256) blocks: strips per block NS = ceil(strips / C) <= 4, row tiles
// MT = 1 or 2.  Four waves (one per SIMD) with two tiles in flight each: against 8 or 16 waves and rings of 1 - 4
// tiles this measured fastest at K = 4096, N = 11008 for every M in {1, 8, 16, 24, 32}, int4 and int8 (graph
// replays; e.g. int4 7.9 / 8.7 / 12.2 us at M = 1 / 16 / 32, where 8 waves with 4 tiles in flight took 9.4 / 10.7 /
// 16.2 us).  Above 32 rows every CU reading all of x costs more than the LDS ring of aq_ring_kernel, which
// shares each activation copy between two strip groups; those batches stay there.
static hipError_t launch_aq_kw_any(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                                   const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int atomic,
                                   hipStream_t st)
{
    const int64_t NBT = N / 16;
    // about 256 blocks; above 1024 strips, blocks of 4 strips (more than one block per CU)
    const int C = aq_blocks(NBT, 4, 256);
    const int64_t ns = (NBT + C - 1) / C;
#define AQ_KW_NS(MT, SPG)                                                                                  \
    switch (ns) {                                                                                           \
    case 1: return launch_aq_kw<MT, 1, 4, 2, SPG>(y, x, wp, int4, scale, offset, g, M, N, K, C, atomic, st); \
    case 2: return launch_aq_kw<MT, 2, 4, 2, SPG>(y, x, wp, int4, scale, offset, g, M, N, K, C, atomic, st); \
    case 3: return launch_aq_kw<MT, 3, 4, 2, SPG>(y, x, wp, int4, scale, offset, g, M, N, K, C, atomic, st); \
    case 4: return launch_aq_kw<MT, 4, 4, 2, SPG>(y, x, wp, int4, scale, offset, g, M, N, K, C, atomic, st); \
    default: return hipErrorInvalidValue;                                                                 \
    }
#define AQ_KW_MT(SPG)                                  \
    do {                                               \
        if (M <= 16) { AQ_KW_NS(1, SPG) }                  \
        if (M <= 32) { AQ_KW_NS(2, SPG) }                  \
        if (M <= 64) { AQ_KW_NS(4, SPG) }                  \
        return hipErrorInvalidValue;                   \
    } while (0)
    // groups of 32 / 64 take 4 / 2 scale and offset rows per k tile of 128; batches up to 64 rows where the LDS ring
    // (which holds every scale row of K in LDS) does not fit: groups this small, or a long K
    if (g == 32) AQ_KW_MT(4);
    if (g == 64) AQ_KW_MT(2);
    AQ_KW_MT(1);
#undef AQ_KW_MT
#undef AQ_KW_NS
}

template <int MT, int NS, int KSW, int ST, bool ROT, int DW = ST>
static void launch_dma(uint16_t* y, const uint16_t* x, const void* wp, bool int4, const uint16_t* scale,
                       const uint16_t* offset, int64_t g, int64_t M, int64_t N, int64_t K, int atomic, hipStream_t st)
{
    const dim3 grid((unsigned)((N / 16 + NS - 1) / NS)), block(NS * KSW * 64);
    const uint8_t* w = (const uint8_t*)wp;
    if (int4) {
        if (offset) launch_k((aq_dma_kernel<MT, NS, KSW, ST, true, true, ROT, DW>), grid, block, 0, st, y, x, w, scale, offset, M, N, K, g, K, atomic);
        else launch_k((aq_dma_kernel<MT, NS, KSW, ST, true, false, ROT, DW>), grid, block, 0, st, y, x, w, scale, offset, M, N, K, g, K, atomic);
    } else {
        if (offset) launch_k((aq_dma_kernel<MT, NS, KSW, ST, false, true, ROT, DW>), grid, block, 0, st, y, x, w, scale, offset, M, N, K, g, K, atomic);
        else launch_k((aq_dma_kernel<MT, NS, KSW, ST, false, false, ROT, DW>), grid, block, 0, st, y, x, w, scale, offset, M, N, K, g, K, atomic);
    }
}


// M is processed in chunks of 64 rows (4 m tiles); decode shapes are a single launch.  The packed weight,
// x and the scales must each stay below 2^31 bytes (buffer offsets; checked by the caller).
hipError_t launch_antiquant_matmul(uint16_t* y, const uint16_t* x, const void* wp, int w_type, const uint16_t* scale,
                                   const uint16_t* offset, int64_t group, int64_t M, int64_t N, int64_t K,
                                   int atomic, hipStream_t st)
{
    const int64_t g = group > 0 ? group : K;
    const bool int4 = w_type == DT_INT4;
    const int64_t NBT = N / 16, KB = K / KT;
    // column-block kernels: groups of 128 << s, or one group over all of K (per channel)
    const bool cols_ok = K % KT == 0 && ((g % KT == 0 && ((g / KT) & (g / KT - 1)) == 0) || g >= K);
    // Above 64 rows: aq_ring_kernel over row blocks (grid.y) -- x shared through the LDS ring by the strip groups of a
    // block, each weight fragment dequantised once per block of rows and multiplied against all of them.  64-row
    // blocks of 6 strips (2 strip groups x 4 k-split waves) while they make about one block per CU, else 128-row blocks
    // of 12 strips (4 strip groups x 2 k-split waves).  Measured at K = 4096, N = 11008 (int4 / int8, M = 128 / 512 /
    // 2048): 27 / 63 / 239 us against 71 / 78 / 250 us for the LDS-staged MFMA GEMM of aq_gemm.hip, which takes the
    // shapes the ring does not (LDS too small for the scale rows), then 64-row passes of the kernels below.  When KW does
    // not divide the k tiles (K = 11008: 86 tiles) the ring's last round is partial.
    if (M > 64 && cols_ok) {
        const int64_t rb64 = (M + 63) / 64, rb128 = (M + 127) / 128;
        const int c64 = aq_blocks(NBT, 6, (int)((256 + rb64 - 1) / rb64));
        hipError_t e = hipErrorInvalidValue;
        if (c64 * rb64 <= 320 && aq_ring_lds<4, 3, 2, 4, 2, 2>(K, offset != nullptr))
            e = launch_aq_ring<4, 3, 2, 4, 2, 2>(y, x, wp, int4, scale, offset, g, M, N, K, c64, atomic, st);
        else if (aq_ring_lds<8, 3, 4, 2, 2, 2>(K, offset != nullptr))
            e = launch_aq_ring<8, 3, 4, 2, 2, 2>(y, x, wp, int4, scale, offset, g, M, N, K,
                                                 aq_blocks(NBT, 12, (int)((256 + rb128 - 1) / rb128)), atomic, st);
        // long K with a scale row per k tile (K = 11008, g = 128: 86 rows) leaves both forms above without LDS for
        // the scale rows; 64-row blocks of two k-split waves halve the activation stages
        else if (aq_ring_lds<4, 3, 2, 2, 2, 2>(K, offset != nullptr))
            e = launch_aq_ring<4, 3, 2, 2, 2, 2>(y, x, wp, int4, scale, offset, g, M, N, K, c64, atomic, st);
        if (e == hipErrorInvalidValue) {
            (void)hipGetLastError();
            e = launch_aq_gemm(y, x, wp, w_type, scale, offset, group, M, N, K, atomic, st);
        }
        if (e != hipErrorInvalidValue) return e;
        (void)hipGetLastError();
    }
    for (int64_t m0 = 0; m0 < M; m0 += 64) {
        const int64_t mc = (M - m0) < 64 ? (M - m0) : 64;
        const uint16_t* xc = x + m0 * K;
        uint16_t* yc = y + m0 * N;
        // Column-block kernels (about 256 workgroups of 1 - 4 strips; shapes measured at K = 4096, N = 11008):
        // M <= 32 with the K-split waves of aq_kw_kernel, larger batches with x streamed through an LDS ring.
        // Shapes they do not take (more than 1024 strips, buffers near 2^31 bytes) go to the earlier forms: x
        // resident in LDS for M <= 16, the LDS ring above, else the one-strip ring of aq_dma_kernel (group a
        // multiple of 128) or activations straight from memory.
        hipError_t e = hipErrorInvalidValue;
        // (past 1024 strips the K-split form runs several blocks per CU: measured at K = 4096, int4, N = 32000 /
        // 128256, M = 16 it takes 18.7 / 61.2 us against 21.4 / 77.7 us for the LDS-resident form below, while a
        // single row stays with that form, 52.2 against 53.8 us at N = 128256)
        if ((cols_ok || g == 32 || g == 64) && (mc <= 32 || !cols_ok) && (NBT <= 1024 || mc > 1 || !cols_ok) &&
            aq_cols_fit(mc, N, K, g, int4))
            e = launch_aq_kw_any(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
        else if (cols_ok && mc <= 16 && KB % 8 == 0 && aq_xs_lds<2, 2, 4, 2>(mc, K, offset != nullptr))
            e = launch_aq_xs<2, 2, 4, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, aq_blocks(NBT, 4, 256), atomic, st);
        else if (cols_ok && mc <= 16 && KB % 4 == 0 && aq_xs_lds<2, 2, 4, 1>(mc, K, offset != nullptr))
            e = launch_aq_xs<2, 2, 4, 1>(yc, xc, wp, int4, scale, offset, g, mc, N, K, aq_blocks(NBT, 4, 256), atomic, st);
        else if (cols_ok && mc > 16 && mc <= 32 && aq_ring_lds<2, 3, 1, 8, 2, 2>(K, offset != nullptr))
            e = launch_aq_ring<2, 3, 1, 8, 2, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, aq_blocks(NBT, 3, 256), atomic, st);
        // (32 < M <= 64: 2 strip groups x 4 k-split waves, weights 1 round ahead, about 256 blocks of <= 4 strips;
        // measured against 172 blocks with 3 rounds ahead and seven other splits: W4 M = 64 17.7 against 18.5-28 us)
        else if (cols_ok && mc > 32 && aq_ring_lds<4, 2, 2, 4, 2, 2>(K, offset != nullptr))
            e = launch_aq_ring<4, 2, 2, 4, 2, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, aq_blocks(NBT, 4, 256), atomic, st);
        // (a long K with a scale row per k tile leaves the ring no LDS for them: the K-split blocks with four row
        // tiles, measured at K = 28672, N = 8192, int4: M = 40 / 64 in 83 / 108 us against 122 / 122 us for a ring of
        // two k-split waves)
        else if (cols_ok && mc > 32 && aq_cols_fit(mc, N, K, g, int4))
            e = launch_aq_kw_any(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
        else {
            if (mc <= 4 && mc * K * 2 + 16 <= 48 * 1024) {
                if (int4) launch_aq<1, 1, 4, 8, true>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
                else launch_aq<1, 1, 8, 4, true>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
            } else if (mc > 4 && g % KT == 0) {
                if (mc <= 16) {
                    if (int4) launch_dma<1, 2, 4, 4, false>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
                    else launch_dma<1, 2, 4, 3, false>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
                } else if (mc <= 32) {
                    launch_dma<2, 4, 4, 4, false>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
                } else {
                    launch_dma<4, 4, 2, 3, true>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
                }
            } else if (mc <= 16) launch_aq<1, 1, 8, 4>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
            else if (mc <= 32) launch_aq<2, 2, 8, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
            else launch_aq<4, 2, 8, 2>(yc, xc, wp, int4, scale, offset, g, mc, N, K, atomic, st);
            e = hipGetLastError();
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace ascq
