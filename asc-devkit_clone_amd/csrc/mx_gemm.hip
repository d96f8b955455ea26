// mx_gemm.hip -- MX-FP4 (E2M1 elements, E8M0 scale per 32 K) block-scaled GEMM on gfx950.
//
// Reference: Matmul<MatmulTypeWithScale<..., fp4x2_e2m1_t, ...>> with SetTensorScaleA/B and IterateAll
// (impl/adv_api/detail/matmul/mx_matmul_impl.h:136-188; MmadMx include/basic_api/kernel_operator_mm_intf.h:348-352),
// fp32 accumulation, F322BF16 (rint) in the fixpipe.  Golden: matmul_mxfp4_high_performance/scripts/gen_data.py.
//
// gfx950 design
//  * v_mfma_scale_f32_16x16x128_f8f6f4 with both formats = FP4 (cbsz = blgp = 4): per lane 32 E2M1 values
//    (16 bytes, one MX block) of row (lane % 16) at k block (lane / 16), and one E8M0 scale byte for that
//    (row, block) -- the hardware applies 2^(e-127) per 32-element block, which is exactly the MX product.
//  * LDS tiles are K-contiguous bytes (two fp4 per byte, even k in the low nibble -- the reference packing,
//    gen_data.py:25-34 -- which is also the MFMA's nibble order): sA[m][k/2], sB[n][k/2], row stride 64+16 B.
//  * Block tile 256 x 256 x 128 on 8 waves (4 x 2), wave tile 64 x 128 = 4 x 8 MFMA tiles; LDS double-buffered.
//  * Scales ride along with the operand tiles: per k step each tile row needs the 4 E8M0 bytes of its 4 k
//    blocks, staged as one dword per row in the same double-buffered LDS stage; a lane reads its byte.
//  * B stored [K, N] (the reference's non-transposed layout, two fp4 per byte along N) is first transposed to
//    [N, K] in a workspace by fp4_transpose_kernel.
#include "common.h"
#include "launch.h"

namespace ascq {

constexpr int MXK = 128;         // K per block step (one MFMA)
constexpr int MXROW = MXK / 2;   // bytes per row per step
constexpr int MXLDS = MXROW + 16;

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(WM * WN * 64) void mx_gemm_kernel(MxGemmArgs p)
{
    constexpr int NT = WM * WN * 64;
    constexpr int WTM = BM / WM, WTN = BN / WN;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int A_CH = BM * MXROW / 16 / NT;
    constexpr int B_CH = BN * MXROW / 16 / NT;
    constexpr int STAGE = (BM + BN) * MXLDS + (BM + BN) * 4;  // operand rows, then one scale dword per row
    constexpr int SC_PER = (BM + BN + NT - 1) / NT;
    static_assert(A_CH >= 1 && B_CH >= 1, "tiling");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_mx[];

    const int64_t M = p.M, N = p.N, K = p.K;
    const int64_t sK = (K + 63) / 64 * 2;
    const int64_t KB2 = K / 2;
    const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
    // XCD-major grouped raster (see gemm_i8.hip)
    int pid = blockIdx.x;
    const int total = tiles_m * tiles_n;
    if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
    constexpr int GROUP_M = 8;
    const int width = GROUP_M * tiles_n, grp = pid / width, first_m = grp * GROUP_M;
    const int gsz = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
    const int tm = first_m + (pid % width) % gsz, tn = (pid % width) / gsz;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int kq = lane >> 4, r16 = lane & 15;

    u32x4 ra[A_CH], rb[B_CH];
    uint32_t rs[SC_PER];
    auto load_global = [&](int64_t k0) {  // k0 in elements
        // scale dword of each tile row: the 4 E8M0 bytes of k blocks k0/32 .. k0/32+3
        const int64_t b0 = k0 / 32;
#pragma unroll
        for (int i = 0; i < SC_PER; ++i) {
            const int r = t + i * NT;
            uint32_t v = 0x7f7f7f7fu;
            if (r < BM) {
                const int64_t gm = m0 + r;
                if (gm < M) {
                    if (p.sa_layout == 0) v = *(const uint32_t*)(p.sA + gm * sK + b0);
                    else v = (uint32_t)*(const uint16_t*)(p.sA + (b0 >> 1) * M * 2 + gm * 2) |
                             ((uint32_t)*(const uint16_t*)(p.sA + ((b0 >> 1) + 1) * M * 2 + gm * 2) << 16);
                }
            } else if (r < BM + BN) {
                const int64_t gn = n0 + (r - BM);
                if (gn < N) {
                    if (p.sb_layout == 1) v = *(const uint32_t*)(p.sB + gn * sK + b0);
                    else v = (uint32_t)*(const uint16_t*)(p.sB + (b0 >> 1) * N * 2 + gn * 2) |
                             ((uint32_t)*(const uint16_t*)(p.sB + ((b0 >> 1) + 1) * N * 2 + gn * 2) << 16);
                }
            }
            rs[i] = v;
        }
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const int c = t + i * NT, row = c >> 2, kc = c & 3;
            const int64_t gm = m0 + row, gb = k0 / 2 + kc * 16;
            ra[i] = (gm < M && gb < KB2) ? *(const u32x4*)(p.A + gm * KB2 + gb) : (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const int c = t + i * NT, row = c >> 2, kc = c & 3;
            const int64_t gn = n0 + row, gb = k0 / 2 + kc * 16;
            rb[i] = (gn < N && gb < KB2) ? *(const u32x4*)(p.B + gn * KB2 + gb) : (u32x4){0u, 0u, 0u, 0u};
        }
    };
    auto store_lds = [&](int buf) {
        uint8_t* sA = smem_mx + buf * STAGE;
        uint8_t* sB = sA + BM * MXLDS;
        uint32_t* sS = (uint32_t*)(sA + (BM + BN) * MXLDS);
#pragma unroll
        for (int i = 0; i < SC_PER; ++i) {
            const int r = t + i * NT;
            if (r < BM + BN) sS[r] = rs[i];
        }
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            const int c = t + i * NT, row = c >> 2, kc = c & 3;
            *(u32x4*)(sA + row * MXLDS + kc * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            const int c = t + i * NT, row = c >> 2, kc = c & 3;
            *(u32x4*)(sB + row * MXLDS + kc * 16) = rb[i];
        }
    };

    v4f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};

    const int64_t nk = (K + MXK - 1) / MXK;
    load_global(0);
    store_lds(0);
    __syncthreads();
    for (int64_t kt = 0; kt < nk; ++kt) {
        const int buf = (int)(kt & 1);
        if (kt + 1 < nk) load_global((kt + 1) * MXK);
        const uint8_t* sA = smem_mx + buf * STAGE;
        const uint8_t* sB = sA + BM * MXLDS;
        const uint8_t* sS = sA + (BM + BN) * MXLDS;
        // scale of this lane's (row, k block kt*4 + kq)
        int sa[FM], sb[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i) sa[i] = sS[(wm * WTM + i * 16 + r16) * 4 + kq];
#pragma unroll
        for (int j = 0; j < FN; ++j) sb[j] = sS[(BM + wn * WTN + j * 16 + r16) * 4 + kq];
        v4i fa[FM];
#pragma unroll
        for (int i = 0; i < FM; ++i) fa[i] = *(const v4i*)(sA + (wm * WTM + i * 16 + r16) * MXLDS + kq * 16);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const v4i fb = *(const v4i*)(sB + (wn * WTN + j * 16 + r16) * MXLDS + kq * 16);
            const v8i b8 = (v8i){fb[0], fb[1], fb[2], fb[3], 0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const v8i a8 = (v8i){fa[i][0], fa[i][1], fa[i][2], fa[i][3], 0, 0, 0, 0};
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a8, b8, acc[i][j], 4, 4, 0, sa[i], 0,
                                                                             sb[j]);
            }
        }
        if (kt + 1 < nk) store_lds(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn * WTN + j * 16 + r16;
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * WTM + i * 16 + kq * 4 + r;
                if (row >= M) continue;
                if (p.c_type == DT_F32) ((float*)p.C)[row * N + col] = acc[i][j][r];
                else ((uint16_t*)p.C)[row * N + col] = f32_to_bf16_sat(acc[i][j][r]);
            }
    }
}

// [K, N] (two fp4 per byte along N) -> [N, K] (two per byte along K).  One thread per output byte.
__global__ __launch_bounds__(256) void fp4_transpose_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                            int64_t K, int64_t N)
{
    const int64_t KB = K / 2, total = N * KB, NB = N / 2;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
        const int64_t n = o / KB, kb = o % KB;
        const int64_t k0 = 2 * kb;
        const uint8_t b0 = src[k0 * NB + (n >> 1)];
        const uint8_t b1 = src[(k0 + 1) * NB + (n >> 1)];
        const uint8_t lo = (n & 1) ? (b0 >> 4) : (b0 & 0xf);
        const uint8_t hi = (n & 1) ? (b1 >> 4) : (b1 & 0xf);
        dst[o] = (uint8_t)(lo | (hi << 4));
    }
}

hipError_t launch_fp4_transpose(uint8_t* dst, const uint8_t* src, int64_t K, int64_t N, hipStream_t st)
{
    int64_t blocks = (N * K / 2 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fp4_transpose_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, src, K, N);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN>
static hipError_t launch_mx_tiled(const MxGemmArgs& a, hipStream_t st)
{
    const size_t lds = 2 * (size_t)(BM + BN) * (MXLDS + 4);
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)mx_gemm_kernel<BM, BN, WM, WN>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const int tiles = (int)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    hipLaunchKernelGGL((mx_gemm_kernel<BM, BN, WM, WN>), dim3(tiles), dim3(WM * WN * 64), lds, st, a);
    return hipGetLastError();
}

hipError_t launch_mx_gemm(const MxGemmArgs& a, hipStream_t st)
{
    if (a.M >= 1024 && a.N >= 1024) return launch_mx_tiled<256, 256, 4, 2>(a, st);
    return launch_mx_tiled<64, 64, 2, 2>(a, st);
}

}  // namespace ascq
