// mx_gemm.hip -- MX-FP4 (E2M1 elements, E8M0 scale per 32 K) block-scaled GEMM on gfx950.
//
// Reference: Matmul<MatmulTypeWithScale<..., fp4x2_e2m1_t, ...>> with SetTensorScaleA/B and IterateAll
// (impl/adv_api/detail/matmul/mx_matmul_impl.h:136-188; MmadMx include/basic_api/kernel_operator_mm_intf.h:348-352),
// fp32 accumulation, F322BF16 (rint) in the fixpipe.  Golden: matmul_mxfp4_high_performance/scripts/gen_data.py.
//
// gfx950 design: the LDS-ring main loop of gemm_core.h with v_mfma_scale_f32_32x32x64_f8f6f4, both formats
// FP4 (cbsz = blgp = 4): per lane 32 E2M1 values (16 bytes, one MX block) of row (lane % 32) at k block
// (lane / 32), and one E8M0 scale byte for that (row, block) -- the hardware applies 2^(e-127) per 32-element
// block, which is exactly the MX product.  Two fp4 per byte, even k in the low nibble: the reference packing
// (gen_data.py:25-34) is also the MFMA's nibble order.  Block tile 256 x 256, 128 fp4 of K per stage, four
// stages, 8 waves (4 x 2), wave tile 64 x 128.  The E8M0 scales, rearranged stage-major by mx_scale_stage_major_kernel, ride in the
// same LDS stage.  B stored [K, N]
// (the reference's non-transposed layout, two fp4 per byte along N) is first transposed to [N, K] in a
// workspace by fp4_transpose_kernel.
#include "common.h"
#include "gemm_core.h"
#include "launch.h"

namespace ascq {

template <int BM, int BN, int WM, int WN, int ST>
__global__ __launch_bounds__(WM * WN * 64) void mx_gemm_kernel(MxGemmArgs p)
{
    using T = GemmCore<BM, BN, WM, WN, ST, true, OP_MXFP4>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_mx[];
    const int64_t M = p.M, N = p.N, K = p.K;
    const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t sK = (K + 63) / 64 * 2;
    CoreArgs c{};
    c.a = make_rsrc(p.A, (uint32_t)(M * (K / 2)));
    c.b = make_rsrc(p.B, (uint32_t)(N * (K / 2)));
    c.lda = c.ldb = (uint32_t)(K / 2);
    c.rows = (int32_t)(M - m0 < BM ? M - m0 : BM);
    c.cols = (int32_t)(N - n0 < BN ? N - n0 : BN);
    c.a0 = (uint32_t)(m0 * (K / 2));
    c.b0 = (uint32_t)(n0 * (K / 2));
    c.kbytes = K / 2;
    // the stage-major scale buffers carry 16 bytes of slack: a 16-byte copy at the end never straddles the range
    c.sa = make_rsrc(p.sA, (uint32_t)(M * sK + 16));
    c.sb = make_rsrc(p.sB, (uint32_t)(N * sK + 16));
    c.sa0_row = (uint32_t)m0;
    c.sb0_row = (uint32_t)n0;
    c.sa_rows = (uint32_t)M;
    c.sb_rows = (uint32_t)N;
    c.sk = (uint32_t)sK;
    typename T::acc_t acc[T::FM][T::FN];
    T::run(c, smem_mx, acc);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
#pragma unroll
    for (int j = 0; j < T::FN; ++j) {
        const int64_t col = n0 + T::frag_col(wn, j, lane);
        if (col >= N) continue;
#pragma unroll
        for (int i = 0; i < T::FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + T::frag_row(wm, i, r, lane);
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
    hipError_t err = hipSuccess;
    if (fp4_transpose_tiled(dst, src, K, N, st, &err)) return err;
    int64_t blocks = (N * K / 2 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(fp4_transpose_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, src, K, N);
    return hipGetLastError();
}

// E8M0 scales -> the stage-major layout the kernel reads: dst word (g, r) = blocks 4g .. 4g + 3 of row r, at
// byte (g * R + r) * 4.  src_layout 0: [R, sK] row-major; 1: [sK/2, R, 2] (pairs of blocks, rows inner).
// One thread per (group, row).
__global__ __launch_bounds__(256) void mx_scale_stage_major_kernel(uint32_t* __restrict__ dst,
                                                                   const uint8_t* __restrict__ src, int64_t R,
                                                                   int64_t sK, int src_layout)
{
    const int64_t groups = sK / 4, total = groups * R;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t g = i / R, r = i % R;
        uint32_t w;
        if (src_layout == 0) {
            w = *(const uint32_t*)(src + r * sK + 4 * g);
        } else {
            const uint16_t* s16 = (const uint16_t*)src;
            w = (uint32_t)s16[(2 * g) * R + r] | ((uint32_t)s16[(2 * g + 1) * R + r] << 16);
        }
        dst[i] = w;
    }
}

hipError_t launch_mx_scale_stage_major(uint8_t* dst, const uint8_t* src, int64_t R, int64_t sK, int src_layout,
                                       hipStream_t st)
{
    int64_t blocks = (R * (sK / 4) + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(mx_scale_stage_major_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (uint32_t*)dst, src, R,
                       sK, src_layout);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int ST>
static hipError_t launch_mx_tiled(const MxGemmArgs& a, hipStream_t st)
{
    using T = GemmCore<BM, BN, WM, WN, ST, true, OP_MXFP4>;
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute((const void*)mx_gemm_kernel<BM, BN, WM, WN, ST>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const int tiles = (int)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    hipLaunchKernelGGL((mx_gemm_kernel<BM, BN, WM, WN, ST>), dim3(tiles), dim3(T::NT), T::LDS_BYTES, st, a);
    return hipGetLastError();
}

// K must be a multiple of 128 (one LDS stage is 128 fp4 of K) and both scale tensors stage-major (the caller
// converts them with launch_mx_scale_stage_major).
hipError_t launch_mx_gemm(const MxGemmArgs& a, hipStream_t st)
{
    if (a.K % 128 != 0) return hipErrorInvalidValue;
    if (a.M >= 1024 && a.N >= 1024) return launch_mx_tiled<256, 256, 4, 2, 4>(a, st);
    return launch_mx_tiled<64, 64, 2, 2, 4>(a, st);
}

}  // namespace ascq
