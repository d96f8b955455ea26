// gemm_i8.hip -- int8 x int8 -> int32 GEMM on CDNA4 MFMA with the fixpipe dequant fused in the epilogue.
//
// Replaces the adv_api Matmul quant scenario (impl/adv_api/detail/matmul/matmul_impl.h:119-137 IterateAll;
// stage/compute/mmad_compute.h:40-90 Mmad int8 -> int32 L0C; stage/copy_cube_out/copy_cube_out_fixpipe.h:339-357
// and quant/quant_processor_fixpipe.h:74-234 for the DEQF16 / QS322BF16_PRE epilogue).
//
// gfx950 design
//  * v_mfma_i32_16x16x64_i8: a wave multiplies 16x64 by 64x16 int8 per instruction (16 cycles); both operands
//    hold 16 consecutive K bytes per lane, so the LDS tiles are K-contiguous: sA[m][k], sB[n][k], row stride
//    BK+16 bytes (the 16-byte pad keeps the 8 lanes of each ds_read_b128 phase on distinct banks).
//  * Block tile BM x BN x 64 on WM x WN waves, each wave BM/WM x BN/WN of 16x16 accumulator tiles; LDS is
//    double-buffered so the global loads of step k+1 are in flight while step k runs on the MFMA pipe.
//  * B given row-major [K, N] (isTransposeB = false, the reference default) is transposed on its way into
//    LDS: each lane loads an 8(k) x 4(n) byte block as 8 dwords, v_perm_b32 turns it into 4 columns of
//    8 K-contiguous bytes, written with ds_write_b64.  B given as [N, K] goes straight in.
//  * Blocks are numbered XCD-major: the hardware deals workgroups to the 8 XCDs round-robin, so the id is
//    remapped to give each XCD a contiguous band of output tiles (its A rows / B columns stay in its own L2).
//  * Epilogue: acc (+ int32 bias) -> f32 (rne) x M1[n] -> f16 / bf16 (rne, saturating); M1 = QUANT_PRE
//    bits [31:13] (accompanying_quantization.md:79-103).  K must be a multiple of 16 (else the generic path).
#include "common.h"
#include "launch.h"

namespace ascq {

constexpr int GK = 64;            // K per block step = K of one MFMA
constexpr int GLDS = GK + 16;     // LDS row stride in bytes

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// 4x4 byte transpose: in r[i] byte j = M[i][j]; out t[j] byte i = M[i][j]
__device__ __forceinline__ void transpose4x4(const uint32_t r0, const uint32_t r1, const uint32_t r2,
                                             const uint32_t r3, uint32_t& t0, uint32_t& t1, uint32_t& t2,
                                             uint32_t& t3)
{
    uint32_t lo01 = perm_b32(r1, r0, 0x05010400u); // r0.b0 r1.b0 r0.b1 r1.b1
    uint32_t hi01 = perm_b32(r1, r0, 0x07030602u); // r0.b2 r1.b2 r0.b3 r1.b3
    uint32_t lo23 = perm_b32(r3, r2, 0x05010400u);
    uint32_t hi23 = perm_b32(r3, r2, 0x07030602u);
    t0 = perm_b32(lo23, lo01, 0x05040100u);        // r0.b0 r1.b0 r2.b0 r3.b0
    t1 = perm_b32(lo23, lo01, 0x07060302u);
    t2 = perm_b32(hi23, hi01, 0x05040100u);
    t3 = perm_b32(hi23, hi01, 0x07060302u);
}

// XCD-aware tile order: consecutive workgroup ids go to different XCDs; give XCD x the ids
// [x*per, (x+1)*per) of a grouped (GROUP_M rows of tiles at a time) raster over the tile grid.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn)
{
    const int total = tiles_m * tiles_n;
    if (total % 8 == 0) {
        const int per = total / 8;
        pid = (pid % 8) * per + pid / 8;
    }
    constexpr int GROUP_M = 8;
    const int width = GROUP_M * tiles_n;
    const int group = pid / width;
    const int first_m = group * GROUP_M;
    const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
    const int in_group = pid % width;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

// Main loop shared by the Matmul and the group-matmul kernels.  A points at the tile's first row (row-major,
// lda), B at the tile's first column (TB: [n][k] with ldb; else [k][n] with ldb).  rows / cols = valid rows of
// A and columns of B in this tile (loads past them read zeros).  acc receives the int32 tile.
template <int BM, int BN, int WM, int WN, bool TB>
struct TileGemmI8 {
    static constexpr int NT = WM * WN * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int FM = WTM / 16, FN = WTN / 16;
    static constexpr int A_CH = BM * GK / 16 / NT;                  // 16-byte chunks of A per thread
    static constexpr int B_CH = TB ? BN * GK / 16 / NT : 1;
    static constexpr int B_BLK = TB ? 1 : (GK / 8) * (BN / 4) / NT; // 8x4 blocks per thread
    static constexpr int STAGE = (BM + BN) * GLDS;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE;
    static_assert(A_CH >= 1 && (BM * GK / 16) % NT == 0, "A tiling");
    static_assert(TB ? ((BN * GK / 16) % NT == 0 && B_CH >= 1) : ((GK / 8) * (BN / 4) % NT == 0 && B_BLK >= 1),
                  "B tiling");

    __device__ __forceinline__ static void run(const int8_t* __restrict__ A, int64_t lda, int64_t rows,
                                               const int8_t* __restrict__ B, int64_t ldb, int64_t cols, int64_t K,
                                               int8_t* smem, v4i (&acc)[FM][FN])
    {
        const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
        const int wm = wave / WN, wn = wave % WN;
        u32x4 ra[A_CH];
        u32x4 rb[B_CH];
        uint32_t rbt[B_BLK][8];

        auto load_global = [&](int64_t k0) {
#pragma unroll
            for (int i = 0; i < A_CH; ++i) {
                const int c = t + i * NT, row = c >> 2, kc = c & 3;
                const int64_t gk = k0 + kc * 16;
                if (row < rows && gk < K) ra[i] = *(const u32x4*)(A + row * lda + gk);
                else ra[i] = (u32x4){0u, 0u, 0u, 0u};
            }
            if constexpr (TB) {
#pragma unroll
                for (int i = 0; i < B_CH; ++i) {
                    const int c = t + i * NT, row = c >> 2, kc = c & 3;
                    const int64_t gk = k0 + kc * 16;
                    if (row < cols && gk < K) rb[i] = *(const u32x4*)(B + row * ldb + gk);
                    else rb[i] = (u32x4){0u, 0u, 0u, 0u};
                }
            } else {
#pragma unroll
                for (int i = 0; i < B_BLK; ++i) {
                    const int b = t + i * NT, nb = b % (BN / 4), kb = b / (BN / 4);
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const int64_t gk = k0 + kb * 8 + r;
                        rbt[i][r] = (nb * 4 < cols && gk < K) ? *(const uint32_t*)(B + gk * ldb + nb * 4) : 0u;
                    }
                }
            }
        };

        auto store_lds = [&](int buf) {
            int8_t* sA = smem + buf * STAGE;
            int8_t* sB = sA + BM * GLDS;
#pragma unroll
            for (int i = 0; i < A_CH; ++i) {
                const int c = t + i * NT, row = c >> 2, kc = c & 3;
                *(u32x4*)(sA + row * GLDS + kc * 16) = ra[i];
            }
            if constexpr (TB) {
#pragma unroll
                for (int i = 0; i < B_CH; ++i) {
                    const int c = t + i * NT, row = c >> 2, kc = c & 3;
                    *(u32x4*)(sB + row * GLDS + kc * 16) = rb[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < B_BLK; ++i) {
                    const int b = t + i * NT, nb = b % (BN / 4), kb = b / (BN / 4);
                    uint32_t lo[4], hi[4];
                    transpose4x4(rbt[i][0], rbt[i][1], rbt[i][2], rbt[i][3], lo[0], lo[1], lo[2], lo[3]);
                    transpose4x4(rbt[i][4], rbt[i][5], rbt[i][6], rbt[i][7], hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) *(u32x2*)(sB + (nb * 4 + j) * GLDS + kb * 8) = (u32x2){lo[j], hi[j]};
                }
            }
        };

#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = (v4i){0, 0, 0, 0};

        const int64_t nk = (K + GK - 1) / GK;
        load_global(0);
        store_lds(0);
        __syncthreads();
        for (int64_t kt = 0; kt < nk; ++kt) {
            const int buf = (int)(kt & 1);
            if (kt + 1 < nk) load_global((kt + 1) * GK);
            const int8_t* sA = smem + buf * STAGE;
            const int8_t* sB = sA + BM * GLDS;
            v4i fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i)
                fa[i] = *(const v4i*)(sA + (wm * WTM + i * 16 + (lane & 15)) * GLDS + (lane >> 4) * 16);
#pragma unroll
            for (int j = 0; j < FN; ++j)
                fb[j] = *(const v4i*)(sB + (wn * WTN + j * 16 + (lane & 15)) * GLDS + (lane >> 4) * 16);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
            if (kt + 1 < nk) store_lds(buf ^ 1);
            __syncthreads();
        }
    }
};

template <int BM, int BN, int WM, int WN, bool TB>
__global__ __launch_bounds__(WM * WN * 64) void gemm_i8_kernel(GemmI8Args p)
{
    using T = TileGemmI8<BM, BN, WM, WN, TB>;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    const int tiles_m = (int)((p.M + BM - 1) / BM), tiles_n = (int)((p.N + BN - 1) / BN);
    int tm, tn;
    tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int8_t* A = p.A + m0 * p.lda;
    const int8_t* B = TB ? p.B + n0 * p.ldb : p.B + n0;
    v4i acc[T::FM][T::FN];
    T::run(A, p.lda, p.M - m0, B, p.ldb, p.N - n0, p.K, smem, acc);

    // epilogue: lane holds rows 4*(lane>>4)+r, column lane&15 of each 16x16 tile
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const float mscalar = quant_pre_m1(p.qscalar);
#pragma unroll
    for (int j = 0; j < T::FN; ++j) {
        const int64_t col = n0 + wn * T::WTN + j * 16 + (lane & 15);
        if (col >= p.N) continue;
        const int32_t bias = p.bias ? p.bias[col] : 0;
        const float m1 = p.qvec ? quant_pre_m1(p.qvec[col]) : mscalar;
#pragma unroll
        for (int i = 0; i < T::FM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * T::WTM + i * 16 + (lane >> 4) * 4 + r;
                if (row >= p.M) continue;
                const int32_t v = (int32_t)((uint32_t)acc[i][j][r] + (uint32_t)bias);
                const int64_t o = row * p.ldc + col;
                if (p.epi == EPI_I32) ((int32_t*)p.C)[o] = v;
                else if (p.epi == EPI_DEQ_F16) ((uint16_t*)p.C)[o] = f32_to_f16_sat((float)v * m1);
                else ((uint16_t*)p.C)[o] = f32_to_bf16_sat((float)v * m1);
            }
        }
    }
}

// QuantGroupMatmul: the m axis is split into G ragged groups (group_list), group g multiplies its rows by
// W[g].  Workgroup slot -> (m-tile of the concatenated groups, n-tile); m-tiles never straddle a group.
// Slots beyond the real tile count exit at once (the grid is sized for ceil(M/BM) + G m-tiles).
template <int BM, int BN, int WM, int WN, bool TB>
__global__ __launch_bounds__(WM * WN * 64) void group_gemm_i8_kernel(GroupGemmArgs p)
{
    using T = TileGemmI8<BM, BN, WM, WN, TB>;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    __shared__ int64_t g_start[65], g_tile[65];
    const int G = (int)p.G;
    if (threadIdx.x == 0) {
        int64_t s = p.list_type == 0 ? p.group_list[0] : 0, tiles = 0;
        for (int g = 0; g < G; ++g) {
            int64_t cnt = p.list_type == 0 ? p.group_list[g + 1] - p.group_list[g] : p.group_list[g];
            if (cnt < 0) cnt = 0;
            g_start[g] = s;
            g_tile[g] = tiles;
            s += cnt;
            tiles += (cnt + BM - 1) / BM;
        }
        g_start[G] = s;
        g_tile[G] = tiles;
    }
    __syncthreads();
    const int tiles_n = (int)((p.N + BN - 1) / BN);
    const int64_t mt = blockIdx.x / tiles_n;
    const int tn = blockIdx.x % tiles_n;
    if (mt >= g_tile[G]) return;
    int g = 0;
    while (g + 1 < G && g_tile[g + 1] <= mt) ++g;
    const int64_t m0 = g_start[g] + (mt - g_tile[g]) * BM;
    int64_t m_end = g_start[g + 1];
    if (m_end > p.M) m_end = p.M;
    if (m0 < 0 || m0 >= m_end) return;  // offsets come from device memory: never form a row outside [0, M)
    const int64_t n0 = (int64_t)tn * BN;
    const int8_t* Wg = p.W + (int64_t)g * p.K * p.N;
    const int8_t* B = TB ? Wg + n0 * p.K : Wg + n0;
    v4i acc[T::FM][T::FN];
    T::run(p.X + m0 * p.K, p.K, m_end - m0, B, TB ? p.K : p.N, p.N - n0, p.K, smem, acc);

    // epilogue (quant_group_matmul_custom.asc:424-452 without the Gelu): AscendDequant acc*scale[g,n] in fp32,
    // Mul by the per-token scale in fp32, one rounding cast to the output type.
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
#pragma unroll
    for (int j = 0; j < T::FN; ++j) {
        const int64_t col = n0 + wn * T::WTN + j * 16 + (lane & 15);
        if (col >= p.N) continue;
        const float sc = p.scale[(int64_t)g * p.N + col];
#pragma unroll
        for (int i = 0; i < T::FM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * T::WTM + i * 16 + (lane >> 4) * 4 + r;
                if (row >= m_end) continue;
                float v = (float)acc[i][j][r] * sc;
                v = v * p.pts[row];
                const int64_t o = row * p.N + col;
                if (p.out_type == DT_F16) ((uint16_t*)p.Y)[o] = f32_to_f16_sat(v);
                else ((uint16_t*)p.Y)[o] = f32_to_bf16_sat(v);
            }
        }
    }
}

// Any shape / layout / alignment: one thread per output element, int32 accumulate, same epilogue.
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(GemmI8Args p)
{
    const int64_t total = p.M * p.N;
    const float mscalar = quant_pre_m1(p.qscalar);
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t m = e / p.N, n = e % p.N;
        uint32_t acc = 0;
        for (int64_t k = 0; k < p.K; ++k) {
            const int32_t a = p.trans_a ? p.A[k * p.lda + m] : p.A[m * p.lda + k];
            const int32_t b = p.trans_b ? p.B[n * p.ldb + k] : p.B[k * p.ldb + n];
            acc += (uint32_t)(a * b);
        }
        const int32_t v = (int32_t)(acc + (uint32_t)(p.bias ? p.bias[n] : 0));
        const float m1 = p.qvec ? quant_pre_m1(p.qvec[n]) : mscalar;
        const int64_t o = m * p.ldc + n;
        if (p.epi == EPI_I32) ((int32_t*)p.C)[o] = v;
        else if (p.epi == EPI_DEQ_F16) ((uint16_t*)p.C)[o] = f32_to_f16_sat((float)v * m1);
        else ((uint16_t*)p.C)[o] = f32_to_bf16_sat((float)v * m1);
    }
}

template <int BM, int BN, int WM, int WN, bool TB>
static hipError_t launch_tiled(const GemmI8Args& a, hipStream_t st)
{
    using T = TileGemmI8<BM, BN, WM, WN, TB>;
    const int tiles = (int)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)gemm_i8_kernel<BM, BN, WM, WN, TB>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((gemm_i8_kernel<BM, BN, WM, WN, TB>), dim3(tiles), dim3(T::NT), T::LDS_BYTES, st, a);
    return hipGetLastError();
}

hipError_t launch_gemm_i8(const GemmI8Args& a, hipStream_t st)
{
    const bool a_ok = !a.trans_a && a.lda % 16 == 0 && ((uintptr_t)a.A % 16 == 0);
    const bool b_ok = a.trans_b ? (a.ldb % 16 == 0 && ((uintptr_t)a.B % 16 == 0))
                                : (a.ldb % 4 == 0 && a.N % 4 == 0 && ((uintptr_t)a.B % 4 == 0));
    if (a_ok && b_ok && a.K % 16 == 0) {
        const bool big = a.M >= 1024 && a.N >= 1024;
        if (a.trans_b) return big ? launch_tiled<256, 256, 4, 2, true>(a, st) : launch_tiled<64, 64, 2, 2, true>(a, st);
        return big ? launch_tiled<256, 256, 4, 2, false>(a, st) : launch_tiled<64, 128, 2, 2, false>(a, st);
    }
    int64_t blocks = (a.M * a.N + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(gemm_i8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

// generic group matmul: one thread per output element (any alignment)
__global__ __launch_bounds__(256) void group_gemm_generic_kernel(GroupGemmArgs p)
{
    const int64_t total = p.M * p.N;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t m = e / p.N, n = e % p.N;
        int64_t s = p.list_type == 0 ? p.group_list[0] : 0;
        int g = -1;
        for (int h = 0; h < (int)p.G; ++h) {
            int64_t cnt = p.list_type == 0 ? p.group_list[h + 1] - p.group_list[h] : p.group_list[h];
            if (cnt < 0) cnt = 0;
            if (m >= s && m < s + cnt) { g = h; break; }
            s += cnt;
        }
        if (g < 0 || m < 0) continue;
        const int8_t* Wg = p.W + (int64_t)g * p.K * p.N;
        uint32_t acc = 0;
        for (int64_t k = 0; k < p.K; ++k)
            acc += (uint32_t)((int32_t)p.X[m * p.K + k] * (int32_t)(p.w_trans ? Wg[n * p.K + k] : Wg[k * p.N + n]));
        float v = (float)(int32_t)acc * p.scale[(int64_t)g * p.N + n];
        v = v * p.pts[m];
        if (p.out_type == DT_F16) ((uint16_t*)p.Y)[m * p.N + n] = f32_to_f16_sat(v);
        else ((uint16_t*)p.Y)[m * p.N + n] = f32_to_bf16_sat(v);
    }
}

template <int BM, int BN, int WM, int WN, bool TB>
static hipError_t launch_group_tiled(const GroupGemmArgs& a, hipStream_t st)
{
    using T = TileGemmI8<BM, BN, WM, WN, TB>;
    const int64_t slots = ((a.M + BM - 1) / BM + a.G) * ((a.N + BN - 1) / BN);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)group_gemm_i8_kernel<BM, BN, WM, WN, TB>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)T::LDS_BYTES);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((group_gemm_i8_kernel<BM, BN, WM, WN, TB>), dim3((unsigned)slots), dim3(T::NT), T::LDS_BYTES,
                       st, a);
    return hipGetLastError();
}

hipError_t launch_group_gemm(const GroupGemmArgs& a, hipStream_t st)
{
    const bool ok = a.K % 16 == 0 && ((uintptr_t)a.X % 16 == 0) &&
                    (a.w_trans ? ((uintptr_t)a.W % 16 == 0) : (a.N % 4 == 0 && (uintptr_t)a.W % 4 == 0)) && a.G <= 64;
    if (ok) {
        if (a.w_trans) return launch_group_tiled<128, 128, 2, 2, true>(a, st);
        return launch_group_tiled<128, 128, 2, 2, false>(a, st);
    }
    int64_t blocks = (a.M * a.N + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(group_gemm_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace ascq
