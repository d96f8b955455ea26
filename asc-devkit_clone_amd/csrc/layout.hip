// layout.hip -- NZ fractal <-> ND converters, so data prepared for the reference's cube format can be fed to the
// ND / K-contiguous kernels of this library (and back).
//
// NZ (CubeFormat::NZ, include/adv_api/matmul/matmul_config.h:23-35; the group-matmul weights of
// examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/quant_group_matmul_high_performance/scripts/
// gen_data.py:62, weight.reshape([G, k/16, 16, n/32, 32]).transpose([0, 3, 1, 2, 4])): a [rows, cols] matrix is
// stored as [ceil(cols / C0)][ceil(rows / 16)][16][C0] with C0 = 32 bytes of elements, i.e. 16 x 32-byte fractals,
// column blocks outermost.  One fractal row (row r, C0 columns) is the same 32 contiguous bytes in both layouts,
// so the conversion moves whole 32-byte segments for every element type; only the tail segment of a row whose
// byte length is not a multiple of 32 is partial (NZ pads it; nd_to_nz writes the padding as zeros).
//
// nz_to_nd with transpose_out (1-byte elements): writes [cols, rows] instead -- the K-contiguous B / [G, N, K]
// expert weights the GEMMs copy straight into LDS -- one 16-byte output chunk (16 consecutive rows of one
// column) per thread, gathered from one fractal at a 32-byte stride.
#include "common.h"
#include "launch.h"

namespace ascq {

struct NzGeom {
    int64_t batch, rows, cols_b;  // cols_b: row length in bytes
    int64_t r16, c32;             // fractal rows (ceil(rows / 16)) and 32-byte column blocks (ceil(cols_b / 32))
    int64_t nz_mat;               // bytes of one NZ matrix: c32 * r16 * 512
};

__device__ __forceinline__ int64_t nz_offset(const NzGeom& g, int64_t b, int64_t r, int64_t cb)
{
    return b * g.nz_mat + ((cb * g.r16 + (r >> 4)) * 16 + (r & 15)) * 32;
}

// one thread per 32-byte segment (b, r, cb) of the ND matrix
template <bool TO_ND>
__global__ __launch_bounds__(256) void nz_nd_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, NzGeom g,
                                                    bool fast)
{
    const int64_t rows_pad = TO_ND ? g.rows : g.r16 * 16;  // nd_to_nz also writes the padding rows
    const int64_t total = g.batch * rows_pad * g.c32;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        const int64_t cb = i % g.c32, r = (i / g.c32) % rows_pad, b = i / (g.c32 * rows_pad);
        const int64_t nz = nz_offset(g, b, r, cb);
        const int64_t nd = (b * g.rows + r) * g.cols_b + cb * 32;
        const int64_t valid = r < g.rows ? (g.cols_b - cb * 32 < 32 ? g.cols_b - cb * 32 : 32) : 0;
        if (TO_ND) {
            if (fast) {
                *(u32x4*)(dst + nd) = *(const u32x4*)(src + nz);
                *(u32x4*)(dst + nd + 16) = *(const u32x4*)(src + nz + 16);
            } else {
                for (int64_t j = 0; j < valid; ++j) dst[nd + j] = src[nz + j];
            }
        } else {
            if (fast && valid == 32) {
                *(u32x4*)(dst + nz) = *(const u32x4*)(src + nd);
                *(u32x4*)(dst + nz + 16) = *(const u32x4*)(src + nd + 16);
            } else {
                for (int64_t j = 0; j < 32; ++j) dst[nz + j] = j < valid ? src[nd + j] : (uint8_t)0;
            }
        }
    }
}

// 1-byte elements, NZ -> [batch][cols][rows]: thread (b, c, kb) writes rows 16 kb .. 16 kb + 15 of column c
__global__ __launch_bounds__(256) void nz_to_nd_t_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                         NzGeom g, bool fast)
{
    const int64_t cols = g.cols_b;
    const int64_t total = g.batch * cols * g.r16;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        // consecutive threads take consecutive columns of one fractal row band, so each of the 16 gathers of a
        // wave reads contiguous bytes
        const int64_t c = i % cols, kb = (i / cols) % g.r16, b = i / (cols * g.r16);
        const uint8_t* f = src + nz_offset(g, b, kb * 16, c >> 5) + (c & 31);
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            w[q] = (uint32_t)f[(4 * q) * 32] | ((uint32_t)f[(4 * q + 1) * 32] << 8) |
                   ((uint32_t)f[(4 * q + 2) * 32] << 16) | ((uint32_t)f[(4 * q + 3) * 32] << 24);
        uint8_t* o = dst + (b * cols + c) * g.rows + kb * 16;
        if (fast) {
            *(u32x4*)o = (u32x4){w[0], w[1], w[2], w[3]};
        } else {
            const int64_t n = g.rows - kb * 16 < 16 ? g.rows - kb * 16 : 16;
            for (int64_t j = 0; j < n; ++j) o[j] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
        }
    }
}

static NzGeom geom(int64_t batch, int64_t rows, int64_t cols, int esize)
{
    NzGeom g;
    g.batch = batch;
    g.rows = rows;
    g.cols_b = cols * esize;
    g.r16 = (rows + 15) / 16;
    g.c32 = (g.cols_b + 31) / 32;
    g.nz_mat = g.c32 * g.r16 * 512;
    return g;
}

static unsigned grid_for(int64_t work)
{
    int64_t blocks = (work + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

size_t nz_bytes(int64_t batch, int64_t rows, int64_t cols, int esize)
{
    const NzGeom g = geom(batch, rows, cols, esize);
    return (size_t)(g.batch * g.nz_mat);
}

hipError_t launch_nz_to_nd(void* dst, const void* src, int esize, int64_t batch, int64_t rows, int64_t cols,
                           int transpose_out, hipStream_t st)
{
    const NzGeom g = geom(batch, rows, cols, esize);
    if (transpose_out) {
        const bool fast = rows % 16 == 0 && (uintptr_t)dst % 16 == 0;
        hipLaunchKernelGGL(nz_to_nd_t_kernel, dim3(grid_for(batch * cols * g.r16)), dim3(256), 0, st, (uint8_t*)dst,
                           (const uint8_t*)src, g, fast);
    } else {
        const bool fast = g.cols_b % 32 == 0 && (uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0;
        hipLaunchKernelGGL(nz_nd_kernel<true>, dim3(grid_for(batch * rows * g.c32)), dim3(256), 0, st, (uint8_t*)dst,
                           (const uint8_t*)src, g, fast);
    }
    return hipGetLastError();
}

hipError_t launch_nd_to_nz(void* dst, const void* src, int esize, int64_t batch, int64_t rows, int64_t cols,
                           hipStream_t st)
{
    const NzGeom g = geom(batch, rows, cols, esize);
    const bool fast = g.cols_b % 32 == 0 && (uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0;
    hipLaunchKernelGGL(nz_nd_kernel<false>, dim3(grid_for(batch * g.r16 * 16 * g.c32)), dim3(256), 0, st,
                       (uint8_t*)dst, (const uint8_t*)src, g, fast);
    return hipGetLastError();
}

}  // namespace ascq
