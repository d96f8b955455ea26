// transpose.hip -- byte and nibble transposes that turn a row-major [K, N] B operand into the K-contiguous
// [N, K] layout the GEMM main loop copies straight into LDS (and the hifloat8 -> bf16 operand decode).
//
// One 256-thread workgroup per 128 (k) x 128 (byte column) tile:
//  * load: 16-byte chunks, eight lanes per 128-byte row segment, into LDS [k][128 bytes]; the dword column
//    of each chunk is XOR-swizzled by ((k / 16) % 4) * 8 so the transposed reads below spread over the banks;
//  * each lane then owns 4 byte columns x 16 k: 16 dword reads (rows k0 .. k0 + 15), four 4x4 byte
//    transposes (v_perm_b32), and per column 16 consecutive k bytes;
//  * int8: out[n][k0 .. k0 + 15] is one 16-byte store, eight lanes per 128-byte output row segment;
//  * fp4 (two E2M1 per byte, even index in the low nibble): byte column c holds n = 2c (low nibbles) and
//    n = 2c + 1 (high nibbles); the 16 k bytes of a column become 8 bytes of row 2c and 8 of row 2c + 1
//    (k pairs packed low nibble first), two 8-byte stores.
// Tiles on the edge load zeros past the matrix and store only inside it; the fast path needs the row length
// in bytes and the row count to be multiples of 16 (the caller falls back to a plain kernel otherwise).
#include "common.h"
#include "launch.h"

namespace ascq {

__device__ __forceinline__ uint32_t tperm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// 4x4 byte transpose: in r[i] byte j = M[i][j]; out t[j] byte i = M[i][j]
__device__ __forceinline__ void tr4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t& t0, uint32_t& t1,
                                      uint32_t& t2, uint32_t& t3)
{
    const uint32_t lo01 = tperm(r1, r0, 0x05010400u);
    const uint32_t hi01 = tperm(r1, r0, 0x07030602u);
    const uint32_t lo23 = tperm(r3, r2, 0x05010400u);
    const uint32_t hi23 = tperm(r3, r2, 0x07030602u);
    t0 = tperm(lo23, lo01, 0x05040100u);
    t1 = tperm(lo23, lo01, 0x07060302u);
    t2 = tperm(hi23, hi01, 0x05040100u);
    t3 = tperm(hi23, hi01, 0x07060302u);
}

// four k bytes (k, k+1, k+2, k+3) of one fp4 byte column -> 16 bits of the even-n row (low nibbles) and 16 bits
// of the odd-n row (high nibbles), each as (k, k+1) packed low nibble first
__device__ __forceinline__ void split_nibbles(uint32_t w, uint32_t& even, uint32_t& odd)
{
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t l2 = lo | (lo >> 4), h2 = hi | (hi >> 4);  // bytes 0 and 2 hold the packed pairs
    even = (l2 & 0xFFu) | ((l2 >> 8) & 0xFF00u);
    odd = (h2 & 0xFFu) | ((h2 >> 8) & 0xFF00u);
}

template <bool FP4>
__global__ __launch_bounds__(256) void transpose_tile_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                             int64_t rows, int64_t cols)
{
    __shared__ __attribute__((aligned(16))) uint32_t tile[128 * 32];  // [k][32 dwords]
    const int64_t tiles_c = (cols + 127) / 128;
    const int64_t k0 = (int64_t)(blockIdx.x / tiles_c) * 128, c0 = (int64_t)(blockIdx.x % tiles_c) * 128;
    const int t = threadIdx.x;
    // all four loads are issued before any is used (a chunk past the matrix edge reads the matrix's first chunk and
    // is zeroed afterwards), so they are in flight together
    u32x4 v[4];
    bool in[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int id = t + i * 256, r = id / 8, ch = id % 8;  // row r, 16-byte chunk ch
        const int64_t k = k0 + r, c = c0 + ch * 16;
        in[i] = k < rows && c < cols;
        v[i] = *(const u32x4*)(src + (in[i] ? k * cols + c : 0));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int id = t + i * 256, r = id / 8, ch = id % 8;
        const int dw = (ch * 4) ^ (((r >> 4) & 3) << 3);
        *(u32x4*)&tile[r * 32 + dw] = in[i] ? v[i] : (u32x4){0u, 0u, 0u, 0u};
    }
    __syncthreads();
    const int lane = t & 63, wave = t >> 6;
    const int kq = lane & 7, cq = (lane >> 3) + 8 * wave;  // 16 k rows (kq), 4 byte columns (cq)
    uint32_t w[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kr = kq * 16 + r;
        w[r] = tile[kr * 32 + (cq ^ (((kr >> 4) & 3) << 3))];
    }
    uint32_t col[4][4];  // col[j][q]: bytes k 4q .. 4q + 3 of byte column 4cq + j
#pragma unroll
    for (int q = 0; q < 4; ++q) tr4x4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3], col[0][q], col[1][q], col[2][q], col[3][q]);
    const int64_t kk = k0 + kq * 16;
    if (kk >= rows) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t c = c0 + cq * 4 + j;
        if (c >= cols) break;
        if constexpr (!FP4) {
            *(u32x4*)(dst + c * rows + kk) = (u32x4){col[j][0], col[j][1], col[j][2], col[j][3]};
        } else {
            uint32_t e[4], o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) split_nibbles(col[j][q], e[q], o[q]);
            const int64_t half = rows / 2;  // output rows are K/2 bytes
            *(u32x2*)(dst + (2 * c) * half + kk / 2) = (u32x2){e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
            *(u32x2*)(dst + (2 * c + 1) * half + kk / 2) = (u32x2){o[0] | (o[1] << 16), o[2] | (o[3] << 16)};
        }
    }
}

// plain int8 transpose for any shape: one thread per output byte
__global__ __launch_bounds__(256) void transpose_i8_plain_kernel(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                                 int64_t rows, int64_t cols)
{
    const int64_t total = rows * cols;
    for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < total; o += (int64_t)gridDim.x * 256) {
        const int64_t c = o / rows, r = o % rows;
        dst[o] = src[r * cols + c];
    }
}

static bool tiled_ok(const void* dst, const void* src, int64_t rows, int64_t cols)
{
    return rows % 16 == 0 && cols % 16 == 0 && (uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0 &&
           rows * cols < (1ll << 40);
}

hipError_t launch_transpose_i8(uint8_t* dst, const uint8_t* src, int64_t rows, int64_t cols, hipStream_t st)
{
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (tiled_ok(dst, src, rows, cols)) {
        const int64_t tiles = ((rows + 127) / 128) * ((cols + 127) / 128);
        if (tiles > 0x7FFFFFFF) return hipErrorInvalidValue;
        hipLaunchKernelGGL(transpose_tile_kernel<false>, dim3((unsigned)tiles), dim3(256), 0, st, dst, src, rows, cols);
        return hipGetLastError();
    }
    log_fallback("transpose_i8_plain_kernel", "rows, columns or pointers not aligned to the 128 x 128 tiles");
    int64_t blocks = (rows * cols + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(transpose_i8_plain_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, src, rows, cols);
    return hipGetLastError();
}

// [K, N] fp4 (two per byte along N) -> [N, K] (two per byte along K); the tiled path needs K % 16 == 0 and
// N % 32 == 0, else the caller uses launch_fp4_transpose's plain kernel.
bool fp4_transpose_tiled(uint8_t* dst, const uint8_t* src, int64_t K, int64_t N, hipStream_t st, hipError_t* err)
{
    if (!tiled_ok(dst, src, K, N / 2) || N % 32 != 0) return false;
    const int64_t tiles = ((K + 127) / 128) * ((N / 2 + 127) / 128);
    if (tiles > 0x7FFFFFFF) return false;
    hipLaunchKernelGGL(transpose_tile_kernel<true>, dim3((unsigned)tiles), dim3(256), 0, st, dst, src, K, N / 2);
    *err = hipGetLastError();
    return true;
}

// int4 (two's complement nibbles, two per byte, even element in the low nibble -- the int4b_t layout of
// examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_int4/scripts/gen_data.py) -> int8, elementwise over
// `bytes` input bytes.  Fast path: 8 input bytes -> 16 output bytes per thread; per byte lane the two's complement
// nibble n becomes offset-binary s = n ^ 8 (value s - 8), and ((s | 0x80) - 8) ^ 0x80 is s - 8 as a byte (the
// subtraction never borrows across bytes); low / high nibbles are then interleaved with v_perm_b32.
__device__ __forceinline__ uint32_t sext_nibbles(uint32_t n)  // four nibbles (one per byte) -> four int8
{
    return (((n ^ 0x08080808u) | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

__global__ __launch_bounds__(256) void unpack_int4_kernel(int8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                          int64_t bytes, bool fast)
{
    if (fast) {
        const int64_t chunks = bytes / 8;
        for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < chunks; i += (int64_t)gridDim.x * 256) {
            const u32x2 w = *(const u32x2*)(src + 8 * i);
            u32x4 o;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t lo = sext_nibbles(w[h] & 0x0F0F0F0Fu), hi = sext_nibbles((w[h] >> 4) & 0x0F0F0F0Fu);
                o[2 * h] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);      // lo.b0 hi.b0 lo.b1 hi.b1
                o[2 * h + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // lo.b2 hi.b2 lo.b3 hi.b3
            }
            *(u32x4*)(dst + 16 * i) = o;
        }
        return;
    }
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < bytes; i += (int64_t)gridDim.x * 256) {
        const uint32_t b = src[i];
        const uint32_t s = sext_nibbles((b & 0xFu) | ((b >> 4) << 8));
        dst[2 * i] = (int8_t)(s & 0xFFu);
        dst[2 * i + 1] = (int8_t)((s >> 8) & 0xFFu);
    }
}

// hifloat8 -> bf16 operand rows for the hifloat8 Matmul: dst [R, ldd] bf16 (ldd a multiple of 8, columns C .. ldd - 1
// written as zero) from src [R, C] (TRANS false) or [C, R] (TRANS true: the [K, M] A of isTransA or the [K, N] B).
// Every HiF8 code is a bf16 value (the finite ones have at most 4 significant bits within 2^-22 .. 2^15, all bf16
// normals; 0x80 is NaN, 0x6F / 0xEF are +-inf): the upper half of hif8_to_f32's bits, looked up in a 256-entry table
// built per workgroup.  TRANS false: a thread writes 8 values (one 16-byte store) of one row; TRANS true: a workgroup
// stages a 64 (c) x 64 (r) byte tile in LDS (loads coalesced along r) and writes 64 rows x 64 values (stores
// coalesced along c).
template <bool TRANS>
__global__ __launch_bounds__(256) void hif8_to_bf16_kernel(uint16_t* __restrict__ dst, int64_t ldd,
                                                          const uint8_t* __restrict__ src, int64_t R, int64_t C)
{
    __shared__ uint16_t lut[256];
    __shared__ uint8_t tile[64][68];
    const int t = threadIdx.x;
    lut[t] = (uint16_t)(__float_as_uint(hif8_to_f32((uint32_t)t)) >> 16);
    __syncthreads();
    if constexpr (!TRANS) {
        const int64_t chunks = ldd / 8, total = R * chunks;
        for (int64_t e = (int64_t)blockIdx.x * 256 + t; e < total; e += (int64_t)gridDim.x * 256) {
            const int64_t r = e / chunks, c0 = (e % chunks) * 8;
            uint32_t h[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = c0 + j < C ? lut[src[r * C + c0 + j]] : 0u;
            *(u32x4*)(dst + r * ldd + c0) = (u32x4){h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                                                    h[6] | (h[7] << 16)};
        }
    } else {
        const int64_t tiles_c = (ldd + 63) / 64;
        const int64_t r0 = (int64_t)(blockIdx.x / tiles_c) * 64, c0 = (int64_t)(blockIdx.x % tiles_c) * 64;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int e = t + 256 * i, cc = e >> 6, rr = e & 63;
            const int64_t c = c0 + cc, r = r0 + rr;
            tile[cc][rr] = (c < C && r < R) ? src[c * R + r] : (uint8_t)0;
        }
        __syncthreads();
        const int rr = t >> 2, q = t & 3;
        const int64_t r = r0 + rr;
        if (r < R) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int cb = 16 * q + 8 * hh;
                if (c0 + cb >= ldd) break;
                uint32_t h[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = lut[tile[cb + j][rr]];
                *(u32x4*)(dst + r * ldd + c0 + cb) = (u32x4){h[0] | (h[1] << 16), h[2] | (h[3] << 16),
                                                             h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
            }
        }
    }
}

hipError_t launch_hif8_to_bf16(uint16_t* dst, int64_t ldd, const uint8_t* src, int64_t R, int64_t C, int transpose,
                              hipStream_t st)
{
    if (R <= 0 || C <= 0) return hipSuccess;
    if (ldd % 8 != 0 || ldd < C || (uintptr_t)dst % 16 != 0) return hipErrorInvalidValue;
    if (transpose) {
        const int64_t tiles = ((R + 63) / 64) * ((ldd + 63) / 64);
        if (tiles > 0x7FFFFFFF) return hipErrorInvalidValue;
        hipLaunchKernelGGL(hif8_to_bf16_kernel<true>, dim3((unsigned)tiles), dim3(256), 0, st, dst, ldd, src, R, C);
    } else {
        int64_t blocks = (R * (ldd / 8) + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(hif8_to_bf16_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st, dst, ldd, src, R, C);
    }
    return hipGetLastError();
}

hipError_t launch_unpack_int4(int8_t* dst, const uint8_t* src, int64_t bytes, hipStream_t st)
{
    if (bytes <= 0) return hipSuccess;
    const bool fast = bytes % 8 == 0 && (uintptr_t)src % 8 == 0 && (uintptr_t)dst % 16 == 0;
    int64_t blocks = ((fast ? bytes / 8 : bytes) + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(unpack_int4_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, src, bytes, fast);
    return hipGetLastError();
}

}  // namespace ascq
