// launch.h -- host-side launchers of the gfx950 kernels (called by api.cpp after argument validation).
// Every launcher enqueues on `st` and returns the launch status; none allocates device memory
// unless its comment says so.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace ascq {

// IterateAll's enAtomic (impl/adv_api/detail/matmul/utils/matmul_config_utils.h:53-55, applied to the copy-out by
// scheduler/base/scheduler_base.h:484-494): 0 stores C; 1 / 2 / 3 combine C = add / max / min (C, v) in C's type,
// one atomic read-modify-write per element (c_atomic), so concurrent IterateAll calls into the same C compose.
enum : int { C_STORE = 0, C_ADD = 1, C_MAX = 2, C_MIN = 3 };

// A launcher took a generic kernel (one thread per output element, or an element-wise kernel without vector loads)
// instead of a tiled / vectorised one: with the environment variable ASCQ_LOG set to 1 or more, one line on stderr
// names the kernel and the reason (api.cpp).
void log_fallback(const char* kernel, const char* reason);

// Raises the dynamic-LDS limit of kernel K to `bytes` once per device (the attribute belongs to the function on
// the current device), thread-safe; K is the kernel itself, so each instantiation keeps its own record.
template <auto K>
inline hipError_t ensure_dynamic_lds(int bytes)
{
    static std::mutex mu;
    static uint64_t done = 0;  // bit d: set on device d (devices 64 and up are set on every call)
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    if (dev < 64 && ((done >> dev) & 1u)) return hipSuccess;
    e = hipFuncSetAttribute((const void*)K, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess && dev < 64) done |= 1ull << dev;
    return e;
}

// One-shot kernel timing hook (ascq_set_launch_events): the next launch_k on this thread records the two events
// at its dispatch's start and end -- hipExtLaunchKernelGGL binds them to the dispatch itself, so no marker packet
// lands between kernels -- and clears them; without events launch_k is a plain launch.  Compute kernels go through
// launch_k, helper kernels (layout transposes, scale rearrangement) do not, so an entry point's events time its
// main kernel.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents& launch_events();  // thread-local; api.cpp

template <typename F, typename... Args>
inline void launch_k(F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t st, Args... args)
{
    LaunchEvents& e = launch_events();
    const hipEvent_t a = e.start, b = e.stop;
    e = LaunchEvents{};
    hipExtLaunchKernelGGL(kernel, grid, block, shm, st, a, b, 0u, args...);  // callers check hipGetLastError()
}

// quant.hip
hipError_t launch_quant_dynamic_per_token(int8_t* q, float* scale_out, const void* x, int src_type, uint32_t m,
                                          uint32_t n, int round_mode, hipStream_t st);
// legacy AscendQuant, arch-3510 form: dst int8 / hifloat8 / fp8; src f16 / bf16 / f32; srcT scale / offset tensors
// of scale_count (scale null: the scalars; offset null with a scale tensor: the scalar offset as a srcT value)
hipError_t launch_quant_legacy(void* q, int dst_type, const void* x, int src_type, const void* scale,
                               const void* offset, float scale_scalar, float offset_scalar, uint32_t cal_count,
                               uint32_t scale_count, hipStream_t st);
// AscendDequant, both forms: rows x cols computed elements at source row stride n and destination row stride ldd;
// smode picks the scale addressing (quant.hip DQ_*: scalar, per column, per row, per group along the row with
// `group` columns, per group down the columns with `group` rows)
hipError_t launch_dequant(void* y, int dst_type, const void* src, int src_type, const void* scale, int scale_type,
                          float scale_scalar, int smode, uint32_t rows, uint32_t cols, uint32_t n, uint32_t ldd,
                          uint32_t group, hipStream_t st);
// f32_arith: int8 / hifloat8 sources in fp32 whatever the scale type (the AntiQuantize form)
hipError_t launch_antiquant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale,
                                   const void* offset, int scale_type, int per_token, int64_t m, int64_t n,
                                   int64_t g, int col_groups, int is_transpose, hipStream_t st, int f32_arith = 0);
hipError_t launch_antiquant(void* dst, int dst_type, const void* src, int src_type, const void* offset,
                            const void* scale, uint32_t K, uint32_t N, uint32_t g, int is_transpose, int arith,
                            hipStream_t st);
// AscendAntiQuant per tensor: dst[i] = (src[i] + offset) * scale with offset / scale the output type's bits
// f32_arith: fp32 arithmetic and one cast whatever the types (the AntiQuantize form)
hipError_t launch_antiquant_scalar(void* dst, int dst_type, const void* src, int src_type, uint16_t offset,
                                   uint16_t scale, int has_offset, int64_t count, hipStream_t st, int f32_arith = 0);
// AscendQuant policy form; scale == null takes scale_scalar for every element (per_token layout, the Quantize
// form's PER_TENSOR); f32_arith: fp32 arithmetic whatever the scale type (the Quantize form)
hipError_t launch_quant_policy(void* dst, int dst_type, const void* src, int src_type, const void* scale,
                               int scale_type, const void* offset, int has_offset, float offset_scalar, int per_token,
                               int64_t m, int64_t n, int64_t g, int k_dim, int round_mode, hipStream_t st,
                               float scale_scalar = 0.0f, int f32_arith = 0);

// gemm_i8.hip
enum : int { EPI_I32 = 0, EPI_DEQ_F16 = 1, EPI_DEQ_BF16 = 2, EPI_REQ8 = 3, EPI_REQ4 = 4 };
struct GemmI8Args {
    const int8_t* A;      // [M, K] row-major (lda), or [K, M] when trans_a
    const int8_t* B;      // [K, N] row-major (ldb), or [N, K] when trans_b
    const int32_t* bias;  // [N] or null
    void* C;              // [M, N] row-major (ldc)
    int64_t M, N, K, lda, ldb, ldc;
    const uint64_t* qvec; // per-channel QUANT_PRE words [N] or null
    uint64_t qscalar;
    int epi;              // EPI_*
    int trans_a, trans_b;
    int atomic;           // C_STORE, or C_ADD / C_MAX / C_MIN (int32 / f16 / bf16 C): IterateAll's enAtomic
    uint8_t* ws;          // decode-sized batches: room for the K-split partials (decode_split_ws_bytes), or null
    size_t ws_bytes;
    int splits;           // (set by the launcher) workgroups per tile of the K-split form
};
hipError_t launch_gemm_i8(const GemmI8Args& a, hipStream_t st);
// Decode-sized batches (M <= 64: one row tile of 32 or 64 rows; K % 256 == 0) -- B given [K, N] (trans_b 0) with long
// K or wide N on x 128 tiles, B given [N, K] with long K and few x 32 tiles -- split each tile's K over several
// workgroups (four waves each) so that about 256 workgroups stream B; their accumulators meet in the workspace and a
// second launch adds them in split order and runs the epilogue.
// decode_splits gives the workgroups per tile (1: the form is not used) and decode_split_ws_bytes the workspace the
// partials need.
int decode_splits(int64_t M, int64_t N, int64_t K, int trans_b);
size_t decode_split_ws_bytes(int64_t M, int64_t N, int64_t K, int trans_b);

// gemm_f8.hip
constexpr int FMT_BF16 = 7;  // operand format code outside the f8f6f4 codes: bf16 elements (OP_BF16)
struct GemmF8Args {
    const uint8_t* A;     // fp8 [M, K] row-major (lda), or [K, M] when trans_a
    const uint8_t* B;     // fp8 [K, N] row-major (ldb), or [N, K] when trans_b
    const float* bias;    // [N] or null
    void* C;              // [M, N] row-major (ldc)
    int64_t M, N, K, lda, ldb, ldc;
    const uint64_t* qvec; // per-channel QUANT_PRE words [N] or null
    uint64_t qscalar;
    int use_quant;        // 1: multiply by M1 (SetQuantScalar / SetQuantVector was called)
    int c_type;           // DT_F16 / DT_BF16 / DT_F32; DT_INT8 / DT_UINT8 (QF322B8); DT_FP8_E4M3 / _E5M2 (QF322FP8);
                          // DT_HIF8 (QF322HIF8); DT_INT4 (QF322S4)
    int fmt_a, fmt_b;     // f8f6f4 codes: 0 e4m3fn, 1 e5m2; FMT_BF16 in both: A / B are bf16 (a hifloat8 Matmul's
                          // operands decoded by the host layer; A [M, K] and B [N, K], K-contiguous, lda / ldb in
                          // elements)
    int trans_a, trans_b;
    int atomic;           // C_STORE, or C_ADD / C_MAX / C_MIN (f32 / f16 / bf16 C): IterateAll's enAtomic
    uint8_t* ws;          // decode-sized batches: room for the K-split partials (decode_split_ws_bytes), or null
    size_t ws_bytes;
    int splits;           // (set by the launcher) workgroups per tile of the K-split form
};
hipError_t launch_gemm_f8(const GemmF8Args& a, hipStream_t st);

// group_gemm.hip
struct GroupGemmArgs {
    void* Y;
    int out_type;             // DT_BF16 / DT_F16
    const int8_t* X;          // [M, K]
    const float* pts;         // [M]
    const int8_t* W;          // [G, K, N] or [G, N, K]
    int w_trans;
    const float* scale;       // [G, N]
    const int64_t* group_list;
    int list_type;            // 0 prefix offsets [G+1], 1 counts [G]
    int64_t G, M, K, N;
    int act;                  // 0 none, 1 FasterGelu
};
hipError_t launch_group_gemm(const GroupGemmArgs& a, hipStream_t st);

// gemv_antiquant.hip
size_t weight_pack_bytes(int w_type, int64_t K, int64_t N);
hipError_t launch_weight_pack(void* packed, const void* w, int w_type, int64_t K, int64_t N, int is_transpose,
                              hipStream_t st);
hipError_t launch_antiquant_matmul(uint16_t* y, const uint16_t* x, const void* wp, int w_type, const uint16_t* scale,
                                   const uint16_t* offset, int64_t group, int64_t M, int64_t N, int64_t K,
                                   int atomic, hipStream_t st);

// aq_gemm.hip: the weight-only antiquant matmul for M > 64 (an LDS-staged f16 GEMM whose weight tiles are dequantised
// once per 256 rows); hipErrorInvalidValue for shapes it does not take (K % 128, N % 16, group not 128 << s, buffers
// of 2^31 bytes)
hipError_t launch_aq_gemm(uint16_t* y, const uint16_t* x, const void* wp, int w_type, const uint16_t* scale,
                          const uint16_t* offset, int64_t group, int64_t M, int64_t N, int64_t K, int atomic,
                          hipStream_t st);

// mx_gemm.hip
struct MxGemmArgs {
    const uint8_t* A;       // [M, K/2] packed E2M1, or [M, K] fp8
    const uint8_t* B;       // [N, K/2] packed, or [N, K] fp8 (after any transpose)
    const uint8_t* sA;      // scales as given: [M, sK] (sa_layout 0) or [sK/2, M, 2] (1)
    const uint8_t* sB;      // [sK/2, N, 2] (sb_layout 0) or [N, sK] (1)
    int sa_layout, sb_layout;
    uint8_t* ws_scales;     // mx_scale_workspace_bytes(M, N, K) bytes: the stage-major copies of both
    int64_t M, N, K;
    void* C;                // [M, N]
    int c_type;             // DT_BF16 / DT_F32
    int fmt_a, fmt_b;       // f8f6f4 codes of the elements: 4 E2M1 (both), or fp8 0 e4m3fn / 1 e5m2 (any mix)
    const float* bias;      // [N] f32, added to the fp32 sums before the output cast, or null
    int atomic;             // C_STORE, or C_ADD / C_MAX / C_MIN: IterateAll's enAtomic
    // fp6 E2M3 (fmt 2, both operands): A / B are the P planes and Aq / Bq the Q planes written by
    // launch_fp4_to_fp6_planes
    const uint8_t* Aq;
    const uint8_t* Bq;
    uint8_t* ws_part;       // decode-sized MX-FP4 batches: room for the K-split partials (mx_decode_split_ws_bytes)
    size_t ws_part_bytes;
    int splits;             // (set by the launcher) workgroups per tile of the K-split form
};
hipError_t launch_mx_gemm(const MxGemmArgs& a, hipStream_t st);
// MX-FP4 at decode-sized batches (M <= 64) with the scales read in place: with few 64 x 64 tiles (N / 64 well under
// 256) K is split across workgroups as well, the partials meeting in the workspace; the workgroups per tile (1: not
// used) and the workspace the partials need
int mx_decode_splits(int64_t M, int64_t N, int64_t K);
size_t mx_decode_split_ws_bytes(int64_t M, int64_t N, int64_t K);
// fp4 (E2M1 or E1M2) [R, K/2] -> fp6 E2M3 split planes: P [R, K/2] (dwords 0-3 of each MX block's six) and Q
// (fp6_q_plane_bytes(R, K): dwords 4-5, 1 KiB per (128 K, 32-row group)); K a multiple of 128
size_t fp6_q_plane_bytes(int64_t R, int64_t K);
hipError_t launch_fp4_to_fp6_planes(uint8_t* P, uint8_t* Q, const uint8_t* src, int64_t R, int64_t K, bool e1m2,
                                    hipStream_t st);
// transpose.hip: int8 [rows, cols] -> [cols, rows]; fp4 [K, N] -> [N, K] tiled fast path (returns false when
// the shape / alignment does not allow it)
hipError_t launch_transpose_i8(uint8_t* dst, const uint8_t* src, int64_t rows, int64_t cols, hipStream_t st);
bool fp4_transpose_tiled(uint8_t* dst, const uint8_t* src, int64_t K, int64_t N, hipStream_t st, hipError_t* err);
size_t mx_scale_workspace_bytes(int64_t M, int64_t N, int64_t K);
// layout.hip: NZ fractal ([ceil(cols*esize/32)][ceil(rows/16)][16][32 bytes]) <-> ND, per matrix of a batch
size_t nz_bytes(int64_t batch, int64_t rows, int64_t cols, int esize);
hipError_t launch_nz_to_nd(void* dst, const void* src, int esize, int64_t batch, int64_t rows, int64_t cols,
                           int transpose_out, hipStream_t st);
hipError_t launch_nd_to_nz(void* dst, const void* src, int esize, int64_t batch, int64_t rows, int64_t cols,
                           hipStream_t st);
// hifloat8 -> bf16 (exact): dst [R, ldd] bf16 (ldd % 8 == 0, columns C .. ldd - 1 zero, dst 16-byte aligned) from
// src [R, C], or from src [C, R] with transpose
hipError_t launch_hif8_to_bf16(uint16_t* dst, int64_t ldd, const uint8_t* src, int64_t R, int64_t C, int transpose,
                              hipStream_t st);
// int4 (two per byte, even element in the low nibble) -> int8, elementwise over `bytes` input bytes
hipError_t launch_unpack_int4(int8_t* dst, const uint8_t* src, int64_t bytes, hipStream_t st);
// transpose a [K, N] packed fp4 matrix (two per byte along N) into [N, K] (two per byte along K)
hipError_t launch_fp4_transpose(uint8_t* dst, const uint8_t* src, int64_t K, int64_t N, hipStream_t st);

}  // namespace ascq
