// gemm_core.h -- the LDS-staged MFMA main loop shared by the int8 Matmul, the MoE group matmul and the MX-FP4
// Matmul (gfx950).
//
// MFMA: the 32x32 forms, v_mfma_i32_32x32x32_i8 and v_mfma_scale_f32_32x32x64_f8f6f4 -- on gfx950 they issue at
// the full int8 / fp4 rate, the 16x16 forms at about half of it (measured: 4.80 vs 2.71 int8 POPS, 9.34 vs
// 4.80 fp4 POPS on one MI355X).  Both consume 32 K bytes per row per instruction, 16 bytes per lane: lane l
// holds row l % 32 at K bytes 16 (l / 32) .. +15 of the step.  One stage holds ROWB = 64*KSTEPS bytes of K for
// every tile row of A and B (int8: 64*KSTEPS elements, fp4: 128*KSTEPS), i.e. 2*KSTEPS MFMA k-steps.
// Layout and schedule:
//  * LDS rows are unpadded, ROWB bytes, and 16-byte chunks are XOR-swizzled: logical chunk c of row r lives at
//    chunk c ^ ((r / (256/ROWB)) % CH).  The 16 lanes an MFMA operand read serves together then hit 16
//    distinct 4-bank groups, and a wave's staging write is 1 KiB contiguous.
//  * Global reads are raw buffer loads: an out-of-range offset returns zeros, so tile edges and the K tail
//    need no branches and the whole loop body stays in one basic block for the scheduler.
//  * Two LDS stages; the loads of stage k+1 are issued before the MFMAs of stage k, a scheduling barrier keeps
//    those MFMAs ahead of the LDS store (whose wait on the loads would otherwise stall them), one barrier per
//    stage.
//  * B given row-major [K, N] (int8 only) is transposed on its way into LDS: each lane loads an 8(k) x 4(n)
//    byte block as 8 dwords and v_perm_b32 turns it into 4 K-contiguous 8-byte pieces.
//  * MX: the E8M0 scales of each tile row for the stage's 4*KSTEPS K blocks ride in the same stage
//    (4*KSTEPS bytes per row); a lane reads the byte of its (row, block) -- k-step s, block 2s + l / 32.
//  * Accumulator layout of one 32x32 tile: lane l, register r holds row 8(r/4) + 4(l/32) + r%4, column l%32.
#pragma once

#include <type_traits>

#include "common.h"

namespace ascq {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t OOB = 0x80000000u;  // buffer offset that is always out of range (num_records < 2^31)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
__device__ __forceinline__ u32x2 bload8(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
__device__ __forceinline__ uint32_t bload2(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// 4x4 byte transpose: in r[i] byte j = M[i][j]; out t[j] byte i = M[i][j]
__device__ __forceinline__ void transpose4x4(uint32_t r0, uint32_t r1, uint32_t r2, uint32_t r3, uint32_t& t0,
                                             uint32_t& t1, uint32_t& t2, uint32_t& t3)
{
    const uint32_t lo01 = perm_b32(r1, r0, 0x05010400u);  // r0.b0 r1.b0 r0.b1 r1.b1
    const uint32_t hi01 = perm_b32(r1, r0, 0x07030602u);  // r0.b2 r1.b2 r0.b3 r1.b3
    const uint32_t lo23 = perm_b32(r3, r2, 0x05010400u);
    const uint32_t hi23 = perm_b32(r3, r2, 0x07030602u);
    t0 = perm_b32(lo23, lo01, 0x05040100u);  // r0.b0 r1.b0 r2.b0 r3.b0
    t1 = perm_b32(lo23, lo01, 0x07060302u);
    t2 = perm_b32(hi23, hi01, 0x05040100u);
    t3 = perm_b32(hi23, hi01, 0x07060302u);
}

// XCD-aware tile order: consecutive workgroup ids go to different XCDs; XCD x gets the ids [x*per, (x+1)*per)
// of a grouped (GROUP_M tile rows at a time) raster, so the tiles one XCD runs together share A rows / B cols.
__device__ __forceinline__ void tile_coords(int pid, int tiles_m, int tiles_n, int& tm, int& tn)
{
    const int total = tiles_m * tiles_n;
    if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
    constexpr int GROUP_M = 8;
    const int width = GROUP_M * tiles_n;
    const int first_m = (pid / width) * GROUP_M;
    const int gm = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
    const int in_group = pid % width;
    tm = first_m + in_group % gm;
    tn = in_group / gm;
}

enum { OP_I8 = 0, OP_MXFP4 = 1 };

struct CoreArgs {
    rsrc_t a, b;          // A: rows of lda bytes; B: rows of ldb bytes ([n][k] when K-contiguous, else [k][n])
    uint32_t lda, ldb;    // leading dimensions in bytes
    int32_t rows, cols;   // valid rows of A / columns of B in this tile (from the tile origin)
    uint32_t a0, b0;      // byte offsets of the tile origin in the A / B buffers
    int64_t kbytes;       // K extent in bytes (int8: K; fp4: K/2)
    // MX scales
    rsrc_t sa, sb;
    uint32_t sa0_row, sb0_row;  // first row / column index of the tile
    uint32_t sa_rows, sb_rows;  // M / N (for the pair layouts)
    uint32_t sk;                // scale blocks per row (sK)
    int sa_pairs, sb_pairs;     // 1: [sK/2][R][2] layout; 0: [R][sK]
};

template <int BM, int BN, int WM, int WN, int KSTEPS, bool B_KCONTIG, int OP>
struct GemmCore {
    static constexpr int NT = WM * WN * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr int ROWB = 64 * KSTEPS;
    static constexpr int CH = ROWB / 16;
    static constexpr int RPW = 256 / ROWB;  // rows per 64-bank wrap
    static constexpr int A_LD = BM * CH / NT;
    static constexpr int B_LD = B_KCONTIG ? BN * CH / NT : 1;
    static constexpr int B_BLK = B_KCONTIG ? 1 : (ROWB / 8) * (BN / 4) / NT;
    static constexpr int SCB = OP == OP_MXFP4 ? 4 * KSTEPS : 0;  // scale bytes per row per stage
    static constexpr int SC_LD = OP == OP_MXFP4 ? (BM + BN + NT - 1) / NT : 1;
    static constexpr int STAGE = (BM + BN) * ROWB + (BM + BN) * SCB;
    static constexpr size_t LDS_BYTES = 2 * (size_t)STAGE;
    typedef typename std::conditional<OP == OP_I8, v16i, v16f>::type acc_t;
    static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");

    // position of accumulator register r of tile (i, j) inside the block tile
    __device__ __forceinline__ static int frag_row(int wm, int i, int r, int lane)
    {
        return wm * WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    }
    __device__ __forceinline__ static int frag_col(int wn, int j, int lane) { return wn * WTN + j * 32 + (lane & 31); }
    static_assert((BM * CH) % NT == 0 && A_LD >= 1, "A staging");
    static_assert(B_KCONTIG ? ((BN * CH) % NT == 0 && B_LD >= 1) : (((ROWB / 8) * (BN / 4)) % NT == 0 && B_BLK >= 1),
                  "B staging");
    static_assert(OP == OP_I8 || B_KCONTIG, "fp4 B must be K-contiguous");

    __device__ __forceinline__ static int swz(int row, int c) { return c ^ ((row / RPW) % CH); }

    __device__ __forceinline__ static void run(const CoreArgs& p, uint8_t* smem, acc_t (&acc)[FM][FN])
    {
        const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
        const int wm = wave / WN, wn = wave % WN;

        u32x4 ra[A_LD];
        u32x4 rb[B_LD];
        uint32_t rbt[B_BLK][8];
        u32x2 rs[SC_LD];

        auto load_global = [&](int64_t kt) {
            const int64_t kb0 = kt * ROWB;
#pragma unroll
            for (int i = 0; i < A_LD; ++i) {
                const int id = t + i * NT, row = id / CH, c = id % CH;
                const int64_t k = kb0 + c * 16;
                const uint32_t off = (row < p.rows && k < p.kbytes) ? p.a0 + (uint32_t)row * p.lda + (uint32_t)k : OOB;
                ra[i] = bload16(p.a, off);
            }
            if constexpr (B_KCONTIG) {
#pragma unroll
                for (int i = 0; i < B_LD; ++i) {
                    const int id = t + i * NT, row = id / CH, c = id % CH;
                    const int64_t k = kb0 + c * 16;
                    const uint32_t off =
                        (row < p.cols && k < p.kbytes) ? p.b0 + (uint32_t)row * p.ldb + (uint32_t)k : OOB;
                    rb[i] = bload16(p.b, off);
                }
            } else {
#pragma unroll
                for (int i = 0; i < B_BLK; ++i) {
                    const int id = t + i * NT, nb = id % (BN / 4), kb = id / (BN / 4);
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        const int64_t k = kb0 + kb * 8 + r;
                        const uint32_t off =
                            (nb * 4 < p.cols && k < p.kbytes) ? p.b0 + (uint32_t)k * p.ldb + (uint32_t)(nb * 4) : OOB;
                        rbt[i][r] = bload4(p.b, off);
                    }
                }
            }
            if constexpr (OP == OP_MXFP4) {
                const uint32_t blk0 = (uint32_t)(kt * 4 * KSTEPS);
#pragma unroll
                for (int i = 0; i < SC_LD; ++i) {
                    const int r = t + i * NT;
                    u32x2 v = (u32x2){0x7f7f7f7fu, 0x7f7f7f7fu};
                    const bool is_a = r < BM;
                    const bool valid = is_a ? (r < p.rows) : (r < BM + BN && (r - BM) < p.cols);
                    const rsrc_t sr = is_a ? p.sa : p.sb;
                    const int pairs = is_a ? p.sa_pairs : p.sb_pairs;
                    const uint32_t idx = is_a ? p.sa0_row + r : p.sb0_row + (r - BM);
                    const uint32_t R = is_a ? p.sa_rows : p.sb_rows;
                    if (valid && blk0 < p.sk) {
                        if (!pairs) {
                            if constexpr (KSTEPS == 2) v = bload8(sr, idx * p.sk + blk0);
                            else v.x = bload4(sr, idx * p.sk + blk0);
                        } else {
                            uint32_t w[2 * KSTEPS];
#pragma unroll
                            for (int q = 0; q < 2 * KSTEPS; ++q) w[q] = bload2(sr, ((blk0 >> 1) + q) * R * 2 + idx * 2);
                            v.x = (w[0] & 0xffffu) | (w[1] << 16);
                            if constexpr (KSTEPS == 2) v.y = (w[2] & 0xffffu) | (w[3] << 16);
                        }
                    }
                    rs[i] = v;
                }
            }
        };

        auto store_lds = [&](int buf) {
            uint8_t* sA = smem + buf * STAGE;
            uint8_t* sB = sA + BM * ROWB;
#pragma unroll
            for (int i = 0; i < A_LD; ++i) {
                const int id = t + i * NT, row = id / CH, c = id % CH;
                *(u32x4*)(sA + row * ROWB + swz(row, c) * 16) = ra[i];
            }
            if constexpr (B_KCONTIG) {
#pragma unroll
                for (int i = 0; i < B_LD; ++i) {
                    const int id = t + i * NT, row = id / CH, c = id % CH;
                    *(u32x4*)(sB + row * ROWB + swz(row, c) * 16) = rb[i];
                }
            } else {
#pragma unroll
                for (int i = 0; i < B_BLK; ++i) {
                    const int id = t + i * NT, nb = id % (BN / 4), kb = id / (BN / 4);
                    uint32_t lo[4], hi[4];
                    transpose4x4(rbt[i][0], rbt[i][1], rbt[i][2], rbt[i][3], lo[0], lo[1], lo[2], lo[3]);
                    transpose4x4(rbt[i][4], rbt[i][5], rbt[i][6], rbt[i][7], hi[0], hi[1], hi[2], hi[3]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int n = nb * 4 + j;
                        *(u32x2*)(sB + n * ROWB + swz(n, kb >> 1) * 16 + (kb & 1) * 8) = (u32x2){lo[j], hi[j]};
                    }
                }
            }
            if constexpr (OP == OP_MXFP4) {
                uint8_t* sS = sA + (BM + BN) * ROWB;
#pragma unroll
                for (int i = 0; i < SC_LD; ++i) {
                    const int r = t + i * NT;
                    if (r < BM + BN) {
                        if constexpr (KSTEPS == 2) *(u32x2*)(sS + r * SCB) = rs[i];
                        else *(uint32_t*)(sS + r * SCB) = rs[i].x;
                    }
                }
            }
        };

#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = (acc_t){};

        const int r32 = lane & 31, kh = lane >> 5;
        const int64_t nk = (p.kbytes + ROWB - 1) / ROWB;
        load_global(0);
        store_lds(0);
        __syncthreads();
        for (int64_t kt = 0; kt < nk; ++kt) {
            const int buf = (int)(kt & 1);
            load_global(kt + 1);  // past the end every offset is out of range: zeros, no memory traffic
            const uint8_t* sA = smem + buf * STAGE;
            const uint8_t* sB = sA + BM * ROWB;
#pragma unroll
            for (int s = 0; s < 2 * KSTEPS; ++s) {
                const int c = s * 2 + kh;  // 16-byte chunk of this lane for k-step s (= MX block index)
                int sa[FM], sb[FN];
                if constexpr (OP == OP_MXFP4) {
                    const uint8_t* sS = sA + (BM + BN) * ROWB;
#pragma unroll
                    for (int i = 0; i < FM; ++i) sa[i] = sS[(wm * WTM + i * 32 + r32) * SCB + c];
#pragma unroll
                    for (int j = 0; j < FN; ++j) sb[j] = sS[(BM + wn * WTN + j * 32 + r32) * SCB + c];
                }
                v4i fa[FM];
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    const int row = wm * WTM + i * 32 + r32;
                    fa[i] = *(const v4i*)(sA + row * ROWB + swz(row, c) * 16);
                }
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int row = wn * WTN + j * 32 + r32;
                    const v4i fb = *(const v4i*)(sB + row * ROWB + swz(row, c) * 16);
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        if constexpr (OP == OP_I8) {
                            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb, acc[i][j], 0, 0, 0);
                        } else {
                            const v8i a8 = (v8i){fa[i][0], fa[i][1], fa[i][2], fa[i][3], 0, 0, 0, 0};
                            const v8i b8 = (v8i){fb[0], fb[1], fb[2], fb[3], 0, 0, 0, 0};
                            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[i][j], 4, 4, 0,
                                                                                         sa[i], 0, sb[j]);
                        }
                    }
                }
            }
            // keep this stage's MFMAs ahead of the LDS store, whose wait on the loads would otherwise stall them
            __builtin_amdgcn_sched_barrier(0);
            store_lds(buf ^ 1);
            __syncthreads();
        }
    }
};

}  // namespace ascq
