// gemm_core.h -- the LDS-staged MFMA main loop shared by the int8 and fp8 Matmuls, the MoE group matmul and
// the MX (FP4 / FP8 element) Matmuls (gfx950).
//
// MFMA: the 32x32 forms, v_mfma_i32_32x32x32_i8 and v_mfma_[scale_]f32_32x32x64_f8f6f4 -- on gfx950 they issue
// at the full int8 / fp8 / fp4 rate, the 16x16 forms at about half of it (measured: 4.80 vs 2.71 int8 POPS,
// 9.34 vs 4.80 fp4 POPS on one MI355X).  A k-step (one instruction) covers 32 int8, 64 fp4 or 64 fp8 of K per
// row: 32, 32 or 64 bytes.  Lane l holds row l % 32.  int8 / fp4: 16 bytes, the K half l / 32 of the step (fp4:
// 32 elements, one MX block).  fp8: 32 bytes in two register quads; the instruction's K order is [quad 0 of
// lanes 0-31, quad 0 of lanes 32-63, quad 1 of lanes 0-31, quad 1 of lanes 32-63], so lane l takes K bytes
// 16 (l / 32) .. +15 into quad 0 and 32 + 16 (l / 32) .. +15 into quad 1, and MX block b (K 32 b .. 32 b + 31)
// is quad b of every lane, its scale supplied by lanes 32 b .. 32 b + 31 (measured with one nonzero K per row
// and different block scales).
// One stage holds ROWB (64 or 128) bytes of K for every tile row of A and B, i.e. ROWB / 32 (int8, fp4) or
// ROWB / 64 (fp8) k-steps.  With ROWB = 128 every copied row is one whole 128-byte cache line, which halves
// the L2 requests per byte.
//
// Pipeline: a ring of STAGES LDS stages.  K-contiguous operands are copied global -> LDS by buffer loads with
// the LDS destination (buffer_load_dwordx4 ... lds): no registers are involved, so STAGES - 1 stages are in
// flight while one is multiplied.  Per iteration each wave waits (s_waitcnt vmcnt) for its own copies of the
// current stage, one barrier publishes them to all waves and frees the stage multiplied last iteration, and
// the copies of the stage STAGES - 1 ahead are issued into that freed slot, a few before each k-step of the
// iteration (so they interleave with the MFMAs instead of stalling the wave in one burst).  Every wave
// issues the same number of copies every iteration (out-of-range copies read zeros), so the vmcnt threshold is
// a compile-time constant.
//
// Layout:
//  * LDS rows are unpadded, ROWB bytes, and 16-byte chunks are XOR-swizzled: logical chunk c of row r lives at
//    chunk c ^ ((r / (256 / ROWB)) % (ROWB / 16)).  The 16 lanes an MFMA operand read serves together then hit
//    16 distinct 4-bank groups.  A copy instruction writes 1 KiB contiguous (lane l -> row l / (ROWB / 16),
//    chunk l % (ROWB / 16)); the swizzle is applied on the global side.
//  * Global reads are raw buffer loads: an out-of-range offset returns zeros, so tile edges and the K tail
//    need no branches.
//  * B given row-major [K, N] (int8 only) goes through registers instead: each lane loads an 8(k) x 4(n) byte
//    block as 8 dwords, v_perm_b32 turns it into 4 K-contiguous 8-byte pieces, and they are written one
//    iteration after they were loaded (two iterations of latency cover; the registers are double-buffered).
//    The row written by store j of a lane is rotated by (n-block / 4) so the 64 lanes of a store spread over
//    the LDS banks.
//  * MX: the E8M0 scales arrive stage-major ([sK/SCB][rows][SCB], SCB = scale bytes per row per stage: ROWB / 16
//    for fp4, ROWB / 32 for fp8), so a stage's scales for 1024 / SCB tile rows are one contiguous 1 KiB copy
//    into the stage.
//    (Row-major scales would cost one cache line per row per stage.)  A lane reads the scale words of its
//    fragment row per pair of k-steps (a 16-bit pair when a stage holds a single fp8 k-step), shifts them by
//    8 * (l / 32), and the MFMA's op_sel picks the byte of block 2s + l / 32 for k-step s.
//  * fp8 without block scales uses the same instruction with zero scale operands, which the compiler emits as
//    the unscaled v_mfma_f32_32x32x64_f8f6f4.
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

// Output tile of an epilogue: a buffer resource whose range ends after the tile's last valid row, so stores of
// rows past the matrix are dropped by the hardware range check, and 32-bit offsets inside the tile (row pitch
// ldc elements of esize bytes; the caller keeps rows * ldc * esize below 2^31).  Columns past the matrix are
// given the out-of-range offset by the caller.
struct TileOut {
    rsrc_t r;
    uint32_t pitch;  // bytes per row
    uint8_t* base;   // the same range as a plain pointer (the enAtomic read-modify-write path)
    uint32_t bytes;
};
__device__ __forceinline__ TileOut tile_out(void* C, int64_t m0, int64_t n0, int64_t ldc, int rows, int cols, int esize)
{
    TileOut t;
    t.base = (uint8_t*)C + (m0 * ldc + n0) * esize;
    t.bytes = (uint32_t)(((int64_t)(rows - 1) * ldc + cols) * esize);
    t.r = make_rsrc(t.base, t.bytes);
    t.pitch = (uint32_t)(ldc * esize);
    return t;
}

// int4 output tile (two codes per byte, even column in the low nibble; ldc even): byte pitch ldc / 2
__device__ __forceinline__ TileOut tile_out_int4(void* C, int64_t m0, int64_t n0, int64_t ldc, int rows, int cols)
{
    TileOut t;
    t.base = (uint8_t*)C + (m0 * ldc + n0) / 2;
    t.bytes = (uint32_t)((int64_t)(rows - 1) * (ldc / 2) + (cols + 1) / 2);
    t.r = make_rsrc(t.base, t.bytes);
    t.pitch = (uint32_t)(ldc / 2);
    return t;
}

// Packs the int4 codes of a 32-column accumulator fragment: lanes 2t and 2t + 1 hold columns 2t and 2t + 1 of the
// same rows, so the even lane stores (own | neighbour << 4); odd lanes, and columns past the tile, store nothing.
// Every lane must call it (the neighbour's code comes through a cross-lane move).
__device__ __forceinline__ void store_int4_pair(const TileOut& o, uint32_t q, int cl, int cols, int lane,
                                                uint32_t row_off)
{
    const uint32_t nb = (uint32_t)__shfl_xor((int)q, 1, 64);
    const uint32_t hi = cl + 1 < cols ? (nb & 0xFu) : 0u;
    const uint32_t off = ((lane & 1) == 0 && cl < cols) ? (uint32_t)(cl >> 1) + row_off : OOB;
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)((q & 0xFu) | (hi << 4)), o.r, off, 0, 0);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// 16 bytes per lane, global (buffer) -> LDS at lds_wave_base + 16 * lane; lds_wave_base must be wave-uniform.
__device__ __forceinline__ void copy16_to_lds(rsrc_t r, uint8_t* lds_wave_base, uint32_t off)
{
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_wave_base, 16, off, 0, 0, 0);
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding: vmcnt[3:0] | expcnt << 4 |
// lgkmcnt << 8 | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// workgroup barrier that the compiler may not move memory accesses across (no hardware fence: the waits are
// explicit)
__device__ __forceinline__ void stage_barrier()
{
    __builtin_amdgcn_sched_barrier(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_sched_barrier(0);
}

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

// operand kinds: int8; MX block-scaled E2M1; fp8 (per-tensor / per-channel dequant in the epilogue); MX
// block-scaled fp8; MX block-scaled fp6 E2M3 in split planes (the E1M2 / mixed fp4 path); bf16 (the hifloat8
// Matmul, whose operands are decoded exactly to bf16 first: v_mfma_f32_32x32x16_bf16, 16 K = 32 bytes per row per
// k-step, a lane holding 8 bf16 of row l % 32 at K 8 (l / 32) .. + 7 -- the int8 fragment's bytes)
enum { OP_I8 = 0, OP_MXFP4 = 1, OP_F8 = 2, OP_MXF8 = 3, OP_MXFP6 = 4, OP_BF16 = 5 };

// f8f6f4 format codes (the MFMA's cbsz / blgp fields)
enum { F8F6F4_E4M3 = 0, F8F6F4_E5M2 = 1, F8F6F4_E2M3 = 2, F8F6F4_E2M1 = 4 };

struct CoreArgs {
    rsrc_t a, b;          // A: rows of lda bytes; B: rows of ldb bytes ([n][k] when K-contiguous, else [k][n])
    uint32_t lda, ldb;    // leading dimensions in bytes
    int32_t rows, cols;   // valid rows of A / columns of B in this tile (from the tile origin)
    uint32_t a0, b0;      // byte offsets of the tile origin in the A / B buffers
    int64_t kbytes;       // K extent in bytes (int8, fp8: K; fp4: K/2); a multiple of 16
    // MX auxiliary data, all read through the one resource `aux` (so a copy's source differs between waves only in
    // its offset, and the copy code needs no branches): the stage-major scales -- the SCB bytes of (stage s, row r)
    // = blocks SCB s .. SCB s + SCB - 1 of row r, at byte sa_base + (s * rows + r) * SCB for A, sb_base + ... for
    // B -- and, for fp6, the Q planes
    rsrc_t aux;
    // SC_DIRECT cores: aux is the A scales as given, row-major [rows, sk] (sk bytes a row), and aux_b the B scales as
    // given: row-major too (SC_DIRECT 1) or in block pairs [sk / 2, sb_rows, 2] (SC_DIRECT 2)
    rsrc_t aux_b;
    uint32_t sa_base, sb_base;  // byte offsets of the A / B stage-major scales in aux
    uint32_t sa0_row, sb0_row;  // first row / column index of the tile
    uint32_t sa_rows, sb_rows;  // M / N: the stage stride in rows
    uint32_t sk;                // scale blocks per row (sK, a multiple of SCB)
    // fp6 Q planes (OP_MXFP6) in aux: byte offset of the tile's first 32-row group in stage 0, and the stage stride
    // (1 KiB x groups)
    uint32_t qa_off, qa_stride, qb_off, qb_stride;
};

// FMT (fp8 ops): f8f6f4 format code of A in bits 0-2 and of B in bits 3-5
// CT (int8 only): the MFMA takes the B fragment as its first operand and the A fragment as its second, so each
// 32 x 32 accumulator holds the transposed block: lane l, register r = 4 q + e holds row (l % 32) and column
// 8 q + 4 (l / 32) + e -- four consecutive columns of one row per register quad, which an epilogue stores as one
// vector (no LDS round trip); ct_row / ct_col give the coordinates.
// SC_DIRECT (MX, 4 scale bytes per row per stage): the E8M0 scales are read where the caller left them instead of
// from a stage-major copy.  A row-major scale tensor [rows, sK] (A always; B when SC_DIRECT == 1): each stage, one
// copy per 64 tile rows moves the stage's 4 bytes of 64 consecutive rows (one 4-byte LDS-DMA load per lane, lane =
// row) into the same [row][4] region the stage-major copies fill.  B in block pairs [sK / 2, N, 2] (SC_DIRECT == 2):
// a stage's two pairs of a row lie in two planes, each 2 bytes a row and contiguous over rows, so one copy moves 128
// rows of one plane (4 bytes = two rows per lane) into a [plane][row] u16 region, and the scale word of a row is its
// two plane entries.
template <int BM, int BN, int WM, int WN, int STAGES, bool B_KCONTIG, int OP, int ROWB_ = 64, int FMT = 0, bool ILV = true,
          bool CT = false, bool B_TR = false, int SC_DIRECT = 0>
struct GemmCore {
    static constexpr bool IS_MX = OP == OP_MXFP4 || OP == OP_MXF8 || OP == OP_MXFP6;
    static constexpr bool IS_F8 = OP == OP_F8 || OP == OP_MXF8;
    static constexpr bool IS_FP6 = OP == OP_MXFP6;
    static_assert(!CT || OP == OP_I8, "transposed accumulators: int8 only");
    static constexpr int CBSZ = OP == OP_MXFP4 ? F8F6F4_E2M1 : (IS_FP6 ? F8F6F4_E2M3 : (FMT & 7));
    static constexpr int BLGP = OP == OP_MXFP4 ? F8F6F4_E2M1 : (IS_FP6 ? F8F6F4_E2M3 : ((FMT >> 3) & 7));
    static constexpr int TBM = BM, TBN = BN, TWN = WN;  // the tile shape, for code outside the template
    static constexpr int NW = WM * WN;
    static constexpr int NT = NW * 64;
    static constexpr int WTM = BM / WM, WTN = BN / WN;
    static constexpr int FM = WTM / 32, FN = WTN / 32;
    static constexpr int ROWB = ROWB_;                // K bytes per row per stage (64 or 128)
    static constexpr int CH = ROWB / 16;              // 16-byte chunks per row
    static constexpr int RPW = 256 / ROWB;            // rows per 256-byte bank window
    static constexpr int ROWS_PER_COPY = 64 / CH;     // rows one wave-wide 1 KiB copy covers
    static constexpr int A_COPIES = BM / ROWS_PER_COPY / NW;              // per wave per stage
    // B_TR (int8, B given [K, N]): B's K rows are copied like A's (16-byte DMA chunks, BN bytes a row, 1 KiB a copy)
    // into a [ROWB][BN] region and each fragment is read with two ds_read_b64_tr_b8 (below)
    static constexpr int B_COPIES = B_KCONTIG ? BN / ROWS_PER_COPY / NW : (B_TR ? ROWB * BN / 1024 / NW : 0);
    static constexpr int CHB = BN / 16;                  // B_TR: 16-byte chunks per K row
    static constexpr int RWB = CHB >= 16 ? 1 : 16 / CHB;  // B_TR: K rows per 256-byte bank window
    static constexpr int KSB = IS_F8 ? 64 : 32;       // K bytes per row per k-step
    static constexpr int LCH = KSB / 32;              // 16-byte chunks per lane per k-step
    static constexpr int KPS = ROWB / KSB;            // k-steps per stage
    static constexpr int NH = KPS >= 2 ? KPS / 2 : 1; // pairs of k-steps per stage (one MX scale word each)
    static constexpr int SPH = KPS >= 2 ? 2 : 1;      // k-steps per pair
    static constexpr int SCB = ROWB / (IS_F8 ? 32 : 16);  // MX scale bytes per row per stage (blocks of 32)
    static constexpr int SC_ROWS = 1024 / SCB;        // rows whose stage scales fill one 1 KiB copy
    // MX scales, stage-major in memory ([sK/SCB][rows][SCB]): the scale bytes of SC_ROWS consecutive rows for
    // one stage are 1 KiB contiguous, one wave-wide 16-byte copy.  SA_REG / SB_REG: the A / B scale regions
    // of a stage.  Every wave issues SC_COPIES copies, so the per-wave copy count (and with it the vmcnt
    // threshold) is the same for all waves; copies past the real ones repeat a real one (the same bytes to the
    // same LDS address, harmless), so no wave needs a dummy destination.
    // fp6 (split planes): the P plane (dwords 0-3 of each block's six) is the operand the copies above stage, ROWB
    // bytes per row like fp4; the Q plane (dwords 4-5) arrives as 1 KiB blocks per (stage, 32-row group) holding
    // the 8-byte pieces of the group's 32 rows block by block ([4 blocks][32 rows][8 bytes] for ROWB = 64), one
    // copy each, staged after the P regions: QA_INSTR + QB_INSTR copies, spread over the waves with the scales.
    // An MFMA read of k-step s then takes 8 consecutive bytes per lane across 32 rows (no bank conflicts).
    static constexpr int QROW = IS_FP6 ? ROWB / 2 : 0;  // Q bytes per row per stage
    static constexpr int QA_INSTR = IS_FP6 ? BM / 32 : 0, QB_INSTR = IS_FP6 ? BN / 32 : 0;
    static constexpr int Q_REG = (QA_INSTR + QB_INSTR) * 1024;
    static constexpr int SA_INSTR = IS_MX ? (BM + SC_ROWS - 1) / SC_ROWS : 0;
    static constexpr int SB_INSTR = IS_MX ? (BN + SC_ROWS - 1) / SC_ROWS : 0;
    static constexpr int SA_REG = SA_INSTR * 1024, SB_REG = SB_INSTR * 1024;
    // SC_DIRECT: copies of 64 rows' scale bytes (64 SCB <= 1 KiB, so the regions above hold them)
    static constexpr int PLANE_B = (BN + 127) / 128 * 256;  // SC_DIRECT 2: bytes of one pair plane of the B region
    static constexpr int DA_INSTR = SC_DIRECT ? BM / 64 : 0;
    static constexpr int DB_INSTR = SC_DIRECT == 1 ? BN / 64 : SC_DIRECT == 2 ? 2 * ((BN + 127) / 128) : 0;
    static constexpr int AUX_INSTR = SC_DIRECT ? DA_INSTR + DB_INSTR : SA_INSTR + SB_INSTR + QA_INSTR + QB_INSTR;
    static constexpr int SC_COPIES = (AUX_INSTR + NW - 1) / NW;
    static constexpr int SC_BYTES = SA_REG + SB_REG;
    static constexpr int COPIES = A_COPIES + B_COPIES + SC_COPIES;
    static constexpr int B_BLK = (B_KCONTIG || B_TR) ? 0 : (ROWB / 8) * (BN / 4) / NT;  // 8x4-byte blocks per lane
    static constexpr int B_LOADS = 8 * B_BLK;         // dword loads per lane per stage for a [K, N] B
    static constexpr int STAGE = (BM + BN) * ROWB + Q_REG + SC_BYTES;
    static constexpr int SC_OFF = (BM + BN) * ROWB + Q_REG;  // the scale regions within a stage
    static constexpr size_t LDS_BYTES = (size_t)STAGES * STAGE;
    // vmem operations of this wave issued after stage kt's copies, at the top of iteration kt
    static constexpr int IN_FLIGHT = (STAGES - 2) * (COPIES + B_LOADS);
    // copies issued before each k-step of a stage (ILV false: all before the first)
    static constexpr int CPS = ILV ? (COPIES + KPS - 1) / KPS : COPIES;
    typedef typename std::conditional<OP == OP_I8, v16i, v16f>::type acc_t;
    static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(BM % (ROWS_PER_COPY * NW) == 0 && A_COPIES >= 1, "A copies must split evenly over the waves");
    static_assert(!B_KCONTIG || (BN % (ROWS_PER_COPY * NW) == 0 && B_COPIES >= 1), "B copies");
    static_assert(B_KCONTIG || B_TR || (((ROWB / 8) * (BN / 4)) % NT == 0 && B_BLK >= 1), "B blocks");
    static_assert(!B_TR || (!B_KCONTIG && (OP == OP_I8 || OP == OP_F8) && 1024 % BN == 0 && BN >= 32 && BN <= 256 &&
                            (ROWB * BN) % (1024 * NW) == 0 && B_COPIES >= 1), "B_TR copies");
    static_assert(!IS_MX || B_KCONTIG, "MX B must be K-contiguous");
    static_assert(OP != OP_BF16 || B_KCONTIG, "bf16 B must be K-contiguous");
    static_assert(!IS_MX || (BM % 64 == 0 && BN % 64 == 0), "scale row groups");
    static_assert(!IS_MX || SCB % 4 == 0 || SCB == 2, "MX stage scale bytes per row");
    // (an LDS-DMA load places lane l's data at 4 l, so only 4-byte rows pack densely)
    static_assert(!SC_DIRECT || (IS_MX && !IS_FP6 && SCB == 4), "direct scales: one 4-byte load a row");
    static_assert(SC_DIRECT != 2 || 2 * PLANE_B <= SB_INSTR * 1024, "pair planes fit the B scale region");
    static_assert(!IS_FP6 || (ROWB == 64 && BM % 32 == 0 && BN % 32 == 0), "fp6 Q blocks: 4 MX blocks per stage");
    static_assert(KPS >= 1, "a stage holds at least one k-step");
    static_assert((STAGES >= 3 || ((B_KCONTIG || B_TR) && STAGES == 2)) && IN_FLIGHT < 64, "stages");
    static_assert(ROWB == 64 || ROWB == 128, "stage row");
    static_assert(LDS_BYTES <= 160 * 1024, "LDS");

    __device__ __forceinline__ static int frag_row(int wm, int i, int r, int lane)
    {
        return wm * WTM + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    }
    __device__ __forceinline__ static int frag_col(int wn, int j, int lane) { return wn * WTN + j * 32 + (lane & 31); }
    // CT layout: the row of fragment (i, *) and the first of the four columns of register quad q of fragment (*, j)
    __device__ __forceinline__ static int ct_row(int wm, int i, int lane) { return wm * WTM + i * 32 + (lane & 31); }
    __device__ __forceinline__ static int ct_col(int wn, int j, int q, int lane)
    {
        return wn * WTN + j * 32 + 8 * q + 4 * (lane >> 5);
    }
    __device__ __forceinline__ static int swz(int row, int c) { return c ^ ((row / RPW) % CH); }
    // B_TR: the physical 16-byte chunk of logical chunk c of K row kr.  A transposed read of k-step s takes 16 K rows
    // (two runs of 8) x 32 bytes; the XOR spreads each run's 8 rows x 2 chunks over 16 distinct 16-byte bank groups
    // (the second run repeats them: two passes, the minimum for 512 bytes)
    __device__ __forceinline__ static int swzb(int kr, int c) { return c ^ (((kr / RWB) & (CHB / 2 - 1)) << 1); }

    // B_TR: the int8 B fragment of k-step s, column block starting at n0 (a multiple of 32), from a [ROWB][BN] region.
    // ds_read_b64_tr_b8 gives lane j of each 16-lane group byte (j % 8) of the 8-byte pieces addressed by lanes
    // 2r + j / 8, r = 0..7: here lanes 2r, 2r + 1 address the two halves of 16 columns of K row k0 + r, so lane j
    // receives K rows k0 .. k0 + 7 of column j -- the group (kh, nh) = (lane / 32, lane / 16 % 2) takes rows
    // 32 s + 16 kh + 8 q + (0..7) and columns n0 + 16 nh + (0..15); two reads (q = 0, 1) give the lane's 16
    // consecutive K bytes, in the order of the A fragment's 16 bytes.
    // The reads are inline assembly: through the builtin the compiler cannot tell them apart from the stage copies'
    // LDS destinations and drains every copy in flight (s_waitcnt vmcnt(0)) before each one, which measured twice
    // the kernel time.  The stage protocol (each wave's counted wait, then the barrier) already orders them after
    // the copies of their stage, and volatile keeps them below that barrier.  All FN fragments of a k-step are read
    // in one block that ends with s_waitcnt lgkmcnt(0), so its outputs hold the data when the block completes (the
    // compiler does not track the loads; a separate wait would let it schedule the MFMAs above it).
    // lane offset in the B region of its first transposed read (k-step 0, q = 0) of the fragment at columns n0 .. n0
    // + 31: the read of k-step s, piece q is 32 s + 8 q rows further down, and swzb is the same for those rows (the
    // step is a multiple of its period for BN <= 256), so this offset is worked out once per fragment column
    __device__ __forceinline__ static uint32_t tr_lane_off(int n0, int lane)
    {
        const int i = lane & 15, g = lane >> 4;
        const int c = (n0 >> 4) + (g & 1);
        const int kr = 16 * (g >> 1) + (i >> 1);
        return (uint32_t)(kr * BN + swzb(kr, c) * 16 + (i & 1) * 8);
    }
    __device__ __forceinline__ static void read_frags_tr(uint32_t region, const uint32_t (&off)[FN], int s, v4i (&f)[FN])
    {
        typedef int v2i_t __attribute__((ext_vector_type(2)));
        static_assert(FN == 1 || FN == 2 || FN == 4, "B_TR fragments per wave");
        v2i_t r[2 * FN];
        uint32_t ad[2 * FN];
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 2; ++q) ad[2 * j + q] = region + off[j] + (uint32_t)((32 * s + 8 * q) * BN);
        if constexpr (FN == 1) {
            asm volatile("ds_read_b64_tr_b8 %0, %2\n\tds_read_b64_tr_b8 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(r[0]), "=&v"(r[1])
                         : "v"(ad[0]), "v"(ad[1]));
        } else if constexpr (FN == 2) {
            asm volatile("ds_read_b64_tr_b8 %0, %4\n\tds_read_b64_tr_b8 %1, %5\n\t"
                         "ds_read_b64_tr_b8 %2, %6\n\tds_read_b64_tr_b8 %3, %7\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
                         : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]));
        } else {
            asm volatile("ds_read_b64_tr_b8 %0, %8\n\tds_read_b64_tr_b8 %1, %9\n\t"
                         "ds_read_b64_tr_b8 %2, %10\n\tds_read_b64_tr_b8 %3, %11\n\t"
                         "ds_read_b64_tr_b8 %4, %12\n\tds_read_b64_tr_b8 %5, %13\n\t"
                         "ds_read_b64_tr_b8 %6, %14\n\tds_read_b64_tr_b8 %7, %15\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),
                           "=&v"(r[7])
                         : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]),
                           "v"(ad[7]));
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) f[j] = (v4i){r[2 * j].x, r[2 * j].y, r[2 * j + 1].x, r[2 * j + 1].y};
    }

    // MX scale bytes of pair h for one tile row: four blocks (a 32-bit word), or two when a stage holds a single
    // fp8 k-step (SCB = 2)
    __device__ __forceinline__ static uint32_t scale_word(const uint8_t* region, int row, int h)
    {
        if constexpr (SCB == 2) return ((const uint16_t*)(region + row * SCB))[0];
        else return ((const uint32_t*)(region + row * SCB))[h];
    }

    // the operand fragment of k-step s for tile row `row` of a stage: 16 bytes (upper half zero) or 32 bytes
    __device__ __forceinline__ static v8i read_frag(const uint8_t* base, int row, int s, int kh)
    {
        if constexpr (LCH == 1) {
            const v4i x = *(const v4i*)(base + row * ROWB + swz(row, s * 2 + kh) * 16);
            return (v8i){x[0], x[1], x[2], x[3], 0, 0, 0, 0};
        } else {
            const int c = s * 4 + kh;
            const v4i x = *(const v4i*)(base + row * ROWB + swz(row, c) * 16);
            const v4i y = *(const v4i*)(base + row * ROWB + swz(row, c + 2) * 16);
            return (v8i){x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
        }
    }

    // fp6: the Q piece (8 bytes) of k-step s, lane half kh, for tile row `row` (a multiple of 32 plus r32) from a Q
    // region ([32-row group][4 blocks][32 rows][8 bytes])
    __device__ __forceinline__ static u32x2 read_q(const uint8_t* qbase, int row, int s, int kh)
    {
        return *(const u32x2*)(qbase + (row >> 5) * 1024 + ((2 * s + kh) * 32 + (row & 31)) * 8);
    }

    // t: the thread's index within the NT threads that run this tile (threadIdx.x, or its lane when each wave of a
    // workgroup runs a one-wave GemmCore on its own k range)
    __device__ __forceinline__ static void run(const CoreArgs& p, uint8_t* smem, acc_t (&acc)[FM][FN],
                                               int t = (int)threadIdx.x)
    {
        const int lane = t & 63;
        const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: copy bases stay scalar
        const int wm = wave / WN, wn = wave % WN;
        typedef uint32_t breg_t[B_BLK > 0 ? B_BLK : 1][8];
        breg_t rb0, rb1;  // two register sets, alternated by the 2x-unrolled main loop (no copies between them)

        // [K, N] B: the 8x4-byte blocks of stage kt into rbt
        auto load_b_regs = [&](breg_t& rbt, int64_t kt) {
            if constexpr (!B_KCONTIG && !B_TR) {
                const int64_t kb0 = kt * ROWB;
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
        };
        // transpose the blocks held in rb and write them K-contiguous into the B part of a slot
        auto store_b_regs = [&](breg_t& rb, int slot) {
            if constexpr (!B_KCONTIG && !B_TR) {
                uint8_t* sB = smem + slot * STAGE + BM * ROWB;
#pragma unroll
                for (int i = 0; i < B_BLK; ++i) {
                    const int id = t + i * NT, nb = id % (BN / 4), kb = id / (BN / 4);
                    uint32_t lo[4], hi[4];
                    transpose4x4(rb[i][0], rb[i][1], rb[i][2], rb[i][3], lo[0], lo[1], lo[2], lo[3]);
                    transpose4x4(rb[i][4], rb[i][5], rb[i][6], rb[i][7], hi[0], hi[1], hi[2], hi[3]);
                    const int rot = (nb >> 2) & 3;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int jj = (j + rot) & 3;
                        const uint32_t l = jj == 0 ? lo[0] : jj == 1 ? lo[1] : jj == 2 ? lo[2] : lo[3];
                        const uint32_t h = jj == 0 ? hi[0] : jj == 1 ? hi[1] : jj == 2 ? hi[2] : hi[3];
                        const int n = nb * 4 + jj;
                        *(u32x2*)(sB + n * ROWB + swz(n, kb >> 1) * 16 + (kb & 1) * 8) = (u32x2){l, h};
                    }
                }
            }
        };

        // MX auxiliary copies of this wave (A scales, B scales, then the fp6 Q blocks of A and of B): their source
        // (offset in p.aux at stage 0, stride per stage) and LDS offset within a stage depend on the wave only, so
        // they are worked out here, once.  The main loop then issues them with no branches: a branch there splits
        // the loop body into blocks, and the compiler sinks each stage's MFMAs (pure operations to it) past the
        // next stage's barrier, which leaves every SIMD without MFMA work between the two barriers.
        struct AuxCopy {
            uint32_t base, stride, dst;
        };
        AuxCopy aux[IS_MX ? SC_COPIES : 1];
        uint32_t aux_is_b[SC_DIRECT ? SC_COPIES : 1], aux_lmul[SC_DIRECT ? SC_COPIES : 1];
        if constexpr (SC_DIRECT) {
            // copy g: 64 rows of A (g < DA_INSTR), lane l taking row 64 g + l (SCB bytes at row * sk + SCB kt); then B:
            // 64 rows the same way (SC_DIRECT 1), or plane j = g' % 2 of 128-row group g' / 2 (SC_DIRECT 2), lane l
            // taking rows 128 (g' / 2) + 2 l, + 1 at ((2 kt + j) N + row) * 2
#pragma unroll
            for (int v = 0; v < SC_COPIES; ++v) {
                const int g = (wave * SC_COPIES + v) % AUX_INSTR;  // wave-uniform; past the real copies: a repeat
                const bool isb = g >= DA_INSTR;
                const int gg = isb ? g - DA_INSTR : g;
                if (isb && SC_DIRECT == 2) {
                    const int j = gg % 2, q = gg / 2;
                    aux[v] = {((uint32_t)j * p.sb_rows + p.sb0_row + (uint32_t)(q * 128)) * 2u, p.sb_rows * 4u,
                              (uint32_t)(SC_OFF + SA_REG + j * PLANE_B + q * 256)};
                    aux_lmul[v] = 4u;
                } else {
                    aux[v] = {((isb ? p.sb0_row : p.sa0_row) + (uint32_t)(gg * 64)) * p.sk, (uint32_t)SCB,
                              (uint32_t)(SC_OFF + (isb ? SA_REG : 0) + gg * 64 * SCB)};
                    aux_lmul[v] = p.sk;
                }
                aux[v].base = __builtin_amdgcn_readfirstlane(aux[v].base);
                aux[v].stride = __builtin_amdgcn_readfirstlane(aux[v].stride);
                aux[v].dst = __builtin_amdgcn_readfirstlane(aux[v].dst);
                aux_is_b[v] = __builtin_amdgcn_readfirstlane((uint32_t)isb);
                aux_lmul[v] = __builtin_amdgcn_readfirstlane(aux_lmul[v]);
            }
        } else if constexpr (IS_MX) {
#pragma unroll
            for (int v = 0; v < SC_COPIES; ++v) {
                const int g = (wave * SC_COPIES + v) % AUX_INSTR;  // wave-uniform; past the real copies: a repeat
                const int q = g - SA_INSTR - SB_INSTR;
                if (g < SA_INSTR)
                    aux[v] = {p.sa_base + (p.sa0_row + (uint32_t)(g * SC_ROWS)) * SCB, p.sa_rows * SCB,
                              (uint32_t)(SC_OFF + g * 1024)};
                else if (q < 0)
                    aux[v] = {p.sb_base + (p.sb0_row + (uint32_t)((g - SA_INSTR) * SC_ROWS)) * SCB, p.sb_rows * SCB,
                              (uint32_t)(SC_OFF + SA_REG + (g - SA_INSTR) * 1024)};
                // (Q groups past the operand's last belong to rows past M / N, whose outputs are dropped: they read
                // the next stage's first groups, or other data past the plane)
                else if (q < QA_INSTR)
                    aux[v] = {p.qa_off + (uint32_t)(q * 1024), p.qa_stride, (uint32_t)((BM + BN) * ROWB + q * 1024)};
                else
                    aux[v] = {p.qb_off + (uint32_t)((q - QA_INSTR) * 1024), p.qb_stride,
                              (uint32_t)((BM + BN) * ROWB + q * 1024)};
                aux[v].base = __builtin_amdgcn_readfirstlane(aux[v].base);
                aux[v].stride = __builtin_amdgcn_readfirstlane(aux[v].stride);
                aux[v].dst = __builtin_amdgcn_readfirstlane(aux[v].dst);
            }
        }

        // copy u (0 <= u < COPIES) of stage kt into slot: A rows, then B rows, then MX scale blocks
        auto issue_copy = [&](int64_t kt, int slot, int u) {
            uint8_t* sA = smem + slot * STAGE;
            uint8_t* sB = sA + BM * ROWB;
            const int64_t kb0 = kt * ROWB;
            const int rin = lane / CH, phys = lane % CH;
            if (u < A_COPIES) {
                const int row0 = (wave * A_COPIES + u) * ROWS_PER_COPY;
                const int row = row0 + rin;
                const int64_t k = kb0 + swz(row, phys) * 16;
                const uint32_t off = (row < p.rows && k < p.kbytes) ? p.a0 + (uint32_t)row * p.lda + (uint32_t)k : OOB;
                copy16_to_lds(p.a, sA + row0 * ROWB, off);
            } else if (u < A_COPIES + B_COPIES) {
                if constexpr (B_TR) {
                    // K rows kr of the stage, BN bytes each; lane's LDS chunk pb of row kr holds logical chunk
                    // swzb(kr, pb) (the XOR is its own inverse); chunks past the tile's columns read zeros
                    const int cc = wave * B_COPIES + (u - A_COPIES);
                    const int kr = cc * (1024 / BN) + lane / CHB, pb = lane % CHB;
                    const int c = swzb(kr, pb);
                    const int64_t k = kb0 + kr;
                    const uint32_t off =
                        (c * 16 < p.cols && k < p.kbytes) ? p.b0 + (uint32_t)k * p.ldb + (uint32_t)(c * 16) : OOB;
                    copy16_to_lds(p.b, sB + cc * 1024, off);
                } else {
                    const int row0 = (wave * B_COPIES + (u - A_COPIES)) * ROWS_PER_COPY;
                    const int row = row0 + rin;
                    const int64_t k = kb0 + swz(row, phys) * 16;
                    const uint32_t off = (row < p.cols && k < p.kbytes) ? p.b0 + (uint32_t)row * p.ldb + (uint32_t)k : OOB;
                    copy16_to_lds(p.b, sB + row0 * ROWB, off);
                }
            } else if constexpr (SC_DIRECT) {
                const int v = u - A_COPIES - B_COPIES;
                const AuxCopy& x = aux[v];
                const bool kval = (uint32_t)(kt * SCB) < p.sk;
                const uint32_t off = kval ? x.base + (uint32_t)kt * x.stride + (uint32_t)lane * aux_lmul[v] : OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(aux_is_b[v] ? p.aux_b : p.aux, (lds_ptr_t)(sA + x.dst), SCB, off,
                                                         0, 0, 0);
            } else if constexpr (IS_MX) {
                const AuxCopy& x = aux[u - A_COPIES - B_COPIES];
                const bool kval = (uint32_t)(kt * SCB) < p.sk;
                copy16_to_lds(p.aux, sA + x.dst, kval ? x.base + (uint32_t)kt * x.stride + (uint32_t)(lane * 16) : OOB);
            }
        };
        auto issue_copies = [&](int64_t kt, int slot) {
#pragma unroll
            for (int u = 0; u < COPIES; ++u) issue_copy(kt, slot, u);
        };

#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = (acc_t){};

        const int r32 = lane & 31, kh = lane >> 5;
        const int64_t nk = (p.kbytes + ROWB - 1) / ROWB;
        uint32_t troff[FN];  // B_TR: this lane's read offsets, one per fragment column
#pragma unroll
        for (int j = 0; j < FN; ++j) troff[j] = B_TR ? tr_lane_off(wn * WTN + j * 32, lane) : 0u;

        // prologue: stages 0 .. STAGES - 2 in flight; a [K, N] B is written for stages 0 .. STAGES - 3 and
        // held in rb1 for stage STAGES - 2 (written at the end of iteration 0)
#pragma unroll
        for (int s = 0; s < STAGES - 1; ++s) {
            if (s < STAGES - 2) load_b_regs(rb0, s);
            else load_b_regs(rb1, s);
            __builtin_amdgcn_sched_barrier(0);
            issue_copies(s, s);
            __builtin_amdgcn_sched_barrier(0);
            if (s < STAGES - 2) store_b_regs(rb0, s);
        }

        // one iteration: stage kt is multiplied; the registers of stage kt + STAGES - 1 are loaded into rb_new and
        // those of stage kt + STAGES - 2 (loaded one iteration ago into rb_old) are written to their slot
        auto iteration = [&](int64_t kt, breg_t& rb_new, breg_t& rb_old) {
            const int slot = (int)(kt % STAGES);
            const int nslot = (int)((kt + STAGES - 1) % STAGES);
            const int pslot = (int)((kt + STAGES - 2) % STAGES);
            __builtin_amdgcn_sched_barrier(0);  // the wait stays below the previous iteration's MFMAs
            wait_vmcnt<IN_FLIGHT>();            // this wave's copies of stage kt have landed
            stage_barrier();                    // ... and every wave's; the slot multiplied last iteration is free
            load_b_regs(rb_new, kt + STAGES - 1);
            __builtin_amdgcn_sched_barrier(0);
            const uint8_t* sA = smem + slot * STAGE;
            const uint8_t* sB = sA + BM * ROWB;
            // k-steps in pairs; a scheduling barrier between pairs keeps the fragment reads of a stage from
            // being hoisted together (they would not fit the register file at two waves per SIMD).  MX: for pair
            // h the scale word of each fragment row (blocks 4h .. 4h + 3), shifted by 8 * (lane / 32) so that
            // byte 2(s % 2) is block 2s + lane / 32 -- the block whose scale this lane supplies for k-step s --
            // and the MFMA's op_sel picks it.
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                if (h > 0) __builtin_amdgcn_sched_barrier(0);
                uint32_t swa[IS_MX ? FM : 1], swb[IS_MX ? FN : 1];
                if constexpr (IS_MX) {
                    const uint8_t* sS = sA + SC_OFF;
#pragma unroll
                    for (int i = 0; i < FM; ++i) swa[i] = scale_word(sS, wm * WTM + i * 32 + r32, h) >> (8 * kh);
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const int row = wn * WTN + j * 32 + r32;
                        if constexpr (SC_DIRECT == 2)  // the row's entries of the two pair planes
                            swb[j] = ((uint32_t)((const uint16_t*)(sS + SA_REG))[row] |
                                      ((uint32_t)((const uint16_t*)(sS + SA_REG + PLANE_B))[row] << 16)) >> (8 * kh);
                        else
                            swb[j] = scale_word(sS + SA_REG, row, h) >> (8 * kh);
                    }
                }
#pragma unroll
                for (int s = SPH * h; s < SPH * h + SPH; ++s) {
                    // the copies of stage kt + STAGES - 1 are spread over the k-steps of this stage (CPS before
                    // each), so no wave stalls on a burst of them in front of its MFMAs (measured 13-14 % faster
                    // than issuing them all after the barrier)
#pragma unroll
                    for (int u = s * CPS; u < (s + 1) * CPS && u < COPIES; ++u) issue_copy(kt + STAGES - 1, nslot, u);
                    __builtin_amdgcn_sched_barrier(0);
                    // this lane's 16-byte chunks of k-step s: s * 2 + kh (int8, fp4), s * 4 + kh and s * 4 + 2 + kh
                    // (fp8)
                    v8i fa[FM];
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        fa[i] = read_frag(sA, wm * WTM + i * 32 + r32, s, kh);
                        if constexpr (IS_FP6) {
                            const u32x2 q = read_q(sA + (BM + BN) * ROWB, wm * WTM + i * 32 + r32, s, kh);
                            fa[i][4] = (int)q[0];
                            fa[i][5] = (int)q[1];
                        }
                    }
                    // B_TR fp8: the 32 bytes of k-step s (lane half kh: K rows 64 s + 16 kh .. and 64 s + 32 + 16 kh ..,
                    // register quads 0 and 1) are the int8-sized transposed reads of steps 2 s and 2 s + 1
                    v4i ftr[FN], ftr2[OP == OP_F8 ? FN : 1];
                    if constexpr (B_TR) {
                        const uint32_t region = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)sB;
                        if constexpr (OP == OP_F8) {
                            read_frags_tr(region, troff, 2 * s, ftr);
                            read_frags_tr(region, troff, 2 * s + 1, ftr2);
                        } else {
                            read_frags_tr(region, troff, s, ftr);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        v8i fb;
                        if constexpr (B_TR && OP == OP_F8) {
                            fb = (v8i){ftr[j][0], ftr[j][1], ftr[j][2], ftr[j][3], ftr2[j][0], ftr2[j][1], ftr2[j][2], ftr2[j][3]};
                        } else if constexpr (B_TR) {
                            fb = (v8i){ftr[j][0], ftr[j][1], ftr[j][2], ftr[j][3], 0, 0, 0, 0};
                        } else {
                            fb = read_frag(sB, wn * WTN + j * 32 + r32, s, kh);
                        }
                        if constexpr (IS_FP6) {
                            const u32x2 q = read_q(sA + (BM + BN) * ROWB + QA_INSTR * 1024, wn * WTN + j * 32 + r32, s, kh);
                            fb[4] = (int)q[0];
                            fb[5] = (int)q[1];
                        }
#pragma unroll
                        for (int i = 0; i < FM; ++i) {
                            if constexpr (OP == OP_I8) {
                                const v4i a4 = (v4i){fa[i][0], fa[i][1], fa[i][2], fa[i][3]};
                                const v4i b4 = (v4i){fb[0], fb[1], fb[2], fb[3]};
                                if constexpr (CT) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b4, a4, acc[i][j], 0, 0, 0);
                                else acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, acc[i][j], 0, 0, 0);
                            } else if constexpr (OP == OP_BF16) {
                                typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));
                                const v4i a4 = (v4i){fa[i][0], fa[i][1], fa[i][2], fa[i][3]};
                                const v4i b4 = (v4i){fb[0], fb[1], fb[2], fb[3]};
                                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf_t, a4),
                                                                                    __builtin_bit_cast(v8bf_t, b4),
                                                                                    acc[i][j], 0, 0, 0);
                            } else if constexpr (OP == OP_F8) {
                                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb, acc[i][j], CBSZ,
                                                                                             BLGP, 0, 0, 0, 0);
                            } else {
                                if ((s & 1) == 0)
                                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                                        fa[i], fb, acc[i][j], CBSZ, BLGP, 0, swa[i], 0, swb[j]);
                                else
                                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                                        fa[i], fb, acc[i][j], CBSZ, BLGP, 2, swa[i], 2, swb[j]);
                            }
                        }
                    }
                }
            }
            if constexpr (!B_KCONTIG && !B_TR) {
                // rb_old's slot was freed two iterations ago and is next read after at least one more barrier
                __builtin_amdgcn_sched_barrier(0);
                store_b_regs(rb_old, pslot);
            }
        };
        int64_t kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            iteration(kt, rb0, rb1);
            iteration(kt + 1, rb1, rb0);
        }
        if (kt < nk) iteration(kt, rb0, rb1);
        // drain: no copy may still target LDS when the caller reuses it or the wave ends
        wait_vmcnt<0>();
    }
};

// A raw buffer resource over the `bytes` bytes at p whose base is p aligned down to 16 bytes; delta = p % 16 is to be
// added to every offset into it.  Multi-dword buffer loads are range-checked per dword, so the range is rounded up to
// whole dwords: the dword that holds the operand's last byte then reads that byte (it lies in the byte's page).
__device__ __forceinline__ rsrc_t make_rsrc_a16(const void* p, uint32_t bytes, uint32_t& delta)
{
    delta = (uint32_t)((uintptr_t)p & 15u);
    return make_rsrc((const uint8_t*)p - delta, (bytes + delta + 3u) & ~3u);
}

// GemmCoreUA: GemmCore's int8 / fp8 tiles, two-stage LDS layout (ROWB = 64), fragment reads and MFMAs for operands of
// any alignment and any K: K not a multiple of 16, leading dimensions and base pointers of any byte alignment.  The
// operands go global -> registers -> LDS.  A lane takes one 16-byte chunk per copy unit -- 16 K bytes of an A row or
// of a K-contiguous B row, or (int8) 16 columns of one K row of a [K, N] B (staged as GemmCore's B_TR region and read
// by its transposed reads) -- as the two 16-byte-aligned blocks that cover it, picks the chunk's five dwords and
// realigns them with v_alignbyte_b32, zeroes its bytes at k >= K, and writes it with one 16-byte LDS store to the
// chunk the swizzle assigns.  Zeroing both operands' bytes past K keeps other rows' (or other groups') bytes out of
// every product, also for a chunk that straddles the end of a row (fp8: a zero byte is +0, so no NaN or infinity
// from past K reaches a sum).
// Every load is 16-byte aligned in memory (the resources' bases are aligned down to 16 bytes, make_rsrc_a16, and the
// offsets carry the difference): a block that holds a byte of the operand lies in that byte's page, and a block that
// starts past the operand is out of the resource's range and reads zeros (the second block is skipped outright
// when the chunk's valid bytes end in the first).
// Pipeline: two register sets hold the chunks of the two stages after the one being multiplied.  Iteration kt: one
// barrier (stage kt is in its slot, the other slot's readers are done), the MFMAs of stage kt, then stage kt + 1
// from its register set into the other slot and the loads of stage kt + 3 into that set -- two stages of MFMAs
// cover each load.
template <int BM, int BN, int WM, int WN, bool B_KCONTIG, bool CT, int OP = OP_I8, int FMT = 0>
struct GemmCoreUA : GemmCore<BM, BN, WM, WN, 2, B_KCONTIG, OP, 64, FMT, true, CT, !B_KCONTIG> {
    using Base = GemmCore<BM, BN, WM, WN, 2, B_KCONTIG, OP, 64, FMT, true, CT, !B_KCONTIG>;
    using acc_t = typename Base::acc_t;
    static_assert(OP == OP_I8 || (OP == OP_F8 && B_KCONTIG), "int8, or fp8 with a K-contiguous B");
    static constexpr int ROWB = 64, CH = 4;
    static constexpr int NT = Base::NT, FM = Base::FM, FN = Base::FN, WTM = Base::WTM, WTN = Base::WTN;
    static constexpr int CHB = BN / 16;                // [K, N] B: chunks per K row
    static constexpr int AC = BM * CH / NT;            // A chunks per thread per stage
    static constexpr int BC = BN * CH / NT;            // B chunks per thread per stage (BN rows or 64 K rows)
    static constexpr int U = AC + BC;
    static_assert(AC >= 1 && BC >= 1 && AC * NT == BM * CH && BC * NT == BN * CH, "chunks per thread");

    struct Regs {
        u32x4 lo[U], hi[U];
    };

    // chunk u of this thread in stage kt: byte offset in its resource (past the resource's delta), the number of its
    // 16 bytes that hold operand data (0: rows past the tile, chunks past K or past the tile's columns) and its
    // offset within an LDS stage
    __device__ __forceinline__ static void chunk(const CoreArgs& p, int t, int64_t kt, int u, uint32_t& off, int& valid,
                                                 uint32_t& lds)
    {
        const int64_t kb0 = kt * ROWB;
        auto kvalid = [&](int64_t k) {
            const int64_t v = p.kbytes - k;
            return v <= 0 ? 0 : (v >= 16 ? 16 : (int)v);
        };
        if (u < AC) {
            const int id = t + u * NT, row = id / CH, c = id % CH;
            const int64_t k = kb0 + c * 16;
            valid = row < p.rows ? kvalid(k) : 0;
            off = p.a0 + (uint32_t)row * p.lda + (uint32_t)k;
            lds = (uint32_t)(row * ROWB + Base::swz(row, c) * 16);
        } else if constexpr (B_KCONTIG) {
            const int id = t + (u - AC) * NT, row = id / CH, c = id % CH;
            const int64_t k = kb0 + c * 16;
            valid = row < p.cols ? kvalid(k) : 0;
            off = p.b0 + (uint32_t)row * p.ldb + (uint32_t)k;
            lds = (uint32_t)(BM * ROWB + row * ROWB + Base::swz(row, c) * 16);
        } else {
            const int id = t + (u - AC) * NT, kr = id / CHB, c = id % CHB;
            const int64_t k = kb0 + kr;
            // columns past the tile's within a chunk are other data: their products land in unstored outputs
            valid = (k < p.kbytes && c * 16 < p.cols) ? 16 : 0;
            off = p.b0 + (uint32_t)k * p.ldb + (uint32_t)(c * 16);
            lds = (uint32_t)(BM * ROWB + kr * BN + Base::swzb(kr, c) * 16);
        }
    }

    __device__ __forceinline__ static void run(const CoreArgs& p, uint8_t* smem, acc_t (&acc)[FM][FN],
                                               int t = (int)threadIdx.x)
    {
        const int lane = t & 63;
        const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
        const int wm = wave / WN, wn = wave % WN;
        const int r32 = lane & 31, kh = lane >> 5;
        const int64_t nk = (p.kbytes + ROWB - 1) / ROWB;

        auto load = [&](Regs& R, int64_t kt) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                uint32_t off, lds;
                int valid;
                chunk(p, t, kt, u, off, valid, lds);
                const rsrc_t r = u < AC ? p.a : p.b;
                const uint32_t o = off & ~15u, s = off & 15u;
                R.lo[u] = bload16(r, valid > 0 ? o : OOB);
                R.hi[u] = bload16(r, (int)s + valid > 16 ? o + 16 : OOB);
            }
        };
        auto store = [&](const Regs& R, int64_t kt, int slot) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                uint32_t off, lds;
                int valid;
                chunk(p, t, kt, u, off, valid, lds);
                const uint32_t s = off & 15u, q = s >> 2, sh = s & 3u;
                const uint32_t w[8] = {R.lo[u][0], R.lo[u][1], R.lo[u][2], R.lo[u][3],
                                       R.hi[u][0], R.hi[u][1], R.hi[u][2], R.hi[u][3]};
                uint32_t d[5];
#pragma unroll
                for (int i = 0; i < 5; ++i)
                    d[i] = q == 0 ? w[i] : (q == 1 ? w[i + 1] : (q == 2 ? w[i + 2] : w[i + 3]));
                u32x4 out;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int nv = valid - 4 * j;  // valid bytes of dword j
                    const uint32_t m = nv >= 4 ? ~0u : (nv <= 0 ? 0u : (1u << (8 * nv)) - 1u);
                    out[j] = __builtin_amdgcn_alignbyte(d[j + 1], d[j], sh) & m;
                }
                *(u32x4*)(smem + slot * Base::STAGE + lds) = out;
            }
        };

        uint32_t troff[FN];  // [K, N] B: this lane's transposed-read offsets, one per fragment column
#pragma unroll
        for (int j = 0; j < FN; ++j) troff[j] = B_KCONTIG ? 0u : Base::tr_lane_off(wn * WTN + j * 32, lane);
        auto compute = [&](int slot) {
            const uint8_t* sA = smem + slot * Base::STAGE;
            const uint8_t* sB = sA + BM * ROWB;
#pragma unroll
            for (int s = 0; s < Base::KPS; ++s) {
                v8i fa[FM];
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[i] = Base::read_frag(sA, wm * WTM + i * 32 + r32, s, kh);
                v4i ftr[FN];
                if constexpr (!B_KCONTIG)
                    Base::read_frags_tr((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)sB, troff,
                                        s, ftr);
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    v8i fb;
                    if constexpr (B_KCONTIG) fb = Base::read_frag(sB, wn * WTN + j * 32 + r32, s, kh);
                    else fb = (v8i){ftr[j][0], ftr[j][1], ftr[j][2], ftr[j][3], 0, 0, 0, 0};
#pragma unroll
                    for (int i = 0; i < FM; ++i) {
                        if constexpr (OP == OP_I8) {
                            const v4i a4 = (v4i){fa[i][0], fa[i][1], fa[i][2], fa[i][3]};
                            const v4i b4 = (v4i){fb[0], fb[1], fb[2], fb[3]};
                            if constexpr (CT) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b4, a4, acc[i][j], 0, 0, 0);
                            else acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, acc[i][j], 0, 0, 0);
                        } else {
                            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[i], fb, acc[i][j], Base::CBSZ,
                                                                                         Base::BLGP, 0, 0, 0, 0);
                        }
                    }
                }
            }
        };

#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = (acc_t){};
        Regs R0, R1;
        load(R0, 0);
        if (nk > 1) load(R1, 1);
        store(R0, 0, 0);
        if (nk > 2) load(R0, 2);
        // Rn holds stage kt + 1 (same parity as kt + 3)
        auto iteration = [&](int64_t kt, Regs& Rn) {
            __syncthreads();
            compute((int)(kt & 1));
            if (kt + 1 < nk) {
                store(Rn, kt + 1, (int)((kt + 1) & 1));
                if (kt + 3 < nk) load(Rn, kt + 3);
            }
        };
        int64_t kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            iteration(kt, R1);
            iteration(kt + 1, R0);
        }
        if (kt < nk) iteration(kt, R1);
    }
};

// the 32 bits of one accumulator element (a value copy: __builtin_bit_cast of a vector-element lvalue reads the
// vector's first element under this compiler)
__device__ __forceinline__ uint32_t acc_bits(float x) { return __float_as_uint(x); }
__device__ __forceinline__ uint32_t acc_bits(int x) { return (uint32_t)x; }

// Rolled epilogue of a GemmCore tile (T): the raw accumulators are parked in LDS -- free once every wave has left
// the main loop -- and a rolled loop then takes one element per thread per step and hands put(tile row, tile
// column, accumulator bits) the element.  Rolling the loop keeps the per-element code (a compare-and-swap, a software
// encoder) and its registers out of an unrolled store path.  A tile that does not fit the LDS at once goes in NCH
// chunks of rows: in chunk ch every wave writes the 32-row fragments that lie in it.
template <class T, class F>
__device__ __forceinline__ void rolled_epilogue(uint8_t* smem, const typename T::acc_t (&acc)[T::FM][T::FN], int rows,
                                                int cols, F put)
{
    constexpr int NCH = (size_t)T::TBM * T::TBN * 4 <= T::LDS_BYTES ? 1 : (size_t)T::TBM * T::TBN * 2 <= T::LDS_BYTES ? 2 : 4;
    constexpr int CHR = T::TBM / NCH;  // rows per chunk
    static_assert((size_t)CHR * T::TBN * 4 <= T::LDS_BYTES && CHR % 32 == 0 && (T::TBN & (T::TBN - 1)) == 0,
                  "rolled epilogue chunks");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / T::TWN, wn = wave % T::TWN;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        __syncthreads();  // the main loop's last LDS reads (or the previous chunk's) are done
#pragma unroll
        for (int i = 0; i < T::FM; ++i) {
            if ((wm * T::WTM + i * 32) / CHR != ch) continue;  // 32-row fragment i lies in chunk ch or not at all
#pragma unroll
            for (int j = 0; j < T::FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    *(uint32_t*)(smem + ((T::frag_row(wm, i, r, lane) - ch * CHR) * T::TBN + T::frag_col(wn, j, lane)) * 4) =
                        acc_bits(acc[i][j][r]);
        }
        __syncthreads();
#pragma unroll 1
        for (int e = threadIdx.x; e < CHR * T::TBN; e += T::NT) {
            const int rr = ch * CHR + e / T::TBN, cc = e % T::TBN;
            if (rr >= rows || cc >= cols) continue;
            put(rr, cc, *(const uint32_t*)(smem + e * 4));
        }
    }
}

// enAtomic epilogue of a GemmCore tile (T): the rolled epilogue with the output conversion conv(tile column,
// accumulator bits) -> C bits combined into C by c_atomic.
template <class T, int DT, class F>
__device__ __forceinline__ void atomic_epilogue(uint8_t* smem, const typename T::acc_t (&acc)[T::FM][T::FN],
                                                const TileOut& out, int rows, int cols, int op, F conv)
{
    constexpr int ES = (DT == DT_INT32 || DT == DT_F32) ? 4 : 2;  // bytes per C element
    rolled_epilogue<T>(smem, acc, rows, cols, [&](int rr, int cc, uint32_t a) {
        c_atomic<DT>(out.base + (uint32_t)rr * out.pitch + (uint32_t)(cc * ES), conv(cc, a), op);
    });
}

}  // namespace ascq
