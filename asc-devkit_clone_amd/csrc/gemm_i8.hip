// gemm_i8.hip -- int8 x int8 -> int32 GEMM on CDNA4 MFMA with the fixpipe dequant / requant fused in the epilogue.
//
// Replaces the adv_api Matmul quant scenario (impl/adv_api/detail/matmul/matmul_impl.h:119-137 IterateAll;
// stage/compute/mmad_compute.h:40-90 Mmad int8 -> int32 L0C; stage/copy_cube_out/copy_cube_out_fixpipe.h:339-357
// and quant/quant_processor_fixpipe.h:74-234 for the DEQF16 / QS322BF16_PRE / REQ8 epilogues).
//
// gfx950 design: the v_mfma_i32_32x32x32_i8 main loop of gemm_core.h (a ring of LDS stages filled by
// global->LDS buffer copies, XOR-swizzled LDS, in-flight byte transpose of a row-major [K, N] B), XCD-aware
// tile order, and the fixpipe epilogue in registers:
//   acc (+ int32 bias) -> f32 (rne) x M1[n] -> f16 / bf16 (rne, saturating), or -> requant8 (int8 / uint8 C:
//   clamp, rint, + offset, saturate by the word's sign flag); M1 = QUANT_PRE bits [31:13]
//   (accompanying_quantization.md:79-103).
#include "common.h"
#include "gemm_core.h"
#include "launch.h"

namespace ascq {

// a value every lane of the wave holds alike, moved to scalar registers
__device__ __forceinline__ int64_t uniform64(int64_t v)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// The int8 main loop of a tile: GemmCore (16-byte-aligned K-contiguous rows, K % 16 == 0), or GemmCoreUA (UA: any
// alignment, any K; two stages of 64 bytes, a [K, N] B staged by K rows)
template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB, bool CT, bool BTR, bool UA>
using I8Core = typename std::conditional<UA, GemmCoreUA<BM, BN, WM, WN, TB, CT>,
                                         GemmCore<BM, BN, WM, WN, ST, TB, OP_I8, RB, 0, true, CT, BTR>>::type;

// KW > 1 (one-wave tiles, WM = WN = 1; store epilogues only): the workgroup's KW waves each run the tile's main loop on
// their own K / KW range (K a multiple of KW * RB, so every wave runs the same stages and meets the same barriers) in
// their own LDS ring, then sum their int32 accumulators through LDS (exact in any order) and wave 0 runs the epilogue.
// For small problems (the W8A8 sample, 32 tiles) this cuts the serial K loop of each tile KW-fold.
// PH (K split across workgroups, decode-sized batches): 1 -- workgroup b runs split b / tiles of tile b % tiles, its
// K range a whole number of KW RB units (the units shared out as evenly as p.splits allows), and stores the tile's
// accumulators in p.ws ([split][tile][fragment][lane]); 2 -- one wave per 32 x 32 fragment of a tile adds the
// splits' accumulators of its fragment in split order (int32: exact) and stores it through the epilogue.
template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB = 64, bool BTR = false, int KW = 1, bool UA = false,
          int PH = 0>
__global__ __launch_bounds__(PH == 2 ? (BM / 32) * (BN / 32) * 64 : WM * WN * 64 * KW) void gemm_i8_kernel(GemmI8Args p)
{
    using T = I8Core<BM, BN, WM, WN, ST, TB, RB, false, BTR, UA>;
    static_assert(!UA || KW == 1, "any-alignment tiles run whole K");
    static_assert(KW == 1 || (WM == 1 && WN == 1), "k-split waves run one-wave tiles");
    static_assert(PH == 0 || (WM == 1 && WN == 1 && !UA && (PH == 2 || KW > 1)), "K split across workgroups");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tiles_m = (int)((p.M + BM - 1) / BM), tiles_n = (int)((p.N + BN - 1) / BN);
    const int ntiles = tiles_m * tiles_n;
    const int tile = PH == 1 ? (int)blockIdx.x % ntiles : (int)blockIdx.x;
    const int split = PH == 1 ? (int)blockIdx.x / ntiles : 0;
    int tm, tn;
    tile_coords(tile, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int kw = KW > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;
    int64_t kg0 = 0, kg = p.K;  // this workgroup's K range
    if constexpr (PH == 1) {
        const int64_t units = p.K / (KW * RB);
        const int64_t u0 = units * split / p.splits, u1 = units * (split + 1) / p.splits;
        kg0 = u0 * KW * RB;
        kg = (u1 - u0) * KW * RB;
    }
    const int64_t kc = kg / KW, k0 = kg0 + kw * kc;  // this wave's K range (KW > 1: a multiple of RB)
    CoreArgs c{};
    const uint32_t a_bytes = (uint32_t)(p.lda * (p.M - 1) + p.K);
    const uint32_t b_bytes = (uint32_t)(TB ? p.ldb * (p.N - 1) + p.K : p.ldb * (p.K - 1) + p.N);
    uint32_t da = 0, db = 0;  // UA: the operands' offsets from their resources' 16-byte-aligned bases
    if constexpr (UA) {
        c.a = make_rsrc_a16(p.A, a_bytes, da);
        c.b = make_rsrc_a16(p.B, b_bytes, db);
    } else {
        c.a = make_rsrc(p.A, a_bytes);
        c.b = make_rsrc(p.B, b_bytes);
    }
    c.lda = (uint32_t)p.lda;
    c.ldb = (uint32_t)p.ldb;
    c.rows = (int32_t)(p.M - m0 < BM ? p.M - m0 : BM);
    c.cols = (int32_t)(p.N - n0 < BN ? p.N - n0 : BN);
    c.a0 = (uint32_t)(m0 * p.lda + k0) + da;
    c.b0 = (uint32_t)(TB ? n0 * p.ldb + k0 : n0 + k0 * p.ldb) + db;
    c.kbytes = kc;
    // KW > 1 (small problems, where the kernel is one chain of latencies): the epilogue's bias and QUANT_PRE words are
    // loaded before the main loop, so their latency hides under it instead of following it.  They are older than the
    // main loop's copies, whose counted waits therefore still cover exactly those copies (loads return in order).
    constexpr bool PRE = KW > 1 && PH == 0;  // the epilogue's words loaded before the main loop
    int32_t pre_bias[T::FN];
    uint64_t pre_w[T::FN];
    if constexpr (PRE) {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(0, j, (int)threadIdx.x & 63);
            const bool cok = cl < c.cols;
            pre_bias[j] = (p.bias && cok) ? p.bias[n0 + cl] : 0;
            pre_w[j] = (p.qvec && cok) ? p.qvec[n0 + cl] : p.qscalar;
        }
    }
    typename T::acc_t acc[T::FM][T::FN];
    constexpr int F = T::FM * T::FN;  // accumulator fragments of the tile
    v16i* part = (v16i*)p.ws;         // PH 1 / 2: [split][tile][F][64 lanes]
    const int fw = PH == 2 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;  // PH 2: this wave's fragment
    if constexpr (PH == 2) {
        const int ln = threadIdx.x & 63;
#pragma unroll
        for (int f = 0; f < F; ++f) {
            acc[f / T::FN][f % T::FN] = typename T::acc_t{};
            if (f != fw) continue;
            acc[f / T::FN][f % T::FN] = part[((int64_t)tile * F + f) * 64 + ln];
            for (int sp = 1; sp < p.splits; ++sp)
                acc[f / T::FN][f % T::FN] += part[(((int64_t)sp * ntiles + tile) * F + f) * 64 + ln];
        }
    } else {
        T::run(c, smem + (KW > 1 ? kw * T::LDS_BYTES : 0), acc, KW > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x);
    }
    if constexpr (KW > 1) {
        __syncthreads();  // every wave's main loop is done with its LDS ring
        v16i* red = (v16i*)smem;  // [KW - 1][F][64 lanes] accumulator fragments
        const int lane = threadIdx.x & 63;
        if (kw > 0) {
#pragma unroll
            for (int f = 0; f < F; ++f) red[((kw - 1) * F + f) * 64 + lane] = acc[f / T::FN][f % T::FN];
        }
        __syncthreads();
        if (kw != 0) return;
#pragma unroll
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
            for (int f = 0; f < F; ++f) acc[f / T::FN][f % T::FN] += red[(w * F + f) * 64 + lane];
    }
    if constexpr (PH == 1) {
        const int ln = threadIdx.x & 63;
#pragma unroll
        for (int f = 0; f < F; ++f) part[(((int64_t)split * ntiles + tile) * F + f) * 64 + ln] = acc[f / T::FN][f % T::FN];
        return;
    }

    // epilogue: per 32x32 accumulator tile, lane holds column lane%32 and 16 rows (GemmCore::frag_row); stores go
    // through a buffer resource over the output tile (rows past M dropped by its range, 32-bit offsets)
    const int lane = threadIdx.x & 63, wave = PH == 2 ? 0 : threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const float mscalar = quant_pre_m1(p.qscalar);
    if (p.epi == EPI_REQ4) {  // (V)REQ4: int4 codes, two per byte
        const TileOut o4 = tile_out_int4(p.C, m0, n0, p.ldc, c.rows, c.cols);
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(wn, j, lane);
            const bool cok = cl < c.cols;
            const int64_t col = n0 + cl;
            const int32_t bias = (p.bias && cok) ? p.bias[col] : 0;
            const uint64_t w = (p.qvec && cok) ? p.qvec[col] : p.qscalar;
            const float m1 = p.qvec ? quant_pre_m1(w) : mscalar;
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int32_t v = (int32_t)((uint32_t)acc[i][j][r] + (uint32_t)bias);
                    store_int4_pair(o4, requant4((float)v * m1, w), cl, c.cols, lane,
                                    (uint32_t)T::frag_row(wm, i, r, lane) * o4.pitch);
                }
        }
        return;
    }
    const int esize = p.epi == EPI_I32 ? 4 : (p.epi == EPI_REQ8 ? 1 : 2);
    const TileOut out = tile_out(p.C, m0, n0, p.ldc, c.rows, c.cols, esize);
    auto store = [&](auto conv, auto put) {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(wn, j, lane);
            const bool cok = cl < c.cols;
            const int64_t col = n0 + cl;
            const int32_t bias = PRE ? pre_bias[j] : (p.bias && cok) ? p.bias[col] : 0;
            const uint64_t w = PRE ? pre_w[j] : (p.qvec && cok) ? p.qvec[col] : p.qscalar;
            const float m1 = p.qvec ? quant_pre_m1(w) : mscalar;
            const uint32_t cbase = cok ? (uint32_t)(cl * esize) : OOB;
#pragma unroll
            for (int i = 0; i < T::FM; ++i) {
                if (PH == 2 && i * T::FN + j != fw) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int32_t v = (int32_t)((uint32_t)acc[i][j][r] + (uint32_t)bias);
                    put(conv(v, m1, w), cbase + (uint32_t)T::frag_row(wm, i, r, lane) * out.pitch);
                }
            }
        }
    };
    if (KW == 1 && p.atomic != C_STORE) {  // enAtomic: int32 / f16 / bf16 C (the host layer refuses the others)
        // acc + bias (int32, wrapping), then x M1 of the column for f16 / bf16 -- the store path's arithmetic
        auto v = [&](int cl, uint32_t a) { return (int32_t)(a + (uint32_t)(p.bias ? p.bias[n0 + cl] : 0)); };
        auto m1 = [&](int cl) { return p.qvec ? quant_pre_m1(p.qvec[n0 + cl]) : mscalar; };
        if (p.epi == EPI_I32)
            atomic_epilogue<T, DT_INT32>(smem, acc, out, c.rows, c.cols, p.atomic,
                                         [&](int cl, uint32_t a) { return (uint32_t)v(cl, a); });
        else if (p.epi == EPI_DEQ_F16)
            atomic_epilogue<T, DT_F16>(smem, acc, out, c.rows, c.cols, p.atomic, [&](int cl, uint32_t a) {
                return (uint32_t)f32_to_f16_sat((float)v(cl, a) * m1(cl));
            });
        else
            atomic_epilogue<T, DT_BF16>(smem, acc, out, c.rows, c.cols, p.atomic, [&](int cl, uint32_t a) {
                return (uint32_t)f32_to_bf16_sat((float)v(cl, a) * m1(cl));
            });
        return;
    }
    if (p.epi == EPI_I32)
        store([](int32_t v, float, uint64_t) { return (uint32_t)v; },
              [&](uint32_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b32(x, out.r, o, 0, 0); });
    else if (p.epi == EPI_DEQ_F16)
        store([](int32_t v, float m1, uint64_t) { return f32_to_f16_sat((float)v * m1); },
              [&](uint16_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b16(x, out.r, o, 0, 0); });
    else if (p.epi == EPI_DEQ_BF16)
        store([](int32_t v, float m1, uint64_t) { return f32_to_bf16_sat((float)v * m1); },
              [&](uint16_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b16(x, out.r, o, 0, 0); });
    else
        store([](int32_t v, float m1, uint64_t w) { return requant8((float)v * m1, w); },
              [&](uint8_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b8(x, out.r, o, 0, 0); });
}

// QuantGroupMatmul: the m axis is split into G ragged groups (group_list), group g multiplies its rows by
// W[g].  The real tiles are ordered group-major, then n-tile, then m-tile within the group, and the order is cut
// into 8 contiguous ranges, one per XCD (workgroup ids go round-robin over the XCDs): an XCD then works on one
// or two experts' column ranges, so its L2 holds the weight columns it streams instead of every XCD fetching
// every expert's weights.  m-tiles never straddle a group.  The grid is sized for ceil(M / BM) + G m-tiles per
// n-tile; ids past the real tile count exit at once.
constexpr int GROUP_MAX = 1024;  // groups the tiled kernel takes (the host refuses more)

// exclusive prefix sum over the workgroup of one value per thread (NT threads); *total gets the full sum
template <int NT>
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* wtot, int64_t* total)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int64_t x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int64_t y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) wtot[w] = x;
    __syncthreads();
    int64_t base = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) {
        if (i < w) base += wtot[i];
        tot += wtot[i];
    }
    __syncthreads();  // wtot may be reused
    *total = tot;
    return base + x - v;
}

// WPE: waves per SIMD the register allocation must allow (2 for two 4-wave workgroups per CU)
// UA: X and W of any alignment and any K (GemmCoreUA)
// KW > 1 (one-wave tiles, few rows per group: decode-sized MoE batches): the workgroup's KW waves each run the tile's
// main loop on their own K / KW range in their own LDS ring, then sum their int32 accumulators through LDS (exact in
// any order) and wave 0 runs the epilogue
template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB = 64, int WPE = 1, bool BTR = false, bool UA = false,
          int KW = 1>
__global__ __launch_bounds__(WM * WN * 64 * KW, WPE) void group_gemm_i8_kernel(GroupGemmArgs p)
{
    // transposed accumulators: four consecutive output columns per register quad, stored as one 8-byte vector;
    // BTR: W given [G, K, N] staged by K rows and read with LDS transpose reads
    using T = I8Core<BM, BN, WM, WN, ST, TB, RB, true, BTR, UA>;
    static_assert(KW == 1 || (WM == 1 && WN == 1 && !UA), "k-split waves run one-wave tiles");
    constexpr int NTT = T::NT * KW;  // threads of the workgroup
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int64_t wtot[NTT / 64];
    __shared__ int64_t tile_info[4];  // group, first row, end row, first m-tile of this workgroup's tile
    // the tile's per-token (BM) and per-channel (BN) scales, copied global -> LDS by one wave-wide copy each
    // (1 KiB: lanes past the scales read zeros)
    static_assert(BM <= 256 && BN <= 256, "one 1 KiB copy per scale vector");
    __shared__ __attribute__((aligned(16))) float s_pt[256], s_sc[256];
    const int G = (int)p.G;
    const int64_t M = p.M;
    // Group g's rows are [start_g, end_g) clamped to [0, M) (rows outside [0, M) exist in no group) and its
    // m-tiles follow those of groups 0 .. g-1.  Thread t owns groups [t * per, (t + 1) * per): two block-wide
    // prefix sums (rows, then m-tiles) give every thread its groups' starts, and the thread owning this
    // workgroup's tile publishes it -- no G-sized table, so the LDS stays with the stage ring.
    const int per = (G + NTT - 1) / NTT, ga = (int)threadIdx.x * per;
    auto count = [&](int g) {
        const int64_t c = p.list_type == 0 ? p.group_list[g + 1] - p.group_list[g] : p.group_list[g];
        return c < 0 ? (int64_t)0 : c;
    };
    auto clampM = [&](int64_t v) { return v < 0 ? (int64_t)0 : (v > M ? M : v); };
    const int64_t base = p.list_type == 0 ? p.group_list[0] : 0;
    int64_t rows_total, tiles_total, mine = 0;
    for (int k = 0; k < per; ++k)
        if (ga + k < G) mine += count(ga + k);
    const int64_t s0 = base + block_exclusive_scan<NTT>(mine, wtot, &rows_total);
    mine = 0;
    {
        int64_t st = s0;
        for (int k = 0; k < per; ++k)
            if (ga + k < G) {
                const int64_t c = count(ga + k);
                mine += (clampM(st + c) - clampM(st) + BM - 1) / BM;
                st += c;
            }
    }
    const int64_t tiles_n = (p.N + BN - 1) / BN;
    const int64_t t0 = block_exclusive_scan<NTT>(mine, wtot, &tiles_total);
    const int64_t total = tiles_total * tiles_n;  // real (m-tile, n-tile) pairs
    const int64_t per_xcd = (total + 7) / 8;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = KW > 1 ? 0 : wave / WN, wn = KW > 1 ? 0 : wave % WN;
    const int kw = KW > 1 ? __builtin_amdgcn_readfirstlane(wave) : 0;
    {
        const int64_t lin = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        if ((int64_t)(blockIdx.x / 8) >= per_xcd || lin >= total) return;
        int64_t st = s0, tf = t0;
        for (int k = 0; k < per; ++k)
            if (ga + k < G) {
                const int64_t c = count(ga + k), a0 = clampM(st), a1 = clampM(st + c);
                const int64_t nt = (a1 - a0 + BM - 1) / BM;
                if (nt > 0 && tf * tiles_n <= lin && lin < (tf + nt) * tiles_n) {
                    tile_info[0] = ga + k;
                    tile_info[1] = a0;
                    tile_info[2] = a1;
                    tile_info[3] = tf;
                }
                st += c;
                tf += nt;
            }
        __syncthreads();
        // every lane reads the same values; readfirstlane keeps them (and the buffer resources built from them)
        // in scalar registers -- a resource in VGPRs costs a waterfall loop around every access
        const int g = __builtin_amdgcn_readfirstlane((int)tile_info[0]);
        const int64_t g_first = uniform64(tile_info[1]), m_end = uniform64(tile_info[2]);
        const int64_t g_tile0 = uniform64(tile_info[3]);
        const int64_t mt_g = (m_end - g_first + BM - 1) / BM;  // m-tiles of group g (>= 1 here)
        const int64_t rem = lin - g_tile0 * tiles_n;
        const int tn = __builtin_amdgcn_readfirstlane((int)(rem / mt_g));
        const int64_t m0 = uniform64(g_first + (rem % mt_g) * BM);
        const int64_t n0 = (int64_t)tn * BN;
        CoreArgs c{};
        uint32_t da = 0, db = 0;  // UA: the operands' offsets from their resources' 16-byte-aligned bases
        if constexpr (UA) {
            c.a = make_rsrc_a16(p.X, (uint32_t)(p.M * p.K), da);
            c.b = make_rsrc_a16(p.W + (int64_t)g * p.K * p.N, (uint32_t)(p.K * p.N), db);
        } else {
            c.a = make_rsrc(p.X, (uint32_t)(p.M * p.K));
            c.b = make_rsrc(p.W + (int64_t)g * p.K * p.N, (uint32_t)(p.K * p.N));
        }
        c.lda = (uint32_t)p.K;
        c.ldb = (uint32_t)(TB ? p.K : p.N);
        c.rows = (int32_t)(m_end - m0 < BM ? m_end - m0 : BM);
        c.cols = (int32_t)(p.N - n0 < BN ? p.N - n0 : BN);
        const int64_t kc = p.K / KW, k0 = kw * kc;  // this wave's K range (KW > 1: K % (KW RB) == 0)
        c.a0 = (uint32_t)(m0 * p.K + k0) + da;
        c.b0 = (uint32_t)(TB ? n0 * p.K + k0 : n0 + k0 * p.N) + db;
        c.kbytes = kc;

        // the epilogue's scales go global -> LDS now (waves 0 and 1, one copy each, no registers held), so their
        // latency hides under the main loop: the copies are older than the main loop's, whose first wait covers
        // them, and its first barrier publishes them.  Rows past the group and columns past N read 0.
        if (wave == 0)
            copy16_to_lds(make_rsrc(p.pts + m0, (uint32_t)(c.rows * 4)), (uint8_t*)s_pt, (uint32_t)lane * 16);
        else if (wave == 1)
            copy16_to_lds(make_rsrc(p.scale + (int64_t)g * p.N + n0, (uint32_t)(c.cols * 4)), (uint8_t*)s_sc,
                          (uint32_t)lane * 16);
        typename T::acc_t acc[T::FM][T::FN];
        T::run(c, smem + (KW > 1 ? kw * T::LDS_BYTES : 0), acc, KW > 1 ? lane : (int)threadIdx.x);
        if constexpr (KW > 1) {
            __syncthreads();  // every wave's main loop is done with its LDS ring
            constexpr int F = T::FM * T::FN;
            typename T::acc_t* red = (typename T::acc_t*)smem;  // [KW - 1][F][64 lanes] accumulator fragments
            if (kw > 0) {
#pragma unroll
                for (int f = 0; f < F; ++f) red[((kw - 1) * F + f) * 64 + lane] = acc[f / T::FN][f % T::FN];
            }
            __syncthreads();
            if (kw != 0) return;
#pragma unroll
            for (int w = 0; w < KW - 1; ++w)
#pragma unroll
                for (int f = 0; f < F; ++f) acc[f / T::FN][f % T::FN] += red[(w * F + f) * 64 + lane];
        }

        // epilogue (quant_group_matmul_custom.asc:424-452): AscendDequant acc*scale[g,n] in fp32 (its int32 -> fp32
        // conversion rounds ties away from zero above 2^24, as every AscendDequant here does), Mul by the
        // per-token scale in fp32, optional FasterGelu in fp32, one rounding cast to the output type.  Stores go
        // through a buffer resource over the output tile: rows past the group's end are out of its range.
        const TileOut out = tile_out(p.Y, m0, n0, p.N, c.rows, c.cols, 2);
        // Lane l holds, for each fragment row (i) and register quad q of each column fragment (j), the four columns
        // ct_col .. ct_col + 3 of row ct_row: with N a multiple of 4 and Y 8-byte aligned they leave as one 8-byte
        // store (a quad is wholly inside or wholly past the tile's columns, whose count is then a multiple of 4),
        // else as four 2-byte stores.
        const bool vec = p.N % 4 == 0 && ((uintptr_t)p.Y & 7) == 0;
        auto store = [&](auto cvt) {
#pragma unroll
            for (int i = 0; i < T::FM; ++i) {
                const int row = T::ct_row(wm, i, lane);
                const float pt = s_pt[row];
                const uint32_t roff = (uint32_t)row * out.pitch;
#pragma unroll
                for (int j = 0; j < T::FN; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int cl = T::ct_col(wn, j, q, lane);
                        const v4f sc = *(const v4f*)(s_sc + cl);
                        uint32_t h[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            float v = i32_to_f32_rna(acc[i][j][4 * q + e]) * sc[e];
                            v = v * pt;
                            h[e] = cvt(p.act ? faster_gelu(v) : v);
                        }
                        if (vec) {
                            const uint32_t off = cl < c.cols ? roff + (uint32_t)(cl * 2) : OOB;
                            __builtin_amdgcn_raw_buffer_store_b64((u32x2){h[0] | (h[1] << 16), h[2] | (h[3] << 16)},
                                                                  out.r, off, 0, 0);
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                __builtin_amdgcn_raw_buffer_store_b16((uint16_t)h[e], out.r,
                                                                      cl + e < c.cols ? roff + (uint32_t)((cl + e) * 2) : OOB,
                                                                      0, 0);
                        }
                    }
            }
        };
        if (p.out_type == DT_F16) store([](float v) { return (uint32_t)f32_to_f16_sat(v); });
        else store([](float v) { return (uint32_t)f32_to_bf16_sat(v); });
    }
}

// Any shape / layout / alignment: one thread per output element, int32 accumulate, same epilogue.
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(GemmI8Args p)
{
    const float mscalar = quant_pre_m1(p.qscalar);
    // acc + bias of element (m, n), int32 wrap-around as the MFMA accumulates
    auto value = [&](int64_t m, int64_t n) {
        uint32_t acc = 0;
        for (int64_t k = 0; k < p.K; ++k) {
            const int32_t a = p.trans_a ? p.A[k * p.lda + m] : p.A[m * p.lda + k];
            const int32_t b = p.trans_b ? p.B[n * p.ldb + k] : p.B[k * p.ldb + n];
            acc += (uint32_t)(a * b);
        }
        return (int32_t)(acc + (uint32_t)(p.bias ? p.bias[n] : 0));
    };
    if (p.epi == EPI_REQ4) {  // one thread per output byte (two int4 codes; N and ldc even)
        const int64_t half = p.N / 2, total = p.M * half;
        for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
            const int64_t m = e / half, n = 2 * (e % half);
            uint32_t q[2];
            for (int h = 0; h < 2; ++h) {
                const uint64_t w = p.qvec ? p.qvec[n + h] : p.qscalar;
                q[h] = requant4((float)value(m, n + h) * (p.qvec ? quant_pre_m1(w) : mscalar), w);
            }
            ((uint8_t*)p.C)[(m * p.ldc + n) / 2] = (uint8_t)(q[0] | (q[1] << 4));
        }
        return;
    }
    const int64_t total = p.M * p.N;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t m = e / p.N, n = e % p.N;
        const int32_t v = value(m, n);
        const uint64_t w = p.qvec ? p.qvec[n] : p.qscalar;
        const float m1 = p.qvec ? quant_pre_m1(w) : mscalar;
        const int64_t o = m * p.ldc + n;
        if (p.atomic != C_STORE) {  // int32 / f16 / bf16 C only (checked by the host layer)
            if (p.epi == EPI_I32) c_atomic<DT_INT32>((uint8_t*)p.C + 4 * o, (uint32_t)v, p.atomic);
            else if (p.epi == EPI_DEQ_F16) c_atomic<DT_F16>((uint8_t*)p.C + 2 * o, f32_to_f16_sat((float)v * m1), p.atomic);
            else c_atomic<DT_BF16>((uint8_t*)p.C + 2 * o, f32_to_bf16_sat((float)v * m1), p.atomic);
        } else if (p.epi == EPI_I32) ((int32_t*)p.C)[o] = v;
        else if (p.epi == EPI_DEQ_F16) ((uint16_t*)p.C)[o] = f32_to_f16_sat((float)v * m1);
        else if (p.epi == EPI_DEQ_BF16) ((uint16_t*)p.C)[o] = f32_to_bf16_sat((float)v * m1);
        else ((uint8_t*)p.C)[o] = requant8((float)v * m1, w);
    }
}

template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB = 64, bool BTR = false, int KW = 1, bool UA = false>
static hipError_t launch_tiled(const GemmI8Args& a, hipStream_t st)
{
    using T = I8Core<BM, BN, WM, WN, ST, TB, RB, false, BTR, UA>;
    const int tiles = (int)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    constexpr size_t lds = T::LDS_BYTES * KW;
    const hipError_t e = ensure_dynamic_lds<gemm_i8_kernel<BM, BN, WM, WN, ST, TB, RB, BTR, KW, UA>>((int)lds);
    if (e != hipSuccess) return e;
    launch_k((gemm_i8_kernel<BM, BN, WM, WN, ST, TB, RB, BTR, KW, UA>), dim3(tiles), dim3(T::NT * KW), (uint32_t)lds, st,
             a);
    return hipGetLastError();
}

// the K split across workgroups of decode-sized batches: 32-row one-wave tiles, four K-split waves per workgroup,
// splits chosen so that tiles x splits is about 256 (one workgroup per CU); K % 256 == 0.  B given [K, N]: 32 x 128
// tiles (whole 128-byte K-row runs), for long K or wide N only -- elsewhere the 32 x 32 K-split tiles measured faster
// (K = 11008 / 14336, N = 4096, M = 1: 36.6 / 45.8 -> 23.3 / 26.0 us; K = N = 8192: 32.1 -> 26.8 us; K = 4096,
// N = 14336: 29.9 -> 23.1 us; slower at K = 4096, N = 8192 / 11008).  B given [N, K]: the 32 x 32 tiles themselves,
// split when they are few (N / 32 well under 256) and K is long (K = 11008 / 14336, N = 4096, M = 16: 21.7 / 23.8 ->
// 17.1 / 19.6 us; slower at K = 4096: 9.1 against 8.4 us)
constexpr int DS_KW = 4, DS_RB = 64;
int decode_split_bn(int trans_b) { return trans_b ? 32 : 128; }
int decode_split_bm(int64_t M) { return M <= 32 ? 32 : 64; }  // one row tile for M <= 64
int decode_splits(int64_t M, int64_t N, int64_t K, int trans_b)
{
    if (M > 64 || M < 1 || N < 1 || K % (DS_KW * DS_RB) != 0) return 1;
    if (!(K >= 8192 || (!trans_b && N >= 12288))) return 1;
    const int64_t tiles = (N + decode_split_bn(trans_b) - 1) / decode_split_bn(trans_b);
    int64_t s = (256 + tiles / 2) / tiles;
    const int64_t units = K / (DS_KW * DS_RB);
    if (s > units) s = units;
    return s < 2 ? 1 : (int)s;
}
size_t decode_split_ws_bytes(int64_t M, int64_t N, int64_t K, int trans_b)
{
    const int s = decode_splits(M, N, K, trans_b), bn = decode_split_bn(trans_b), bm = decode_split_bm(M);
    return s < 2 ? 0 : (size_t)s * (size_t)((N + bn - 1) / bn) * (bm / 32) * (bn / 32) * 64 * 64;
}

template <bool TB, bool BTR, int BM, int BN, int ST>
static hipError_t launch_i8_split(GemmI8Args a, hipStream_t st)
{
    using T = I8Core<BM, BN, 1, 1, ST, TB, DS_RB, false, BTR, false>;
    const int tiles = (int)((a.N + BN - 1) / BN);
    constexpr size_t lds = T::LDS_BYTES * DS_KW;
    static_assert((size_t)(DS_KW - 1) * T::FM * T::FN * 64 * sizeof(typename T::acc_t) <= lds, "k-split reduction");
    hipError_t e = ensure_dynamic_lds<gemm_i8_kernel<BM, BN, 1, 1, ST, TB, DS_RB, BTR, DS_KW, false, 1>>((int)lds);
    if (e != hipSuccess) return e;
    launch_k((gemm_i8_kernel<BM, BN, 1, 1, ST, TB, DS_RB, BTR, DS_KW, false, 1>), dim3(tiles * a.splits),
             dim3(64 * DS_KW), (uint32_t)lds, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_k((gemm_i8_kernel<BM, BN, 1, 1, ST, TB, DS_RB, BTR, 1, false, 2>), dim3(tiles), dim3(T::FM * T::FN * 64), 0u,
             st, a);
    return hipGetLastError();
}

hipError_t launch_gemm_i8(const GemmI8Args& a, hipStream_t st)
{
    const bool a_ok = !a.trans_a && a.lda % 16 == 0 && ((uintptr_t)a.A % 16 == 0) && a.lda * a.M < (1ll << 31);
    const bool b_ok = a.trans_b ? (a.ldb % 16 == 0 && ((uintptr_t)a.B % 16 == 0) && a.ldb * a.N < (1ll << 31))
                                : (a.ldb % 4 == 0 && a.N % 4 == 0 && ((uintptr_t)a.B % 4 == 0) && a.ldb * a.K < (1ll << 31));
    // the tiled epilogue addresses a 256-row output tile with 32-bit offsets
    if (a_ok && b_ok && a.K % 16 == 0 && a.ldc < (1ll << 21)) {
        const bool big = a.M >= 1024 && a.N >= 1024;
        // small problems (the W8A8 sample, 128 x 256 x 512: 4 tiles of 64 x 128) take 32 x 32 single-wave tiles so
        // that at least 32 workgroups share the work
        const bool tiny = ((a.M + 63) / 64) * ((a.N + 127) / 128) < 32;
        // ... and, when K holds four 64-byte stages per wave and C is stored (not combined by enAtomic), each tile's K
        // split over four waves of one workgroup, so a tile's loads are all in flight at once.  Decode-sized batches
        // (B streamed once) take the same tiles up to 32 rows, and up to 64 while 64 x 64 tiles would leave fewer than
        // 160 workgroups (measured, DEQF16: K = 11008, N = 4096, M = 1 / 16 / 64 in 15.6 / 21.0 / 25.5 us against
        // 35.4 / 35.5 / 44.5 us on 64 x 64 tiles; at K = 4096, N = 11008, M = 64 the 172 tiles of 64 x 64 keep it, 18.8
        // against 21.4 us)
        const int64_t t64 = ((a.M + 63) / 64) * ((a.N + 63) / 64);
        const bool skinny = a.M <= 32 || (a.M <= 64 && t64 < 160);
        const bool ksplit = (tiny || skinny) && a.K % 256 == 0 && a.atomic == C_STORE;
        // decode-sized batches (up to 64 rows, one row tile of 32 or 64) with a workspace for the partials: the K split
        // across workgroups as well, where decode_splits finds it faster (B [K, N]: x 128 tiles; B [N, K]: x 32)
        const int splits = decode_splits(a.M, a.N, a.K, a.trans_b);
        if (!tiny && splits > 1 && a.atomic == C_STORE && a.epi != EPI_REQ4 && a.ws &&
            a.ws_bytes >= decode_split_ws_bytes(a.M, a.N, a.K, a.trans_b)) {
            GemmI8Args b = a;
            b.splits = splits;
            const bool m32 = a.M <= 32;
            if (a.trans_b)
                return m32 ? launch_i8_split<true, false, 32, 32, 4>(b, st) : launch_i8_split<true, false, 64, 32, 4>(b, st);
            if (a.ldb % 16 == 0 && (uintptr_t)a.B % 16 == 0)
                return m32 ? launch_i8_split<false, true, 32, 128, 3>(b, st)
                           : launch_i8_split<false, true, 64, 128, 3>(b, st);
        }
        // (33-64 rows: one 64-row tile per 32 columns, B read by one workgroup, where those tiles make one nearly full
        // round of 225-256 workgroups -- K = N = 8192, M = 64: 28.7 -> 23.2 us; K = 4096, N = 8192: 16.5 -> 14.7 us;
        // at N = 4096 / 2048 the two 32-row tiles are faster, 9.7 / 6.9 against 11.7 / 9.1 us, and at N = 9216
        // (288 such tiles, B [K, N]) 33.9 against 36.1 us)
        const bool m64x32 = a.M > 32 && a.N > 7168 && a.N <= 8192;
        if (ksplit && a.trans_b)
            return m64x32 ? launch_tiled<64, 32, 1, 1, 4, true, 64, false, 4>(a, st)
                          : launch_tiled<32, 32, 1, 1, 4, true, 64, false, 4>(a, st);
        // (B [K, N]: 32 x 64 tiles -- 64-byte K-row runs -- while they still give about 160 workgroups or more:
        // K = 4096, N = 11008, M = 1 / 16: 22.1 / 23.8 -> 18.1 / 19.7 us; at N = 4096 / 8192 the 32 x 32 tiles are
        // faster, 16.9 / 18.0 against 18.8 / 20.2 us)
        if (ksplit && a.ldb % 16 == 0 && (uintptr_t)a.B % 16 == 0)
            return a.N >= 10240 ? launch_tiled<32, 64, 1, 1, 4, false, 64, true, 4>(a, st)
                   : m64x32   ? launch_tiled<64, 32, 1, 1, 4, false, 64, true, 4>(a, st)
                                : launch_tiled<32, 32, 1, 1, 4, false, 64, true, 4>(a, st);
        if (a.trans_b)
            return big ? (a.K % 128 == 0 ? launch_tiled<256, 256, 4, 2, 2, true, 128>(a, st)
                                         : launch_tiled<256, 256, 4, 2, 4, true>(a, st))
                       : (tiny ? launch_tiled<32, 32, 1, 1, 4, true>(a, st) : launch_tiled<64, 64, 2, 2, 4, true>(a, st));
        // B [K, N] with 16-byte K rows (small and medium problems; the host transposes a large one first): the K
        // rows are copied like A's and read by LDS transpose reads.  For 256 x 256 tiles that measured slower than
        // the transpose plus the K-contiguous kernel (632.7 against 602 us at 8192^3: the 128-byte-stage form spills)
        if (!big && a.ldb % 16 == 0 && (uintptr_t)a.B % 16 == 0)
            return tiny ? launch_tiled<32, 32, 1, 1, 4, false, 64, true>(a, st)
                        : launch_tiled<64, 128, 2, 2, 4, false, 64, true>(a, st);
        if (tiny) return launch_tiled<32, 32, 1, 1, 4, false>(a, st);
        return big ? launch_tiled<256, 256, 4, 2, 4, false>(a, st) : launch_tiled<64, 128, 2, 2, 4, false>(a, st);
    }
    // K not a multiple of 16, or operands / leading dimensions not 16-byte (A, K-contiguous B) or 4-byte ([K, N] B)
    // aligned: the any-alignment tiles (GemmCoreUA), 64 x 64 while that leaves fewer than 256 workgroups of 128 x 128
    const int64_t a_span = a.lda * (a.M - 1) + a.K, b_span = a.trans_b ? a.ldb * (a.N - 1) + a.K : a.ldb * (a.K - 1) + a.N;
    const char* why = a.trans_a                            ? "A given [K, M]"
                      : (a_span >= (1ll << 31) - 16 || b_span >= (1ll << 31) - 16) ? "an operand spans 2^31 bytes"
                      : a.ldc >= (1ll << 21)               ? "ldc >= 2^21"
                                                           : nullptr;
    if (!why) {
        const bool small = ((a.M + 127) / 128) * ((a.N + 127) / 128) < 256;
        if (a.trans_b)
            return small ? launch_tiled<64, 64, 2, 2, 2, true, 64, false, 1, true>(a, st)
                         : launch_tiled<128, 128, 2, 2, 2, true, 64, false, 1, true>(a, st);
        return small ? launch_tiled<64, 64, 2, 2, 2, false, 64, true, 1, true>(a, st)
                     : launch_tiled<128, 128, 2, 2, 2, false, 64, true, 1, true>(a, st);
    }
    log_fallback("gemm_i8_generic_kernel", why);
    int64_t blocks = (a.M * a.N + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    launch_k(gemm_i8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
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
        float v = i32_to_f32_rna((int32_t)acc) * p.scale[(int64_t)g * p.N + n];
        v = v * p.pts[m];
        if (p.act) v = faster_gelu(v);
        if (p.out_type == DT_F16) ((uint16_t*)p.Y)[m * p.N + n] = f32_to_f16_sat(v);
        else ((uint16_t*)p.Y)[m * p.N + n] = f32_to_bf16_sat(v);
    }
}

template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB = 64, int WPE = 1, bool BTR = false, bool UA = false,
          int KW = 1>
static hipError_t launch_group_tiled(const GroupGemmArgs& a, hipStream_t st)
{
    using T = I8Core<BM, BN, WM, WN, ST, TB, RB, true, BTR, UA>;
    constexpr int LDS = (int)T::LDS_BYTES * KW;
    static_assert(KW == 1 || (size_t)(KW - 1) * T::FM * T::FN * 64 * sizeof(typename T::acc_t) <= (size_t)LDS,
                  "k-split reduction");
    const int64_t upper = ((a.M + BM - 1) / BM + a.G) * ((a.N + BN - 1) / BN);  // tiles, at most
    const hipError_t e = ensure_dynamic_lds<group_gemm_i8_kernel<BM, BN, WM, WN, ST, TB, RB, WPE, BTR, UA, KW>>(LDS);
    if (e != hipSuccess) return e;
    launch_k((group_gemm_i8_kernel<BM, BN, WM, WN, ST, TB, RB, WPE, BTR, UA, KW>), dim3((unsigned)((upper + 7) / 8 * 8)),
             dim3(T::NT * KW), LDS, st, a);
    return hipGetLastError();
}

hipError_t launch_group_gemm(const GroupGemmArgs& a, hipStream_t st)
{
    const char* why = a.G > GROUP_MAX                                          ? "more than 1024 groups"
                      : (a.M * a.K >= (1ll << 31) - 16 || a.K * a.N >= (1ll << 31) - 16) ? "an operand spans 2^31 bytes"
                      : a.N >= (1ll << 21)                                     ? "N >= 2^21"
                                                                               : nullptr;
    if (why) {
        log_fallback("group_gemm_generic_kernel", why);
        int64_t blocks = (a.M * a.N + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        if (blocks < 1) blocks = 1;
        launch_k(group_gemm_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    const bool aligned = a.K % 16 == 0 && ((uintptr_t)a.X % 16 == 0) &&
                         (a.w_trans ? ((uintptr_t)a.W % 16 == 0) : (a.N % 4 == 0 && (uintptr_t)a.W % 4 == 0));
    // K not a multiple of 16 or X / W not aligned: 128 x 128 tiles of GemmCoreUA, two workgroups per CU
    if (!aligned)
        return a.w_trans ? launch_group_tiled<128, 128, 2, 2, 2, true, 64, 2, false, true>(a, st)
                         : launch_group_tiled<128, 128, 2, 2, 2, false, 64, 2, true, true>(a, st);
    // decode-sized MoE batches (at most 16 rows per group on average, so most groups fill one 32-row tile and every
    // expert's weights are streamed about once): 32 x 32 tiles, each tile's K split over four waves of one
    // workgroup, so many more workgroups stream the weights than the 128 x 256 tiles give
    if (a.M <= 16 * a.G && a.K % 256 == 0) {
        if (a.w_trans) return launch_group_tiled<32, 32, 1, 1, 4, true, 64, 1, false, false, 4>(a, st);
        // (W [G, K, N]: 32 x 64 tiles -- 64-byte K-row runs -- from 8 rows per expert on average: 256 tokens over 16
        // experts in 41.9 against 46.9 us; at 64 tokens the 32 x 32 tiles are faster, 37.5 against 39.0 us)
        if (a.N % 16 == 0 && (uintptr_t)a.W % 16 == 0)
            return a.M >= 8 * a.G ? launch_group_tiled<32, 64, 1, 1, 4, false, 64, 1, true, false, 4>(a, st)
                                  : launch_group_tiled<32, 32, 1, 1, 4, false, 64, 1, true, false, 4>(a, st);
    }
    {
        // 128 x 256 tiles.  Short K (the reference sample's K = 1024): 4 waves with 64 x 128 wave tiles and
        // 64-byte stages, two workgroups per CU, so one's epilogue and its store / load latencies overlap the
        // other's MFMAs (measured 110-120 us against 145-150 us for one 8-wave workgroup per CU).  Long K (the
        // MoE shape, 4096 tokens, 16 experts, K = 4096, N = 1408: ~250 tiles, one per CU): 8 waves, 128-byte
        // stages (16 MFMAs per wave per barrier), three stages keep two in flight.
        if (a.w_trans && a.K <= 2048) return launch_group_tiled<128, 256, 2, 2, 3, true, 64, 2>(a, st);
        if (a.w_trans && a.K % 128 == 0) return launch_group_tiled<128, 256, 2, 4, 3, true, 128>(a, st);
        if (a.w_trans) return launch_group_tiled<128, 256, 2, 4, 6, true>(a, st);
        // W [G, K, N] with 16-byte K rows: the same tiles, K rows copied like A's and read by LDS transpose reads
        // (the 4-wave, two-workgroups-per-CU form of the short-K case spills here: 8 waves for every K)
        if (a.N % 16 == 0 && (uintptr_t)a.W % 16 == 0) {
            if (a.K % 128 == 0) return launch_group_tiled<128, 256, 2, 4, 3, false, 128, 1, true>(a, st);
            return launch_group_tiled<128, 256, 2, 4, 6, false, 64, 1, true>(a, st);
        }
        return launch_group_tiled<128, 128, 2, 2, 4, false>(a, st);
    }
}

}  // namespace ascq
