// gemm_f8.hip -- fp8 (e4m3fn / e5m2, any mix) x fp8 -> fp32 GEMM on CDNA4 MFMA with the fixpipe epilogue fused.
//
// Replaces the adv_api Matmul with fp8 A / B (examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_fp8/
// matmul_fp8.asc; L0C type fp32, impl/adv_api/detail/matmul/utils/matmul_utils.h:134-175) and its
// QF322F16_PRE / QF322BF16_PRE / QF322F32_PRE epilogue (stage/copy_cube_out/quant/quant_processor_fixpipe.h:101-115,
// mode rules quant_processor_utils.h:39-43):
//   out = cast((acc + bias[n]) * M1)   with M1 from SetQuantScalar / SetQuantVector (QUANT_PRE bits [31:13]),
//   out = cast(acc + bias[n])          without a quant word (F322F16 / F322BF16 / F32);
// int8 / uint8 C is (V)QF322B8_PRE (requant8: clamp, rint, + the word's offset, saturate by its sign flag) and
// fp8 C is (V)QF322FP8_PRE (f32_to_fp8: rne, e4m3 saturating at 448), both with a quant word.
// The float bias seeds the accumulator in the reference (MmadCompute with isBias, mmad_compute.h:40-90); adding
// it to the finished fp32 sum differs only by fp32 rounding.
//
// gfx950 design: the gemm_core.h main loop with v_mfma_f32_32x32x64_f8f6f4 (the f8f6f4 MFMA with zero scale
// operands), cbsz / blgp selecting e4m3 (0) or e5m2 (1) per operand: per lane 32 fp8 of one row in two
// register quads, 64 K per instruction (K order in gemm_core.h).  The instruction sums each group of 16
// consecutive K products (one register quad) aligned to the group's largest product and drops what falls below
// 2^(e_max - 13) (measured: 1 + 2^-15 gives 1 within a group and 1 + 2^-15 across groups or k-steps), so
// results differ from an fp32-accumulated sum by up to ~2^-13 of the group maxima.  gfx950's fp8 formats are
// the OCP ones: e4m3 with no infinities and S.1111.111 as NaN (fp8_e4m3fn_t) and IEEE-like e5m2 (fp8_e5m2_t).
// Tiles, stages and the [K, N] B register transpose are those of the int8 GEMM (fp8 operands are bytes like
// int8).
// hifloat8 operands (the sample's default scenario, MatmulFp8Kernel<hifloat8_t, hifloat8_t, float, float>,
// matmul_fp8.asc:229; A and B both hifloat8, README_en.md) have no gfx950 MFMA format, but every HiF8 value (a
// significand of at most 4 bits, 2^-22 .. 2^15, +-inf, NaN) is a bf16 value -- a normal one, where f16 would need
// subnormals below 2^-14 -- so the host layer decodes both operands to bf16 K-contiguous rows in the workspace and
// this kernel runs them through v_mfma_f32_32x32x16_bf16 (fmt code FMT_BF16, GemmCore OP_BF16) with the same fp32
// accumulators and epilogue.  C may be hifloat8 for either operand kind
// ((V)QF322HIF8_PRE, quant_processor_fixpipe.h:106-107: ties away from zero, saturating at +-32768, NaN -> 0 -- the
// saturation-mode row of matrix_compute_move_out_interface_boundary_value_summary.md:68-70).
#include "common.h"
#include "gemm_core.h"
#include "launch.h"

namespace ascq {

// fp8 bits -> fp32 (common.h), the format picked by its f8f6f4 code
__device__ __forceinline__ float fp8_to_f32(uint8_t v, int fmt) { return fp8_bits_to_f32(v, fmt != F8F6F4_E4M3); }
// element idx of an operand: fp8 bytes, or bf16 for FMT_BF16
__device__ __forceinline__ float op_elem(const uint8_t* p, int64_t idx, int fmt)
{
    return fmt == FMT_BF16 ? bf16_to_f32(((const uint16_t*)p)[idx]) : fp8_to_f32(p[idx], fmt);
}

// a 1-byte C element: (V)QF322B8_PRE for int8 / uint8, (V)QF322FP8_PRE, (V)QF322HIF8_PRE
__device__ __forceinline__ uint8_t byte_out(float v, uint64_t w, int c_type)
{
    if (c_type == DT_INT8 || c_type == DT_UINT8) return requant8(v, w);
    if (c_type == DT_HIF8) return (uint8_t)hif8_code_rna_sat(v);
    return f32_to_fp8(v, c_type == DT_FP8_E5M2 ? 1 : 0);
}

// w: the column's QUANT_PRE word (offset and sign flag of QF322B8); atomic: IterateAll's enAtomic (f32 / f16 /
// bf16 C only, checked by the host layer)
__device__ __forceinline__ void store_f8_out(void* C, int c_type, int64_t o, float v, uint64_t w, int atomic)
{
    if (atomic != C_STORE) {
        if (c_type == DT_F32) c_atomic<DT_F32>((uint8_t*)C + 4 * o, __float_as_uint(v), atomic);
        else if (c_type == DT_F16) c_atomic<DT_F16>((uint8_t*)C + 2 * o, f32_to_f16_sat(v), atomic);
        else c_atomic<DT_BF16>((uint8_t*)C + 2 * o, f32_to_bf16_sat(v), atomic);
    } else if (c_type == DT_F32) ((float*)C)[o] = v;
    else if (c_type == DT_F16) ((uint16_t*)C)[o] = f32_to_f16_sat(v);
    else if (c_type == DT_BF16) ((uint16_t*)C)[o] = f32_to_bf16_sat(v);
    else ((uint8_t*)C)[o] = byte_out(v, w, c_type);
}

// FMT: f8f6f4 codes of A (bits 0-2) and B (bits 3-5), or FMT_BF16 in both for bf16 operands
template <int FMT>
constexpr int op_of_fmt = (FMT == (FMT_BF16 | (FMT_BF16 << 3))) ? OP_BF16 : OP_F8;

// KW > 1 (one-wave tiles, B K-contiguous, f32 / f16 / bf16 C stored, not combined by enAtomic): the workgroup's KW
// waves each run the tile's main loop on their own K / KW range in their own LDS ring, then wave 0 adds the other
// waves' fp32 accumulators in wave order (one fixed order, so the result does not vary between calls) and runs the
// epilogue.  For decode-sized batches this puts a tile's whole K in flight at once instead of one serial ring.
// BTR (B given [K, N], 16-byte K rows): B's K rows are staged like A's and read by LDS transpose reads
// PH (K split across workgroups, decode-sized batches): 1 -- workgroup b runs split b / tiles of tile b % tiles, its K
// range a whole number of KW RB units (shared out as evenly as p.splits allows), and stores the tile's fp32
// accumulators in p.ws ([split][tile][fragment][lane]); 2 -- one wave per 32 x 32 fragment of a tile adds the
// splits' accumulators of its fragment in split order (one fixed order, so the result does not vary between calls)
// and stores it through the epilogue.
template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB, int FMT, bool UA = false, int KW = 1, bool BTR = false,
          int PH = 0>
__global__ __launch_bounds__(PH == 2 ? (BM / 32) * (BN / 32) * 64 : WM * WN * 64 * KW) void gemm_f8_kernel(GemmF8Args p)
{
    constexpr int OP = op_of_fmt<FMT>;
    constexpr int ES = OP == OP_BF16 ? 2 : 1;  // bytes per operand element
    // UA (fp8, B K-contiguous): operands of any alignment and any K (GemmCoreUA)
    using T = typename std::conditional<UA, GemmCoreUA<BM, BN, WM, WN, TB, false, OP, FMT>,
                                        GemmCore<BM, BN, WM, WN, ST, TB, OP, RB, FMT, true, false, BTR>>::type;
    static_assert(KW == 1 || (WM == 1 && WN == 1 && (TB || BTR) && !UA),
                  "k-split waves run one-wave tiles of a K-contiguous or LDS-transposed B");
    static_assert(PH == 0 || (WM == 1 && WN == 1 && !UA && ES == 1 && (PH == 2 || KW > 1)), "K split across workgroups");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_f8[];
    const int tiles_m = (int)((p.M + BM - 1) / BM), tiles_n = (int)((p.N + BN - 1) / BN);
    const int ntiles = tiles_m * tiles_n;
    const int tile = PH == 1 ? (int)blockIdx.x % ntiles : (int)blockIdx.x;
    const int split = PH == 1 ? (int)blockIdx.x / ntiles : 0;
    int tm, tn;
    tile_coords(tile, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    CoreArgs c{};
    const uint32_t a_bytes = (uint32_t)((p.lda * (p.M - 1) + p.K) * ES);
    const uint32_t b_bytes = (uint32_t)(TB ? (p.ldb * (p.N - 1) + p.K) * ES : p.ldb * (p.K - 1) + p.N);
    uint32_t da = 0, db = 0;  // UA: the operands' offsets from their resources' 16-byte-aligned bases
    if constexpr (UA) {
        c.a = make_rsrc_a16(p.A, a_bytes, da);
        c.b = make_rsrc_a16(p.B, b_bytes, db);
    } else {
        c.a = make_rsrc(p.A, a_bytes);
        c.b = make_rsrc(p.B, b_bytes);
    }
    c.lda = (uint32_t)(p.lda * ES);
    c.ldb = (uint32_t)(TB ? p.ldb * ES : p.ldb);
    c.rows = (int32_t)(p.M - m0 < BM ? p.M - m0 : BM);
    c.cols = (int32_t)(p.N - n0 < BN ? p.N - n0 : BN);
    const int kw = KW > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;
    int64_t kg0 = 0, kg = p.K;  // this workgroup's K range
    if constexpr (PH == 1) {
        const int64_t units = p.K / (KW * RB);
        const int64_t u0 = units * split / p.splits, u1 = units * (split + 1) / p.splits;
        kg0 = u0 * KW * RB;
        kg = (u1 - u0) * KW * RB;
    }
    const int64_t kc = kg / KW, k0 = kg0 + kw * kc;  // this wave's K range (KW > 1: K ES % (KW RB) == 0)
    c.a0 = (uint32_t)((m0 * p.lda + k0) * ES) + da;
    c.b0 = (uint32_t)(TB ? (n0 * p.ldb + k0) * ES : n0 + k0 * p.ldb) + db;
    c.kbytes = kc * ES;
    // KW > 1: the epilogue's bias and QUANT_PRE words are loaded before the main loop (their latency hides under it;
    // they are older than the main loop's copies, so its counted waits still cover exactly those copies)
    constexpr bool PRE = KW > 1 && PH == 0;
    float pre_bias[T::FN];
    uint64_t pre_w[T::FN];
    if constexpr (PRE) {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(0, j, (int)threadIdx.x & 63);
            const bool cok = cl < c.cols;
            pre_bias[j] = (p.bias && cok) ? p.bias[n0 + cl] : 0.0f;
            pre_w[j] = (p.qvec && cok) ? p.qvec[n0 + cl] : p.qscalar;
        }
    }
    typedef typename T::acc_t acc_t;
    acc_t acc[T::FM][T::FN];
    constexpr int F = T::FM * T::FN;  // accumulator fragments of the tile
    acc_t* part = (acc_t*)p.ws;       // PH 1 / 2: [split][tile][F][64 lanes]
    const int fw = PH == 2 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6) : 0;  // PH 2: this wave's fragment
    if constexpr (PH == 2) {
        const int ln = threadIdx.x & 63;
#pragma unroll
        for (int f = 0; f < F; ++f) {
            acc[f / T::FN][f % T::FN] = acc_t{};
            if (f != fw) continue;
            acc[f / T::FN][f % T::FN] = part[((int64_t)tile * F + f) * 64 + ln];
            for (int sp = 1; sp < p.splits; ++sp)
                acc[f / T::FN][f % T::FN] += part[(((int64_t)sp * ntiles + tile) * F + f) * 64 + ln];
        }
    } else {
        T::run(c, smem_f8 + (KW > 1 ? kw * T::LDS_BYTES : 0), acc, KW > 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x);
    }
    if constexpr (KW > 1) {
        __syncthreads();  // every wave's main loop is done with its LDS ring
        acc_t* red = (acc_t*)smem_f8;  // [KW - 1][F][64 lanes] accumulator fragments
        const int ln = threadIdx.x & 63;
        if (kw > 0) {
#pragma unroll
            for (int f = 0; f < F; ++f) red[((kw - 1) * F + f) * 64 + ln] = acc[f / T::FN][f % T::FN];
        }
        __syncthreads();
        if (kw != 0) return;
#pragma unroll
        for (int w = 0; w < KW - 1; ++w)
#pragma unroll
            for (int f = 0; f < F; ++f) acc[f / T::FN][f % T::FN] += red[(w * F + f) * 64 + ln];
    }
    if constexpr (PH == 1) {
        const int ln = threadIdx.x & 63;
#pragma unroll
        for (int f = 0; f < F; ++f) part[(((int64_t)split * ntiles + tile) * F + f) * 64 + ln] = acc[f / T::FN][f % T::FN];
        return;
    }

    // epilogue through a buffer resource over the output tile (rows past M dropped by its range)
    const int lane = threadIdx.x & 63, wave = PH == 2 ? 0 : threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const float mscalar = quant_pre_m1(p.qscalar);
    if (p.c_type == DT_INT4) {  // (V)QF322S4_PRE: int4 codes, two per byte
        const TileOut o4 = tile_out_int4(p.C, m0, n0, p.ldc, c.rows, c.cols);
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(wn, j, lane);
            const bool cok = cl < c.cols;
            const int64_t col = n0 + cl;
            const float bias = (p.bias && cok) ? p.bias[col] : 0.0f;
            const uint64_t w = (p.qvec && cok) ? p.qvec[col] : p.qscalar;
            const float m1 = p.qvec ? quant_pre_m1(w) : mscalar;
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = acc[i][j][r];
                    if (p.bias) v = v + bias;
                    store_int4_pair(o4, requant4(v * m1, w), cl, c.cols, lane,
                                    (uint32_t)T::frag_row(wm, i, r, lane) * o4.pitch);
                }
        }
        return;
    }
    const int esize = p.c_type == DT_F32 ? 4 : ((p.c_type == DT_F16 || p.c_type == DT_BF16) ? 2 : 1);
    const TileOut out = tile_out(p.C, m0, n0, p.ldc, c.rows, c.cols, esize);
    auto store = [&](auto conv, auto put) {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(wn, j, lane);
            const bool cok = cl < c.cols;
            const int64_t col = n0 + cl;
            const float bias = PRE ? pre_bias[j] : (p.bias && cok) ? p.bias[col] : 0.0f;
            const uint64_t w = PRE ? pre_w[j] : (p.qvec && cok) ? p.qvec[col] : p.qscalar;
            const float m1 = p.qvec ? quant_pre_m1(w) : mscalar;
            const uint32_t cbase = cok ? (uint32_t)(cl * esize) : OOB;
#pragma unroll
            for (int i = 0; i < T::FM; ++i) {
                if (PH == 2 && i * T::FN + j != fw) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = acc[i][j][r];
                    if (p.bias) v = v + bias;
                    if (p.use_quant) v = v * m1;
                    put(conv(v, w), cbase + (uint32_t)T::frag_row(wm, i, r, lane) * out.pitch);
                }
            }
        }
    };
    if (KW == 1 && p.atomic != C_STORE) {  // enAtomic: f32 / f16 / bf16 C (the host layer refuses the others)
        // (acc + bias) x M1 of the column -- the store path's arithmetic
        auto v = [&](int cl, uint32_t a) {
            float x = __uint_as_float(a);
            if (p.bias) x = x + p.bias[n0 + cl];
            if (p.use_quant) x = x * (p.qvec ? quant_pre_m1(p.qvec[n0 + cl]) : mscalar);
            return x;
        };
        if (p.c_type == DT_F32)
            atomic_epilogue<T, DT_F32>(smem_f8, acc, out, c.rows, c.cols, p.atomic,
                                       [&](int cl, uint32_t a) { return __float_as_uint(v(cl, a)); });
        else if (p.c_type == DT_F16)
            atomic_epilogue<T, DT_F16>(smem_f8, acc, out, c.rows, c.cols, p.atomic,
                                       [&](int cl, uint32_t a) { return (uint32_t)f32_to_f16_sat(v(cl, a)); });
        else
            atomic_epilogue<T, DT_BF16>(smem_f8, acc, out, c.rows, c.cols, p.atomic,
                                        [&](int cl, uint32_t a) { return (uint32_t)f32_to_bf16_sat(v(cl, a)); });
        return;
    }
    auto put32 = [&](uint32_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b32(x, out.r, o, 0, 0); };
    auto put16 = [&](uint16_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b16(x, out.r, o, 0, 0); };
    auto put8 = [&](uint8_t x, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b8(x, out.r, o, 0, 0); };
    if (p.c_type == DT_F32) store([](float v, uint64_t) { return __float_as_uint(v); }, put32);
    else if (p.c_type == DT_F16) store([](float v, uint64_t) { return f32_to_f16_sat(v); }, put16);
    else if (p.c_type == DT_BF16) store([](float v, uint64_t) { return f32_to_bf16_sat(v); }, put16);
    else {
        // the 1-byte C types -- int8 / uint8 (QF322B8), fp8 (QF322FP8), hifloat8 (QF322HIF8) -- in the rolled
        // epilogue: one more unrolled store loop (the hifloat8 encoder alone is ~30 instructions per element) grew
        // the kernel until the compiler kept the accumulators in scratch memory in the main loop
        rolled_epilogue<T>(smem_f8, acc, c.rows, c.cols, [&](int rr, int cc, uint32_t a) {
            float v = __uint_as_float(a);
            const int64_t col = n0 + cc;
            if (p.bias) v = v + p.bias[col];
            const uint64_t w = p.qvec ? p.qvec[col] : p.qscalar;
            if (p.use_quant) v = v * (p.qvec ? quant_pre_m1(w) : mscalar);
            __builtin_amdgcn_raw_buffer_store_b8(byte_out(v, w, p.c_type), out.r, (uint32_t)rr * out.pitch + (uint32_t)cc,
                                                 0, 0);
        });
    }
}

// Any shape / layout / alignment: one thread per output element, fp32 accumulation in k order.
__global__ __launch_bounds__(256) void gemm_f8_generic_kernel(GemmF8Args p)
{
    const float mscalar = quant_pre_m1(p.qscalar);
    // (acc + bias) * M1 of element (m, n), fp32 accumulation in k order
    auto value = [&](int64_t m, int64_t n, uint64_t w) {
        float acc = 0.0f;
        for (int64_t k = 0; k < p.K; ++k) {
            const float a = op_elem(p.A, p.trans_a ? k * p.lda + m : m * p.lda + k, p.fmt_a);
            const float b = op_elem(p.B, p.trans_b ? n * p.ldb + k : k * p.ldb + n, p.fmt_b);
            acc = acc + a * b;  // the product of two fp8 (or two decoded hifloat8) values is exact in fp32
        }
        if (p.bias) acc = acc + p.bias[n];
        if (p.use_quant) acc = acc * (p.qvec ? quant_pre_m1(w) : mscalar);
        return acc;
    };
    if (p.c_type == DT_INT4) {  // one thread per output byte (two int4 codes; N and ldc even)
        const int64_t half = p.N / 2, total = p.M * half;
        for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
            const int64_t m = e / half, n = 2 * (e % half);
            uint32_t q[2];
            for (int h = 0; h < 2; ++h) {
                const uint64_t w = p.qvec ? p.qvec[n + h] : p.qscalar;
                q[h] = requant4(value(m, n + h, w), w);
            }
            ((uint8_t*)p.C)[(m * p.ldc + n) / 2] = (uint8_t)(q[0] | (q[1] << 4));
        }
        return;
    }
    const int64_t total = p.M * p.N;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t m = e / p.N, n = e % p.N;
        const uint64_t w = p.qvec ? p.qvec[n] : p.qscalar;
        store_f8_out(p.C, p.c_type, m * p.ldc + n, value(m, n, w), w, p.atomic);
    }
}

template <int BM, int BN, int WM, int WN, int ST, bool TB, int RB, int FMT, bool UA = false, int KW = 1, bool BTR = false>
static hipError_t launch_f8_tiled(const GemmF8Args& a, hipStream_t st)
{
    using T = typename std::conditional<UA, GemmCoreUA<BM, BN, WM, WN, TB, false, op_of_fmt<FMT>, FMT>,
                                        GemmCore<BM, BN, WM, WN, ST, TB, op_of_fmt<FMT>, RB, FMT, true, false, BTR>>::type;
    constexpr int LDS = (int)T::LDS_BYTES * KW;
    static_assert(KW == 1 || (size_t)(KW - 1) * T::FM * T::FN * 64 * sizeof(typename T::acc_t) <= (size_t)LDS,
                  "k-split reduction");
    const int tiles = (int)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    const hipError_t e = ensure_dynamic_lds<gemm_f8_kernel<BM, BN, WM, WN, ST, TB, RB, FMT, UA, KW, BTR>>(LDS);
    if (e != hipSuccess) return e;
    launch_k((gemm_f8_kernel<BM, BN, WM, WN, ST, TB, RB, FMT, UA, KW, BTR>), dim3(tiles), dim3(T::NT * KW), LDS, st, a);
    return hipGetLastError();
}

// the K split across workgroups of decode-sized batches (decode_splits): one-wave tiles of 32 or 64 rows (one row
// tile; B [K, N]: x 128, K rows read by LDS transpose reads; B [N, K]: x 32), four K-split waves per workgroup; fp32
// partials in a.ws, added in split order by the second launch
template <int FMT, bool TB, int BM, int BN, int ST>
static hipError_t launch_f8_split(GemmF8Args a, hipStream_t st)
{
    constexpr int KWS = 4, RB = 64;
    constexpr bool BTR = !TB;
    using T = GemmCore<BM, BN, 1, 1, ST, TB, op_of_fmt<FMT>, RB, FMT, true, false, BTR>;
    const int tiles = (int)((a.N + BN - 1) / BN);
    constexpr size_t lds = T::LDS_BYTES * KWS;
    static_assert((size_t)(KWS - 1) * T::FM * T::FN * 64 * sizeof(typename T::acc_t) <= lds, "k-split reduction");
    hipError_t e = ensure_dynamic_lds<gemm_f8_kernel<BM, BN, 1, 1, ST, TB, RB, FMT, false, KWS, BTR, 1>>((int)lds);
    if (e != hipSuccess) return e;
    launch_k((gemm_f8_kernel<BM, BN, 1, 1, ST, TB, RB, FMT, false, KWS, BTR, 1>), dim3(tiles * a.splits),
             dim3(64 * KWS), (uint32_t)lds, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_k((gemm_f8_kernel<BM, BN, 1, 1, ST, TB, RB, FMT, false, 1, BTR, 2>), dim3(tiles), dim3(T::FM * T::FN * 64), 0u,
             st, a);
    return hipGetLastError();
}

template <int FMT>
static hipError_t launch_f8_fmt(const GemmF8Args& a, bool ua, hipStream_t st)
{
    constexpr int ES = op_of_fmt<FMT> == OP_BF16 ? 2 : 1;
    // fp8 operands of any alignment / any K with a K-contiguous B: GemmCoreUA tiles, 64 x 64 while 128 x 128 would
    // leave fewer than 256 workgroups
    if constexpr (ES == 1) {
        if (ua)
            return ((a.M + 127) / 128) * ((a.N + 127) / 128) < 256 ? launch_f8_tiled<64, 64, 2, 2, 2, true, 64, FMT, true>(a, st)
                                                                  : launch_f8_tiled<128, 128, 2, 2, 2, true, 64, FMT, true>(a, st);
    }
    if (ua) return hipErrorInvalidValue;
    const bool big = a.M >= 1024 && a.N >= 1024;
    // decode-sized batches (B streamed once) with a K-contiguous B and f32 / f16 / bf16 C stored: 32 x 32 tiles,
    // each tile's K split over four waves of one workgroup, up to 32 rows, and up to 64 while 64 x 64 tiles would
    // leave fewer than 160 workgroups (the int8 Matmul's rule; 33-64 rows take 64 x 32 tiles where those make one
    // nearly full round of 225-256 workgroups: K = N = 8192, M = 64: 29.1 -> 24.6 us)
    const int64_t t64 = ((a.M + 63) / 64) * ((a.N + 63) / 64);
    const bool skinny = a.M <= 32 || (a.M <= 64 && t64 < 160);
    const bool c_wide = a.c_type == DT_F32 || a.c_type == DT_F16 || a.c_type == DT_BF16;
    const bool m64x32 = a.M > 32 && a.N > 7168 && a.N <= 8192;
    if constexpr (ES == 1) {
        // with a workspace for the partials, the K split across workgroups as well where decode_splits (the int8
        // Matmul's rule) finds it faster: B [N, K] on the 32 x 32 tiles, B [K, N] (16-byte K rows) on 32 x 128 tiles
        const int splits = decode_splits(a.M, a.N, a.K, a.trans_b);
        const bool b_tr = !a.trans_b && a.ldb % 16 == 0 && (uintptr_t)a.B % 16 == 0;
        if ((a.trans_b || b_tr) && splits > 1 && c_wide && a.atomic == C_STORE && a.ws &&
            a.ws_bytes >= decode_split_ws_bytes(a.M, a.N, a.K, a.trans_b) &&
            ((a.M + 63) / 64) * ((a.N + 127) / 128) >= 32) {
            GemmF8Args b = a;
            b.splits = splits;
            if (a.M <= 32)
                return a.trans_b ? launch_f8_split<FMT, true, 32, 32, 4>(b, st)
                                 : launch_f8_split<FMT, false, 32, 128, 3>(b, st);
            return a.trans_b ? launch_f8_split<FMT, true, 64, 32, 4>(b, st) : launch_f8_split<FMT, false, 64, 128, 3>(b, st);
        }
        if (a.trans_b && skinny && c_wide && a.atomic == C_STORE && a.K % 256 == 0)
            return m64x32 ? launch_f8_tiled<64, 32, 1, 1, 4, true, 64, FMT, false, 4>(a, st)
                          : launch_f8_tiled<32, 32, 1, 1, 4, true, 64, FMT, false, 4>(a, st);
        // ... and with B given [K, N] (16-byte K rows): B's K rows staged like A's, read by LDS transpose reads
        // (32 x 64 tiles from N = 10240 on, as the int8 Matmul: K = 4096, N = 11008, M = 1 / 16: 22.8 / 24.6 ->
        // 21.4 / 21.6 us)
        if (b_tr && skinny && c_wide && a.atomic == C_STORE && a.K % 256 == 0)
            return a.N >= 10240 ? launch_f8_tiled<32, 64, 1, 1, 4, false, 64, FMT, false, 4, true>(a, st)
                   : m64x32   ? launch_f8_tiled<64, 32, 1, 1, 4, false, 64, FMT, false, 4, true>(a, st)
                                : launch_f8_tiled<32, 32, 1, 1, 4, false, 64, FMT, false, 4, true>(a, st);
    }
    if (a.trans_b) {
        if (big) return (a.K * ES) % 128 == 0 ? launch_f8_tiled<256, 256, 4, 2, 2, true, 128, FMT>(a, st)
                                              : launch_f8_tiled<256, 256, 4, 2, 4, true, 64, FMT>(a, st);
        return launch_f8_tiled<64, 64, 2, 2, 4, true, 64, FMT>(a, st);
    }
    // a large [K, N] B is transposed by the host layer first; this in-loop transpose serves the rest (fp8 only: the
    // bf16 operands of a hifloat8 Matmul are always K-contiguous)
    // (16-byte K rows: staged like A's and read by LDS transpose reads, as the int8 Matmul does -- K = 4096,
    // N = 11008, M = 64: 37.8 -> 23.6 us; otherwise the in-register byte transpose)
    if constexpr (ES == 1) {
        if (a.ldb % 16 == 0 && (uintptr_t)a.B % 16 == 0)
            return launch_f8_tiled<64, 128, 2, 2, 4, false, 64, FMT, false, 1, true>(a, st);
        return launch_f8_tiled<64, 128, 2, 2, 4, false, 64, FMT>(a, st);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemm_f8(const GemmF8Args& a, hipStream_t st)
{
    const bool bf = a.fmt_a == FMT_BF16 && a.fmt_b == FMT_BF16;
    if (!bf &&
        ((a.fmt_a != F8F6F4_E4M3 && a.fmt_a != F8F6F4_E5M2) || (a.fmt_b != F8F6F4_E4M3 && a.fmt_b != F8F6F4_E5M2)))
        return hipErrorInvalidValue;
    if (bf && (a.trans_a || !a.trans_b)) return hipErrorInvalidValue;
    const int64_t es = bf ? 2 : 1;
    const bool a_ok = !a.trans_a && (a.lda * es) % 16 == 0 && ((uintptr_t)a.A % 16 == 0) && a.lda * es * a.M < (1ll << 31);
    const bool b_ok = a.trans_b ? ((a.ldb * es) % 16 == 0 && ((uintptr_t)a.B % 16 == 0) && a.ldb * es * a.N < (1ll << 31))
                                : (a.ldb % 4 == 0 && a.N % 4 == 0 && ((uintptr_t)a.B % 4 == 0) && a.ldb * a.K < (1ll << 31));
    // the tiled epilogue addresses a 256-row output tile with 32-bit offsets
    const bool tiled = a_ok && b_ok && (a.K * es) % 16 == 0 && a.ldc < (1ll << 21);
    // otherwise fp8 with A [M, K] and B [N, K] (any alignment, any K) takes the any-alignment tiles
    const char* why = tiled ? nullptr
                      : bf ? "bf16 operands: K not a multiple of 8"
                      : a.trans_a ? "A given [K, M]"
                      : !a.trans_b ? "B given [K, N] with K not a multiple of 16 or operands not aligned"
                      : (a.lda * (a.M - 1) + a.K >= (1ll << 31) - 16 || a.ldb * (a.N - 1) + a.K >= (1ll << 31) - 16)
                          ? "an operand spans 2^31 bytes"
                      : a.ldc >= (1ll << 21) ? "ldc >= 2^21"
                                             : nullptr;
    if (!why) {
        if (bf) return launch_f8_fmt<FMT_BF16 | (FMT_BF16 << 3)>(a, false, st);
        switch (a.fmt_a | (a.fmt_b << 3)) {
        case F8F6F4_E4M3 | (F8F6F4_E4M3 << 3): return launch_f8_fmt<F8F6F4_E4M3 | (F8F6F4_E4M3 << 3)>(a, !tiled, st);
        case F8F6F4_E5M2 | (F8F6F4_E5M2 << 3): return launch_f8_fmt<F8F6F4_E5M2 | (F8F6F4_E5M2 << 3)>(a, !tiled, st);
        case F8F6F4_E4M3 | (F8F6F4_E5M2 << 3): return launch_f8_fmt<F8F6F4_E4M3 | (F8F6F4_E5M2 << 3)>(a, !tiled, st);
        default: return launch_f8_fmt<F8F6F4_E5M2 | (F8F6F4_E4M3 << 3)>(a, !tiled, st);
        }
    }
    log_fallback("gemm_f8_generic_kernel", why);
    int64_t blocks = (a.M * a.N + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    launch_k(gemm_f8_generic_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace ascq
