// mx_gemm.hip -- MX block-scaled GEMM on gfx950: E2M1 (MX-FP4) or fp8 e4m3fn / e5m2 (MX-FP8) elements with one
// E8M0 scale per 32 K.
//
// Reference: Matmul<MatmulTypeWithScale<..., fp4x2_e2m1_t | fp8_e4m3fn_t | fp8_e5m2_t, ...>> with
// SetTensorScaleA/B and IterateAll (impl/adv_api/detail/matmul/mx_matmul_impl.h:136-188; MmadMx
// include/basic_api/kernel_operator_mm_intf.h:348-352), fp32 accumulation, F322BF16 (rint) in the fixpipe.
// Golden: matmul_mxfp4_high_performance/scripts/gen_data.py; the MX-FP8 sample is
// examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_mx/matmul_mx.asc:90-244 (e5m2 elements, fp32 C).
//
// gfx950 design: the LDS-ring main loop of gemm_core.h with v_mfma_scale_f32_32x32x64_f8f6f4, both formats
// FP4 (cbsz = blgp = 4): per lane 32 E2M1 values (16 bytes, one MX block) of row (lane % 32) at k block
// (lane / 32), and one E8M0 scale byte for that (row, block) -- the hardware applies 2^(e-127) per 32-element
// block, which is exactly the MX product.  Two fp4 per byte, even k in the low nibble: the reference packing
// (gen_data.py:25-34) is also the MFMA's nibble order.  Block tile 256 x 256, 256 fp4 of K per stage (128-byte
// rows, four k-steps per barrier), two stages, 8 waves (4 x 2), wave tile 64 x 128.  The E8M0 scales, rearranged
// stage-major by mx_scale_stage_major_kernel, ride in the same LDS stage.  B stored [K, N]
// (the reference's non-transposed layout, two fp4 per byte along N) is first transposed to [N, K] in a
// workspace by fp4_transpose_kernel.
//
// E1M2 elements (fp4x2_e1m2_t, the reference's high-performance MX sample) have no gfx950 format, but every E1M2
// value k/4 (k = 0..7) is exact in fp6 E2M3, a native format of the same instruction at the fp4 rate, and so is
// every E2M1 value.  When either operand is E1M2 both are rewritten to fp6 by fp4_to_fp6_planes_kernel and
// multiplied by the OP_MXFP6 form of the core (cbsz = blgp = 2): per lane 32 fp6 of row (lane % 32), MX block
// (lane / 32), packed 6 bits each (element i at bits 6i .. 6i + 5 of six registers: the layout measured for the
// fp6 operand matches fp4's lane / block assignment).  The six registers are split into two planes so the P
// plane (registers 0-3) is staged exactly like fp4 and the Q plane (registers 4-5) rides in 1 KiB blocks like
// the scales; three stages of 256 x 256 (50 KiB each) fit the 160 KiB of LDS.
//
// MX-FP8 uses the same instruction with fp8 format codes: per lane 32 fp8 of one row (32 bytes, two register
// quads; MX block b of a k-step is quad b of all 64 lanes, see gemm_core.h);
// 128 fp8 of K per 128-byte stage row (two k-steps, a 32-bit word of scales per row), two stages of 256 x 256.
// A [K, N] fp8 B is transposed to [N, K] by the byte transpose first.
#include "common.h"
#include "gemm_core.h"
#include "launch.h"

namespace ascq {

// scale blocks per row in the stage-major copies: sK rounded up to whole groups of the largest stage (8 blocks)
__host__ __device__ inline int64_t sk_stage_major(int64_t K) { return ((K + 63) / 64 * 2 + 7) / 8 * 8; }

// DIRECT (the core's SC_DIRECT): the scales are read as given -- A row-major [M, sK], B row-major [N, sK] (1) or in
// block pairs [sK / 2, N, 2] (2) -- by the core's copies (sa_sm / sb_sm unused); 0: from the stage-major copies at
// sa_sm / sb_sm
// PH (K split across workgroups; decode tiles with direct scales): 1 -- workgroup b runs split b / tiles of tile
// b % tiles over a whole number of stages (shared out as evenly as p.splits allows; the scale resources start at the
// split's first stage) and stores its waves' fp32 accumulators in p.ws_part ([split][tile][wave][fragment][lane]);
// 2 -- the same waves add the splits' accumulators in split order and run the epilogue.
template <int BM, int BN, int WM, int WN, int ST, int RB, int OP, int FMT, bool ILV = true, int DIRECT = 0, int PH = 0>
__global__ __launch_bounds__(WM * WN * 64) void mx_gemm_kernel(MxGemmArgs p, const uint8_t* __restrict__ sa_sm,
                                                                const uint8_t* __restrict__ sb_sm)
{
    using T = GemmCore<BM, BN, WM, WN, ST, true, OP, RB, FMT, ILV, false, false, DIRECT>;
    static_assert(PH == 0 || (DIRECT && OP != OP_MXFP6), "K split across workgroups: tiles with direct scales");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem_mx[];
    const int64_t M = p.M, N = p.N, K = p.K;
    const int64_t KB = OP == OP_MXF8 ? K : K / 2;  // bytes per row (fp6: of the P plane)
    const int tiles_m = (int)((M + BM - 1) / BM), tiles_n = (int)((N + BN - 1) / BN);
    const int ntiles = tiles_m * tiles_n;
    const int tile = PH == 1 ? (int)blockIdx.x % ntiles : (int)blockIdx.x;
    const int split = PH == 1 ? (int)blockIdx.x / ntiles : 0;
    int tm, tn;
    tile_coords(tile, tiles_m, tiles_n, tm, tn);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t sK = (K + 63) / 64 * 2;
    CoreArgs c{};
    c.a = make_rsrc(p.A, (uint32_t)(M * KB));
    c.b = make_rsrc(p.B, (uint32_t)(N * KB));
    c.lda = c.ldb = (uint32_t)KB;
    c.rows = (int32_t)(M - m0 < BM ? M - m0 : BM);
    c.cols = (int32_t)(N - n0 < BN ? N - n0 : BN);
    int64_t u0 = 0;  // PH 1: this workgroup's first stage; its K bytes (otherwise the whole row, a last stage partial)
    c.kbytes = KB;
    if constexpr (PH == 1) {
        const int64_t units = KB / RB;
        u0 = units * split / p.splits;
        c.kbytes = (units * (split + 1) / p.splits - u0) * RB;
    }
    c.a0 = (uint32_t)(m0 * KB + u0 * RB);
    c.b0 = (uint32_t)(n0 * KB + u0 * RB);
    // One resource over every auxiliary region (launch_mx_gemm checks the layout): the stage-major scales (which
    // carry 16 bytes of slack, so a 16-byte copy at the end never straddles the range) and, for fp6, the Q planes
    // before them: [Aq][P plane of B][Bq][scales of A][scales of B].
    if constexpr (DIRECT) {
        // from stage u0 on: row-major rows advance SCB bytes a stage, pair planes SCB N bytes
        const int64_t sa_off = u0 * T::SCB, sb_off = u0 * T::SCB * (DIRECT == 2 ? N : 1);
        c.aux = make_rsrc(p.sA + sa_off, (uint32_t)(M * sK - sa_off));
        c.aux_b = make_rsrc(p.sB + sb_off, (uint32_t)(N * sK - sb_off));
    } else {
        const uint8_t* aux = OP == OP_MXFP6 ? p.Aq : sa_sm;
        c.aux = make_rsrc(aux, (uint32_t)(sb_sm - aux) + (uint32_t)(N * sk_stage_major(K) + 16));
        c.sa_base = (uint32_t)(sa_sm - aux);
        c.sb_base = (uint32_t)(sb_sm - aux);
    }
    if constexpr (OP == OP_MXFP6) {
        const uint32_t ga = (uint32_t)((M + 31) / 32), gb = (uint32_t)((N + 31) / 32);
        c.qa_stride = ga * 1024u;
        c.qb_stride = gb * 1024u;
        c.qa_off = (uint32_t)(m0 / 32) * 1024u;
        c.qb_off = (uint32_t)(p.Bq - p.Aq) + (uint32_t)(n0 / 32) * 1024u;
    }
    c.sa0_row = (uint32_t)m0;
    c.sb0_row = (uint32_t)n0;
    c.sa_rows = (uint32_t)M;
    c.sb_rows = (uint32_t)N;
    c.sk = (uint32_t)sK;
    typedef typename T::acc_t acc_t;
    acc_t acc[T::FM][T::FN];
    constexpr int F = T::FM * T::FN;  // accumulator fragments of a wave
    acc_t* part = (acc_t*)p.ws_part;  // PH 1 / 2: [split][tile][wave][F][64 lanes]
    const int pw = (int)threadIdx.x >> 6, pl = (int)threadIdx.x & 63;
    if constexpr (PH == 2) {
#pragma unroll
        for (int f = 0; f < F; ++f) acc[f / T::FN][f % T::FN] = part[(((int64_t)tile * T::NW + pw) * F + f) * 64 + pl];
        for (int sp = 1; sp < p.splits; ++sp)
#pragma unroll
            for (int f = 0; f < F; ++f)
                acc[f / T::FN][f % T::FN] += part[((((int64_t)sp * ntiles + tile) * T::NW + pw) * F + f) * 64 + pl];
    } else {
        T::run(c, smem_mx, acc);
    }
    if constexpr (PH == 1) {
#pragma unroll
        for (int f = 0; f < F; ++f)
            part[((((int64_t)split * ntiles + tile) * T::NW + pw) * F + f) * 64 + pl] = acc[f / T::FN][f % T::FN];
        return;
    }

    // epilogue through a buffer resource over the output tile (rows past M dropped by its range)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int esize = p.c_type == DT_F32 ? 4 : 2;
    const TileOut out = tile_out(p.C, m0, n0, N, c.rows, c.cols, esize);
    auto store = [&](auto put) {
#pragma unroll
        for (int j = 0; j < T::FN; ++j) {
            const int cl = T::frag_col(wn, j, lane);
            const uint32_t cbase = cl < c.cols ? (uint32_t)(cl * esize) : OOB;
            const float bias = (p.bias && cl < c.cols) ? p.bias[n0 + cl] : 0.0f;
#pragma unroll
            for (int i = 0; i < T::FM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = acc[i][j][r];
                    if (p.bias) v = v + bias;
                    put(v, cbase + (uint32_t)T::frag_row(wm, i, r, lane) * out.pitch);
                }
        }
    };
    if (p.atomic != C_STORE) {  // enAtomic: acc + bias, then the output cast -- the store path's arithmetic
        auto v = [&](int cl, uint32_t a) { return p.bias ? __uint_as_float(a) + p.bias[n0 + cl] : __uint_as_float(a); };
        if (p.c_type == DT_F32)
            atomic_epilogue<T, DT_F32>(smem_mx, acc, out, c.rows, c.cols, p.atomic,
                                       [&](int cl, uint32_t a) { return __float_as_uint(v(cl, a)); });
        else
            atomic_epilogue<T, DT_BF16>(smem_mx, acc, out, c.rows, c.cols, p.atomic,
                                        [&](int cl, uint32_t a) { return (uint32_t)f32_to_bf16_sat(v(cl, a)); });
        return;
    }
    if (p.c_type == DT_F32)
        store([&](float v, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), out.r, o, 0, 0); });
    else
        store([&](float v, uint32_t o) { __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_sat(v), out.r, o, 0, 0); });
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

// fp4 -> fp6 E2M3 split planes.  A nibble s|abc is E1M2 (sign, 1-bit exponent, 2-bit mantissa, value abc / 4) or
// E2M1 (sign, 2-bit exponent, 1-bit mantissa, bias 1); its E2M3 code (sign, 2-bit exponent, 3-bit mantissa,
// bias 1) is s|0abc|0 for E1M2 (abc / 4 = a.bc, or 0.bc when a = 0) and s|abc|00 for E2M1 -- both exact, signed
// zero included.  Each MX block's 32 codes pack into six dwords (element i at bits 6i .. 6i + 5); dwords 0-3 go to
// P (block b of row r at byte r K/2 + 16 b) and dwords 4-5 to Q ([stage t = b / 4][32-row group][b % 4][row % 32]
// x 8 bytes).  Workgroup (x: pair of stages, y: 32-row group) of 256 = 2 stages x 4 blocks x 32 rows, so each row's
// 128 bytes are one cache line in and out and each Q block is written as 1 KiB contiguous.  Rows past R write zero
// Q pieces (read by the GEMM's last group only for rows it drops).
__global__ __launch_bounds__(256) void fp4_to_fp6_planes_kernel(uint8_t* __restrict__ P, uint8_t* __restrict__ Q,
                                                                const uint8_t* __restrict__ src, int64_t R, int64_t K,
                                                                int e1m2)
{
    const int r32 = threadIdx.x & 31, b4 = (threadIdx.x >> 5) & 3;
    const int64_t t = 2 * (int64_t)blockIdx.x + (threadIdx.x >> 7);
    const int64_t groups = gridDim.y, g = blockIdx.y;
    if (t >= K / 128) return;
    const int64_t r = g * 32 + r32, b = t * 4 + b4;
    uint32_t in[4] = {0u, 0u, 0u, 0u};
    if (r < R) {
        const u32x4 v = *(const u32x4*)(src + r * (K / 2) + b * 16);
        in[0] = v[0];
        in[1] = v[1];
        in[2] = v[2];
        in[3] = v[3];
    }
    const uint32_t msh = e1m2 ? 1u : 2u;
    uint32_t out[6] = {0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const uint32_t n = (in[i / 8] >> (4 * (i % 8))) & 0xFu;
        const uint32_t c = ((n & 8u) << 2) | ((n & 7u) << msh);
        const int bit = 6 * i;
        out[bit / 32] |= c << (bit % 32);
        if (bit % 32 > 26) out[bit / 32 + 1] |= c >> (32 - bit % 32);
    }
    if (r < R) *(u32x4*)(P + r * (K / 2) + b * 16) = (u32x4){out[0], out[1], out[2], out[3]};
    *(u32x2*)(Q + (((t * groups + g) * 4 + b4) * 32 + r32) * 8) = (u32x2){out[4], out[5]};
}

size_t fp6_q_plane_bytes(int64_t R, int64_t K) { return (size_t)((K / 128) * ((R + 31) / 32) * 1024); }

hipError_t launch_fp4_to_fp6_planes(uint8_t* P, uint8_t* Q, const uint8_t* src, int64_t R, int64_t K, bool e1m2,
                                    hipStream_t st)
{
    const int64_t groups = (R + 31) / 32, pairs = (K / 128 + 1) / 2;
    if (K % 128 != 0 || groups > 65535 || pairs < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fp4_to_fp6_planes_kernel, dim3((unsigned)pairs, (unsigned)groups), dim3(256), 0, st, P, Q, src,
                       R, K, e1m2 ? 1 : 0);
    return hipGetLastError();
}

// E8M0 scales -> the stage-major layout the kernel reads: the SCB bytes of (group g, row r) are blocks
// SCB g .. SCB g + SCB - 1 of row r, at byte (g * R + r) * SCB, for ceil(sK / SCB) groups; blocks past sK (the
// K tail of a stage, whose elements the GEMM reads as zeros) get the scale 127 = 2^0, so no NaN code (0xFF)
// meets them.  src_layout 0: [R, sK] row-major; 1: [sK/2, R, 2] (pairs of blocks, rows inner).  sK is even.
// One thread per (group, row).
// Both operands' scales in one launch (the rearrangement of one operand is ~2 MB at 8192 x 8192 and costs little
// beyond its launch): workgroups [0, blocks_a) rearrange A, the rest B.
struct ScaleJob {
    uint8_t* dst;
    const uint8_t* src;
    int64_t R;
    int src_layout;
};

template <int SCB>
__global__ __launch_bounds__(256) void mx_scale_stage_major_kernel(ScaleJob ja, ScaleJob jb, int64_t sK,
                                                                   uint32_t blocks_a)
{
    const bool is_a = blockIdx.x < blocks_a;
    const ScaleJob j = is_a ? ja : jb;
    uint8_t* __restrict__ dst = j.dst;
    const uint8_t* __restrict__ src = j.src;
    const int64_t R = j.R;
    const int src_layout = j.src_layout;
    const int64_t bid = is_a ? blockIdx.x : blockIdx.x - blocks_a, nb = is_a ? blocks_a : gridDim.x - blocks_a;
    const int64_t groups = (sK + SCB - 1) / SCB, total = groups * R;
    const uint16_t* s16 = (const uint16_t*)src;
    // the 16-bit pair of blocks (b, b + 1), b even; past sK the neutral scale
    auto pair = [&](int64_t b, int64_t r) -> uint32_t {
        if (b >= sK) return 0x7F7Fu;
        return src_layout == 0 ? *(const uint16_t*)(src + r * sK + b) : s16[(b / 2) * R + r];
    };
    for (int64_t i = bid * 256 + threadIdx.x; i < total; i += nb * 256) {
        const int64_t g = i / R, r = i % R;
        if constexpr (SCB == 2) {
            ((uint16_t*)dst)[i] = (uint16_t)pair(2 * g, r);
        } else {
#pragma unroll
            for (int q = 0; q < SCB / 4; ++q) {
                const int64_t b = SCB * g + 4 * q;
                ((uint32_t*)dst)[i * (SCB / 4) + q] = pair(b, r) | (pair(b + 2, r) << 16);
            }
        }
    }
}

template <int SCB>
static hipError_t launch_scale_stage_major(const ScaleJob& a, const ScaleJob& b, int64_t sK, hipStream_t st)
{
    const auto blocks_for = [&](int64_t R) {
        int64_t n = (R * ((sK + SCB - 1) / SCB) + 255) / 256;
        return n > 32768 ? (int64_t)32768 : (n < 1 ? (int64_t)1 : n);
    };
    const int64_t ba = blocks_for(a.R), bb = blocks_for(b.R);
    hipLaunchKernelGGL(mx_scale_stage_major_kernel<SCB>, dim3((unsigned)(ba + bb)), dim3(256), 0, st, a, b, sK,
                       (uint32_t)ba);
    return hipGetLastError();
}

size_t mx_scale_workspace_bytes(int64_t M, int64_t N, int64_t K)
{
    const int64_t sKp = sk_stage_major(K);
    return (size_t)((M * sKp + 16 + 255) / 256 * 256 + (N * sKp + 16 + 255) / 256 * 256);
}

// the decode tiles' K split across workgroups (64 x 64 tiles of four waves, 128 fp4 of K per stage): splits so that
// tiles x splits is about 256, for few tiles only
int mx_decode_splits(int64_t M, int64_t N, int64_t K)
{
    if (M > 64 || M < 1 || N < 1 || K % 128 != 0) return 1;
    const int64_t tiles = (N + 63) / 64, units = K / 128;
    int64_t s = (256 + tiles / 2) / tiles;
    if (s > units) s = units;
    return s < 2 ? 1 : (int)s;
}
size_t mx_decode_split_ws_bytes(int64_t M, int64_t N, int64_t K)
{
    const int s = mx_decode_splits(M, N, K);
    return s < 2 ? 0 : (size_t)s * (size_t)((N + 63) / 64) * 4 * 64 * 64;
}

template <int DIRECT>
static hipError_t launch_mx_split(MxGemmArgs a, hipStream_t st)
{
    using T = GemmCore<64, 64, 2, 2, 4, true, OP_MXFP4, 64, 0, true, false, false, DIRECT>;
    const int tiles = (int)((a.N + 63) / 64);
    hipError_t e = ensure_dynamic_lds<mx_gemm_kernel<64, 64, 2, 2, 4, 64, OP_MXFP4, 0, true, DIRECT, 1>>((int)T::LDS_BYTES);
    if (e != hipSuccess) return e;
    launch_k((mx_gemm_kernel<64, 64, 2, 2, 4, 64, OP_MXFP4, 0, true, DIRECT, 1>), dim3(tiles * a.splits), dim3(T::NT),
             T::LDS_BYTES, st, a, (const uint8_t*)nullptr, (const uint8_t*)nullptr);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_k((mx_gemm_kernel<64, 64, 2, 2, 4, 64, OP_MXFP4, 0, true, DIRECT, 2>), dim3(tiles), dim3(T::NT), 0u, st, a,
             (const uint8_t*)nullptr, (const uint8_t*)nullptr);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int ST, int RB, int OP, int FMT, bool ILV = true, int DIRECT = 0>
static hipError_t launch_mx_tiled(const MxGemmArgs& a, hipStream_t st)
{
    using T = GemmCore<BM, BN, WM, WN, ST, true, OP, RB, FMT, ILV, false, false, DIRECT>;
    constexpr int SCB = T::SCB;
    const int64_t sK = (a.K + 63) / 64 * 2;
    uint8_t* sa_sm = a.ws_scales;
    uint8_t* sb_sm = a.ws_scales + (a.M * sk_stage_major(a.K) + 16 + 255) / 256 * 256;
    hipError_t e = hipSuccess;
    if (!DIRECT) {
        e = launch_scale_stage_major<SCB>(ScaleJob{sa_sm, a.sA, a.M, a.sa_layout == 1 ? 1 : 0},
                                          ScaleJob{sb_sm, a.sB, a.N, a.sb_layout == 0 ? 1 : 0}, sK, st);
        if (e != hipSuccess) return e;
    }
    e = ensure_dynamic_lds<mx_gemm_kernel<BM, BN, WM, WN, ST, RB, OP, FMT, ILV, DIRECT>>((int)T::LDS_BYTES);
    if (e != hipSuccess) return e;
    const int tiles = (int)(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN));
    launch_k((mx_gemm_kernel<BM, BN, WM, WN, ST, RB, OP, FMT, ILV, DIRECT>), dim3(tiles), dim3(T::NT), T::LDS_BYTES, st,
             a, sa_sm, sb_sm);
    return hipGetLastError();
}

template <int FMT>
static hipError_t launch_mx_f8(const MxGemmArgs& a, hipStream_t st)
{
    const bool big = a.M >= 1024 && a.N >= 1024;
    if (big) return launch_mx_tiled<256, 256, 4, 2, 2, 128, OP_MXF8, FMT>(a, st);
    return launch_mx_tiled<64, 64, 2, 2, 4, 64, OP_MXF8, FMT>(a, st);
}

// K must be a multiple of one LDS stage row: 128 fp4 (64 bytes) or 64 fp8 (64 bytes); the scales are rearranged
// stage-major into a.ws_scales (mx_scale_workspace_bytes) before the GEMM.
hipError_t launch_mx_gemm(const MxGemmArgs& a, hipStream_t st)
{
    const bool fp4 = a.fmt_a == F8F6F4_E2M1 && a.fmt_b == F8F6F4_E2M1;
    const bool fp6 = a.fmt_a == F8F6F4_E2M3 && a.fmt_b == F8F6F4_E2M3;
    // (the epilogue addresses a 256-row output tile with 32-bit offsets: N < 2^21)
    if (a.K % (fp4 || fp6 ? 128 : 64) != 0 || !a.ws_scales || a.N >= (1ll << 21)) return hipErrorInvalidValue;
    const bool big = a.M >= 1024 && a.N >= 1024;
    {
        // the auxiliary regions the kernel reads through one resource: (fp6) Aq < Bq < the scale workspace, all
        // within 2 GiB of the first
        const uint8_t* base = fp6 ? a.Aq : a.ws_scales;
        if (fp6 && (!a.Aq || !a.Bq || a.Bq - a.Aq < (int64_t)fp6_q_plane_bytes(a.M, a.K) ||
                    a.ws_scales - a.Bq < (int64_t)fp6_q_plane_bytes(a.N, a.K)))
            return hipErrorInvalidValue;
        if ((a.ws_scales - base) + (int64_t)mx_scale_workspace_bytes(a.M, a.N, a.K) >= (1ll << 31))
            return hipErrorInvalidValue;
    }
    if (fp6) {
        if (big) return launch_mx_tiled<256, 256, 4, 2, 3, 64, OP_MXFP6, 0>(a, st);
        return launch_mx_tiled<64, 64, 2, 2, 4, 64, OP_MXFP6, 0>(a, st);
    }
    if (fp4) {
        if (big) return launch_mx_tiled<256, 256, 4, 2, 2, 128, OP_MXFP4, 0>(a, st);
        // decode-sized batches (M <= 64) with A's scales row-major [M, sK] and B's row-major [N, sK] or in block
        // pairs [sK / 2, N, 2] (N even; 4-byte aligned): the 64 x 64 tiles read the scales as given, so no
        // rearrangement launch precedes the GEMM (measured, K = 4096, N = 11008, row-major B scales: M = 1 / 16 / 64
        // in 11.9 / 12.7 / 16.3 us against 17.5 / 17.6 / 19.5 us; at M = 256 the per-row reads, 64 cache lines a
        // copy, cost more than the launch: 45.4 against 38.0 us at K = N = 8192)
        if (a.M <= 64 && a.sa_layout == 0 && (uintptr_t)a.sA % 4 == 0 && (uintptr_t)a.sB % 4 == 0) {
            // ... with few tiles (N / 64 well under 256) and a workspace for the partials, K split across workgroups
            // too, the fp32 partials added in split order by a second launch
            const int splits = mx_decode_splits(a.M, a.N, a.K);
            const bool split = splits > 1 && a.atomic == C_STORE && a.ws_part &&
                               a.ws_part_bytes >= mx_decode_split_ws_bytes(a.M, a.N, a.K);
            MxGemmArgs b = a;
            b.splits = splits;
            if (a.sb_layout == 1)
                return split ? launch_mx_split<1>(b, st) : launch_mx_tiled<64, 64, 2, 2, 4, 64, OP_MXFP4, 0, true, 1>(a, st);
            if (a.N % 2 == 0)
                return split ? launch_mx_split<2>(b, st) : launch_mx_tiled<64, 64, 2, 2, 4, 64, OP_MXFP4, 0, true, 2>(a, st);
        }
        return launch_mx_tiled<64, 64, 2, 2, 4, 64, OP_MXFP4, 0>(a, st);
    }
    switch (a.fmt_a | (a.fmt_b << 3)) {
    case F8F6F4_E4M3 | (F8F6F4_E4M3 << 3): return launch_mx_f8<F8F6F4_E4M3 | (F8F6F4_E4M3 << 3)>(a, st);
    case F8F6F4_E5M2 | (F8F6F4_E5M2 << 3): return launch_mx_f8<F8F6F4_E5M2 | (F8F6F4_E5M2 << 3)>(a, st);
    case F8F6F4_E4M3 | (F8F6F4_E5M2 << 3): return launch_mx_f8<F8F6F4_E4M3 | (F8F6F4_E5M2 << 3)>(a, st);
    case F8F6F4_E5M2 | (F8F6F4_E4M3 << 3): return launch_mx_f8<F8F6F4_E5M2 | (F8F6F4_E4M3 << 3)>(a, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace ascq
