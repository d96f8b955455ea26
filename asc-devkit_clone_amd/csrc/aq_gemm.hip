// aq_gemm.hip -- weight-only antiquant matmul (W8A16 / W4A16) for batches above the decode shapes (M > 64) on gfx950.
//
// Reference: AscendAntiQuant per group (include/adv_api/quantization/ascend_antiquant.h:47-62;
// impl/adv_api/detail/quantization/antiquant/ascend_antiquant_impl.h:63-96, 366-411) composed with a half Matmul whose
// L0C is fp32 (impl/adv_api/detail/matmul/utils/matmul_utils.h:171-174): y = f16( x @ w_f16 ), fp32 accumulation,
// w_f16 = half( half(q + offset) * scale ) per group of K.
//
// The decode kernels (gemv_antiquant.hip) dequantise each weight fragment in registers for a block of at most 64 rows;
// for a prefill batch that would dequantise and read the weight once per 64 rows.  Here a workgroup computes a
// BM x BN output tile as an LDS-staged GEMM on v_mfma_f32_32x32x16_f16:
//  * one LDS stage holds 64 k (128 bytes) of every tile row of x and of the dequantised weight, in a ring of ST
//    stages; 16-byte chunk c of row r sits at chunk c ^ ((r / 2) % 8), so the 16 rows an MFMA operand read serves
//    together hit 16 distinct bank groups;
//  * x goes global -> LDS by buffer loads with an LDS destination (no registers; rows past M read zeros);
//  * the packed weight (ascq_weight_pack's layout: 16-column x 128-k tiles, lane l holding column l % 16 and, per 32-k
//    step j, k = 32 j + 8 (l / 16) .. + 7) goes global -> registers for the stage ST - 1 ahead, and one iteration later
//    each thread dequantises its units (one 8-element fragment = 8 consecutive k of one column per step, bit-exactly as
//    AscendAntiQuant) and writes them K-contiguous into the stage, so each weight is read and dequantised once per BM
//    rows;
//  * MFMA fragments: lane l takes row l % 32 and the 16-byte chunk 2 s + l / 32 of k-step s (16 k) for both operands.
// Accumulator layout of a 32x32 tile: lane l, register r holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
#include "aq_frag.h"
#include "common.h"
#include "launch.h"

namespace ascq {

namespace {

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
constexpr uint32_t OOB = 0x80000000u;  // an always out-of-range buffer offset (every range here is below 2^31)

__device__ __forceinline__ rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int N>
__device__ __forceinline__ void wait_vm()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

}  // namespace

struct AqGemmArgs {
    uint16_t* y;            // [M, N] f16
    const uint16_t* x;      // [M, K] f16
    const uint8_t* wp;      // packed weight
    const uint16_t* scale;  // [K / g, N] f16
    const uint16_t* offset; // [K / g, N] f16 or null
    uint32_t M, N, K;
    uint32_t gshift;        // g = 128 << gshift
    uint32_t x_bytes, w_bytes, s_bytes;
    int atomic;
};

// EB: weight register sets beyond two (iterations of extra lookahead for the weight stream)
template <int BM, int BN, int WM, int WN, int ST, int EB, bool INT4, bool HAS_OFF>
__global__ __launch_bounds__(WM * WN * 64) void aq_gemm_kernel(AqGemmArgs p)
{
    constexpr int NW = WM * WN, NT = NW * 64;
    constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
    constexpr int ROWB = 128;                   // K bytes per row per stage (64 k)
    constexpr int A_BYTES = BM * ROWB, STAGE = (BM + BN) * ROWB;
    constexpr int A_COPIES = A_BYTES / 1024 / NW;  // 1 KiB (8 rows) per wave-wide copy
    constexpr int BU = (BN / 16) * 64 / NT;      // weight units (strip, lane) per thread per stage
    constexpr int TILE_BYTES = INT4 ? 1024 : 2048, LANE_BYTES = INT4 ? 16 : 32;
    constexpr int B_LOADS = BU * (HAS_OFF ? 3 : 2);  // weight, scale (and offset) loads per thread per stage
    // vector memory operations of this wave issued after stage kt's x copies, at the top of iteration kt: each
    // iteration (and prologue step) issues its weight loads, then its x copies
    constexpr int IN_FLIGHT = (ST - 2) * (A_COPIES + B_LOADS);
    static_assert(IN_FLIGHT < 64, "vmcnt range");
    static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
    static_assert(A_BYTES % (1024 * NW) == 0 && A_COPIES >= 1, "x copies split evenly over the waves");
    static_assert(((BN / 16) * 64) % NT == 0 && BU >= 1, "weight units split evenly over the threads");
    // three stages: the prologue loads the weights of stages 0 .. EB + 1 into distinct register sets before it
    // dequantises stage 0 (with more stages a set would be reloaded before its stage is written)
    static_assert(ST == 3 && ST * STAGE <= 160 * 1024, "stages");
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const uint32_t tiles_n = (p.N + BN - 1) / BN;
    const uint32_t m0 = (blockIdx.x / tiles_n) * BM, n0 = (blockIdx.x % tiles_n) * BN;
    const uint32_t KB = p.K / 128, nk = p.K / 64;  // packed k tiles, stages
    const rsrc_t rx = rsrc(p.x, p.x_bytes), rw = rsrc(p.wp, p.w_bytes);
    const rsrc_t rs = rsrc(p.scale, p.s_bytes), ro = rsrc(HAS_OFF ? p.offset : p.scale, p.s_bytes);
    const uint32_t magic = half_magic_vgpr();
    auto swz = [](uint32_t row, uint32_t c) { return c ^ ((row >> 1) & 7u); };

    // x copies of this wave (stage-independent parts): copy u fills rows 8 (wave A_COPIES + u) .. + 7, lane l the
    // physical chunk l % 8 of row l / 8, which holds logical chunk swz(row, l % 8)
    uint32_t xoff[A_COPIES];
#pragma unroll
    for (int u = 0; u < A_COPIES; ++u) {
        const uint32_t row = 8 * (wave * A_COPIES + u) + lane / 8;
        xoff[u] = m0 + row < p.M ? ((m0 + row) * p.K * 2 + swz(row, lane % 8) * 16) : OOB;
    }
    auto issue_x = [&](uint32_t kt, int slot) {
#pragma unroll
        for (int u = 0; u < A_COPIES; ++u) {
            const uint32_t off = kt < nk ? xoff[u] + kt * ROWB : OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(smem + slot * STAGE + 8 * (wave * A_COPIES + u) * ROWB),
                                                     16, off, 0, 0, 0);
        }
    };

    // weight units of this thread: unit i = t + i NT is (strip i / 64 of the tile, lane i % 64 of the packed tile)
    struct BRegs {
        uint32_t w[BU][INT4 ? 2 : 4];
        uint32_t sc[BU], of[BU];
    };
    uint32_t wbase[BU], sbase[BU];
#pragma unroll
    for (int i = 0; i < BU; ++i) {
        const uint32_t u = (uint32_t)t + (uint32_t)i * NT, strip = n0 / 16 + u / 64, l = u % 64;
        const bool ok = strip * 16 < p.N;
        wbase[i] = ok ? strip * KB * TILE_BYTES + l * LANE_BYTES : OOB;
        sbase[i] = ok ? (strip * 16 + (l & 15)) * 2 : OOB;
    }
    auto load_b = [&](uint32_t kt, BRegs& r) {
        const uint32_t kb = kt / 2, half = kt & 1;
        const uint32_t soff = (kb >> p.gshift) * p.N * 2;
#pragma unroll
        for (int i = 0; i < BU; ++i) {
            const uint32_t off = kt < nk ? wbase[i] + kb * TILE_BYTES + half * (LANE_BYTES / 2) : OOB;
            if constexpr (INT4) {
                const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rw, off, 0, 0);
                r.w[i][0] = v[0];
                r.w[i][1] = v[1];
            } else {
                const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
#pragma unroll
                for (int q = 0; q < 4; ++q) r.w[i][q] = v[q];
            }
            const uint32_t so = kt < nk ? sbase[i] + soff : OOB;
            r.sc[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0);
            if constexpr (HAS_OFF) r.of[i] = __builtin_amdgcn_raw_buffer_load_b16(ro, so, 0, 0);
        }
    };
    // dequantise unit i held in r and write it K-contiguous into the weight part of a slot: unit (strip, l) gives
    // column 16 strip + l % 16 and, per step jj of the stage, logical chunk 4 jj + l / 16
    auto store_b_unit = [&](const BRegs& r, int slot, int i) {
        uint8_t* sB = smem + slot * STAGE + A_BYTES;
        {
            const uint32_t u = (uint32_t)t + (uint32_t)i * NT, n = (u / 64) * 16 + (u & 15), q = (u % 64) / 16;
            const _Float16 sv = __builtin_bit_cast(_Float16, (uint16_t)r.sc[i]);
            const _Float16 ov = HAS_OFF ? __builtin_bit_cast(_Float16, (uint16_t)r.of[i]) : (_Float16)0.0f;
            const h2 s2 = (h2){sv, sv}, o2 = (h2){ov, ov};
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const h8 f = INT4 ? dequant8<true, HAS_OFF>(r.w[i][jj], 0u, o2, s2, magic)
                                  : dequant8<false, HAS_OFF>(r.w[i][2 * jj], r.w[i][2 * jj + 1], o2, s2, magic);
                *(h8*)(sB + n * ROWB + swz(n, 4 * jj + q) * 16) = f;
            }
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v16f){};

    // weight registers: a ring of RB = EB + 2 sets.  Stage t's weights are loaded EB + 1 iterations before the
    // iteration (t - ST + 2) that dequantises them into their slot, so EB extra iterations of HBM latency are covered
    // without LDS (the slot of a stage must stay free until one iteration before it is multiplied).
    constexpr int RB = EB + 2;
    BRegs rb[RB];
    // prologue: the weights of stages 0 .. EB - 1, then ST - 1 steps shaped like an iteration (the weights of stage
    // s + EB, then the x copies of stage s), so every iteration's counted wait sees the same operations after the x
    // copies it waits for; stages 0 .. ST - 3 are dequantised here
#pragma unroll
    for (int s = 0; s < EB; ++s) load_b((uint32_t)s, rb[s % RB]);
#pragma unroll
    for (int s = 0; s < ST - 1; ++s) {
        __builtin_amdgcn_sched_barrier(0);
        load_b((uint32_t)(s + EB), rb[(s + EB) % RB]);
        __builtin_amdgcn_sched_barrier(0);
        issue_x((uint32_t)s, s);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < ST - 2; ++s)
#pragma unroll
        for (int i = 0; i < BU; ++i) store_b_unit(rb[s % RB], s, i);

    const uint32_t r32 = lane & 31, kh = lane >> 5;
    // iteration kt: stage kt is multiplied; the weights of stage kt + ST - 1 + EB are loaded into their set and those of
    // stage kt + ST - 2 are dequantised into its slot (freed two iterations ago, read after at least one more barrier)
    auto iteration = [&](uint32_t kt, BRegs& rb_new, BRegs& rb_old) {
        const int slot = (int)(kt % ST), nslot = (int)((kt + ST - 1) % ST), pslot = (int)((kt + ST - 2) % ST);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<IN_FLIGHT>();                 // this wave's x copies of stage kt have landed (the compiler waits for
                                              // the weight registers where they are used)
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this thread's weight writes of stage kt are done
        __builtin_amdgcn_sched_barrier(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();         // ... and every wave's; the slot multiplied last iteration is free
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_sched_barrier(0);
        load_b(kt + ST - 1 + EB, rb_new);
        __builtin_amdgcn_sched_barrier(0);
        issue_x(kt + ST - 1, nslot);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* sA = smem + slot * STAGE;
        const uint8_t* sB = sA + A_BYTES;
#pragma unroll
        for (int s = 0; s < 4; ++s) {  // k-steps of 16 k
            // the weight units of stage kt + ST - 2 are dequantised and written between the k-steps (a quarter of them
            // before each), so their vector-ALU work issues while the MFMAs run
#pragma unroll
            for (int i = s * BU / 4; i < (s + 1) * BU / 4; ++i) store_b_unit(rb_old, pslot, i);
            h8 fa[FM];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint32_t row = wm * WTM + 32 * i + r32;
                fa[i] = *(const h8*)(sA + row * ROWB + swz(row, 2 * s + kh) * 16);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const uint32_t col = wn * WTN + 32 * j + r32;
                const h8 fb = *(const h8*)(sB + col * ROWB + swz(col, 2 * s + kh) * 16);
#pragma unroll
                for (int i = 0; i < FM; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb, acc[i][j], 0, 0, 0);
            }
        }
    };
    // RB iterations per pass, so every register set is named statically; iterations past the last stage are skipped
    for (uint32_t k0 = 0; k0 < nk; k0 += RB) {
#pragma unroll
        for (int u = 0; u < RB; ++u)
            if (k0 + u < nk) iteration(k0 + u, rb[(u + ST - 1 + EB) % RB], rb[(u + ST - 2) % RB]);
    }
    wait_vm<0>();  // no copy may still target LDS when the wave ends

    // epilogue: rows past M and columns past N are not written
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const uint32_t col = n0 + wn * WTN + 32 * j + r32;
            if (col >= p.N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t row = m0 + wm * WTM + 32 * i + 8 * (r / 4) + 4 * kh + (r & 3);
                if (row >= p.M) continue;
                uint16_t* yp = p.y + (uint64_t)row * p.N + col;
                const uint16_t v = f32_to_f16_sat(acc[i][j][r]);
                if (p.atomic == C_STORE) *yp = v;
                else c_atomic<DT_F16>((uint8_t*)yp, v, p.atomic);
            }
        }
}

template <int BM, int BN, int WM, int WN, int ST, int EB>
static hipError_t launch_aq_gemm_t(const AqGemmArgs& a, bool int4, hipStream_t st)
{
    constexpr size_t lds = (size_t)ST * (BM + BN) * 128;
    const uint32_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
#define AQG_LAUNCH(I4, OF)                                                                       \
    do {                                                                                         \
        constexpr auto kern = aq_gemm_kernel<BM, BN, WM, WN, ST, EB, I4, OF>;                         \
        hipError_t e = ensure_dynamic_lds<kern>((int)lds);                                       \
        if (e != hipSuccess) return e;                                                           \
        launch_k(kern, dim3(tiles), dim3(WM * WN * 64), (uint32_t)lds, st, a);                   \
    } while (0)
    if (int4) {
        if (a.offset) AQG_LAUNCH(true, true);
        else AQG_LAUNCH(true, false);
    } else {
        if (a.offset) AQG_LAUNCH(false, true);
        else AQG_LAUNCH(false, false);
    }
#undef AQG_LAUNCH
    return hipGetLastError();
}

// M > 64, K % 128 == 0, N % 16 == 0, group 128 << s (checked here), every buffer below 2^31 - 2^16 bytes
hipError_t launch_aq_gemm(uint16_t* y, const uint16_t* x, const void* wp, int w_type, const uint16_t* scale,
                          const uint16_t* offset, int64_t group, int64_t M, int64_t N, int64_t K, int atomic,
                          hipStream_t st)
{
    const int64_t g = group > 0 ? group : K;
    const bool int4 = w_type == DT_INT4;
    const uint64_t lim = 0x7FFF0000ull;
    const uint64_t w_bytes = (uint64_t)K * N / (int4 ? 2 : 1), s_bytes = (uint64_t)((K + g - 1) / g) * N * 2;
    const uint64_t x_bytes = (uint64_t)M * K * 2;
    if (K % 128 != 0 || N % 16 != 0 || g % 128 != 0 || ((g / 128) & (g / 128 - 1)) != 0 || w_bytes >= lim ||
        s_bytes >= lim || x_bytes >= lim || M * N >= (int64_t)lim)
        return hipErrorInvalidValue;
    AqGemmArgs a;
    a.y = y;
    a.x = x;
    a.wp = (const uint8_t*)wp;
    a.scale = scale;
    a.offset = offset;
    a.M = (uint32_t)M;
    a.N = (uint32_t)N;
    a.K = (uint32_t)K;
    a.gshift = (uint32_t)__builtin_ctzll((unsigned long long)(g / 128));
    a.x_bytes = (uint32_t)x_bytes;
    a.w_bytes = (uint32_t)w_bytes;
    a.s_bytes = (uint32_t)s_bytes;
    a.atomic = atomic;
    // 256 x 128 tiles, 8 waves of 64 x 64, four extra weight register sets: measured against 128 x 256 / 128 x 128
    // tiles with 4 or 8 waves and 0 - 6 extra sets at K = 4096, N = 11008 (M = 512: 79 against 81 - 121 us)
    return launch_aq_gemm_t<256, 128, 4, 2, 3, 4>(a, int4, st);
}

}  // namespace ascq
