/*
 * ascq.h -- C ABI of the MI355X (gfx950) quantized-inference library (libascq.so).
 *
 * The library re-implements, for one AMD Instinct MI355X, the quantized hot path of the
 * Ascend C devkit (asc-devkit 9.3.0): the adv_api Matmul on int8 / fp8 / MX-FP4 operands
 * with the fused dequant epilogue, AscendQuant / AscendDequant / AscendAntiQuant, the
 * weight-only antiquant matmul and the quantized group matmul used for MoE.
 *
 * In the reference these are C++ templates instantiated inside a device kernel; here each
 * becomes one host call that validates its arguments and enqueues hand-written HIP kernels
 * on the caller's stream.  Each declaration names the reference interface it replaces
 * (paths relative to the asc-devkit source tree).
 *
 * Conventions
 *  - All tensor pointers are device pointers owned by the caller (the reference's
 *    GlobalTensor is likewise a non-owning view, matmul_quant.asc:79-83).
 *  - `stream` is a hipStream_t passed as void*; NULL is the default stream.  Calls are
 *    stream-ordered and asynchronous.
 *  - f16 / bf16 scalars are passed as their uint16_t bit patterns.
 *  - Return codes: ASCQ_OK (0) or a negative ascq_status; invalid arguments are rejected on
 *    the host before anything is launched (the reference's host tiling returns -1 on bad
 *    input, impl/adv_api/tiling/matmul/matmul_tiling.cpp:26-33; its device-side checks,
 *    impl/adv_api/detail/api_check/kernel_api_check.h:25-33, exist only in CPU debug).
 *  - ascq_last_error() returns a text description of the last failure on this thread.
 *  - Handles are not thread-safe; use one handle per host thread / stream.
 */
#ifndef ASCQ_H
#define ASCQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t ascq_status;
#define ASCQ_OK 0
#define ASCQ_E_INVALID_ARG (-1) /* mirrors GetTiling's -1 (matmul_tiling.cpp:26-33) */
#define ASCQ_E_UNSUPPORTED (-2) /* a dtype / layout / mode combination this library does not implement */
#define ASCQ_E_HIP (-3)         /* a HIP runtime call failed (see ascq_last_error) */
#define ASCQ_E_STATE (-4)       /* calls out of order, e.g. IterateAll before SetTensorA */

/* Element types.  Mirrors the reference's device types (int8_t, int4b_t, half, bfloat16_t,
 * fp8_e4m3fn_t, fp8_e5m2_t, fp4x2_e2m1_t, fp8_e8m0_t; include/basic_api/kernel_type.h and
 * impl/adv_api/detail/matmul/utils/matmul_type_def.h:114-131). */
typedef enum {
    ASCQ_DT_INT8 = 1,
    ASCQ_DT_UINT8 = 2,
    ASCQ_DT_INT4 = 3,      /* int4b_t, two per byte, even element in the low nibble */
    ASCQ_DT_INT32 = 4,
    ASCQ_DT_F16 = 5,
    ASCQ_DT_BF16 = 6,
    ASCQ_DT_F32 = 7,
    ASCQ_DT_U64 = 8,       /* uint64 deq-scale words (low 32 bits = fp32 scale) */
    ASCQ_DT_FP8_E4M3 = 9,  /* fp8_e4m3fn_t */
    ASCQ_DT_FP8_E5M2 = 10, /* fp8_e5m2_t */
    ASCQ_DT_FP4_E2M1 = 11, /* fp4x2_e2m1_t, two per byte, even element in the low nibble */
    ASCQ_DT_E8M0 = 12,     /* fp8_e8m0_t shared exponent */
    ASCQ_DT_INT64 = 13,
    ASCQ_DT_FP4_E1M2 = 14, /* fp4x2_e1m2_t: sign | 1-bit exponent (bias 1) | 2-bit mantissa, magnitudes k / 4,
                              k = 0..7; two per byte, even element in the low nibble */
    ASCQ_DT_HIF8 = 15      /* hifloat8_t: sign | dot field (11 / 10 / 01 / 001 / 0001 / 0000) | exponent | mantissa
                              (layout of impl/utils/debug/npu_arch_9201/asc_type_conversion_utils.h:62-149); finite
                              range 2^-22 .. 2^15, 0x80 NaN, 0x6F / 0xEF +-inf */
} ascq_dtype;

/* RoundMode (impl/basic_api/utils/kernel_utils_mode.h:103-118). NONE acts as RINT on lossy casts. */
typedef enum {
    ASCQ_ROUND_NONE = 0,
    ASCQ_ROUND_RINT = 1,  /* half to even */
    ASCQ_ROUND_FLOOR = 2,
    ASCQ_ROUND_CEIL = 3,
    ASCQ_ROUND_ROUND = 4, /* half away from zero */
    ASCQ_ROUND_TRUNC = 5
} ascq_round_mode;

/* AscendQuantPolicy / AscendDeQuantPolicy (include/adv_api/quantization/ascend_quant_utils.h:74-81,
 * ascend_dequant_utils.h:37) plus the legacy per-tensor / per-channel forms. */
typedef enum {
    ASCQ_POLICY_PER_TENSOR = 0,
    ASCQ_POLICY_PER_CHANNEL = 1,
    ASCQ_POLICY_PER_TOKEN = 2,
    ASCQ_POLICY_PER_GROUP = 3
} ascq_policy;

/* Arithmetic of AscendAntiQuant: half ops (arch 2201, ascend_antiquant_impl.h:63-96) or fp32 ops
 * with one final rint cast (bf16 output, ascend_antiquant_c220_impl.h:46-75; arch 3510 fp16 path). */
typedef enum { ASCQ_ARITH_F16 = 0, ASCQ_ARITH_F32 = 1 } ascq_arith;

/* ------------------------------------------------------------------------------------------
 * Library
 * ------------------------------------------------------------------------------------------ */
const char* ascq_last_error(void);
const char* ascq_version(void);
/* Number of HIP devices visible (0 without a GPU); makes no other HIP call. */
int32_t ascq_device_count(void);
/* Kernel timing hook, no counterpart in the reference (for benchmarks and profilers that need a kernel's own
 * duration without marker packets between kernels): start / stop are hipEvent_t handles (both or neither); the
 * next entry point called on this thread records them at the start and end of its main kernel's dispatch
 * (hipExtLaunchKernelGGL), then the hook clears itself.  Every entry point that launches kernels disarms the hook
 * when it returns, also when it fails its argument checks and launches nothing.  Where one call runs its main
 * kernel more than once (ascq_antiquant_matmul and a weight-only IterateAll with M > 64 go in 64-row chunks), the
 * events time the first launch only. */
ascq_status ascq_set_launch_events(void* start, void* stop);

/* Pack an fp32 multiplier, a 9-bit offset and the sign flag into a QUANT_PRE word
 * (docs/zh/api/SIMD-API/c_api/cube_datamove/cube_store_key_features/accompanying_quantization.md:79-103;
 * the reference sample packs (uint64)(*(uint32*)&f), matmul_quant.asc:111-113).  Host only. */
uint64_t ascq_pack_quant_pre(float m1, int32_t offset9, int32_t sign_flag);

/* ------------------------------------------------------------------------------------------
 * Matmul high-level API
 * Replaces AscendC::Matmul<MatmulType<GM,ND,A>, <B>, <C>, <Bias>, CFG> and
 * MatmulTypeWithScale (include/adv_api/matmul/matmul.h:54-400; matmul_intf.h:42-111;
 * impl/adv_api/detail/matmul/utils/matmul_type_def.h:114-131) together with
 * REGIST_MATMUL_OBJ / Init(TCubeTiling*) (matmul_intf.h:40).  One handle computes the whole
 * singleShape block; the gfx950 tile decomposition replaces TCubeTiling.
 *
 * Supported type combinations (A, B, C, Bias) and epilogues:
 *  int8, int8, f16,   int32   + SetQuantScalar/Vector -> DEQF16 / VDEQF16
 *  int8, int8, bf16,  int32   + SetQuantScalar/Vector -> QS322BF16_PRE / VQS322BF16_PRE
 *  int8, int8, int32, int32   (no quant)              -> raw int32 accumulators
 *  int8, int8, int8|uint8, int32 + SetQuantScalar/Vector -> REQ8 / VREQ8: sat8(rint(clamp(f32(acc) * M1,
 *                               -256, 255)) + offset), the word's sign flag picking int8 or uint8 saturation
 *                               (quant_processor_fixpipe.h:93-94, 211-212)
 *  int4, int4, int32|f16 (or any int8 C above), int32 bias -> the int8 epilogues on exact int32 sums
 *                               (matmul_int4/matmul_int4.asc:151; A not transposed, K and N even): both operands
 *                               are unpacked to int8 in the workspace, B given [K, N] nibble-transposed first
 *  f16,  int8|int4, f16, f32  + SetAntiQuantScalar/Vector (weight-only, optional groups)
 *  fp8_e4m3|fp8_e5m2 (any mix), f16|bf16|f32, f32 bias
 *                               (+ SetQuantScalar/Vector -> QF322F16 / QF322BF16 / QF322F32 _PRE; without a
 *                               quant word a plain cast; quant_processor_fixpipe.h:101-115)
 *  int8, int8, int4, int32 + SetQuantScalar/Vector -> REQ4 / VREQ4: sat4(rint(clamp(f32(acc) * M1, -256, 255))
 *                               + offset), C packed two codes per byte (even column in the low nibble, N even);
 *                               a fixpipe mode of the reference (asc_set_l0c_copy_prequant.md:37-41, boundary table
 *                               matrix_compute_move_out_interface_boundary_value_summary.md:110-111) that the
 *                               Matmul's own mode table does not select
 *  fp8, fp8, int4 + SetQuantScalar/Vector -> QF322S4_PRE (as REQ4 on the fp32 accumulator)
 *  fp8, fp8, int8|uint8 + SetQuantScalar/Vector -> QF322B8_PRE (as REQ8 on the fp32 accumulator)
 *  fp8, fp8, fp8_e4m3|fp8_e5m2 + SetQuantScalar/Vector -> QF322FP8_PRE (rne; e4m3 saturates at +-448, NaN -> 0)
 *  fp8, fp8, hifloat8 + SetQuantScalar/Vector -> QF322HIF8_PRE (ties away from zero, saturating at +-32768,
 *                               NaN -> 0: the saturation-mode row of
 *                               matrix_compute_move_out_interface_boundary_value_summary.md:68-70)
 *  hifloat8, hifloat8 (both; matmul_fp8/README_en.md), any C of the fp8 rows above or hifloat8, f32 bias
 *                               (matmul_fp8.asc:229, the sample's default MatmulFp8Kernel<hifloat8_t, hifloat8_t,
 *                               float, float>; mode table quant_processor_utils.h:36-41): both operands are decoded
 *                               exactly to bf16 in the workspace (every HiF8 value is a bf16 value) and multiplied
 *                               with fp32 accumulation, then the fp8 rows' epilogues
 *  fp4_e2m1|fp4_e1m2 (any mix), bf16|f32, f32 bias, with E8M0 scales (SetTensorScaleA/B) -> MX block-scaled
 *                               (K % 128 == 0; fp4x2_e1m2_t operands, the high-performance MX sample
 *                               matmul_mxfp4_high_performance/matmul_mx.h:117-133, run as exact fp6 E2M3 after a
 *                               conversion pass into the workspace)
 *  fp8_e4m3|fp8_e5m2 (any mix), bf16|f32, f32 bias, with E8M0 scales -> MX-FP8 (matmul_mx.asc:90-244, bias
 *                               :99-116,199-201; K % 64 == 0)
 * int8 / fp8 A given [K, M] (isTransA) and a large [K, N] B are transposed into the workspace first.
 * ------------------------------------------------------------------------------------------ */
typedef struct ascq_matmul_s* ascq_matmul_t;

/* CubeFormat of B (MatmulType<TPosition, CubeFormat, T>, impl/adv_api/detail/matmul/utils/matmul_type_def.h:40;
 * CubeFormat include/adv_api/matmul/matmul_config.h:23-35):
 * ND is the reference's row-major layout; PACKED is the output of ascq_weight_pack (weight-only only); NZ is the
 * reference's fractal layout (the one ascq_nz_to_nd reads: B [K, N], or [N, K] with isTransposeB, as [K, N] / [N, K]
 * NZ matrices) for int8 and fp8 B, turned into a K-contiguous [N, K] copy in the workspace at every IterateAll. */
typedef enum { ASCQ_FORMAT_ND = 0, ASCQ_FORMAT_PACKED = 1, ASCQ_FORMAT_NZ = 2 } ascq_format;

typedef struct {
    int32_t a_type;     /* ascq_dtype of A */
    int32_t b_type;     /* ascq_dtype of B */
    int32_t c_type;     /* ascq_dtype of C */
    int32_t bias_type;  /* ascq_dtype of the bias (0 = no bias type) */
    int32_t scale_type; /* ASCQ_DT_E8M0 for MX operands (MatmulTypeWithScale), else 0 */
    int32_t b_format;   /* ascq_format of B */
} ascq_matmul_types;

/* REGIST_MATMUL_OBJ + Init (matmul_intf.h:40; matmul.h:79-95) */
ascq_status ascq_matmul_create(const ascq_matmul_types* types, ascq_matmul_t* out);

/* The reference's host tiling result, TCubeTiling (include/adv_api/matmul/matmul_tilingdata.h:21-72): the same
 * int32 fields in the same order, so host code that fills, copies or serialises one passes it unchanged.  Only
 * the shape fields are read here; the rest describe the Ascend core split and buffers and are ignored. */
typedef struct {
    int32_t usedCoreNum, M, N, Ka, Kb, singleCoreM, singleCoreN, singleCoreK, baseM, baseN, baseK, depthA1, depthB1,
        stepM, stepN, isBias, transLength, iterateOrder, shareMode, shareL1Size, shareL0CSize, shareUbSize, batchM,
        batchN, singleBatchM, singleBatchN, stepKa, stepKb, depthAL1CacheUB, depthBL1CacheUB, dbL0A, dbL0B, dbL0C,
        ALayoutInfoB, ALayoutInfoS, ALayoutInfoN, ALayoutInfoG, ALayoutInfoD, BLayoutInfoB, BLayoutInfoS,
        BLayoutInfoN, BLayoutInfoG, BLayoutInfoD, CLayoutInfoB, CLayoutInfoS1, CLayoutInfoN, CLayoutInfoG,
        CLayoutInfoS2, BatchNum, mxTypePara;
} ascq_cube_tiling;

/* Init(const TCubeTiling*) (matmul.h:79-95): the org shape becomes (M, N, Ka); Ka must equal Kb.  The per-core
 * split (usedCoreNum, singleCoreM/N/K) is not applied: one IterateAll computes the whole org shape, which is
 * what the reference's cores compute together (set_single_shape still restricts a call to a block). */
ascq_status ascq_matmul_init(ascq_matmul_t h, const ascq_cube_tiling* tiling);
/* SetOrgShape(orgM, orgN, orgK) (matmul.h:94): full matrix shape; sets the leading dimensions */
ascq_status ascq_matmul_set_org_shape(ascq_matmul_t h, int64_t m, int64_t n, int64_t k);
/* SetSingleShape / SetTail (matmul.h:110, :117): the block this call computes (defaults to org shape) */
ascq_status ascq_matmul_set_single_shape(ascq_matmul_t h, int64_t m, int64_t n, int64_t k);
ascq_status ascq_matmul_set_tail(ascq_matmul_t h, int64_t tail_m, int64_t tail_n, int64_t tail_k);
/* SetTensorA / SetTensorB (matmul.h:123-129; impl matmul_impl_base.h:560-638) */
ascq_status ascq_matmul_set_tensor_a(ascq_matmul_t h, const void* a, int32_t is_transpose_a);
ascq_status ascq_matmul_set_tensor_b(ascq_matmul_t h, const void* b, int32_t is_transpose_b);
/* SetBias / DisableBias (matmul.h:134, :224) */
ascq_status ascq_matmul_set_bias(ascq_matmul_t h, const void* bias);
ascq_status ascq_matmul_disable_bias(ascq_matmul_t h);
/* SetQuantScalar / SetQuantVector (matmul.h:175-185; quant_processor_fixpipe.h:74-117,209-234) */
ascq_status ascq_matmul_set_quant_scalar(ascq_matmul_t h, uint64_t quant_scalar);
ascq_status ascq_matmul_set_quant_vector(ascq_matmul_t h, const uint64_t* quant_vector /* [N] */);
/* SetAntiQuantScalar / SetAntiQuantVector (matmul.h:161-170; antiquant_processor_using_ub.h:32-136).
 * group_size 0 = per-channel vectors [N] (the reference's only form); group_size g > 0 = [K/g, N]
 * vectors (per-group, an extension).  offset may be NULL (scale only). */
ascq_status ascq_matmul_set_antiquant_scalar(ascq_matmul_t h, uint16_t offset_f16, uint16_t scale_f16);
ascq_status ascq_matmul_set_antiquant_vector(ascq_matmul_t h, const void* offset, const void* scale,
                                             int64_t group_size);
/* SetTensorScaleA / SetTensorScaleB (mx_matmul_impl.h:136-188; examples/01_simd_cpp_api/04_advanced_api/00_matmul/matmul_mx/matmul_mx.asc:194-203).
 * scaleA: [M, sK] (transpose: [sK/2, M, 2]); scaleB: [sK/2, N, 2] (transpose: [N, sK]); sK = ceil(K/64)*2. */
ascq_status ascq_matmul_set_tensor_scale_a(ascq_matmul_t h, const uint8_t* scale_a, int32_t is_transpose_scale_a);
ascq_status ascq_matmul_set_tensor_scale_b(ascq_matmul_t h, const uint8_t* scale_b, int32_t is_transpose_scale_b);
/* Optional device workspace for handles that need one (int8 / fp8 with isTransA or a large [K,N] B; MX; hifloat8;
 * W4/W8 with ND B):
 * ascq_matmul_workspace_size() bytes.  Without it IterateAll allocates on first use. */
ascq_status ascq_matmul_workspace_size(ascq_matmul_t h, size_t* bytes);
ascq_status ascq_matmul_set_workspace(ascq_matmul_t h, void* workspace, size_t bytes);
/* IterateAll(GlobalTensor<C>, enAtomic) (matmul.h:255-265; matmul_impl.h:119-137).  en_atomic (ATOMIC_ADD / MAX /
 * MIN = 1 / 2 / 3, matmul_config_utils.h:53-55; scheduler_base.h:484-494) combines the result into C instead of
 * storing it: C = add / max / min(C, result) per element in C's type, as one atomic read-modify-write, so
 * concurrent calls into one C compose.  int32 C: wrapping add, signed max / min; f32 / f16 / bf16 C: the exact sum
 * rounded once (rne, overflow to inf), max / min by comparison (a NaN neither replaces nor is replaced).  For a
 * uint8 / int4 / fp8 C the reference's SetAtomic does nothing and the result is stored; int8 C with en_atomic != 0
 * is refused (ASCQ_E_UNSUPPORTED); en_atomic > 3 is ASCQ_E_INVALID_ARG. */
#define ASCQ_ATOMIC_NONE 0
#define ASCQ_ATOMIC_ADD 1
#define ASCQ_ATOMIC_MAX 2
#define ASCQ_ATOMIC_MIN 3
ascq_status ascq_matmul_iterate_all(ascq_matmul_t h, void* c, uint8_t en_atomic, void* stream);
/* IterateAll that allocates nothing -- no counterpart in the reference; for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * results as ascq_matmul_iterate_all, but a handle that needs a workspace (ascq_matmul_workspace_size > 0) uses
 * the library's static per-device scratch of ASCQ_NOALLOC_SCRATCH_BYTES instead of its own workspace or a
 * hipMalloc; a handle needing more is rejected with ASCQ_E_UNSUPPORTED before anything is launched.  Every call
 * on one device shares that device's scratch: calls that overlap on a device (other streams, other threads) race.
 * Nothing of the scratch's previous contents is read. */
#define ASCQ_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
ascq_status ascq_matmul_iterate_all_noalloc(ascq_matmul_t h, void* c, uint8_t en_atomic, void* stream);
/* End (matmul.h:358): releases per-call bindings; the handle may be re-bound and reused */
ascq_status ascq_matmul_end(ascq_matmul_t h);
ascq_status ascq_matmul_destroy(ascq_matmul_t h);

/* ------------------------------------------------------------------------------------------
 * AscendQuant
 * ------------------------------------------------------------------------------------------ */
/* AscendQuantParam{m, n, calCount, groupSize} + AscendQuantConfig{hasOffset, kDim, roundMode}
 * (include/adv_api/quantization/ascend_quant_utils.h:31-89) */
typedef struct {
    uint32_t m;
    uint32_t n;
    uint32_t cal_count;
    uint32_t group_size;
    int32_t has_offset;
    int32_t kdim;
    int32_t round_mode; /* ascq_round_mode */
} ascq_quant_param;

/* AscendQuant<int8_t, srcT, float, false, config, PER_TOKEN>(dst, src, scale[m], offset[m], para)
 * (ascend_quant.h:714-777; impl ascend_quant_per_group_3510_impl.h:142-178, 1341-1367, 1455-1501).
 * src_type: F16, BF16 or F32.  q = sat_s8(round(f32(x)*scale[row] (+offset[row]))).
 * cal_count must be a multiple of n (ascend_quant_per_group_3510_impl.h:1476-1477); m = cal_count/n rows. */
ascq_status ascq_ascend_quant_per_token(int8_t* dst, const void* src, int32_t src_type, const float* scale,
                                        const float* offset, const ascq_quant_param* para, void* stream);
/* Dynamic per-token quant: per-row absmax, multiplier 127/absmax, the PER_TOKEN quant above with that
 * multiplier, and scale_out[row] = absmax/127 for the dequant.  (The reference leaves the absmax
 * reduction to the caller; this entry point is that caller plus AscendQuant PER_TOKEN.) */
ascq_status ascq_ascend_quant_dynamic_per_token(int8_t* dst, float* scale_out, const void* src,
                                                int32_t src_type, uint32_t m, uint32_t n, int32_t round_mode,
                                                void* stream);
/* AscendQuant<dstT, srcT, scaleT, false, config{hasOffset, kDim, roundMode}, policy>(dst, src, scale, offset, para),
 * the arch-3510 policy form (include/adv_api/quantization/ascend_quant.h:714-777; impl
 * impl/adv_api/detail/quantization/quant/ascend_quant_per_group_3510_impl.h:33-1340, dispatch :1451-1504;
 * TransRegForFp8 / S8 / Fp4 ascend_quant_3510_impl.h:888-1036).  src / dst [rows, n] row-major with
 * rows = cal_count / n; para->group_size, has_offset, kdim and round_mode as in the config.
 * Scale (and offset) index of element (r, c):
 *   PER_TOKEN: scale[r];
 *   PER_GROUP, kdim 1: scale[r][c / group] ([rows][ceil(n/group)]); kdim 0: scale[r / group][c]
 *              ([ceil(rows/group)][n]); group_size a positive multiple of 32.
 * dst_type and arithmetic:
 *   INT8: y = x * scale (+ offset), each op rounded in scale_type, then clamp(round_mode(y), -128, 127), NaN -> 0;
 *   FP8_E4M3 / FP8_E5M2: the same ops in fp32 whatever scale_type, then rint with saturation (overflow and
 *         inf -> +-max finite, NaN -> 0); round_mode is not used (every mode is rint, :888-896);
 *   HIF8: the INT8 arithmetic (in scale_type), then ties away from zero with saturation at +-32768, NaN -> 0
 *         (TransRegForHif8, ascend_quant_3510_impl.h:899-933: every round mode but CAST_HYBRID, which this library does
 *         not take, is CAST_ROUND);
 *   FP4_E2M1 (PER_GROUP only; offset ignored, :1385): y = x * scale in scale_type; an f16 / f32 y is rounded to
 *         bf16 (rne, saturating, NaN -> 0); then E2M1 in round_mode with saturation at +-6; two codes a byte, even
 *         element in the low nibble (n even);
 *   FP4_E1M2: as FP4_E2M1, with E1M2 codes in round_mode saturating at +-1.75 (the same per-group kernels,
 *         ascend_quant_per_group_3510_impl.h:1383-1440, serve both fp4 types).
 * src_type F16, BF16 or F32; scale_type F16, BF16 or F32.  For INT8 / FP4 a 16-bit scale_type needs a source
 * of the same type (a 16-bit source meets an F32 scale as fp32); FP8 accepts every pair.
 * Offset (para->has_offset): the tensor `offset` (scale_type, indexed like scale) or, when it is NULL, the scalar
 * offset_scalar rounded (rne) to scale_type -- the overloads taking `const scaleT offset` (ascend_quant.h:737-777).
 */
ascq_status ascq_ascend_quant_policy(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                     const void* scale, const void* offset, float offset_scalar, int32_t scale_type,
                                     int32_t policy, const ascq_quant_param* para, void* stream);
/* Legacy AscendQuant, the arch-3510 form (include/adv_api/quantization/ascend_quant.h:64-293, 360-460; impl
 * impl/adv_api/detail/quantization/quant/ascend_quant_3510_impl.h:35-620):
 *   scale == NULL: AscendQuant(dst, src, const float scale, const float offset, calCount) -- scale_scalar and
 *     offset_scalar for every element (offset must be NULL too);
 *   scale != NULL: the per-channel overloads, element i using channel i % scale_count of `scale` and `offset`
 *     (srcT tensors of scale_count elements); offset == NULL is the `const T offset` overload, offset_scalar rounded
 *     (rne) to srcT.  calCount must be a multiple of 32 and of scale_count (ascend_quant_3510_impl.h:551-557).
 * src_type F16, BF16 or F32.  dst_type and arithmetic:
 *   INT8 / HIF8: half arithmetic -- source and srcT tensors cast to half with rne and saturation, the float scalars
 *     with rne (static_cast<half>); t = half(x * s); t = half(t + o); INT8: rint with saturation (NaN -> 0); HIF8:
 *     ties away from zero with saturation (+-32768; NaN -> 0);
 *   FP8_E4M3 / FP8_E5M2: fp32 arithmetic (exact conversions), rint with saturation, NaN -> 0.
 * dst holds cal_count bytes. */
ascq_status ascq_ascend_quant(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                              const void* offset, float scale_scalar, float offset_scalar, uint32_t cal_count,
                              uint32_t scale_count, void* stream);

/* ------------------------------------------------------------------------------------------
 * AscendDequant
 * ------------------------------------------------------------------------------------------ */
/* DequantParams{m, n, calCount} (include/adv_api/quantization/ascend_dequant_utils.h:26-30) */
typedef struct {
    uint32_t m;
    uint32_t n;
    uint32_t cal_count;
} ascq_dequant_param;

/* DeQuantMode (impl/basic_api/utils/kernel_utils_mode.h:193-196): how the legacy form reads params {1, m*n, n} */
typedef enum { ASCQ_DEQUANT_SINGLE_ROW = 0, ASCQ_DEQUANT_MULTI_ROW = 1 } ascq_dequant_mode;

/* Legacy AscendDequant<dstT, scaleT, mode>(dst, src, deqScale, params) and its scalar-deqScale overload
 * (include/adv_api/quantization/ascend_dequant.h:38-291), with arch 3510's kernels
 * (DequantPerchannelVFImpl / DequantPertensorVFImpl, impl/adv_api/detail/quantization/dequant/
 * ascend_dequant_3510_impl.h:37-210):
 *   policy PER_CHANNEL: the deqScale tensor `scale` (scale_type); PER_TENSOR: the scalar scale_scalar of
 *     scale_type (a BF16 scale_type rounds it to bf16, rne, first).
 *   mode SINGLE_ROW (the reference's default): {1, n, calCount} whose calCount is a whole number of 32-byte dst
 *     blocks and divides n is processed as {n / calCount, calCount, calCount} (UpdateDequantParams,
 *     ascend_dequant_common_impl.h:208-223); MULTI_ROW takes params as given.
 *   For each row i < m and column j < calCount: dst[i * ldd + j] = cast(f32(src[i * n + j]) * scale), with
 *     ldd = n rounded up to a whole 32-byte block of dst elements (dstInner, ascend_dequant_3510_impl.h:44, 99):
 *     dst holds m * ldd elements (ascq_ascend_dequant_dst_shape gives m and ldd after the SINGLE_ROW rule); columns
 *     >= calCount and the padding are not written.  int32 -> fp32 rounds ties away from zero (MrgZRndA, :61);
 *     cast = rne + saturating to f16 / bf16, or a plain f32 store.  A U64 deqScale contributes the low 32 bits
 *     of each word as an fp32 (:62-64).
 *   src_type INT32 (INT8 is accepted too: widened to int32, exact).
 *   (scale_type, dst_type) as IsTemplateValid allows (ascend_dequant_common_impl.h:126-155): tensor (U64, F16),
 *     (F32, F32), (BF16, F32), (BF16, BF16), (F32, BF16); scalar (BF16, BF16), (BF16, F32), (F32, F32), (F32, BF16).
 *   Argument checks of the reference's CPU-debug build (api_check/kernel_check/quantization/dequant/
 *     dequant_check_common.h): n % 8 == 0 and 0 < calCount <= n. */
ascq_status ascq_ascend_dequant(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                                int32_t scale_type, float scale_scalar, int32_t policy, int32_t mode,
                                const ascq_dequant_param* params, void* stream);
/* Rows and dst row stride (elements) that ascq_ascend_dequant writes for these params: the SINGLE_ROW rule of
 * UpdateDequantParams (ascend_dequant_common_impl.h:208-223) and dstInner (ascend_dequant_3510_impl.h:44, 99).
 * Host only. */
ascq_status ascq_ascend_dequant_dst_shape(int32_t dst_type, int32_t mode, const ascq_dequant_param* params,
                                          uint32_t* rows, uint32_t* row_stride);

/* AscendDeQuantParam{m, n, calCount, groupSize} + AscendDeQuantConfig{hasOffset, kDim}
 * (include/adv_api/quantization/ascend_dequant_utils.h:32-44) */
typedef struct {
    uint32_t m;
    uint32_t n;
    uint32_t cal_count;
    uint32_t group_size;
    int32_t has_offset;
    int32_t kdim;
} ascq_dequant_policy_param;

/* AscendDequant<dstT, srcT, scaleT, config, policy>(dst, src, scale, offset, para), the arch-3510 policy form
 * (include/adv_api/quantization/ascend_dequant.h:293-315; impl ascend_dequant_3510_impl.h:254-598, dispatch
 * :643-690).  src and dst [rows, n] row-major, rows = cal_count / n:
 *   PER_TOKEN: dst[r][c] = cast(f32(src[r][c]) * scale[r]);
 *   PER_GROUP, kdim 1: scale[r][c / group] ([rows][ceil(n / group)]); kdim 0: scale[r / group][c]
 *     ([ceil(rows / group)][n]); group_size a positive multiple of 32.
 * src_type INT32 (ties-away conversion) or F32 (INT8 accepted too, widened exactly); scale_type F16, BF16 or F32
 * (widened exactly); dst_type F16 / BF16 (rne, saturating) or F32.  The reference's kernels never read the
 * offset tensor, and neither does this one (offset and has_offset are accepted and unused). */
ascq_status ascq_ascend_dequant_policy(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                       const void* scale, const void* offset, int32_t scale_type, int32_t policy,
                                       const ascq_dequant_policy_param* para, void* stream);

/* ------------------------------------------------------------------------------------------
 * AscendAntiQuant
 * ------------------------------------------------------------------------------------------ */
/* AscendAntiQuant<InputDataType, OutputDataType, isTranspose>(dst, src, offset, scale, tmp, K, shapeInfo)
 * (include/adv_api/quantization/ascend_antiquant.h:47-225; AntiQuantShapeInfo ascend_antiquant_utils.h:26-31;
 * impl ascend_antiquant_impl.h:48-96, 285-411, ascend_antiquant_c220_impl.h:46-100).
 *   dst = (src + offset) * scale.  src_type INT8 or INT4; dst_type F16 or BF16 (offset/scale are dst_type).
 *   src_type HIF8 / FP8_E4M3 / FP8_E5M2 (arch 3510, per channel only: group_size 0; AntiQuantPerchannelImpl
 *   ascend_antiquant_3510_impl.h:752-770): fp8 in fp32 ops with one rne cast; hifloat8 in half ops to F16, in bf16 ops
 *   to BF16 when not transposed (PerchannelNoTransposeForB8 :470-495) and in fp32 ops when transposed
 *   (PerchannelTransposeForB8 :646-687); `arith` applies to INT8 / INT4 only.
 *   is_transpose 0: src [K, N], offset/scale [K/group, N];  1: src [N, K], offset/scale [N, K/group].
 *   group_size 0 = per-channel ([1, N] / [N, 1]).  offset NULL = scale only.  arith: ascq_arith
 *   (BF16 output always uses fp32 arithmetic). */
ascq_status ascq_ascend_antiquant(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                  const void* offset, const void* scale, uint32_t k, uint32_t n,
                                  uint32_t group_size, int32_t is_transpose, int32_t arith, void* stream);
/* AscendAntiQuant with scalar offset and scale of the output type, per tensor
 * (include/adv_api/quantization/ascend_antiquant.h:136-210; arch 3510 AntiQuantPertensorImpl,
 * impl/adv_api/detail/quantization/antiquant/ascend_antiquant_3510_impl.h:301-415):
 *   dst[i] = (src[i] + offset) * scale for i < count (has_offset 0: the scale-only overload, :166-190);
 * offset / scale are f16 or bf16 bit patterns of dst_type.  src INT8, INT4, HIF8: half ops for F16, fp32 ops and one
 * rne cast for BF16 (PerTensorProcessForB8 :334-392); FP8_E4M3 / FP8_E5M2: fp32 ops (PerTensorProcessForFp8 :301-333). */
ascq_status ascq_ascend_antiquant_scalar(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                         uint16_t offset, uint16_t scale, int32_t has_offset, uint64_t count,
                                         void* stream);

/* AscendAntiQuant<dstT, srcT, scaleT, config{hasOffset, isTranspose, kDim}, policy>(dst, src, scale, offset,
 * {m, n, calCount = m * n, groupSize}), the arch-3510 policy form (include/adv_api/quantization/ascend_antiquant.h:
 * 235-259; AscendAntiQuantConfig / Policy / Param impl/adv_api/detail/quantization/antiquant/
 * ascend_antiquant_common.h:46-66; impl ascend_antiquant_3510_impl.h:1386-1412, 1458-2110, dispatch :2175-2221).
 * src / dst [m, n] row-major.  Scale (and offset, NULL = config.hasOffset false) index of element (r, c):
 *   PER_TOKEN: scale[r] (is_transpose: scale[c]);
 *   PER_GROUP: along the columns, scale[r][c / group] ([m][ceil(n/group)]), when (k_dim == 1 && !is_transpose) ||
 *              (k_dim == 0 && is_transpose); else along the rows, scale[r / group][c] ([ceil(m/group)][n]);
 *              group_size a positive multiple of 32.
 * Arithmetic:
 *   src INT8 / HIF8: (src + offset) * scale, each op rounded in scale_type (F16 / BF16 / F32); a 16-bit scale_type
 *             writes dst of that type, F32 writes F32 or casts rne + saturating to F16 / BF16;
 *   src FP8_E4M3 / FP8_E5M2: the same in fp32 whatever scale_type (F16 / BF16 / F32), cast to dst;
 *   src FP4_E2M1 ([m, n/2] bytes, even element in the low nibble; n even): PER_GROUP only, scale_type E8M0
 *             (2^(e-127); e = 0 -> 2^-127, e = 255 -> NaN), no offset; bf16(src) * bf16(scale) rounded to bf16,
 *             dst BF16 or F16 (saturating cast);
 *   src FP4_E1M2: as FP4_E2M1 with E1M2 codes (exact in bf16; :2144-2159 route both fp4 types alike).
 * (ConvertSrc / StoreF32Res: ascend_antiquant_3510_impl.h:1363-1403; fp4 kernels :1724-1828) */
ascq_status ascq_ascend_antiquant_policy(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                         const void* scale, const void* offset, int32_t scale_type, int32_t policy,
                                         int64_t m, int64_t n, int64_t group_size, int32_t k_dim, int32_t is_transpose,
                                         void* stream);

/* ------------------------------------------------------------------------------------------
 * Quantize / Dequantize / AntiQuantize: the newer interface of include/adv_api/quantization/quantize.h:55-94,
 * dequantize.h:59-95 and antiquantize.h:61-98, on the kernels of the AscendQuant / AscendDequant / AscendAntiQuant
 * entry points above.  Tensors are [m, n] row-major; n is the element count of a row.
 * ------------------------------------------------------------------------------------------ */
/* QuantizeConfig{policy, hasOffset, roundMode, kDim} + QuantizeParams{m, n, groupSize}
 * (include/adv_api/quantization/quantize_utils.h:32-46); DequantizeConfig / AntiQuantizeConfig and their params carry
 * the same fields without roundMode (impl/adv_api/detail/quantization/dequantize/dequantize_common.h:27-44,
 * antiquantize/antiquantize_common.h:27-44) -- round_mode is read by ascq_quantize only. */
typedef struct {
    int32_t policy;     /* ascq_policy */
    int32_t has_offset;
    int32_t round_mode; /* ascq_round_mode */
    int32_t kdim;
    uint32_t m;
    uint32_t n;
    uint32_t group_size;
} ascq_quantize_param;

/* Quantize<config>(dst, src, scale, offset, params) (quantize.h:55-63; impl impl/adv_api/detail/quantization/
 * quantize/quantize_impl.h:1006-1066).  Every policy computes in fp32: y = f32(x) * f32(s), then + f32(o) when
 * has_offset (one fp32 rounding each; QuantizePerGroupForKColCommonVF :361-364, the other policies alike), and casts
 * y to dst_type:
 *   INT8: clamp(round_mode(y), -128, 127), NaN -> 0 (TransRegForS8 :128-190; modes other than rint / round / floor /
 *         ceil / trunc are rint);
 *   FP8_E4M3 / FP8_E5M2: rint with saturation, NaN -> 0 (TransRegForFp8 :80-90);
 *   HIF8: ties away from zero, saturating at +-32768, NaN -> 0 (TransRegForHif8 :92-126);
 *   FP4_E2M1 / FP4_E1M2 (PER_GROUP only, no offset, n even): y rounded to bf16 (rne, saturating, NaN -> 0), then
 *         the fp4 code in round_mode (TransRegForFp4 :192-230); two codes a byte, even element in the low nibble.
 * Scale (and offset) of element (r, c), by policy (:701-966, 446-700):
 *   PER_TENSOR: the scalars scale_scalar / offset_scalar (scale and offset must be NULL);
 *   PER_CHANNEL: scale[c] ([n]);  PER_TOKEN: scale[r] ([m]);
 *   PER_GROUP: kdim 1: scale[r][c / group] ([m][ceil(n / group)]); kdim 0: scale[r / group][c]
 *              ([ceil(m / group)][n]); group_size a positive multiple of 32.
 *   offset: a tensor indexed like scale, or (offset NULL, has_offset) the scalar offset_scalar.  Scalars are values
 *   of scale_type (rounded rne to it).
 * (src_type, scale_type) as CheckApiDtypeValid allows (:33-61): (F16, F16), (BF16, BF16), (F32, F32), (F16, F32),
 * (BF16, F32).  params.n must be a multiple of 32 (quantize_impl.h:1020).  dst holds m * n bytes (fp4: m * n / 2). */
ascq_status ascq_quantize(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                          const void* offset, float scale_scalar, float offset_scalar, int32_t scale_type,
                          const ascq_quantize_param* params, void* stream);

/* Dequantize<config>(dst, src, scale, offset, params) (dequantize.h:59-67; impl impl/adv_api/detail/quantization/
 * dequantize/dequantize_impl.h:254-290), a dispatch onto AscendDequant (type pairs IsDataTypeValid :67-92):
 *   PER_TENSOR: src INT32, the scalar scale_scalar (scale_type BF16 or F32; dst BF16 or F32) -- the legacy per-tensor
 *     kernel with params {m, n, n} in DEQUANT_WITH_MULTI_ROW (:94-116);
 *   PER_CHANNEL: src INT32, scale [n]: (U64, F16), (F32, F32), (BF16, F32), (BF16, BF16), (F32, BF16) -- the legacy
 *     per-channel kernel, {m, n, n}, MULTI_ROW (:118-138);
 *   PER_TOKEN / PER_GROUP: src INT32 or F32, scale [m] / as AscendDequant's policy form by kdim: (F16, F16),
 *     (BF16, BF16), (F32, F32), (F32, F16), (F32, BF16) (:140-195).
 * dst = cast(f32(src) * scale), int32 -> fp32 ties away from zero.  has_offset must be 0 (:102, 125, 148, 172: "do
 * not support offset currently").  n * sizeof(src) and n * sizeof(dst) must be multiples of 32 bytes. */
ascq_status ascq_dequantize(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                            float scale_scalar, int32_t scale_type, const ascq_quantize_param* params, void* stream);

/* AntiQuantize<config>(dst, src, scale, offset, params) (antiquantize.h:61-69; impl impl/adv_api/detail/
 * quantization/antiquantize/antiquantize_impl.h:284-302, antiquantize_3510_impl.h:38-396).  Every int8 / hifloat8 /
 * fp8 policy computes in fp32: y = (f32(src) + f32(o)) * f32(s) (+ o only when has_offset), one cast to dst_type
 * (rne, saturating; a plain store for F32):
 *   PER_TENSOR: src INT8 / HIF8 / FP8_E4M3 / FP8_E5M2, scalars scale_scalar / offset_scalar of dst_type = scale_type
 *     (F16 or BF16; rounded rne to it) (:76-102, 3510 :266-326);
 *   PER_CHANNEL: the same sources, scale / offset [n] of dst_type = scale_type (F16 or BF16) (:104-129, 3510
 *     :328-396);
 *   PER_TOKEN: scale / offset [m] (:131-159);  PER_GROUP: kdim 1 [m][ceil(n / group)], kdim 0 [ceil(m / group)][n],
 *     group_size a positive multiple of 32 (:161-226);  (scale_type, dst_type) for both: (F16, F16), (BF16, BF16),
 *     (F32, F32), (F32, F16), (F32, BF16) (IsDataTypeValid :46-74);
 *   PER_GROUP fp4: src FP4_E2M1 / FP4_E1M2 ([m, n / 2] bytes, n % 64 == 0), E8M0 scales, no offset, dst F16 or BF16:
 *     bf16(src) * bf16(scale) rounded to bf16 (ascq_ascend_antiquant_policy's fp4 rule).
 * n * sizeof(src) must be a multiple of 32 bytes (antiquantize_impl.h:99-100, 126-127, 153-154, 194). */
ascq_status ascq_antiquantize(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                              const void* offset, float scale_scalar, float offset_scalar, int32_t scale_type,
                              const ascq_quantize_param* params, void* stream);

/* ------------------------------------------------------------------------------------------
 * Weight-only antiquant matmul (W8A16 / W4A16)
 * The reference composes AscendAntiQuant (per group) with a half Matmul (fp32 L0C, half out);
 * here one fused kernel dequantises B in registers and feeds fp16 MFMA.
 * ------------------------------------------------------------------------------------------ */
/* Bytes of the packed B for a [K, N] weight of w_type INT8 or INT4 (K % 128 == 0, N % 16 == 0). */
ascq_status ascq_weight_pack_size(int32_t w_type, int64_t k, int64_t n, size_t* bytes);
/* Repack a row-major weight (is_transpose 0: [K, N]; 1: [N, K]) into the MFMA-native tile layout used by
 * ascq_antiquant_matmul -- the counterpart of the reference's ND -> NZ weight conversion
 * (examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/quant_group_matmul_high_performance/
 * scripts/gen_data.py:62; layout described in asc-devkit_clone_amd/csrc/gemv_antiquant.hip).
 * Device to device, on `stream`. */
ascq_status ascq_weight_pack(void* packed, const void* w, int32_t w_type, int64_t k, int64_t n,
                             int32_t is_transpose, void* stream);
/* y[M,N] (f16) = x[M,K] (f16) @ antiquant(w_packed) with fp32 accumulation: AscendAntiQuant per group
 * (ascend_antiquant_impl.h:63-96, 366-411) fused with a half Matmul whose L0C is fp32
 * (impl/adv_api/detail/matmul/utils/matmul_utils.h:171-174).
 * scale/offset: f16 [K/group_size, N]; offset may be NULL; group_size a multiple of 32 dividing K,
 * or 0 for per-channel [1, N].  M >= 1 (any value; decode shapes M in {1..64} are the fast path). */
ascq_status ascq_antiquant_matmul(uint16_t* y, const uint16_t* x, const void* w_packed, int32_t w_type,
                                  const uint16_t* scale, const uint16_t* offset, int64_t group_size, int64_t m,
                                  int64_t n, int64_t k, void* stream);

/* ------------------------------------------------------------------------------------------
 * Quantized group matmul (MoE)
 * ------------------------------------------------------------------------------------------ */
/* Activation of the group-matmul epilogue: none, or the sample's FasterGelu x / (1 + exp(-1.702 x)) in fp32
 * (quant_group_matmul_custom.asc:442-445; impl/adv_api/detail/activation/gelu/gelu_3510_impl.h:113-122). */
typedef enum { ASCQ_ACT_NONE = 0, ASCQ_ACT_FASTER_GELU = 1 } ascq_activation;

/* ------------------------------------------------------------------------------------------
 * Replaces quant_group_matmul_custom (examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/
 * quant_group_matmul_high_performance/quant_group_matmul_custom.asc:89-452, formula README_en.md:36-60):
 *   for group g, rows [s_g, s_g + cnt_g):  y = cast( act( (f32(x_g @ W_g) * scale[g, n]) * per_token_scale[m] ) )
 * x int8 [M, K]; per_token_scale f32 [M]; w int8 [G, K, N] (w_trans: [G, N, K]); scale f32 [G, N];
 * group_list int64 on the device: list_type 0 = G+1 prefix offsets, 1 = G counts (the reference form,
 * :263).  Rows outside every group are not written.  out_type BF16 or F16.  activation: ascq_activation (the
 * sample applies ASCQ_ACT_FASTER_GELU with f16 output).
 * ------------------------------------------------------------------------------------------ */
ascq_status ascq_quant_group_matmul(void* y, int32_t out_type, const int8_t* x, const float* per_token_scale,
                                    const int8_t* w, int32_t w_trans, const float* scale,
                                    const int64_t* group_list, int32_t list_type, int64_t num_groups, int64_t m,
                                    int64_t k, int64_t n, int32_t activation, void* stream);

/* ------------------------------------------------------------------------------------------
 * NZ fractal <-> ND layout converters
 * CubeFormat::NZ (include/adv_api/matmul/matmul_config.h:23-35): each [rows, cols] matrix of a batch is stored
 * [ceil(cols / C0)][ceil(rows / 16)][16][C0], C0 = 32 bytes of elements (int8 / fp8: 32, f16 / bf16: 16,
 * f32 / int32: 8) -- e.g. the group-matmul weights, weight.reshape([G, K/16, 16, N/32, 32]).transpose(0, 3, 1, 2, 4)
 * (examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/quant_group_matmul_high_performance/scripts/
 * gen_data.py:62).  Device to device on `stream`.
 * ------------------------------------------------------------------------------------------ */
/* Bytes of the NZ form of `batch` [rows, cols] matrices of `dtype` (padding included); 0 on bad arguments. */
size_t ascq_nz_size(int32_t dtype, int64_t batch, int64_t rows, int64_t cols);
/* NZ -> ND [batch][rows][cols]; transpose_out = 1 (1-byte types) writes [batch][cols][rows] instead: NZ int8
 * expert weights [G, K, N] become the K-contiguous [G, N, K] that ascq_quant_group_matmul takes with w_trans. */
ascq_status ascq_nz_to_nd(void* dst, const void* src, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                          int32_t transpose_out, void* stream);
/* ND [batch][rows][cols] -> NZ (padding written as zero) */
ascq_status ascq_nd_to_nz(void* dst, const void* src, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                          void* stream);

#ifdef __cplusplus
}
#endif
#endif /* ASCQ_H */
