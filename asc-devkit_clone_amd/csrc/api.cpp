// api.cpp -- the C ABI of libascq (include/ascq.h): argument validation, the Matmul handle and dispatch to
// the gfx950 kernels.  Every entry point checks its arguments on the host and returns a negative status
// before launching anything; there is no CPU fallback -- every compute path is a HIP kernel.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "../../include/ascq.h"
#include "launch.h"

namespace {

thread_local std::string g_err;
thread_local ascq::LaunchEvents g_launch_events;

// Host log, gated by the environment variable ASCQ_LOG (read once): unset or 0 = silent; 1 = the message of every
// failed call and every launch that takes a generic (fallback) kernel, on stderr; 2 = also one line per accepted call
// of the main entry points (name, types, shape).
int log_level()
{
    static const int level = [] {
        const char* e = std::getenv("ASCQ_LOG");
        return e ? std::atoi(e) : 0;
    }();
    return level;
}

void trace(const char* fmt, ...)
{
    if (log_level() < 2) return;
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    std::fprintf(stderr, "ascq: %s\n", buf);
}

ascq_status fail(ascq_status code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    if (log_level() >= 1) std::fprintf(stderr, "ascq: error %d: %s\n", (int)code, buf);
    return code;
}

ascq_status hip_status(hipError_t e, const char* what)
{
    if (e == hipSuccess) return ASCQ_OK;
    return fail(ASCQ_E_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Per-call state of an entry point that launches kernels: a HIP error left on this thread by an unrelated earlier
// call is cleared first, so the status the entry point returns is that of its own launches, and launch events armed
// by ascq_set_launch_events are disarmed on every return -- including argument-check failures that launch nothing,
// which would otherwise leave them armed for whatever kernel the thread launches next.
struct CallScope {
    CallScope() { (void)hipGetLastError(); }
    ~CallScope() { g_launch_events = ascq::LaunchEvents{}; }
    CallScope(const CallScope&) = delete;
    CallScope& operator=(const CallScope&) = delete;
};

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline bool valid_round(int32_t r) { return r >= ASCQ_ROUND_NONE && r <= ASCQ_ROUND_TRUNC; }

}  // namespace

namespace ascq {
void log_fallback(const char* kernel, const char* reason)
{
    if (log_level() >= 1) std::fprintf(stderr, "ascq: fallback: %s (%s)\n", kernel, reason);
}
}  // namespace ascq

// Scratch of ascq_matmul_iterate_all_noalloc: one array per device (the code object's copy on each GPU), held
// until the process ends.  Host code never uses the array's name as an address: it is looked up once per device
// with hipGetSymbolAddress and only that per-device pointer is handed to kernels.
static __device__ __align__(256) uint8_t scratch[ASCQ_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// the current device's scratch address (looked up on the first call on each device)
ascq_status scratch_for_current_device(void** out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(ASCQ_E_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
        if (!ptr) return fail(ASCQ_E_HIP, "hipGetSymbolAddress(scratch) returned a null address");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return ASCQ_OK;
}
}  // namespace

struct ascq_matmul_s {
    ascq_matmul_types ty{};
    int64_t M = 0, N = 0, K = 0;        // org shape
    int64_t sm = -1, sn = -1, sk = -1;  // single shape (-1: the org shape)
    const void* a = nullptr;
    int32_t trans_a = 0;
    const void* b = nullptr;
    int32_t trans_b = 0;
    const void* bias = nullptr;
    bool quant_set = false;
    const uint64_t* qvec = nullptr;
    uint64_t qscalar = 0;
    bool aq_set = false;
    bool aq_vec = false;
    uint16_t aq_off = 0, aq_scale = 0;
    const void* aq_off_vec = nullptr;
    const void* aq_scale_vec = nullptr;
    int64_t aq_group = 0;
    const uint8_t* scale_a = nullptr;
    int32_t trans_sa = 0;
    const uint8_t* scale_b = nullptr;
    int32_t trans_sb = 1;  // SetTensorScaleB defaults isTransposeScaleB = true (mx_matmul_impl.h:148)
    void* ws = nullptr;
    size_t ws_bytes = 0;
    bool ws_owned = false;
};

namespace {

enum Kind { K_NONE, K_INT8, K_ANTIQUANT, K_MX, K_F8, K_INT4, K_HIF8 };

bool is_f8(int32_t t) { return t == ASCQ_DT_FP8_E4M3 || t == ASCQ_DT_FP8_E5M2; }
bool is_fp4(int32_t t) { return t == ASCQ_DT_FP4_E2M1 || t == ASCQ_DT_FP4_E1M2; }
// f8f6f4 format code of an fp8 / fp4 element type (the MFMA's cbsz / blgp field)
int f8f6f4_code(int32_t t) { return t == ASCQ_DT_FP8_E5M2 ? 1 : (t == ASCQ_DT_FP4_E2M1 ? 4 : 0); }
constexpr int kF8F6F4Fp6E2M3 = 2;  // the code of fp6 E2M3 (the operand format of the E1M2 path)

Kind kind_of(const ascq_matmul_types& t)
{
    if (t.a_type == ASCQ_DT_INT8 && t.b_type == ASCQ_DT_INT8) return K_INT8;
    if (t.a_type == ASCQ_DT_INT4 && t.b_type == ASCQ_DT_INT4) return K_INT4;
    if (t.a_type == ASCQ_DT_F16 && (t.b_type == ASCQ_DT_INT8 || t.b_type == ASCQ_DT_INT4)) return K_ANTIQUANT;
    if (t.scale_type == ASCQ_DT_E8M0 &&
        ((is_fp4(t.a_type) && is_fp4(t.b_type)) || (is_f8(t.a_type) && is_f8(t.b_type))))
        return K_MX;
    if (t.scale_type == 0 && is_f8(t.a_type) && is_f8(t.b_type)) return K_F8;
    // hifloat8 A and B (the same type for both, matmul_fp8/README_en.md; quant_processor_utils.h:36-41)
    if (t.scale_type == 0 && t.a_type == ASCQ_DT_HIF8 && t.b_type == ASCQ_DT_HIF8) return K_HIF8;
    return K_NONE;
}

bool mx_is_fp4(const ascq_matmul_s* h) { return is_fp4(h->ty.a_type); }
// an E1M2 operand: both operands are rewritten to fp6 E2M3 planes (exact) for the f8f6f4 MFMA
bool mx_is_fp6(const ascq_matmul_s* h)
{
    return mx_is_fp4(h) && (h->ty.a_type == ASCQ_DT_FP4_E1M2 || h->ty.b_type == ASCQ_DT_FP4_E1M2);
}

// DEQF16 / QS322BF16_PRE for int8 with f16 / bf16 C; QF322{F16,BF16,F32}_PRE for fp8 (quant_processor_utils.h:31-55)
bool has_quant_epilogue(const ascq_matmul_types& t)
{
    const Kind k = kind_of(t);
    return ((k == K_INT8 || k == K_INT4) && t.c_type != ASCQ_DT_INT32) || k == K_F8 || k == K_HIF8;
}

// hifloat8 Matmul: both operands are decoded to bf16 rows of hif8_k_pad(K) values (K rounded up to a whole 16-byte
// chunk, the padding zero) in the workspace, A as [M, Kp] and B as [N, Kp]
int64_t hif8_k_pad(int64_t K) { return (K + 7) / 8 * 8; }

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// int8 / fp8 B given [K, N]: for large problems the whole org B is transposed to [N, K] in the workspace first,
// so the GEMM copies both operands straight into LDS (the transpose costs 2 K N bytes of traffic; the in-loop byte
// transpose of the [K, N] path roughly halves the GEMM's rate).  Below the 256 x 256 tile sizes (M or N < 1024) an
// int8 B [K, N] with N % 16 == 0 is not transposed: its GEMM copies the K rows into LDS and reads them with LDS
// transpose reads.
bool bytes_transposes_b(const ascq_matmul_s* h)
{
    if (h->ty.b_format == ASCQ_FORMAT_NZ) return false;  // converted from NZ instead (bytes_nz_b)
    if (kind_of(h->ty) == K_INT8 && h->N % 16 == 0 && (h->M < 1024 || h->N < 1024)) return false;
    return !h->trans_b && h->M >= 512 && h->N % 16 == 0 && h->K % 16 == 0;
}

// int8 / fp8 A given [K, M] (isTransA): the whole org A is transposed to [M, K] in the workspace (the tiled
// GEMM reads K-contiguous A rows only)
bool bytes_transposes_a(const ascq_matmul_s* h) { return h->trans_a != 0; }

// int8 / fp8 B in the NZ fractal layout: converted to a K-contiguous [N, K] copy in the workspace at every IterateAll
bool bytes_nz_b(const ascq_matmul_s* h) { return h->ty.b_format == ASCQ_FORMAT_NZ; }

// the operand copies of an int8 / fp8 Matmul (transposed or NZ-converted B, transposed A)
size_t bytes_operands(const ascq_matmul_s* h)
{
    size_t need = bytes_transposes_b(h) || bytes_nz_b(h) ? align256((size_t)h->N * (size_t)h->K) : 0;
    if (bytes_transposes_a(h)) need += align256((size_t)h->M * (size_t)h->K);
    return need;
}

// ... then, for decode-sized batches, the accumulators of the K split across workgroups
size_t bytes_workspace(const ascq_matmul_s* h)
{
    const int tb = h->trans_b || bytes_transposes_b(h) || bytes_nz_b(h);  // B as the GEMM sees it
    return bytes_operands(h) + align256(ascq::decode_split_ws_bytes(h->M, h->N, h->K, tb));
}

size_t workspace_need(const ascq_matmul_s* h)
{
    switch (kind_of(h->ty)) {
    case K_INT8:
    case K_F8: return bytes_workspace(h);
    case K_HIF8:
        return align256((size_t)h->M * (size_t)hif8_k_pad(h->K) * 2) + align256((size_t)h->N * (size_t)hif8_k_pad(h->K) * 2);
    case K_INT4:  // A and B unpacked to int8 [M, K] / [N, K]; a [K, N] B is nibble-transposed to [N, K/2] first
        return align256((size_t)h->M * (size_t)h->K) + align256((size_t)h->N * (size_t)h->K) +
               (h->trans_b ? 0 : align256((size_t)h->N * (size_t)h->K / 2));
    case K_ANTIQUANT: {
        size_t need = 0;
        if (h->ty.b_format == ASCQ_FORMAT_ND) need += ascq::weight_pack_bytes(h->ty.b_type, h->K, h->N);
        if (h->aq_set && !h->aq_vec) need += 2 * ((size_t)h->N * 2 + 256);
        return need;
    }
    case K_MX: {
        // [K, N] B transposed to [N, K]; both scale tensors rearranged stage-major; 256-byte aligned parts
        // fp6 (an E1M2 operand): the P and Q planes of A and of B as well
        const size_t kb = mx_is_fp4(h) ? (size_t)(h->K / 2) : (size_t)h->K;
        size_t need = h->trans_b ? 0 : align256((size_t)h->N * kb);
        need += ascq::mx_scale_workspace_bytes(h->M, h->N, h->K);
        if (mx_is_fp4(h) && !mx_is_fp6(h)) need += align256(ascq::mx_decode_split_ws_bytes(h->M, h->N, h->K));
        if (mx_is_fp6(h))
            need += align256((size_t)h->M * kb) + align256(ascq::fp6_q_plane_bytes(h->M, h->K)) +
                    align256((size_t)h->N * kb) + align256(ascq::fp6_q_plane_bytes(h->N, h->K));
        return need;
    }
    default: return 0;
    }
}

ascq_status ensure_workspace(ascq_matmul_s* h)
{
    const size_t need = workspace_need(h);
    if (need == 0 || h->ws_bytes >= need) return ASCQ_OK;
    if (h->ws && !h->ws_owned) return fail(ASCQ_E_INVALID_ARG, "workspace of %zu bytes is smaller than %zu", h->ws_bytes, need);
    if (h->ws_owned && h->ws) (void)hipFree(h->ws);
    h->ws = nullptr;
    h->ws_bytes = 0;
    hipError_t e = hipMalloc(&h->ws, need);
    if (e != hipSuccess) return hip_status(e, "hipMalloc(workspace)");
    h->ws_bytes = need;
    h->ws_owned = true;
    return ASCQ_OK;
}

// the K-split partials' region of the workspace for this call (null when the call cannot use it: no split form for
// these sizes, enAtomic, or a caller's workspace too small for it -- then the call runs without the split)
ascq_status split_region(ascq_matmul_s* h, int64_t m, int64_t n, int64_t k, uint8_t en_atomic, uint8_t** ws,
                         size_t* bytes)
{
    *ws = nullptr;
    *bytes = 0;
    const int tb = h->trans_b || bytes_transposes_b(h) || bytes_nz_b(h);  // B as the GEMM sees it
    const size_t need = ascq::decode_split_ws_bytes(m, n, k, tb);
    if (need == 0 || en_atomic != 0) return ASCQ_OK;
    const size_t off = bytes_operands(h);
    if (h->ws && !h->ws_owned) {  // the caller's workspace: used when it has room, never replaced
        if (h->ws_bytes < off + need) return ASCQ_OK;
    } else {
        ascq_status s = ensure_workspace(h);
        if (s != ASCQ_OK) return s;
        if (h->ws_bytes < off + need) return ASCQ_OK;
    }
    *ws = (uint8_t*)h->ws + off;
    *bytes = h->ws_bytes - off;
    return ASCQ_OK;
}

// int8 / fp8 operands after the workspace transposes (bytes_transposes_a / _b): pointers, leading dimensions
// (org shape) and the layouts the GEMM sees
struct ByteOperands {
    const uint8_t* A;
    const uint8_t* B;
    int64_t lda, ldb;
    int trans_a, trans_b;
};

ascq_status prepare_byte_operands(ascq_matmul_s* h, hipStream_t st, ByteOperands& o)
{
    o.A = (const uint8_t*)h->a;
    o.B = (const uint8_t*)h->b;
    o.lda = h->trans_a ? h->M : h->K;
    o.ldb = h->trans_b ? h->K : h->N;
    o.trans_a = h->trans_a;
    o.trans_b = h->trans_b;
    const bool tb = bytes_transposes_b(h), ta = bytes_transposes_a(h), nz = bytes_nz_b(h);
    if (!tb && !ta && !nz) return ASCQ_OK;
    ascq_status s = ensure_workspace(h);
    if (s != ASCQ_OK) return s;
    uint8_t* ws = (uint8_t*)h->ws;
    if (nz) {  // NZ B [K, N] (transposed on the way out) or [N, K] -> ND [N, K]
        hipError_t e = h->trans_b ? ascq::launch_nz_to_nd(ws, h->b, 1, 1, h->N, h->K, 0, st)
                                  : ascq::launch_nz_to_nd(ws, h->b, 1, 1, h->K, h->N, 1, st);
        if (e != hipSuccess) return hip_status(e, "NZ B to ND");
        o.B = ws;
        o.ldb = h->K;
        o.trans_b = 1;
        ws += align256((size_t)h->N * (size_t)h->K);
    }
    if (tb) {  // B [K, N] -> [N, K]
        hipError_t e = ascq::launch_transpose_i8(ws, (const uint8_t*)h->b, h->K, h->N, st);
        if (e != hipSuccess) return hip_status(e, "transpose B");
        o.B = ws;
        o.ldb = h->K;
        o.trans_b = 1;
        ws += align256((size_t)h->N * (size_t)h->K);
    }
    if (ta) {  // A [K, M] -> [M, K]
        hipError_t e = ascq::launch_transpose_i8(ws, (const uint8_t*)h->a, h->K, h->M, st);
        if (e != hipSuccess) return hip_status(e, "transpose A");
        o.A = ws;
        o.lda = h->K;
        o.trans_a = 0;
    }
    return ASCQ_OK;
}

__global__ void fill_u16_kernel(uint16_t* p, int64_t n, uint16_t v)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

}  // namespace

ascq::LaunchEvents& ascq::launch_events() { return g_launch_events; }

extern "C" {

const char* ascq_last_error(void) { return g_err.c_str(); }

ascq_status ascq_set_launch_events(void* start, void* stop)
{
    if ((start == nullptr) != (stop == nullptr))
        return fail(ASCQ_E_INVALID_ARG, "set_launch_events: give both events or neither");
    g_launch_events.start = reinterpret_cast<hipEvent_t>(start);
    g_launch_events.stop = reinterpret_cast<hipEvent_t>(stop);
    return ASCQ_OK;
}

const char* ascq_version(void) { return "ascq 0.1 (gfx950)"; }

int32_t ascq_device_count(void)
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

uint64_t ascq_pack_quant_pre(float m1, int32_t offset9, int32_t sign_flag)
{
    uint32_t u;
    std::memcpy(&u, &m1, 4);
    return (uint64_t)u | ((uint64_t)((uint32_t)offset9 & 0x1ffu) << 37) | ((uint64_t)(sign_flag & 1) << 46);
}

// ------------------------------------------------------------------------------------------------
// Matmul
// ------------------------------------------------------------------------------------------------
ascq_status ascq_matmul_create(const ascq_matmul_types* types, ascq_matmul_t* out)
{
    if (!types || !out) return fail(ASCQ_E_INVALID_ARG, "matmul_create: null argument");
    *out = nullptr;
    const Kind k = kind_of(*types);
    if (k == K_NONE)
        return fail(ASCQ_E_UNSUPPORTED, "matmul_create: unsupported A/B types (%d, %d)", types->a_type, types->b_type);
    if (k == K_INT8 || k == K_INT4) {
        if (types->c_type != ASCQ_DT_F16 && types->c_type != ASCQ_DT_BF16 && types->c_type != ASCQ_DT_INT32 &&
            types->c_type != ASCQ_DT_INT8 && types->c_type != ASCQ_DT_UINT8 && types->c_type != ASCQ_DT_INT4)
            return fail(ASCQ_E_UNSUPPORTED,
                        "matmul_create: int8 matmul supports C = f16, bf16, int32, int8, uint8 or int4");
        if (types->bias_type != 0 && types->bias_type != ASCQ_DT_INT32)
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: int8 matmul bias must be int32");
        if (types->b_format != ASCQ_FORMAT_ND && !(k == K_INT8 && types->b_format == ASCQ_FORMAT_NZ))
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: int8 B must be ND or NZ, int4 B ND");
    } else if (k == K_ANTIQUANT) {
        if (types->c_type != ASCQ_DT_F16) return fail(ASCQ_E_UNSUPPORTED, "matmul_create: weight-only matmul supports C = f16");
        if (types->b_format != ASCQ_FORMAT_ND && types->b_format != ASCQ_FORMAT_PACKED)
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: weight-only B must be ND or PACKED");
        if (types->bias_type != 0) return fail(ASCQ_E_UNSUPPORTED, "matmul_create: weight-only matmul has no bias path");
    } else if (k == K_F8 || k == K_HIF8) {
        const char* what = k == K_F8 ? "fp8" : "hifloat8";
        if (types->c_type != ASCQ_DT_F16 && types->c_type != ASCQ_DT_BF16 && types->c_type != ASCQ_DT_F32 &&
            types->c_type != ASCQ_DT_INT8 && types->c_type != ASCQ_DT_UINT8 && types->c_type != ASCQ_DT_INT4 &&
            !is_f8(types->c_type) && types->c_type != ASCQ_DT_HIF8)
            return fail(ASCQ_E_UNSUPPORTED,
                        "matmul_create: %s matmul supports C = f16, bf16, f32, int8, uint8, int4, fp8_e4m3, fp8_e5m2 or "
                        "hifloat8", what);
        if (types->bias_type != 0 && types->bias_type != ASCQ_DT_F32)
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: %s matmul bias must be f32", what);
        if (types->b_format != ASCQ_FORMAT_ND && !(k == K_F8 && types->b_format == ASCQ_FORMAT_NZ))
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: %s B must be ND%s", what, k == K_F8 ? " or NZ" : "");
    } else {
        if (types->c_type != ASCQ_DT_BF16 && types->c_type != ASCQ_DT_F32)
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: MX matmul supports C = bf16 or f32");
        if (types->bias_type != 0 && types->bias_type != ASCQ_DT_F32)
            return fail(ASCQ_E_UNSUPPORTED, "matmul_create: MX matmul bias must be f32");
        if (types->b_format != ASCQ_FORMAT_ND) return fail(ASCQ_E_UNSUPPORTED, "matmul_create: MX B must be ND");
    }
    auto* h = new (std::nothrow) ascq_matmul_s();
    if (!h) return fail(ASCQ_E_INVALID_ARG, "matmul_create: out of host memory");
    h->ty = *types;
    *out = h;
    return ASCQ_OK;
}

ascq_status ascq_matmul_init(ascq_matmul_t h, const ascq_cube_tiling* t)
{
    if (!h || !t) return fail(ASCQ_E_INVALID_ARG, "matmul_init: null argument");
    if (t->M <= 0 || t->N <= 0 || t->Ka <= 0) return fail(ASCQ_E_INVALID_ARG, "matmul_init: tiling shape must be positive");
    if (t->Kb != t->Ka) return fail(ASCQ_E_INVALID_ARG, "matmul_init: Ka (%d) and Kb (%d) differ", t->Ka, t->Kb);
    h->M = t->M;
    h->N = t->N;
    h->K = t->Ka;
    h->sm = h->sn = h->sk = -1;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_org_shape(ascq_matmul_t h, int64_t m, int64_t n, int64_t k)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    if (m <= 0 || n <= 0 || k <= 0) return fail(ASCQ_E_INVALID_ARG, "set_org_shape: shape must be positive");
    h->M = m;
    h->N = n;
    h->K = k;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_single_shape(ascq_matmul_t h, int64_t m, int64_t n, int64_t k)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    if (m <= 0 || n <= 0 || k <= 0) return fail(ASCQ_E_INVALID_ARG, "set_single_shape: shape must be positive");
    h->sm = m;
    h->sn = n;
    h->sk = k;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_tail(ascq_matmul_t h, int64_t tail_m, int64_t tail_n, int64_t tail_k)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    // SetTail(-1) keeps a dimension (matmul.h:117 default arguments)
    if (tail_m > 0) h->sm = tail_m;
    if (tail_n > 0) h->sn = tail_n;
    if (tail_k > 0) h->sk = tail_k;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_tensor_a(ascq_matmul_t h, const void* a, int32_t is_transpose_a)
{
    if (!h || !a) return fail(ASCQ_E_INVALID_ARG, "set_tensor_a: null argument");
    h->a = a;
    h->trans_a = is_transpose_a ? 1 : 0;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_tensor_b(ascq_matmul_t h, const void* b, int32_t is_transpose_b)
{
    if (!h || !b) return fail(ASCQ_E_INVALID_ARG, "set_tensor_b: null argument");
    h->b = b;
    h->trans_b = is_transpose_b ? 1 : 0;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_bias(ascq_matmul_t h, const void* bias)
{
    if (!h || !bias) return fail(ASCQ_E_INVALID_ARG, "set_bias: null argument");
    if (h->ty.bias_type != ASCQ_DT_INT32 && h->ty.bias_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "set_bias: the handle has no bias type");
    if (!aligned(bias, 4)) return fail(ASCQ_E_INVALID_ARG, "set_bias: pointer must be 4-byte aligned");
    h->bias = bias;
    return ASCQ_OK;
}

ascq_status ascq_matmul_disable_bias(ascq_matmul_t h)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    h->bias = nullptr;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_quant_scalar(ascq_matmul_t h, uint64_t quant_scalar)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    if (!has_quant_epilogue(h->ty))
        return fail(ASCQ_E_UNSUPPORTED, "set_quant_scalar: no quant epilogue for this type combination");
    h->quant_set = true;
    h->qvec = nullptr;
    h->qscalar = quant_scalar;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_quant_vector(ascq_matmul_t h, const uint64_t* quant_vector)
{
    if (!h || !quant_vector) return fail(ASCQ_E_INVALID_ARG, "set_quant_vector: null argument");
    if (!has_quant_epilogue(h->ty))
        return fail(ASCQ_E_UNSUPPORTED, "set_quant_vector: no quant epilogue for this type combination");
    if (!aligned(quant_vector, 8)) return fail(ASCQ_E_INVALID_ARG, "set_quant_vector: pointer must be 8-byte aligned");
    h->quant_set = true;
    h->qvec = quant_vector;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_antiquant_scalar(ascq_matmul_t h, uint16_t offset_f16, uint16_t scale_f16)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    if (kind_of(h->ty) != K_ANTIQUANT) return fail(ASCQ_E_UNSUPPORTED, "set_antiquant_scalar: not a weight-only handle");
    h->aq_set = true;
    h->aq_vec = false;
    h->aq_off = offset_f16;
    h->aq_scale = scale_f16;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_antiquant_vector(ascq_matmul_t h, const void* offset, const void* scale, int64_t group_size)
{
    if (!h || !scale) return fail(ASCQ_E_INVALID_ARG, "set_antiquant_vector: null argument");
    if (kind_of(h->ty) != K_ANTIQUANT) return fail(ASCQ_E_UNSUPPORTED, "set_antiquant_vector: not a weight-only handle");
    if (group_size < 0 || (group_size > 0 && group_size % 32 != 0))
        return fail(ASCQ_E_INVALID_ARG, "set_antiquant_vector: group_size must be 0 or a multiple of 32");
    h->aq_set = true;
    h->aq_vec = true;
    h->aq_off_vec = offset;
    h->aq_scale_vec = scale;
    h->aq_group = group_size;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_tensor_scale_a(ascq_matmul_t h, const uint8_t* scale_a, int32_t is_transpose_scale_a)
{
    if (!h || !scale_a) return fail(ASCQ_E_INVALID_ARG, "set_tensor_scale_a: null argument");
    if (kind_of(h->ty) != K_MX) return fail(ASCQ_E_UNSUPPORTED, "set_tensor_scale_a: not an MX handle");
    h->scale_a = scale_a;
    h->trans_sa = is_transpose_scale_a ? 1 : 0;
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_tensor_scale_b(ascq_matmul_t h, const uint8_t* scale_b, int32_t is_transpose_scale_b)
{
    if (!h || !scale_b) return fail(ASCQ_E_INVALID_ARG, "set_tensor_scale_b: null argument");
    if (kind_of(h->ty) != K_MX) return fail(ASCQ_E_UNSUPPORTED, "set_tensor_scale_b: not an MX handle");
    h->scale_b = scale_b;
    h->trans_sb = is_transpose_scale_b ? 1 : 0;
    return ASCQ_OK;
}

ascq_status ascq_matmul_workspace_size(ascq_matmul_t h, size_t* bytes)
{
    if (!h || !bytes) return fail(ASCQ_E_INVALID_ARG, "workspace_size: null argument");
    *bytes = workspace_need(h);
    return ASCQ_OK;
}

ascq_status ascq_matmul_set_workspace(ascq_matmul_t h, void* workspace, size_t bytes)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    if (h->ws_owned && h->ws) (void)hipFree(h->ws);
    h->ws = workspace;
    h->ws_bytes = workspace ? bytes : 0;
    h->ws_owned = false;
    return ASCQ_OK;
}

ascq_status ascq_matmul_iterate_all(ascq_matmul_t h, void* c, uint8_t en_atomic, void* stream)
{
    CallScope scope;
    if (!h || !c) return fail(ASCQ_E_INVALID_ARG, "iterate_all: null argument");
    if (en_atomic > 3) return fail(ASCQ_E_INVALID_ARG, "iterate_all: enAtomic must be 0 (store), 1 (add), 2 (max) or 3 (min)");
    // The copy-out combines into C only for the C types SetAtomic takes (scheduler_base.h:484-494: float, half,
    // int16_t, int32_t, int8_t, bfloat16_t); for the others (uint8, int4, fp8) the reference stores, and so does this.
    // int8 C is refused: the saturation of the int8 accumulation is not published.
    const int32_t ct = h->ty.c_type;
    int atomic = en_atomic;
    if (ct != ASCQ_DT_INT32 && ct != ASCQ_DT_F32 && ct != ASCQ_DT_F16 && ct != ASCQ_DT_BF16) {
        if (ct == ASCQ_DT_INT8 && atomic != 0)
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: enAtomic with an int8 C is not supported");
        atomic = ascq::C_STORE;
    }
    if (!h->a || !h->b) return fail(ASCQ_E_STATE, "iterate_all: SetTensorA and SetTensorB must precede IterateAll");
    if (h->M <= 0) return fail(ASCQ_E_STATE, "iterate_all: SetOrgShape must precede IterateAll");
    const int64_t m = h->sm > 0 ? h->sm : h->M, n = h->sn > 0 ? h->sn : h->N, k = h->sk > 0 ? h->sk : h->K;
    if (m > h->M || n > h->N || k > h->K) return fail(ASCQ_E_INVALID_ARG, "iterate_all: single shape exceeds org shape");
    hipStream_t st = S(stream);
    trace("iterate_all: A %d B %d C %d kind %d, M %lld N %lld K %lld, transA %d transB %d, enAtomic %d", h->ty.a_type,
          h->ty.b_type, h->ty.c_type, (int)kind_of(h->ty), (long long)m, (long long)n, (long long)k, h->trans_a,
          h->trans_b, atomic);
    switch (kind_of(h->ty)) {
    case K_INT8: {
        if (h->ty.c_type != ASCQ_DT_INT32 && !h->quant_set)
            return fail(ASCQ_E_STATE, "iterate_all: f16/bf16/int8/uint8/int4 output needs SetQuantScalar or SetQuantVector");
        if (h->ty.c_type == ASCQ_DT_INT4 && (h->N % 2 != 0 || n % 2 != 0))
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: int4 C packs two codes per byte: N must be even");
        ascq::GemmI8Args g{};
        g.A = (const int8_t*)h->a;
        g.B = (const int8_t*)h->b;
        g.bias = (const int32_t*)h->bias;
        g.C = c;
        g.M = m;
        g.N = n;
        g.K = k;
        g.lda = h->trans_a ? h->M : h->K;
        g.ldb = h->trans_b ? h->K : h->N;
        g.ldc = h->N;
        g.qvec = h->qvec;
        g.qscalar = h->qscalar;
        switch (h->ty.c_type) {
        case ASCQ_DT_INT32: g.epi = ascq::EPI_I32; break;
        case ASCQ_DT_F16: g.epi = ascq::EPI_DEQ_F16; break;
        case ASCQ_DT_BF16: g.epi = ascq::EPI_DEQ_BF16; break;
        case ASCQ_DT_INT4: g.epi = ascq::EPI_REQ4; break;  // (V)REQ4
        default: g.epi = ascq::EPI_REQ8; break;            // int8 / uint8: (V)REQ8
        }
        ByteOperands o;
        ascq_status s = prepare_byte_operands(h, st, o);
        if (s != ASCQ_OK) return s;
        g.A = (const int8_t*)o.A;
        g.B = (const int8_t*)o.B;
        g.lda = o.lda;
        g.ldb = o.ldb;
        g.trans_a = o.trans_a;
        g.trans_b = o.trans_b;
        g.atomic = atomic;
        s = split_region(h, m, n, k, atomic, &g.ws, &g.ws_bytes);
        if (s != ASCQ_OK) return s;
        return hip_status(ascq::launch_gemm_i8(g, st), "gemm_i8");
    }
    case K_INT4: {
        // int4b_t A / B (matmul_int4.asc:151; README constraints: A not transposed, C int32 or half): both are
        // unpacked to int8 in the workspace, then the int8 GEMM and its epilogues run unchanged (exact: int4 x int4
        // products sum in int32 as on the cube unit)
        if (h->trans_a) return fail(ASCQ_E_UNSUPPORTED, "iterate_all: an int4 A cannot be transposed");
        if (h->K % 2 != 0 || h->N % 2 != 0)
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: int4 operands pack two per byte: K and N must be even");
        if (h->ty.c_type != ASCQ_DT_INT32 && !h->quant_set)
            return fail(ASCQ_E_STATE, "iterate_all: f16/bf16/int8/uint8/int4 output needs SetQuantScalar or SetQuantVector");
        if (h->ty.c_type == ASCQ_DT_INT4 && n % 2 != 0)
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: int4 C packs two codes per byte: N must be even");
        ascq_status s = ensure_workspace(h);
        if (s != ASCQ_OK) return s;
        int8_t* a8 = (int8_t*)h->ws;
        int8_t* b8 = a8 + align256((size_t)h->M * (size_t)h->K);
        hipError_t e = ascq::launch_unpack_int4(a8, (const uint8_t*)h->a, h->M * h->K / 2, st);
        if (e != hipSuccess) return hip_status(e, "unpack A");
        const uint8_t* bsrc = (const uint8_t*)h->b;
        if (!h->trans_b) {  // [K, N/2] packed along N -> [N, K/2] packed along K
            uint8_t* bt = (uint8_t*)b8 + align256((size_t)h->N * (size_t)h->K);
            e = ascq::launch_fp4_transpose(bt, bsrc, h->K, h->N, st);
            if (e != hipSuccess) return hip_status(e, "transpose B");
            bsrc = bt;
        }
        e = ascq::launch_unpack_int4(b8, bsrc, h->N * h->K / 2, st);
        if (e != hipSuccess) return hip_status(e, "unpack B");
        ascq::GemmI8Args g{};
        g.A = a8;
        g.B = b8;
        g.bias = (const int32_t*)h->bias;
        g.C = c;
        g.M = m;
        g.N = n;
        g.K = k;
        g.lda = h->K;
        g.ldb = h->K;
        g.ldc = h->N;
        g.qvec = h->qvec;
        g.qscalar = h->qscalar;
        g.trans_a = 0;
        g.trans_b = 1;
        g.atomic = atomic;
        switch (h->ty.c_type) {
        case ASCQ_DT_INT32: g.epi = ascq::EPI_I32; break;
        case ASCQ_DT_F16: g.epi = ascq::EPI_DEQ_F16; break;
        case ASCQ_DT_BF16: g.epi = ascq::EPI_DEQ_BF16; break;
        case ASCQ_DT_INT4: g.epi = ascq::EPI_REQ4; break;
        default: g.epi = ascq::EPI_REQ8; break;
        }
        return hip_status(ascq::launch_gemm_i8(g, st), "gemm_i8 (int4 operands)");
    }
    case K_HIF8: {
        // hifloat8 A / B (matmul_fp8.asc:229): both decoded exactly to bf16 K-contiguous rows in the workspace (every
        // HiF8 value is a bf16 value), then the bf16-MFMA form of the fp8 GEMM with the same fp32 accumulators and
        // QF322*_PRE epilogues
        const int32_t ct = h->ty.c_type;
        if ((ct == ASCQ_DT_INT8 || ct == ASCQ_DT_UINT8 || ct == ASCQ_DT_INT4 || is_f8(ct) || ct == ASCQ_DT_HIF8) &&
            !h->quant_set)
            return fail(ASCQ_E_STATE,
                        "iterate_all: int8/uint8/int4/fp8/hifloat8 output needs SetQuantScalar or SetQuantVector");
        if (ct == ASCQ_DT_INT4 && (h->N % 2 != 0 || n % 2 != 0))
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: int4 C packs two codes per byte: N must be even");
        const int64_t kp = hif8_k_pad(h->K);
        ascq_status s = ensure_workspace(h);
        if (s != ASCQ_OK) return s;
        uint16_t* a16 = (uint16_t*)h->ws;
        uint16_t* b16 = (uint16_t*)((uint8_t*)h->ws + align256((size_t)h->M * (size_t)kp * 2));
        hipError_t e = ascq::launch_hif8_to_bf16(a16, kp, (const uint8_t*)h->a, h->M, h->K, h->trans_a, st);
        if (e == hipSuccess) e = ascq::launch_hif8_to_bf16(b16, kp, (const uint8_t*)h->b, h->N, h->K, !h->trans_b, st);
        if (e != hipSuccess) return hip_status(e, "hifloat8 -> bf16");
        ascq::GemmF8Args g{};
        g.A = (const uint8_t*)a16;
        g.B = (const uint8_t*)b16;
        g.lda = kp;
        g.ldb = kp;
        g.trans_a = 0;
        g.trans_b = 1;
        g.bias = (const float*)h->bias;
        g.C = c;
        g.M = m;
        g.N = n;
        g.K = k == h->K ? kp : k;  // the zero padding adds nothing
        g.ldc = h->N;
        g.qvec = h->qvec;
        g.qscalar = h->qscalar;
        g.use_quant = h->quant_set ? 1 : 0;
        g.c_type = ct;
        g.fmt_a = g.fmt_b = ascq::FMT_BF16;
        g.atomic = atomic;
        return hip_status(ascq::launch_gemm_f8(g, st), "gemm_f8 (hifloat8 operands)");
    }
    case K_F8: {
        const int32_t ct = h->ty.c_type;
        if ((ct == ASCQ_DT_INT8 || ct == ASCQ_DT_UINT8 || ct == ASCQ_DT_INT4 || is_f8(ct) || ct == ASCQ_DT_HIF8) &&
            !h->quant_set)
            return fail(ASCQ_E_STATE,
                        "iterate_all: int8/uint8/int4/fp8/hifloat8 output needs SetQuantScalar or SetQuantVector");
        if (ct == ASCQ_DT_INT4 && (h->N % 2 != 0 || n % 2 != 0))
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: int4 C packs two codes per byte: N must be even");
        ascq::GemmF8Args g{};
        ByteOperands o;
        ascq_status s = prepare_byte_operands(h, st, o);
        if (s != ASCQ_OK) return s;
        g.A = o.A;
        g.B = o.B;
        g.lda = o.lda;
        g.ldb = o.ldb;
        g.trans_a = o.trans_a;
        g.trans_b = o.trans_b;
        g.bias = (const float*)h->bias;
        g.C = c;
        g.M = m;
        g.N = n;
        g.K = k;
        g.ldc = h->N;
        g.qvec = h->qvec;
        g.qscalar = h->qscalar;
        g.use_quant = h->quant_set ? 1 : 0;
        g.c_type = h->ty.c_type;  // ascq_dtype codes equal the device DT_* codes
        g.fmt_a = f8f6f4_code(h->ty.a_type);
        g.fmt_b = f8f6f4_code(h->ty.b_type);
        g.atomic = atomic;
        s = split_region(h, m, n, k, atomic, &g.ws, &g.ws_bytes);
        if (s != ASCQ_OK) return s;
        return hip_status(ascq::launch_gemm_f8(g, st), "gemm_f8");
    }
    case K_ANTIQUANT: {
        if (!h->aq_set) return fail(ASCQ_E_STATE, "iterate_all: SetAntiQuantScalar/Vector must precede IterateAll");
        if (m != h->M || n != h->N || k != h->K)
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: weight-only matmul computes the full org shape only");
        if (h->trans_a) return fail(ASCQ_E_UNSUPPORTED, "iterate_all: weight-only matmul needs A = [M, K]");
        if (h->K % 128 != 0 || h->N % 16 != 0)
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: weight-only matmul needs K %% 128 == 0 and N %% 16 == 0");
        if (h->aq_vec && h->aq_group > 0 && h->K % h->aq_group != 0)
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: group_size must divide K");
        if (!aligned(h->a, 16)) return fail(ASCQ_E_INVALID_ARG, "iterate_all: A must be 16-byte aligned");
        ascq_status s = ensure_workspace(h);
        if (s != ASCQ_OK) return s;
        uint8_t* ws = (uint8_t*)h->ws;
        const void* wp = h->b;
        if (h->K * h->N >= (1ll << 31))
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: the weight must stay below 2^31 elements");
        if (h->ty.b_format == ASCQ_FORMAT_ND) {
            hipError_t e = ascq::launch_weight_pack(ws, h->b, h->ty.b_type, h->K, h->N, h->trans_b, st);
            if (e != hipSuccess) return hip_status(e, "weight_pack");
            wp = ws;
            ws += (ascq::weight_pack_bytes(h->ty.b_type, h->K, h->N) + 255) / 256 * 256;
        } else if (!aligned(h->b, 16)) {
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: packed B must be 16-byte aligned");
        }
        const uint16_t* sc = (const uint16_t*)h->aq_scale_vec;
        const uint16_t* of = (const uint16_t*)h->aq_off_vec;
        int64_t grp = h->aq_group;
        if (!h->aq_vec) {
            uint16_t* s16 = (uint16_t*)ws;
            uint16_t* o16 = s16 + (h->N + 127) / 128 * 128;
            hipLaunchKernelGGL(fill_u16_kernel, dim3(64), dim3(256), 0, st, s16, h->N, h->aq_scale);
            hipLaunchKernelGGL(fill_u16_kernel, dim3(64), dim3(256), 0, st, o16, h->N, h->aq_off);
            sc = s16;
            of = o16;
            grp = 0;
        }
        return hip_status(ascq::launch_antiquant_matmul((uint16_t*)c, (const uint16_t*)h->a, wp, h->ty.b_type, sc, of,
                                                        grp, h->M, h->N, h->K, atomic, st),
                          "antiquant_matmul");
    }
    case K_MX: {
        if (!h->scale_a || !h->scale_b) return fail(ASCQ_E_STATE, "iterate_all: SetTensorScaleA/B must precede IterateAll");
        if (m != h->M || n != h->N || k != h->K)
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: MX matmul computes the full org shape only");
        if (h->trans_a) return fail(ASCQ_E_UNSUPPORTED, "iterate_all: MX matmul needs A = [M, K]");
        const bool fp4 = mx_is_fp4(h);
        if (h->K % (fp4 ? 128 : 64) != 0)
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: MX matmul needs K %% %d == 0", fp4 ? 128 : 64);
        const int64_t kb = fp4 ? h->K / 2 : h->K;  // bytes per row
        if (h->M * kb >= (1ll << 31) || h->N * kb >= (1ll << 31))
            return fail(ASCQ_E_UNSUPPORTED, "iterate_all: MX operands must stay below 2 GiB");
        if (fp4 && !h->trans_b && h->N % 2 != 0) return fail(ASCQ_E_INVALID_ARG, "iterate_all: [K, N] fp4 B needs even N");
        if (!aligned(h->a, 16) || !aligned(h->b, 16) || !aligned(h->scale_a, 4) || !aligned(h->scale_b, 4))
            return fail(ASCQ_E_INVALID_ARG, "iterate_all: MX operands must be 16-byte (scales 4-byte) aligned");
        // a caller's workspace sized without the decode partials runs the call without the K split across workgroups
        const size_t part = fp4 && !mx_is_fp6(h) ? align256(ascq::mx_decode_split_ws_bytes(h->M, h->N, h->K)) : 0;
        const size_t need = workspace_need(h);
        const bool no_part = h->ws && !h->ws_owned && h->ws_bytes < need && h->ws_bytes + part >= need;
        if (!no_part) {
            ascq_status s = ensure_workspace(h);
            if (s != ASCQ_OK) return s;
        }
        const uint8_t* at = (const uint8_t*)h->a;
        const uint8_t* bt = (const uint8_t*)h->b;
        const uint8_t* sa = h->scale_a;
        const uint8_t* sb = h->scale_b;
        uint8_t* ws = (uint8_t*)h->ws;
        if (!h->trans_b) {
            hipError_t e = fp4 ? ascq::launch_fp4_transpose(ws, (const uint8_t*)h->b, h->K, h->N, st)
                               : ascq::launch_transpose_i8(ws, (const uint8_t*)h->b, h->K, h->N, st);
            if (e != hipSuccess) return hip_status(e, "transpose B");
            bt = ws;
            ws += align256((size_t)h->N * (size_t)(fp4 ? h->K / 2 : h->K));
        }
        const bool fp6 = mx_is_fp6(h);
        const uint8_t* aq = nullptr;
        const uint8_t* bq = nullptr;
        if (fp6) {  // both operands -> fp6 E2M3 P / Q planes
            uint8_t* pa = ws;
            uint8_t* qa = pa + align256((size_t)h->M * (size_t)(h->K / 2));
            uint8_t* pb = qa + align256(ascq::fp6_q_plane_bytes(h->M, h->K));
            uint8_t* qb = pb + align256((size_t)h->N * (size_t)(h->K / 2));
            ws = qb + align256(ascq::fp6_q_plane_bytes(h->N, h->K));
            hipError_t e = ascq::launch_fp4_to_fp6_planes(pa, qa, at, h->M, h->K, h->ty.a_type == ASCQ_DT_FP4_E1M2, st);
            if (e == hipSuccess)
                e = ascq::launch_fp4_to_fp6_planes(pb, qb, bt, h->N, h->K, h->ty.b_type == ASCQ_DT_FP4_E1M2, st);
            if (e != hipSuccess) return hip_status(e, "fp4 -> fp6 planes");
            at = pa;
            bt = pb;
            aq = qa;
            bq = qb;
        }
        ascq::MxGemmArgs g{};
        g.A = at;
        g.B = bt;
        g.Aq = aq;
        g.Bq = bq;
        g.sA = sa;
        g.sB = sb;
        g.sa_layout = h->trans_sa ? 1 : 0;  // scaleA [M, sK], or [sK/2, M, 2] with isTransposeScaleA
        g.sb_layout = h->trans_sb ? 1 : 0;  // scaleB [sK/2, N, 2], or [N, sK] with isTransposeScaleB
        g.ws_scales = ws;  // after the B transpose (if any); the GEMM rearranges both scale tensors here
        if (part && !no_part) {  // then the decode partials
            g.ws_part = ws + align256(ascq::mx_scale_workspace_bytes(h->M, h->N, h->K));
            g.ws_part_bytes = part;
        }
        g.M = h->M;
        g.N = h->N;
        g.K = h->K;
        g.C = c;
        g.c_type = h->ty.c_type;  // ascq_dtype codes equal the device DT_* codes
        g.fmt_a = fp6 ? kF8F6F4Fp6E2M3 : f8f6f4_code(h->ty.a_type);
        g.fmt_b = fp6 ? kF8F6F4Fp6E2M3 : f8f6f4_code(h->ty.b_type);
        g.bias = (const float*)h->bias;
        g.atomic = atomic;
        return hip_status(ascq::launch_mx_gemm(g, st), "mx_gemm");
    }
    default: return fail(ASCQ_E_UNSUPPORTED, "iterate_all: unsupported handle");
    }
}

ascq_status ascq_matmul_iterate_all_noalloc(ascq_matmul_t h, void* c, uint8_t en_atomic, void* stream)
{
    CallScope scope;
    if (!h || !c) return fail(ASCQ_E_INVALID_ARG, "iterate_all_noalloc: null argument");
    const size_t need = workspace_need(h);
    if (need > ASCQ_NOALLOC_SCRATCH_BYTES)
        return fail(ASCQ_E_UNSUPPORTED,
                    "iterate_all_noalloc: this handle needs %zu bytes of workspace, above the %zu-byte static scratch "
                    "(use ascq_matmul_iterate_all with a workspace)", need, (size_t)ASCQ_NOALLOC_SCRATCH_BYTES);
    void* ptr = nullptr;
    if (need > 0) {
        ascq_status s = scratch_for_current_device(&ptr);
        if (s != ASCQ_OK) return s;
    }
    // run IterateAll on a copy of the handle whose workspace is the scratch (ensure_workspace then sees enough room
    // and allocates nothing); the caller's handle is only read, so it never holds the scratch as its workspace
    ascq_matmul_s tmp = *h;
    tmp.ws = ptr;
    tmp.ws_bytes = need > 0 ? (size_t)ASCQ_NOALLOC_SCRATCH_BYTES : 0;
    tmp.ws_owned = false;
    return ascq_matmul_iterate_all(&tmp, c, en_atomic, stream);
}

ascq_status ascq_matmul_end(ascq_matmul_t h)
{
    if (!h) return fail(ASCQ_E_INVALID_ARG, "null handle");
    h->a = h->b = h->bias = nullptr;
    h->quant_set = h->aq_set = false;
    h->qvec = nullptr;
    h->scale_a = h->scale_b = nullptr;
    h->sm = h->sn = h->sk = -1;
    return ASCQ_OK;
}

ascq_status ascq_matmul_destroy(ascq_matmul_t h)
{
    if (!h) return ASCQ_OK;
    if (h->ws_owned && h->ws) (void)hipFree(h->ws);
    delete h;
    return ASCQ_OK;
}

// ------------------------------------------------------------------------------------------------
// AscendQuant / AscendDequant / AscendAntiQuant
// ------------------------------------------------------------------------------------------------
ascq_status ascq_ascend_quant_per_token(int8_t* dst, const void* src, int32_t src_type, const float* scale,
                                        const float* offset, const ascq_quant_param* para, void* stream)
{
    CallScope scope;
    if (!dst || !src || !scale || !para) return fail(ASCQ_E_INVALID_ARG, "quant_per_token: null argument");
    if (src_type != ASCQ_DT_F16 && src_type != ASCQ_DT_BF16 && src_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "quant_per_token: src must be f16, bf16 or f32");
    if (para->n == 0) return fail(ASCQ_E_INVALID_ARG, "quant_per_token: n must be positive");
    if (para->cal_count % para->n != 0)
        return fail(ASCQ_E_INVALID_ARG, "quant_per_token: calCount must be an integer multiple of n");
    if (!valid_round(para->round_mode)) return fail(ASCQ_E_INVALID_ARG, "quant_per_token: bad round mode");
    if (para->has_offset && !offset) return fail(ASCQ_E_INVALID_ARG, "quant_per_token: has_offset needs an offset tensor");
    const uint32_t m = para->cal_count / para->n;
    if (m == 0) return ASCQ_OK;
    // the PER_TOKEN policy form with an f32 scale computes exactly this (f32 product and offset, round mode,
    // saturation), through the vectorised policy kernels
    return hip_status(ascq::launch_quant_policy(dst, ASCQ_DT_INT8, src, src_type, scale, ASCQ_DT_F32, offset,
                                                para->has_offset ? 1 : 0, 0.0f, 1, m, para->n, 0, 1, para->round_mode,
                                                S(stream)),
                      "quant_per_token");
}

ascq_status ascq_ascend_quant_policy(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                     const void* scale, const void* offset, float offset_scalar, int32_t scale_type,
                                     int32_t policy, const ascq_quant_param* para, void* stream)
{
    CallScope scope;
    if (!para) return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: null argument");
    const auto fp_type = [](int32_t t) { return t == ASCQ_DT_F16 || t == ASCQ_DT_BF16 || t == ASCQ_DT_F32; };
    if (!fp_type(src_type)) return fail(ASCQ_E_UNSUPPORTED, "ascend_quant_policy: src must be f16, bf16 or f32");
    if (!fp_type(scale_type)) return fail(ASCQ_E_UNSUPPORTED, "ascend_quant_policy: scale must be f16, bf16 or f32");
    const bool fp8 = dst_type == ASCQ_DT_FP8_E4M3 || dst_type == ASCQ_DT_FP8_E5M2;
    const bool fp4 = dst_type == ASCQ_DT_FP4_E2M1 || dst_type == ASCQ_DT_FP4_E1M2;
    if (!fp8 && !fp4 && dst_type != ASCQ_DT_INT8 && dst_type != ASCQ_DT_HIF8)
        return fail(ASCQ_E_UNSUPPORTED,
                    "ascend_quant_policy: dst must be int8, hifloat8, fp8_e4m3, fp8_e5m2, fp4_e2m1 or fp4_e1m2");
    if (policy != ASCQ_POLICY_PER_TOKEN && policy != ASCQ_POLICY_PER_GROUP)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_quant_policy: policy must be PER_TOKEN or PER_GROUP");
    if (policy == ASCQ_POLICY_PER_TOKEN && fp4)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_quant_policy: PER_TOKEN writes int8, hifloat8 or fp8");
    if (policy == ASCQ_POLICY_PER_GROUP) {
        if (para->kdim != 0 && para->kdim != 1) return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: kdim must be 0 or 1");
        if (para->group_size == 0 || para->group_size % 32 != 0)
            return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: group_size must be a positive multiple of 32");
    }
    if (!fp8 && scale_type != ASCQ_DT_F32 && scale_type != src_type)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_quant_policy: a 16-bit scale needs a source of the same type");
    if (!valid_round(para->round_mode)) return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: bad round mode");
    if (para->n == 0) return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: n must be positive");
    if (para->cal_count % para->n != 0)
        return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: calCount must be an integer multiple of n");
    if (fp4 && para->n % 2 != 0) return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: fp4 rows pack two per byte (n even)");
    const int64_t rows = para->cal_count / para->n;
    if (rows == 0) return ASCQ_OK;  // calCount = 0: nothing to do (empty tensors may carry null pointers)
    if (!dst || !src || !scale) return fail(ASCQ_E_INVALID_ARG, "ascend_quant_policy: null argument");
    return hip_status(ascq::launch_quant_policy(dst, dst_type, src, src_type, scale, scale_type, offset,
                                                para->has_offset ? 1 : 0, offset_scalar,
                                                policy == ASCQ_POLICY_PER_TOKEN ? 1 : 0, rows, para->n,
                                                para->group_size, para->kdim, para->round_mode, S(stream)),
                      "ascend_quant_policy");
}

ascq_status ascq_ascend_quant_dynamic_per_token(int8_t* dst, float* scale_out, const void* src, int32_t src_type,
                                                uint32_t m, uint32_t n, int32_t round_mode, void* stream)
{
    CallScope scope;
    if (!dst || !scale_out || !src) return fail(ASCQ_E_INVALID_ARG, "quant_dynamic_per_token: null argument");
    if (src_type != ASCQ_DT_F16 && src_type != ASCQ_DT_BF16 && src_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "quant_dynamic_per_token: src must be f16, bf16 or f32");
    if (!valid_round(round_mode)) return fail(ASCQ_E_INVALID_ARG, "quant_dynamic_per_token: bad round mode");
    if (m == 0 || n == 0) return ASCQ_OK;
    return hip_status(ascq::launch_quant_dynamic_per_token(dst, scale_out, src, src_type, m, n, round_mode, S(stream)),
                      "quant_dynamic_per_token");
}

ascq_status ascq_ascend_quant(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                              const void* offset, float scale_scalar, float offset_scalar, uint32_t cal_count,
                              uint32_t scale_count, void* stream)
{
    CallScope scope;
    if (src_type != ASCQ_DT_F16 && src_type != ASCQ_DT_BF16 && src_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_quant: src must be f16, bf16 or f32");
    if (dst_type != ASCQ_DT_INT8 && dst_type != ASCQ_DT_HIF8 && dst_type != ASCQ_DT_FP8_E4M3 &&
        dst_type != ASCQ_DT_FP8_E5M2)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_quant: dst must be int8, hifloat8, fp8_e4m3 or fp8_e5m2");
    if (offset && !scale)
        return fail(ASCQ_E_INVALID_ARG, "ascend_quant: an offset tensor needs a scale tensor (per-channel form)");
    if (scale) {  // the per-channel checks of ascend_quant_3510_impl.h:551-557
        if (scale_count == 0) return fail(ASCQ_E_INVALID_ARG, "ascend_quant: scaleCount must be positive");
        if (cal_count % scale_count != 0 || cal_count % 32 != 0)
            return fail(ASCQ_E_INVALID_ARG, "ascend_quant: calCount must be an integer multiple of 32 and scaleCount");
    }
    if (cal_count == 0) return ASCQ_OK;
    if (!dst || !src) return fail(ASCQ_E_INVALID_ARG, "ascend_quant: null argument");
    return hip_status(ascq::launch_quant_legacy(dst, dst_type, src, src_type, scale, offset, scale_scalar,
                                                offset_scalar, cal_count, scale ? scale_count : 0u, S(stream)),
                      "ascend_quant");
}

// quant.hip's scale addressing codes (DQ_*)
enum { DQ_SCALAR = 0, DQ_COL = 1, DQ_ROW = 2, DQ_GROUP_COL = 3, DQ_GROUP_ROW = 4 };

ascq_status ascq_ascend_dequant_dst_shape(int32_t dst_type, int32_t mode, const ascq_dequant_param* params,
                                          uint32_t* rows, uint32_t* row_stride)
{
    if (!params || !rows || !row_stride) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_dst_shape: null argument");
    if (dst_type != ASCQ_DT_F16 && dst_type != ASCQ_DT_BF16 && dst_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant_dst_shape: dst must be f16, bf16 or f32");
    if (mode != ASCQ_DEQUANT_SINGLE_ROW && mode != ASCQ_DEQUANT_MULTI_ROW)
        return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_dst_shape: bad DeQuantMode %d", mode);
    uint32_t m = params->m, n = params->n;
    const uint32_t blk = dst_type == ASCQ_DT_F32 ? 8u : 16u, cal = params->cal_count;  // dst elements per 32 bytes
    // UpdateDequantParams (ascend_dequant_common_impl.h:208-223)
    if (mode == ASCQ_DEQUANT_SINGLE_ROW && m == 1 && cal > 0 && cal % blk == 0 && n % cal == 0) {
        m = n / cal;
        n = cal;
    }
    *rows = m;
    *row_stride = (n + blk - 1) / blk * blk;  // dstInner
    return ASCQ_OK;
}

ascq_status ascq_ascend_dequant(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                                int32_t scale_type, float scale_scalar, int32_t policy, int32_t mode,
                                const ascq_dequant_param* params, void* stream)
{
    CallScope scope;
    if (!params) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant: null params");
    if (dst_type != ASCQ_DT_F16 && dst_type != ASCQ_DT_BF16 && dst_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant: dst must be f16, bf16 or f32");
    if (src_type != ASCQ_DT_INT32 && src_type != ASCQ_DT_INT8)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant: src must be int32 (or int8)");
    if (policy != ASCQ_POLICY_PER_TENSOR && policy != ASCQ_POLICY_PER_CHANNEL)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant: the legacy form takes a deqScale tensor (PER_CHANNEL) or a "
                                        "scalar (PER_TENSOR); PER_TOKEN / PER_GROUP are ascq_ascend_dequant_policy");
    if (mode != ASCQ_DEQUANT_SINGLE_ROW && mode != ASCQ_DEQUANT_MULTI_ROW)
        return fail(ASCQ_E_INVALID_ARG, "ascend_dequant: bad DeQuantMode %d", mode);
    // IsTemplateValid (ascend_dequant_common_impl.h:126-155)
    const bool tensor = policy == ASCQ_POLICY_PER_CHANNEL;
    const int32_t s = scale_type, d = dst_type;
    const bool ok = tensor ? ((s == ASCQ_DT_U64 && d == ASCQ_DT_F16) || (s == ASCQ_DT_F32 && d == ASCQ_DT_F32) ||
                              (s == ASCQ_DT_BF16 && d == ASCQ_DT_F32) || (s == ASCQ_DT_BF16 && d == ASCQ_DT_BF16) ||
                              (s == ASCQ_DT_F32 && d == ASCQ_DT_BF16))
                           : ((s == ASCQ_DT_BF16 || s == ASCQ_DT_F32) && (d == ASCQ_DT_BF16 || d == ASCQ_DT_F32));
    if (!ok)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant: deqScale type %d with dst type %d is not a combination the "
                                        "reference accepts", s, d);
    // the reference's CPU-debug checks (dequant_check_common.h)
    if (params->n % 8 != 0) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant: params.n must be divisible by 8");
    if (params->cal_count == 0 || params->cal_count > params->n)
        return fail(ASCQ_E_INVALID_ARG, "ascend_dequant: params.calCount must be in (0, n]");
    if (params->m == 0) return ASCQ_OK;
    if (!dst || !src || (tensor && !scale)) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant: null argument");
    uint32_t rows = 0, ldd = 0;
    ascq_status st = ascq_ascend_dequant_dst_shape(dst_type, mode, params, &rows, &ldd);
    if (st != ASCQ_OK) return st;
    const uint32_t n = rows == params->m ? params->n : params->cal_count;
    if ((uint64_t)rows * ldd >= (1ull << 40)) return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant: tensor too large");
    float ss = scale_scalar;
    if (!tensor && scale_type == ASCQ_DT_BF16) {  // the scalar is a bfloat16_t value
        uint32_t u;
        std::memcpy(&u, &ss, 4);
        if ((u & 0x7fffffffu) <= 0x7f800000u) u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
        std::memcpy(&ss, &u, 4);
    }
    return hip_status(ascq::launch_dequant(dst, dst_type, src, src_type, scale, scale_type, ss,
                                           tensor ? DQ_COL : DQ_SCALAR, rows, params->cal_count, n, ldd, 0,
                                           S(stream)),
                      "ascend_dequant");
}

ascq_status ascq_ascend_dequant_policy(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                       const void* scale, const void* offset, int32_t scale_type, int32_t policy,
                                       const ascq_dequant_policy_param* para, void* stream)
{
    CallScope scope;
    (void)offset;  // never read by the reference's policy kernels (ascend_dequant_3510_impl.h:254-598)
    if (!para) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_policy: null argument");
    if (dst_type != ASCQ_DT_F16 && dst_type != ASCQ_DT_BF16 && dst_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant_policy: dst must be f16, bf16 or f32");
    if (src_type != ASCQ_DT_INT32 && src_type != ASCQ_DT_F32 && src_type != ASCQ_DT_INT8)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant_policy: src must be int32 or f32 (or int8)");
    if (scale_type != ASCQ_DT_F16 && scale_type != ASCQ_DT_BF16 && scale_type != ASCQ_DT_F32)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant_policy: scale must be f16, bf16 or f32");
    if (policy != ASCQ_POLICY_PER_TOKEN && policy != ASCQ_POLICY_PER_GROUP)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_dequant_policy: policy must be PER_TOKEN or PER_GROUP");
    if (policy == ASCQ_POLICY_PER_GROUP) {
        if (para->kdim != 0 && para->kdim != 1) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_policy: kdim must be 0 or 1");
        if (para->group_size == 0 || para->group_size % 32 != 0)
            return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_policy: group_size must be a positive multiple of 32");
    }
    if (para->n == 0) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_policy: n must be positive");
    const uint32_t rows = para->cal_count / para->n;
    if (rows == 0) return ASCQ_OK;  // calCount < n: nothing to do (empty tensors may carry null pointers)
    if (!dst || !src || !scale) return fail(ASCQ_E_INVALID_ARG, "ascend_dequant_policy: null argument");
    int smode = DQ_ROW;
    uint32_t group = 0;
    if (policy == ASCQ_POLICY_PER_GROUP) {
        smode = para->kdim == 1 ? DQ_GROUP_COL : DQ_GROUP_ROW;
        group = para->group_size;
    }
    return hip_status(ascq::launch_dequant(dst, dst_type, src, src_type, scale, scale_type, 0.0f, smode, rows, para->n,
                                           para->n, para->n, group, S(stream)),
                      "ascend_dequant_policy");
}

ascq_status ascq_ascend_antiquant(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* offset,
                                  const void* scale, uint32_t k, uint32_t n, uint32_t group_size, int32_t is_transpose,
                                  int32_t arith, void* stream)
{
    CallScope scope;
    if (!dst || !src || !scale) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant: null argument");
    if (dst_type != ASCQ_DT_F16 && dst_type != ASCQ_DT_BF16)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant: dst must be f16 or bf16");
    const bool b8 = src_type == ASCQ_DT_HIF8 || src_type == ASCQ_DT_FP8_E4M3 || src_type == ASCQ_DT_FP8_E5M2;
    if (src_type != ASCQ_DT_INT8 && src_type != ASCQ_DT_INT4 && !b8)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant: src must be int8, int4, hifloat8, fp8_e4m3 or fp8_e5m2");
    if (b8 && group_size != 0)  // AntiQuantPerchannelImpl (ascend_antiquant_3510_impl.h:752-770): per channel only
        return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant: hifloat8 / fp8 sources are per channel (group_size 0)");
    if (arith != ASCQ_ARITH_F16 && arith != ASCQ_ARITH_F32) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant: bad arith");
    if (group_size && k % group_size != 0) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant: group_size must divide K");
    if (src_type == ASCQ_DT_INT4 && ((uint64_t)k * n) % 2 != 0)
        return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant: int4 needs an even element count");
    if (k == 0 || n == 0) return ASCQ_OK;
    const uint32_t g = group_size ? group_size : k;
    return hip_status(ascq::launch_antiquant(dst, dst_type, src, src_type, offset, scale, k, n, g, is_transpose ? 1 : 0,
                                             dst_type == ASCQ_DT_BF16 ? 1 : arith, S(stream)),
                      "ascend_antiquant");
}

ascq_status ascq_ascend_antiquant_scalar(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                         uint16_t offset, uint16_t scale, int32_t has_offset, uint64_t count,
                                         void* stream)
{
    CallScope scope;
    if (dst_type != ASCQ_DT_F16 && dst_type != ASCQ_DT_BF16)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_scalar: dst must be f16 or bf16");
    if (src_type != ASCQ_DT_INT8 && src_type != ASCQ_DT_INT4 && src_type != ASCQ_DT_HIF8 &&
        src_type != ASCQ_DT_FP8_E4M3 && src_type != ASCQ_DT_FP8_E5M2)
        return fail(ASCQ_E_UNSUPPORTED,
                    "ascend_antiquant_scalar: src must be int8, int4, hifloat8, fp8_e4m3 or fp8_e5m2");
    if (src_type == ASCQ_DT_INT4 && count % 2 != 0)
        return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_scalar: int4 needs an even element count");
    if (count >= (1ull << 40)) return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_scalar: tensor too large");
    if (count == 0) return ASCQ_OK;
    if (!dst || !src) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_scalar: null argument");
    return hip_status(ascq::launch_antiquant_scalar(dst, dst_type, src, src_type, offset, scale, has_offset ? 1 : 0,
                                                    (int64_t)count, S(stream)),
                      "ascend_antiquant_scalar");
}

ascq_status ascq_ascend_antiquant_policy(void* dst, int32_t dst_type, const void* src, int32_t src_type,
                                         const void* scale, const void* offset, int32_t scale_type, int32_t policy,
                                         int64_t m, int64_t n, int64_t group_size, int32_t k_dim, int32_t is_transpose,
                                         void* stream)
{
    CallScope scope;
    if (m < 0 || n < 0) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_policy: negative shape");
    if (policy != ASCQ_POLICY_PER_TOKEN && policy != ASCQ_POLICY_PER_GROUP)
        return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_policy: policy must be PER_TOKEN or PER_GROUP");
    if (k_dim != 0 && k_dim != 1) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_policy: k_dim must be 0 or 1");
    if (policy == ASCQ_POLICY_PER_GROUP && (group_size <= 0 || group_size % 32 != 0))
        return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_policy: group_size must be a positive multiple of 32");
    const bool fp8 = src_type == ASCQ_DT_FP8_E4M3 || src_type == ASCQ_DT_FP8_E5M2;
    const bool out_ok = dst_type == ASCQ_DT_F16 || dst_type == ASCQ_DT_BF16 || dst_type == ASCQ_DT_F32;
    if (src_type == ASCQ_DT_FP4_E2M1 || src_type == ASCQ_DT_FP4_E1M2) {
        if (policy != ASCQ_POLICY_PER_GROUP || scale_type != ASCQ_DT_E8M0 || offset)
            return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_policy: fp4 takes PER_GROUP E8M0 scales and no offset");
        if (dst_type != ASCQ_DT_F16 && dst_type != ASCQ_DT_BF16)
            return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_policy: fp4 output must be f16 or bf16");
        if (n % 2 != 0) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_policy: fp4 rows pack two per byte (n even)");
    } else if (src_type == ASCQ_DT_INT8 || src_type == ASCQ_DT_HIF8 || fp8) {
        if (scale_type != ASCQ_DT_F16 && scale_type != ASCQ_DT_BF16 && scale_type != ASCQ_DT_F32)
            return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_policy: scale must be f16, bf16 or f32");
        if (!out_ok) return fail(ASCQ_E_UNSUPPORTED, "ascend_antiquant_policy: dst must be f16, bf16 or f32");
        if (!fp8 && scale_type != ASCQ_DT_F32 && dst_type != scale_type)
            return fail(ASCQ_E_UNSUPPORTED,
                        "ascend_antiquant_policy: int8 / hifloat8 with a 16-bit scale writes the scale type");
    } else {
        return fail(ASCQ_E_UNSUPPORTED,
                    "ascend_antiquant_policy: src must be int8, hifloat8, fp8_e4m3, fp8_e5m2, fp4_e2m1 or fp4_e1m2");
    }
    if (m == 0 || n == 0) return ASCQ_OK;  // empty tensors may carry null pointers
    if (!dst || !src || !scale) return fail(ASCQ_E_INVALID_ARG, "ascend_antiquant_policy: null argument");
    const int col_groups = (k_dim == 1 && !is_transpose) || (k_dim == 0 && is_transpose);
    return hip_status(ascq::launch_antiquant_policy(dst, dst_type, src, src_type, scale, offset, scale_type,
                                                    policy == ASCQ_POLICY_PER_TOKEN ? 1 : 0, m, n, group_size, col_groups,
                                                    is_transpose ? 1 : 0, S(stream)),
                      "ascend_antiquant_policy");
}

// ------------------------------------------------------------------------------------------------
// Quantize / Dequantize / AntiQuantize (quantize.h, dequantize.h, antiquantize.h): the AscendQuant / AscendDequant /
// AscendAntiQuant kernels with fp32 arithmetic (Quantize, AntiQuantize) and the newer interface's type rules
// ------------------------------------------------------------------------------------------------
namespace {

bool valid_policy(int32_t p) { return p >= ASCQ_POLICY_PER_TENSOR && p <= ASCQ_POLICY_PER_GROUP; }

// bits of v rounded (rne) to the 16-bit float type t (F16 / BF16)
uint16_t half_bits_of(float v, int32_t t)
{
    if (t == ASCQ_DT_F16) {
        const _Float16 h = (_Float16)v;
        uint16_t b;
        std::memcpy(&b, &h, 2);
        return b;
    }
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays NaN
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// one group covering every row: scale[r / g][c] is then scale[c] (PER_CHANNEL through the per-group kernels, whose
// row blocks need a group size that is a multiple of 32)
int64_t whole_column_group(uint32_t m) { return ((int64_t)(m > 0 ? m : 1) + 31) / 32 * 32; }

}  // namespace

ascq_status ascq_quantize(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                          const void* offset, float scale_scalar, float offset_scalar, int32_t scale_type,
                          const ascq_quantize_param* p, void* stream)
{
    CallScope scope;
    if (!p) return fail(ASCQ_E_INVALID_ARG, "quantize: null params");
    if (!valid_policy(p->policy)) return fail(ASCQ_E_INVALID_ARG, "quantize: bad policy %d", p->policy);
    const auto fp_type = [](int32_t t) { return t == ASCQ_DT_F16 || t == ASCQ_DT_BF16 || t == ASCQ_DT_F32; };
    if (!fp_type(src_type)) return fail(ASCQ_E_UNSUPPORTED, "quantize: src must be f16, bf16 or f32");
    // CheckApiDtypeValid (quantize_impl.h:33-61): (src, scale) = (f16, f16), (bf16, bf16), (f32, f32), (f16, f32),
    // (bf16, f32)
    if (!fp_type(scale_type) || (scale_type != ASCQ_DT_F32 && scale_type != src_type))
        return fail(ASCQ_E_UNSUPPORTED, "quantize: the scale is f32 or of the source's type");
    const bool fp4 = dst_type == ASCQ_DT_FP4_E2M1 || dst_type == ASCQ_DT_FP4_E1M2;
    if (dst_type != ASCQ_DT_INT8 && dst_type != ASCQ_DT_HIF8 && dst_type != ASCQ_DT_FP8_E4M3 &&
        dst_type != ASCQ_DT_FP8_E5M2 && !fp4)
        return fail(ASCQ_E_UNSUPPORTED, "quantize: dst must be int8, hifloat8, fp8_e4m3, fp8_e5m2, fp4_e2m1 or fp4_e1m2");
    if (fp4 && p->policy != ASCQ_POLICY_PER_GROUP)
        return fail(ASCQ_E_UNSUPPORTED, "quantize: fp4 outputs are PER_GROUP only (quantize_impl.h:1021-1053)");
    if (p->policy == ASCQ_POLICY_PER_GROUP) {
        if (p->kdim != 0 && p->kdim != 1) return fail(ASCQ_E_INVALID_ARG, "quantize: kdim must be 0 or 1");
        if (p->group_size == 0 || p->group_size % 32 != 0)
            return fail(ASCQ_E_INVALID_ARG, "quantize: group_size must be a positive multiple of 32");
    }
    if (p->policy == ASCQ_POLICY_PER_TENSOR && (scale || offset))
        return fail(ASCQ_E_INVALID_ARG, "quantize: PER_TENSOR takes scalar scale and offset (pass NULL tensors)");
    if (!valid_round(p->round_mode)) return fail(ASCQ_E_INVALID_ARG, "quantize: bad round mode");
    if (p->n % 32 != 0) return fail(ASCQ_E_INVALID_ARG, "quantize: params.n must be a multiple of 32");
    if (p->m == 0 || p->n == 0) return ASCQ_OK;
    if (!dst || !src || (p->policy != ASCQ_POLICY_PER_TENSOR && !scale))
        return fail(ASCQ_E_INVALID_ARG, "quantize: null argument");
    const bool scalar_layout = p->policy == ASCQ_POLICY_PER_TENSOR || p->policy == ASCQ_POLICY_PER_TOKEN;
    const bool channel = p->policy == ASCQ_POLICY_PER_CHANNEL;
    trace("quantize: policy %d, dst %d src %d scale %d, m %u n %u group %u kdim %d offset %d", p->policy, dst_type,
          src_type, scale_type, p->m, p->n, p->group_size, p->kdim, p->has_offset);
    return hip_status(ascq::launch_quant_policy(dst, dst_type, src, src_type, scale, scale_type, offset,
                                                p->has_offset ? 1 : 0, offset_scalar, scalar_layout ? 1 : 0, p->m,
                                                p->n, channel ? whole_column_group(p->m) : (int64_t)p->group_size,
                                                channel ? 0 : p->kdim, p->round_mode, S(stream), scale_scalar, 1),
                      "quantize");
}

ascq_status ascq_dequantize(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                            float scale_scalar, int32_t scale_type, const ascq_quantize_param* p, void* stream)
{
    CallScope scope;
    if (!p) return fail(ASCQ_E_INVALID_ARG, "dequantize: null params");
    if (!valid_policy(p->policy)) return fail(ASCQ_E_INVALID_ARG, "dequantize: bad policy %d", p->policy);
    if (p->has_offset) return fail(ASCQ_E_UNSUPPORTED, "dequantize: offset is not supported (dequantize_impl.h:102)");
    const int32_t s = scale_type, d = dst_type;
    const bool legacy = p->policy == ASCQ_POLICY_PER_TENSOR || p->policy == ASCQ_POLICY_PER_CHANNEL;
    // IsDataTypeValid (dequantize_impl.h:67-92)
    bool ok;
    if (p->policy == ASCQ_POLICY_PER_CHANNEL)
        ok = (s == ASCQ_DT_U64 && d == ASCQ_DT_F16) || (s == ASCQ_DT_F32 && d == ASCQ_DT_F32) ||
             (s == ASCQ_DT_BF16 && d == ASCQ_DT_F32) || (s == ASCQ_DT_BF16 && d == ASCQ_DT_BF16) ||
             (s == ASCQ_DT_F32 && d == ASCQ_DT_BF16);
    else if (p->policy == ASCQ_POLICY_PER_TENSOR)
        ok = (s == ASCQ_DT_BF16 || s == ASCQ_DT_F32) && (d == ASCQ_DT_BF16 || d == ASCQ_DT_F32);
    else
        ok = (s == ASCQ_DT_F16 && d == ASCQ_DT_F16) || (s == ASCQ_DT_BF16 && d == ASCQ_DT_BF16) ||
             (s == ASCQ_DT_F32 && (d == ASCQ_DT_F32 || d == ASCQ_DT_F16 || d == ASCQ_DT_BF16));
    if (!ok) return fail(ASCQ_E_UNSUPPORTED, "dequantize: scale type %d with dst type %d is not accepted", s, d);
    if (src_type != ASCQ_DT_INT32 && (legacy || src_type != ASCQ_DT_F32))
        return fail(ASCQ_E_UNSUPPORTED, "dequantize: src must be int32 (PER_TOKEN / PER_GROUP: int32 or f32)");
    const uint32_t dsz = d == ASCQ_DT_F32 ? 4 : 2;
    if ((p->n * 4u) % 32 != 0 || (p->n * dsz) % 32 != 0)
        return fail(ASCQ_E_INVALID_ARG, "dequantize: rows of src and dst must be whole 32-byte blocks");
    if (p->m == 0 || p->n == 0) return ASCQ_OK;
    if (p->policy == ASCQ_POLICY_PER_GROUP) {
        if (p->kdim != 0 && p->kdim != 1) return fail(ASCQ_E_INVALID_ARG, "dequantize: kdim must be 0 or 1");
        if (p->group_size == 0 || p->group_size % 32 != 0)
            return fail(ASCQ_E_INVALID_ARG, "dequantize: group_size must be a positive multiple of 32");
    }
    if ((uint64_t)p->m * p->n >= (1ull << 32)) return fail(ASCQ_E_UNSUPPORTED, "dequantize: tensor too large");
    if (legacy) {
        const ascq_dequant_param dp{p->m, p->n, p->n};
        return ascq_ascend_dequant(dst, dst_type, src, src_type, scale, scale_type, scale_scalar, p->policy,
                                   ASCQ_DEQUANT_MULTI_ROW, &dp, stream);
    }
    const ascq_dequant_policy_param pp{p->m, p->n, p->m * p->n, p->group_size, 0, p->kdim};
    return ascq_ascend_dequant_policy(dst, dst_type, src, src_type, scale, nullptr, scale_type, p->policy, &pp, stream);
}

ascq_status ascq_antiquantize(void* dst, int32_t dst_type, const void* src, int32_t src_type, const void* scale,
                              const void* offset, float scale_scalar, float offset_scalar, int32_t scale_type,
                              const ascq_quantize_param* p, void* stream)
{
    CallScope scope;
    if (!p) return fail(ASCQ_E_INVALID_ARG, "antiquantize: null params");
    if (!valid_policy(p->policy)) return fail(ASCQ_E_INVALID_ARG, "antiquantize: bad policy %d", p->policy);
    const bool b8 = src_type == ASCQ_DT_INT8 || src_type == ASCQ_DT_HIF8 || src_type == ASCQ_DT_FP8_E4M3 ||
                    src_type == ASCQ_DT_FP8_E5M2;
    const bool fp4 = src_type == ASCQ_DT_FP4_E2M1 || src_type == ASCQ_DT_FP4_E1M2;
    const int32_t s = scale_type, d = dst_type;
    if (p->policy == ASCQ_POLICY_PER_TENSOR || p->policy == ASCQ_POLICY_PER_CHANNEL) {
        if (!b8) return fail(ASCQ_E_UNSUPPORTED, "antiquantize: src must be int8, hifloat8, fp8_e4m3 or fp8_e5m2");
        if (!((s == ASCQ_DT_F16 && d == ASCQ_DT_F16) || (s == ASCQ_DT_BF16 && d == ASCQ_DT_BF16)))
            return fail(ASCQ_E_UNSUPPORTED, "antiquantize: PER_TENSOR / PER_CHANNEL take f16 or bf16 scales of the dst type");
    } else if (fp4) {
        if (p->policy != ASCQ_POLICY_PER_GROUP || s != ASCQ_DT_E8M0 || (d != ASCQ_DT_F16 && d != ASCQ_DT_BF16))
            return fail(ASCQ_E_UNSUPPORTED, "antiquantize: fp4 takes PER_GROUP E8M0 scales and f16 / bf16 dst");
        if (p->has_offset) return fail(ASCQ_E_UNSUPPORTED, "antiquantize: fp4 takes no offset (antiquantize_impl.h:191)");
        if (p->n % 64 != 0) return fail(ASCQ_E_INVALID_ARG, "antiquantize: fp4 rows must be a multiple of 64");
    } else {
        if (!b8) return fail(ASCQ_E_UNSUPPORTED, "antiquantize: src must be int8, hifloat8, fp8 or fp4");
        const bool ok = (s == ASCQ_DT_F16 && d == ASCQ_DT_F16) || (s == ASCQ_DT_BF16 && d == ASCQ_DT_BF16) ||
                        (s == ASCQ_DT_F32 && (d == ASCQ_DT_F32 || d == ASCQ_DT_F16 || d == ASCQ_DT_BF16));
        if (!ok) return fail(ASCQ_E_UNSUPPORTED, "antiquantize: scale type %d with dst type %d is not accepted", s, d);
    }
    if (p->policy == ASCQ_POLICY_PER_GROUP) {
        if (p->kdim != 0 && p->kdim != 1) return fail(ASCQ_E_INVALID_ARG, "antiquantize: kdim must be 0 or 1");
        if (p->group_size == 0 || p->group_size % 32 != 0)
            return fail(ASCQ_E_INVALID_ARG, "antiquantize: group_size must be a positive multiple of 32");
    }
    if (b8 && p->n % 32 != 0) return fail(ASCQ_E_INVALID_ARG, "antiquantize: rows must be whole 32-byte blocks");
    if (p->policy == ASCQ_POLICY_PER_TENSOR && (scale || offset))
        return fail(ASCQ_E_INVALID_ARG, "antiquantize: PER_TENSOR takes scalar scale and offset (pass NULL tensors)");
    if (p->policy != ASCQ_POLICY_PER_TENSOR && p->has_offset && !offset)
        return fail(ASCQ_E_INVALID_ARG, "antiquantize: has_offset needs an offset tensor");
    if (p->m == 0 || p->n == 0) return ASCQ_OK;
    if (!dst || !src || (p->policy != ASCQ_POLICY_PER_TENSOR && !scale))
        return fail(ASCQ_E_INVALID_ARG, "antiquantize: null argument");
    trace("antiquantize: policy %d, dst %d src %d scale %d, m %u n %u group %u kdim %d offset %d", p->policy, d,
          src_type, s, p->m, p->n, p->group_size, p->kdim, p->has_offset);
    if (p->policy == ASCQ_POLICY_PER_TENSOR)
        return hip_status(ascq::launch_antiquant_scalar(dst, d, src, src_type, half_bits_of(offset_scalar, s),
                                                        half_bits_of(scale_scalar, s), p->has_offset ? 1 : 0,
                                                        (int64_t)p->m * p->n, S(stream), 1),
                          "antiquantize");
    const bool channel = p->policy == ASCQ_POLICY_PER_CHANNEL;
    const int col_groups = p->policy == ASCQ_POLICY_PER_GROUP && p->kdim == 1;
    return hip_status(ascq::launch_antiquant_policy(dst, d, src, src_type, scale, p->has_offset ? offset : nullptr, s,
                                                    p->policy == ASCQ_POLICY_PER_TOKEN ? 1 : 0, p->m, p->n,
                                                    channel ? whole_column_group(p->m) : (int64_t)p->group_size,
                                                    col_groups, 0, S(stream), 1),
                      "antiquantize");
}

// ------------------------------------------------------------------------------------------------
// weight-only antiquant matmul
// ------------------------------------------------------------------------------------------------
ascq_status ascq_weight_pack_size(int32_t w_type, int64_t k, int64_t n, size_t* bytes)
{
    if (!bytes) return fail(ASCQ_E_INVALID_ARG, "weight_pack_size: null argument");
    if (w_type != ASCQ_DT_INT8 && w_type != ASCQ_DT_INT4) return fail(ASCQ_E_UNSUPPORTED, "weight_pack_size: int8 or int4");
    if (k <= 0 || n <= 0 || k % 128 != 0 || n % 16 != 0)
        return fail(ASCQ_E_INVALID_ARG, "weight_pack_size: K %% 128 == 0 and N %% 16 == 0 required");
    *bytes = ascq::weight_pack_bytes(w_type, k, n);
    return ASCQ_OK;
}

ascq_status ascq_weight_pack(void* packed, const void* w, int32_t w_type, int64_t k, int64_t n, int32_t is_transpose,
                             void* stream)
{
    CallScope scope;
    size_t bytes = 0;
    ascq_status s = ascq_weight_pack_size(w_type, k, n, &bytes);
    if (s != ASCQ_OK) return s;
    if (!packed || !w) return fail(ASCQ_E_INVALID_ARG, "weight_pack: null argument");
    if (!aligned(packed, 16)) return fail(ASCQ_E_INVALID_ARG, "weight_pack: output must be 16-byte aligned");
    return hip_status(ascq::launch_weight_pack(packed, w, w_type, k, n, is_transpose ? 1 : 0, S(stream)), "weight_pack");
}

ascq_status ascq_antiquant_matmul(uint16_t* y, const uint16_t* x, const void* w_packed, int32_t w_type,
                                  const uint16_t* scale, const uint16_t* offset, int64_t group_size, int64_t m,
                                  int64_t n, int64_t k, void* stream)
{
    CallScope scope;
    if (!y || !x || !w_packed || !scale) return fail(ASCQ_E_INVALID_ARG, "antiquant_matmul: null argument");
    if (w_type != ASCQ_DT_INT8 && w_type != ASCQ_DT_INT4) return fail(ASCQ_E_UNSUPPORTED, "antiquant_matmul: int8 or int4");
    if (m <= 0 || n <= 0 || k <= 0) return fail(ASCQ_E_INVALID_ARG, "antiquant_matmul: shape must be positive");
    if (k % 128 != 0 || n % 16 != 0)
        return fail(ASCQ_E_INVALID_ARG, "antiquant_matmul: K %% 128 == 0 and N %% 16 == 0 required");
    if (group_size < 0 || (group_size > 0 && (group_size % 32 != 0 || k % group_size != 0)))
        return fail(ASCQ_E_INVALID_ARG, "antiquant_matmul: group_size must be 0 or a multiple of 32 dividing K");
    if (!aligned(x, 16) || !aligned(w_packed, 16))
        return fail(ASCQ_E_INVALID_ARG, "antiquant_matmul: x and the packed weight must be 16-byte aligned");
    if (k * n >= (1ll << 31) || 64 * k * 2 >= (1ll << 31))
        return fail(ASCQ_E_UNSUPPORTED, "antiquant_matmul: the weight must stay below 2^31 elements");
    trace("antiquant_matmul: W %d, M %lld N %lld K %lld, group %lld, offset %d", w_type, (long long)m, (long long)n,
          (long long)k, (long long)group_size, offset ? 1 : 0);
    return hip_status(ascq::launch_antiquant_matmul(y, x, w_packed, w_type, scale, offset, group_size, m, n, k,
                                                    ascq::C_STORE, S(stream)),
                      "antiquant_matmul");
}

// ------------------------------------------------------------------------------------------------
// quantized group matmul
// ------------------------------------------------------------------------------------------------
ascq_status ascq_quant_group_matmul(void* y, int32_t out_type, const int8_t* x, const float* per_token_scale,
                                    const int8_t* w, int32_t w_trans, const float* scale, const int64_t* group_list,
                                    int32_t list_type, int64_t num_groups, int64_t m, int64_t k, int64_t n,
                                    int32_t activation, void* stream)
{
    CallScope scope;
    if (!y || !x || !per_token_scale || !w || !scale || !group_list)
        return fail(ASCQ_E_INVALID_ARG, "quant_group_matmul: null argument");
    if (out_type != ASCQ_DT_BF16 && out_type != ASCQ_DT_F16)
        return fail(ASCQ_E_UNSUPPORTED, "quant_group_matmul: output must be bf16 or f16");
    if (list_type != 0 && list_type != 1) return fail(ASCQ_E_INVALID_ARG, "quant_group_matmul: list_type must be 0 or 1");
    if (activation != ASCQ_ACT_NONE && activation != ASCQ_ACT_FASTER_GELU)
        return fail(ASCQ_E_INVALID_ARG, "quant_group_matmul: unknown activation %d", activation);
    if (num_groups <= 0 || num_groups > 1024) return fail(ASCQ_E_INVALID_ARG, "quant_group_matmul: 1 <= groups <= 1024");
    if (m <= 0 || k <= 0 || n <= 0) return fail(ASCQ_E_INVALID_ARG, "quant_group_matmul: shape must be positive");
    ascq::GroupGemmArgs g{};
    g.Y = y;
    g.out_type = out_type;
    g.X = x;
    g.pts = per_token_scale;
    g.W = w;
    g.w_trans = w_trans ? 1 : 0;
    g.scale = scale;
    g.group_list = group_list;
    g.list_type = list_type;
    g.G = num_groups;
    g.M = m;
    g.K = k;
    g.N = n;
    g.act = activation;
    trace("quant_group_matmul: out %d, G %lld M %lld K %lld N %lld, w_trans %d, list_type %d, act %d", out_type,
          (long long)num_groups, (long long)m, (long long)k, (long long)n, g.w_trans, list_type, activation);
    return hip_status(ascq::launch_group_gemm(g, S(stream)), "quant_group_matmul");
}

// ------------------------------------------------------------------------------------------------
// NZ fractal <-> ND
// ------------------------------------------------------------------------------------------------
namespace {
int elem_bytes(int32_t dtype)
{
    switch (dtype) {
    case ASCQ_DT_INT8:
    case ASCQ_DT_UINT8:
    case ASCQ_DT_FP8_E4M3:
    case ASCQ_DT_FP8_E5M2: return 1;
    case ASCQ_DT_F16:
    case ASCQ_DT_BF16: return 2;
    case ASCQ_DT_INT32:
    case ASCQ_DT_F32: return 4;
    default: return 0;
    }
}

ascq_status check_nz_args(const char* what, const void* dst, const void* src, int32_t dtype, int64_t batch,
                          int64_t rows, int64_t cols)
{
    if (!dst || !src) return fail(ASCQ_E_INVALID_ARG, "%s: null argument", what);
    if (elem_bytes(dtype) == 0) return fail(ASCQ_E_UNSUPPORTED, "%s: unsupported element type %d", what, dtype);
    if (batch <= 0 || rows <= 0 || cols <= 0) return fail(ASCQ_E_INVALID_ARG, "%s: shape must be positive", what);
    if (ascq::nz_bytes(batch, rows, cols, elem_bytes(dtype)) >= ((size_t)1 << 40))
        return fail(ASCQ_E_UNSUPPORTED, "%s: matrix too large", what);
    return ASCQ_OK;
}
}  // namespace

size_t ascq_nz_size(int32_t dtype, int64_t batch, int64_t rows, int64_t cols)
{
    const int e = elem_bytes(dtype);
    if (e == 0 || batch <= 0 || rows <= 0 || cols <= 0) return 0;
    return ascq::nz_bytes(batch, rows, cols, e);
}

ascq_status ascq_nz_to_nd(void* dst, const void* src, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                          int32_t transpose_out, void* stream)
{
    CallScope scope;
    ascq_status s = check_nz_args("nz_to_nd", dst, src, dtype, batch, rows, cols);
    if (s != ASCQ_OK) return s;
    if (transpose_out && elem_bytes(dtype) != 1)
        return fail(ASCQ_E_UNSUPPORTED, "nz_to_nd: transpose_out needs a 1-byte element type");
    return hip_status(ascq::launch_nz_to_nd(dst, src, elem_bytes(dtype), batch, rows, cols, transpose_out ? 1 : 0,
                                            S(stream)),
                      "nz_to_nd");
}

ascq_status ascq_nd_to_nz(void* dst, const void* src, int32_t dtype, int64_t batch, int64_t rows, int64_t cols,
                          void* stream)
{
    CallScope scope;
    ascq_status s = check_nz_args("nd_to_nz", dst, src, dtype, batch, rows, cols);
    if (s != ASCQ_OK) return s;
    return hip_status(ascq::launch_nd_to_nz(dst, src, elem_bytes(dtype), batch, rows, cols, S(stream)), "nd_to_nz");
}

}  // extern "C"
