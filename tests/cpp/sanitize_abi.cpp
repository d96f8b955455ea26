// Host argument checks of the C ABI under AddressSanitizer + UndefinedBehaviorSanitizer: every call below is
// rejected (or answered) on the host before any device work, so no GPU is needed.  Exit status 0 = every
// expectation held and the sanitizers reported nothing.
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "ascq.h"

static int failures = 0;
#define EXPECT(call, want)                                                                                        \
    do {                                                                                                          \
        const ascq_status got_ = (call);                                                                          \
        if (got_ != (want)) {                                                                                     \
            std::printf("line %d: %s returned %d, expected %d (%s)\n", __LINE__, #call, got_, (want),             \
                        ascq_last_error());                                                                       \
            ++failures;                                                                                           \
        } else if ((want) != ASCQ_OK && std::strlen(ascq_last_error()) == 0) {                                    \
            std::printf("line %d: %s failed without a message\n", __LINE__, #call);                               \
            ++failures;                                                                                           \
        }                                                                                                         \
    } while (0)

int main()
{
    void* const d = reinterpret_cast<void*>(0x1000);  // never dereferenced: every call below fails its checks
    if (!ascq_version() || !*ascq_version()) ++failures;
    if (ascq_pack_quant_pre(1.0f, 3, 1) != (0x3F800000ull | (3ull << 37) | (1ull << 46))) ++failures;

    // Matmul handle state machine and type table
    ascq_matmul_t h = nullptr;
    ascq_matmul_types bad{ASCQ_DT_F16, ASCQ_DT_F16, ASCQ_DT_F16, 0, 0, 0};
    EXPECT(ascq_matmul_create(&bad, &h), ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_matmul_create(nullptr, &h), ASCQ_E_INVALID_ARG);
    ascq_matmul_types t{ASCQ_DT_INT8, ASCQ_DT_INT8, ASCQ_DT_F16, ASCQ_DT_INT32, 0, 0};
    EXPECT(ascq_matmul_create(&t, &h), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, 0, nullptr), ASCQ_E_STATE);
    EXPECT(ascq_matmul_set_tensor_a(h, d, 0), ASCQ_OK);
    EXPECT(ascq_matmul_set_tensor_b(h, d, 0), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, 0, nullptr), ASCQ_E_STATE);
    EXPECT(ascq_matmul_set_org_shape(h, 128, 256, 512), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, 0, nullptr), ASCQ_E_STATE);
    EXPECT(ascq_matmul_iterate_all(h, d, 4, nullptr), ASCQ_E_INVALID_ARG);
    EXPECT(ascq_matmul_set_antiquant_scalar(h, 0, 0), ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_matmul_set_tensor_scale_a(h, reinterpret_cast<const uint8_t*>(d), 0), ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_matmul_set_single_shape(h, 256, 256, 512), ASCQ_OK);
    EXPECT(ascq_matmul_set_quant_scalar(h, 0x3F800000u), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, 0, nullptr), ASCQ_E_INVALID_ARG);
    size_t ws = 0;
    EXPECT(ascq_matmul_workspace_size(h, &ws), ASCQ_OK);
    EXPECT(ascq_matmul_workspace_size(h, nullptr), ASCQ_E_INVALID_ARG);
    EXPECT(ascq_matmul_end(h), ASCQ_OK);
    EXPECT(ascq_matmul_destroy(h), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(nullptr, d, 0, nullptr), ASCQ_E_INVALID_ARG);
    ascq_matmul_types i8{ASCQ_DT_INT8, ASCQ_DT_INT8, ASCQ_DT_INT8, 0, 0, 0};
    EXPECT(ascq_matmul_create(&i8, &h), ASCQ_OK);
    EXPECT(ascq_matmul_set_org_shape(h, 64, 64, 64), ASCQ_OK);
    EXPECT(ascq_matmul_set_tensor_a(h, d, 0), ASCQ_OK);
    EXPECT(ascq_matmul_set_tensor_b(h, d, 0), ASCQ_OK);
    EXPECT(ascq_matmul_set_quant_scalar(h, 0x3F800000u), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, ASCQ_ATOMIC_ADD, nullptr), ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_matmul_destroy(h), ASCQ_OK);
    ascq_matmul_types mx{ASCQ_DT_FP4_E1M2, ASCQ_DT_FP4_E2M1, ASCQ_DT_BF16, ASCQ_DT_F32, ASCQ_DT_E8M0, 0};
    EXPECT(ascq_matmul_create(&mx, &h), ASCQ_OK);
    EXPECT(ascq_matmul_set_org_shape(h, 128, 128, 96), ASCQ_OK);
    EXPECT(ascq_matmul_set_tensor_a(h, d, 0), ASCQ_OK);
    EXPECT(ascq_matmul_set_tensor_b(h, d, 1), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, 0, nullptr), ASCQ_E_STATE);  // no scales
    EXPECT(ascq_matmul_set_tensor_scale_a(h, reinterpret_cast<const uint8_t*>(d), 0), ASCQ_OK);
    EXPECT(ascq_matmul_set_tensor_scale_b(h, reinterpret_cast<const uint8_t*>(d), 1), ASCQ_OK);
    EXPECT(ascq_matmul_iterate_all(h, d, 0, nullptr), ASCQ_E_UNSUPPORTED);  // K % 128
    EXPECT(ascq_matmul_destroy(h), ASCQ_OK);
    ascq_cube_tiling tiling;
    std::memset(&tiling, 0, sizeof(tiling));
    EXPECT(ascq_matmul_init(nullptr, &tiling), ASCQ_E_INVALID_ARG);

    // quant / dequant / antiquant argument checks
    ascq_quant_param qp{4, 100, 400, 0, 0, 1, ASCQ_ROUND_RINT};
    EXPECT(ascq_ascend_quant_per_token(nullptr, d, ASCQ_DT_F16, reinterpret_cast<const float*>(d), nullptr, &qp, nullptr),
           ASCQ_E_INVALID_ARG);
    qp.cal_count = 401;  // not a multiple of n
    EXPECT(ascq_ascend_quant_per_token(reinterpret_cast<int8_t*>(d), d, ASCQ_DT_F16, reinterpret_cast<const float*>(d),
                                       nullptr, &qp, nullptr), ASCQ_E_INVALID_ARG);
    EXPECT(ascq_ascend_quant_dynamic_per_token(nullptr, nullptr, d, ASCQ_DT_F16, 4, 8, 1, nullptr), ASCQ_E_INVALID_ARG);
    EXPECT(ascq_ascend_quant_policy(d, ASCQ_DT_INT8, d, 99, d, nullptr, 0.0f, ASCQ_DT_F32, 2, &qp, nullptr),
           ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_ascend_quant(d, ASCQ_DT_INT32, d, ASCQ_DT_F16, d, nullptr, 1.0f, 0.0f, 64, 64, nullptr),
           ASCQ_E_UNSUPPORTED);
    ascq_dequant_param dp{4, 30, 30};  // n % 8 != 0
    EXPECT(ascq_ascend_dequant(d, ASCQ_DT_F16, d, ASCQ_DT_INT32, d, ASCQ_DT_U64, 0.0f, 1, ASCQ_DEQUANT_SINGLE_ROW, &dp,
                               nullptr), ASCQ_E_INVALID_ARG);
    uint32_t rows = 0, stride = 0;
    ascq_dequant_param dq{1, 16, 8};
    EXPECT(ascq_ascend_dequant_dst_shape(ASCQ_DT_F32, ASCQ_DEQUANT_SINGLE_ROW, &dq, &rows, &stride), ASCQ_OK);
    if (rows != 2 || stride != 8) {
        std::printf("dst_shape {1,16,8} f32: rows %u stride %u\n", rows, stride);
        ++failures;
    }
    ascq_dequant_policy_param pp{4, 64, 256, 30, 0, 1};  // group % 32 != 0
    EXPECT(ascq_ascend_dequant_policy(d, ASCQ_DT_F16, d, ASCQ_DT_INT32, d, nullptr, ASCQ_DT_F32, 3, &pp, nullptr),
           ASCQ_E_INVALID_ARG);
    EXPECT(ascq_ascend_antiquant(d, ASCQ_DT_F16, d, ASCQ_DT_INT32, nullptr, d, 128, 64, 0, 0, 0, nullptr),
           ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_ascend_antiquant_scalar(nullptr, ASCQ_DT_F16, d, ASCQ_DT_INT8, 0, 0x3C00, 0, 16, nullptr),
           ASCQ_E_INVALID_ARG);
    EXPECT(ascq_ascend_antiquant_policy(d, ASCQ_DT_F16, d, ASCQ_DT_INT8, d, nullptr, ASCQ_DT_F16, 3, 4, 64, 20, 1, 0,
                                        nullptr), ASCQ_E_INVALID_ARG);

    // weight-only, group matmul, layout
    size_t wb = 0;
    EXPECT(ascq_weight_pack_size(ASCQ_DT_INT4, 4096, 11008, &wb), ASCQ_OK);
    if (wb != 4096ull * 11008 / 2) ++failures;
    EXPECT(ascq_weight_pack_size(ASCQ_DT_F16, 4096, 11008, &wb), ASCQ_E_UNSUPPORTED);
    EXPECT(ascq_antiquant_matmul(reinterpret_cast<uint16_t*>(d), reinterpret_cast<const uint16_t*>(d), d, ASCQ_DT_INT4,
                                 reinterpret_cast<const uint16_t*>(d), nullptr, 128, 1, 11008, 4000, nullptr),
           ASCQ_E_INVALID_ARG);
    EXPECT(ascq_quant_group_matmul(d, ASCQ_DT_BF16, reinterpret_cast<const int8_t*>(d), reinterpret_cast<const float*>(d),
                                   reinterpret_cast<const int8_t*>(d), 1, reinterpret_cast<const float*>(d),
                                   reinterpret_cast<const int64_t*>(d), 1, 2000, 64, 64, 64, 0, nullptr),
           ASCQ_E_INVALID_ARG);
    EXPECT(ascq_quant_group_matmul(nullptr, ASCQ_DT_BF16, nullptr, nullptr, nullptr, 0, nullptr, nullptr, 0, 1, 1, 1, 1,
                                   0, nullptr), ASCQ_E_INVALID_ARG);
    if (ascq_nz_size(ASCQ_DT_INT8, 8, 1024, 8192) != 8ull * 1024 * 8192) ++failures;
    EXPECT(ascq_nz_to_nd(nullptr, d, ASCQ_DT_INT8, 1, 16, 32, 0, nullptr), ASCQ_E_INVALID_ARG);

    std::printf("%s: %d failure(s)\n", failures ? "FAIL" : "ok", failures);
    return failures ? 1 : 0;
}
