// ascq_matmul.hpp -- header-only C++ mirror of the reference's Matmul call sequence on top of the C ABI.
//
// The reference instantiates AscendC::Matmul<MatmulType<GM, ND, A>, <B>, <C>, <Bias>, CFG> inside a device
// kernel and drives it with SetTensorA / SetTensorB / SetBias / SetQuantScalar / SetQuantVector / IterateAll /
// End (include/adv_api/matmul/matmul.h:54-400).  This class keeps those names and argument meanings on the
// host: each method forwards to one ascq_matmul_* function (include/ascq.h); errors throw ascq::Error.
#pragma once

#include <stdexcept>
#include <string>

#include "ascq.h"

namespace ascq {

struct Error : std::runtime_error {
    ascq_status status;
    Error(ascq_status s, const std::string& what) : std::runtime_error(what), status(s) {}
};

inline void check(ascq_status s, const char* what)
{
    if (s != ASCQ_OK) throw Error(s, std::string(what) + ": " + ascq_last_error());
}

class Matmul {
public:
    Matmul(ascq_dtype a, ascq_dtype b, ascq_dtype c, int32_t bias = 0, int32_t scale = 0,
           ascq_format b_format = ASCQ_FORMAT_ND)
    {
        ascq_matmul_types t{a, b, c, bias, scale, b_format};
        check(ascq_matmul_create(&t, &h_), "Matmul");
    }
    ~Matmul() { ascq_matmul_destroy(h_); }
    Matmul(const Matmul&) = delete;
    Matmul& operator=(const Matmul&) = delete;

    void SetOrgShape(int64_t m, int64_t n, int64_t k) { check(ascq_matmul_set_org_shape(h_, m, n, k), "SetOrgShape"); }
    void SetSingleShape(int64_t m, int64_t n, int64_t k)
    {
        check(ascq_matmul_set_single_shape(h_, m, n, k), "SetSingleShape");
    }
    void SetTail(int64_t m = -1, int64_t n = -1, int64_t k = -1) { check(ascq_matmul_set_tail(h_, m, n, k), "SetTail"); }
    void SetTensorA(const void* a, bool isTransposeA = false)
    {
        check(ascq_matmul_set_tensor_a(h_, a, isTransposeA), "SetTensorA");
    }
    void SetTensorB(const void* b, bool isTransposeB = false)
    {
        check(ascq_matmul_set_tensor_b(h_, b, isTransposeB), "SetTensorB");
    }
    void SetBias(const void* bias) { check(ascq_matmul_set_bias(h_, bias), "SetBias"); }
    void DisableBias() { check(ascq_matmul_disable_bias(h_), "DisableBias"); }
    void SetQuantScalar(uint64_t quant) { check(ascq_matmul_set_quant_scalar(h_, quant), "SetQuantScalar"); }
    void SetQuantVector(const uint64_t* quant) { check(ascq_matmul_set_quant_vector(h_, quant), "SetQuantVector"); }
    void SetAntiQuantScalar(uint16_t offset_f16, uint16_t scale_f16)
    {
        check(ascq_matmul_set_antiquant_scalar(h_, offset_f16, scale_f16), "SetAntiQuantScalar");
    }
    void SetAntiQuantVector(const void* offset, const void* scale, int64_t group_size = 0)
    {
        check(ascq_matmul_set_antiquant_vector(h_, offset, scale, group_size), "SetAntiQuantVector");
    }
    void SetTensorScaleA(const uint8_t* s, bool isTransposeScaleA = false)
    {
        check(ascq_matmul_set_tensor_scale_a(h_, s, isTransposeScaleA), "SetTensorScaleA");
    }
    void SetTensorScaleB(const uint8_t* s, bool isTransposeScaleB = true)
    {
        check(ascq_matmul_set_tensor_scale_b(h_, s, isTransposeScaleB), "SetTensorScaleB");
    }
    void IterateAll(void* c, uint8_t enAtomic = 0, void* stream = nullptr)
    {
        check(ascq_matmul_iterate_all(h_, c, enAtomic, stream), "IterateAll");
    }
    void End() { check(ascq_matmul_end(h_), "End"); }
    ascq_matmul_t handle() const { return h_; }

private:
    ascq_matmul_t h_ = nullptr;
};

}  // namespace ascq
