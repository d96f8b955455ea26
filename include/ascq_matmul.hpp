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

    // Init(const TCubeTiling*) / REGIST_MATMUL_OBJ(..., &tiling): the org shape from the tiling
    void Init(const ascq_cube_tiling* tiling) { check(ascq_matmul_init(h_, tiling), "Init"); }
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

// Host tiling builder with the reference's call sequence (matmul_tiling::MultiCoreMatmulTiling,
// include/adv_api/matmul/matmul_tiling_base.h:329-556): SetAType / SetBType / SetCType / SetBiasType / SetShape /
// SetOrgShape / SetBias / SetDequantType / SetBufferSpace / GetTiling.  GetTiling returns -1, as the reference
// does (impl/adv_api/tiling/matmul/matmul_tiling.cpp:28-35), when the description is incomplete or the type
// combination has no kernel here; otherwise 0 and a tiling whose shape fields Matmul::Init reads.  The Ascend
// buffer / core-split settings have no meaning for one gfx950 launch and are accepted and ignored.
enum class TPosition { GM, VECIN, VECCALC, VECOUT, A1, A2, B1, B2, CO1, CO2, TSCM };
enum class CubeFormat { ND, NZ, ZN, ZZ, NN, ND_ALIGN, SCALAR, VECTOR };
enum class DequantType { SCALAR, TENSOR };

class MultiCoreMatmulTiling {
public:
    MultiCoreMatmulTiling() = default;
    int32_t SetDim(int32_t) { return 0; }
    int32_t SetAType(TPosition, CubeFormat f, ascq_dtype t, bool isTrans = false) { return set(a_, f, t, isTrans); }
    int32_t SetBType(TPosition, CubeFormat f, ascq_dtype t, bool isTrans = false) { return set(b_, f, t, isTrans); }
    int32_t SetCType(TPosition, CubeFormat f, ascq_dtype t) { return set(c_, f, t, false); }
    int32_t SetBiasType(TPosition, CubeFormat f, ascq_dtype t) { return set(bias_, f, t, false); }
    int32_t SetDequantType(DequantType) { return 0; }
    int32_t SetShape(int32_t m, int32_t n, int32_t k)
    {
        m_ = m;
        n_ = n;
        k_ = k;
        return 0;
    }
    int32_t SetOrgShape(int32_t m, int32_t n, int32_t k) { return SetOrgShape(m, n, k, k); }
    int32_t SetOrgShape(int32_t m, int32_t n, int32_t ka, int32_t kb)
    {
        om_ = m;
        on_ = n;
        oka_ = ka;
        okb_ = kb;
        return 0;
    }
    int32_t SetBias(bool isBias = false)
    {
        isBias_ = isBias;
        return 0;
    }
    int32_t SetBufferSpace(int32_t = -1, int32_t = -1, int32_t = -1, int32_t = -1) { return 0; }
    int32_t SetFixSplit(int32_t = -1, int32_t = -1, int32_t = -1) { return 0; }

    int64_t GetTiling(ascq_cube_tiling& t) const
    {
        const int32_t M = om_ > 0 ? om_ : m_, N = on_ > 0 ? on_ : n_, Ka = oka_ > 0 ? oka_ : k_;
        const int32_t Kb = okb_ > 0 ? okb_ : Ka;
        if (!a_.set || !b_.set || !c_.set || M <= 0 || N <= 0 || Ka <= 0 || Ka != Kb) return -1;
        if (m_ > M || n_ > N || k_ > Ka) return -1;
        // A and C row-major; B row-major or NZ (int8 / fp8 B: Matmul(..., ASCQ_FORMAT_NZ) takes it as it is)
        if (a_.fmt != CubeFormat::ND || c_.fmt != CubeFormat::ND) return -1;
        if (b_.fmt != CubeFormat::ND && b_.fmt != CubeFormat::NZ) return -1;
        // the type combination must have a kernel: the library decides (a transient handle)
        ascq_matmul_types ty{a_.type, b_.type, c_.type, bias_.set && isBias_ ? bias_.type : 0, 0,
                             b_.fmt == CubeFormat::NZ ? ASCQ_FORMAT_NZ : ASCQ_FORMAT_ND};
        ascq_matmul_t h = nullptr;
        if (ascq_matmul_create(&ty, &h) != ASCQ_OK) return -1;
        ascq_matmul_destroy(h);
        t = ascq_cube_tiling{};
        t.usedCoreNum = 1;  // one launch covers the whole shape
        t.M = M;
        t.N = N;
        t.Ka = Ka;
        t.Kb = Kb;
        t.singleCoreM = m_ > 0 ? m_ : M;
        t.singleCoreN = n_ > 0 ? n_ : N;
        t.singleCoreK = k_ > 0 ? k_ : Ka;
        t.isBias = isBias_ ? 1 : 0;
        t.BatchNum = 1;
        return 0;
    }

private:
    struct Desc {
        bool set = false;
        CubeFormat fmt = CubeFormat::ND;
        int32_t type = 0;
        bool trans = false;
    };
    static int32_t set(Desc& d, CubeFormat f, ascq_dtype t, bool trans)
    {
        d.set = true;
        d.fmt = f;
        d.type = t;
        d.trans = trans;
        return 0;
    }
    Desc a_, b_, c_, bias_;
    int32_t m_ = -1, n_ = -1, k_ = -1, om_ = -1, on_ = -1, oka_ = -1, okb_ = -1;
    bool isBias_ = false;
};

}  // namespace ascq
