// Host-only check of the TCubeTiling mirror and the MultiCoreMatmulTiling / Matmul::Init shim
// (include/ascq_matmul.hpp), written the way the reference's matmul_quant.asc host code builds its tiling
// (SetAType / SetBType / SetCType / SetBiasType / SetShape / SetOrgShape / SetBias / SetDequantType /
// SetBufferSpace / GetTiling).  Prints one line per check; exit status 0 when all hold.  No GPU needed.
#include <cstddef>
#include <cstdio>

#include "ascq_matmul.hpp"

static int fails = 0;
#define EXPECT(c)                                        \
    do {                                                 \
        if (!(c)) {                                      \
            std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); \
            ++fails;                                     \
        }                                                \
    } while (0)

int main()
{
    // layout: 50 int32 fields, in the reference's order
    EXPECT(sizeof(ascq_cube_tiling) == 50 * sizeof(int32_t));
    EXPECT(offsetof(ascq_cube_tiling, M) == 4);
    EXPECT(offsetof(ascq_cube_tiling, Ka) == 12);
    EXPECT(offsetof(ascq_cube_tiling, isBias) == 15 * 4);
    EXPECT(offsetof(ascq_cube_tiling, BatchNum) == 48 * 4);
    EXPECT(offsetof(ascq_cube_tiling, mxTypePara) == 49 * 4);

    using ascq::CubeFormat;
    using ascq::TPosition;
    ascq::MultiCoreMatmulTiling tiling;
    tiling.SetDim(1);
    tiling.SetAType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT8);
    tiling.SetBType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT8);
    tiling.SetCType(TPosition::GM, CubeFormat::ND, ASCQ_DT_F16);
    tiling.SetBiasType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT32);
    tiling.SetShape(128, 256, 512);
    tiling.SetOrgShape(128, 256, 512);
    tiling.SetBias(true);
    tiling.SetDequantType(ascq::DequantType::TENSOR);
    tiling.SetBufferSpace(-1, -1, -1);
    ascq_cube_tiling t;
    EXPECT(tiling.GetTiling(t) == 0);
    EXPECT(t.M == 128 && t.N == 256 && t.Ka == 512 && t.Kb == 512 && t.isBias == 1);
    EXPECT(t.singleCoreM == 128 && t.singleCoreN == 256 && t.singleCoreK == 512);

    ascq::Matmul mm(ASCQ_DT_INT8, ASCQ_DT_INT8, ASCQ_DT_F16, ASCQ_DT_INT32);
    mm.Init(&t);  // org shape from the tiling
    size_t ws = 1;
    EXPECT(ascq_matmul_workspace_size(mm.handle(), &ws) == ASCQ_OK);

    // GetTiling's -1 cases: a type combination without a kernel, missing types, Ka != Kb, an NZ A, an NZ B of a
    // type without an NZ path (int4)
    ascq::MultiCoreMatmulTiling bad;
    bad.SetAType(TPosition::GM, CubeFormat::ND, ASCQ_DT_F32);
    bad.SetBType(TPosition::GM, CubeFormat::ND, ASCQ_DT_F32);
    bad.SetCType(TPosition::GM, CubeFormat::ND, ASCQ_DT_F32);
    bad.SetShape(16, 16, 16);
    EXPECT(bad.GetTiling(t) == -1);
    ascq::MultiCoreMatmulTiling none;
    none.SetShape(16, 16, 16);
    EXPECT(none.GetTiling(t) == -1);
    ascq::MultiCoreMatmulTiling kk;
    kk.SetAType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT8);
    kk.SetBType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT8);
    kk.SetCType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT32);
    kk.SetOrgShape(16, 16, 32, 48);
    EXPECT(kk.GetTiling(t) == -1);
    ascq::MultiCoreMatmulTiling nza;
    nza.SetAType(TPosition::GM, CubeFormat::NZ, ASCQ_DT_INT8);
    nza.SetBType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT8);
    nza.SetCType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT32);
    nza.SetShape(16, 16, 16);
    EXPECT(nza.GetTiling(t) == -1);
    ascq::MultiCoreMatmulTiling nz4;
    nz4.SetAType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT4);
    nz4.SetBType(TPosition::GM, CubeFormat::NZ, ASCQ_DT_INT4);
    nz4.SetCType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT32);
    nz4.SetShape(16, 16, 16);
    EXPECT(nz4.GetTiling(t) == -1);

    // an NZ int8 B (the group-matmul sample's MatmulType<GM, NZ, int8_t>, quant_group_matmul_custom.asc:110): a
    // tiling, and a handle created with ASCQ_FORMAT_NZ that counts the ND copy of B in its workspace
    ascq::MultiCoreMatmulTiling nz;
    nz.SetAType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT8);
    nz.SetBType(TPosition::GM, CubeFormat::NZ, ASCQ_DT_INT8);
    nz.SetCType(TPosition::GM, CubeFormat::ND, ASCQ_DT_INT32);
    nz.SetShape(64, 96, 128);
    EXPECT(nz.GetTiling(t) == 0);
    ascq::Matmul mnz(ASCQ_DT_INT8, ASCQ_DT_INT8, ASCQ_DT_INT32, 0, 0, ASCQ_FORMAT_NZ);
    mnz.Init(&t);
    EXPECT(ascq_matmul_workspace_size(mnz.handle(), &ws) == ASCQ_OK && ws >= (size_t)96 * 128);

    // Init rejects Ka != Kb
    ascq_cube_tiling t2 = {};
    t2.M = 8;
    t2.N = 8;
    t2.Ka = 16;
    t2.Kb = 32;
    EXPECT(ascq_matmul_init(mm.handle(), &t2) == ASCQ_E_INVALID_ARG);
    std::printf("%s\n", fails ? "FAILED" : "ok");
    return fails ? 1 : 0;
}
