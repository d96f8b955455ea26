// aq_frag.h -- the weight-fragment dequantisation shared by the weight-only antiquant matmul kernels
// (gemv_antiquant.hip, aq_gemm.hip): AscendAntiQuant's per-group half arithmetic (impl/adv_api/detail/quantization/
// antiquant/ascend_antiquant_impl.h:63-96), w = half( half(q + offset) * scale ), on one 8-element fragment of the
// packed weight layout (ascq_weight_pack: offset-binary codes; int4 element e of a 32-k step at bits 4 (e / 2) +
// 16 (e % 2) of its word, int8 elements as the bytes of two words in k order).
#pragma once

#include "common.h"

namespace ascq {

// 0x64006400 (two binary16 1024.0) held in a VGPR: with both masks as literals the compiler cannot fuse the
// and / or of the int4 unpacking into one v_and_or_b32 (a VOP3 instruction takes no literal operand here)
__device__ __forceinline__ uint32_t half_magic_vgpr()
{
    uint32_t m;
    asm("v_mov_b32 %0, 0x64006400" : "=v"(m));
    return m;
}

// dequantise one 8-element B fragment: codes -> half(half(q + off) * scale)
template <bool INT4, bool HAS_OFF>
__device__ __forceinline__ h8 dequant8(uint32_t w0, uint32_t w1, h2 off, h2 sc, uint32_t magic)
{
    uint32_t d[4];
    h2 qv[4];
    if constexpr (INT4) {
        // w0 holds all 8 nibbles of the step.  Pairs 0 / 2 (bits 0-3 / 8-11 of each half) OR under the exponent of
        // 1024 as 1024 + c; pairs 1 / 3 (bits 4-7 / 12-15) are masked in place, giving 1024 + 16 c, and
        // 1024 + 16 c -> c - 8 is one exact fma (x / 16 - 72), so no shift by 4 or 12 is needed
        const uint32_t w8 = w0 >> 8;
        d[0] = (w0 & 0x000F000Fu) | magic;
        d[1] = (w0 & 0x00F000F0u) | magic;
        d[2] = (w8 & 0x000F000Fu) | magic;
        d[3] = (w8 & 0x00F000F0u) | magic;
        const h2 bias = (h2){(_Float16)1032.0f, (_Float16)1032.0f};
        const h2 sixteenth = (h2){(_Float16)0.0625f, (_Float16)0.0625f}, b16 = (h2){(_Float16)-72.0f, (_Float16)-72.0f};
        qv[0] = __builtin_bit_cast(h2, d[0]) - bias;                                       // exact
        qv[1] = __builtin_elementwise_fma(__builtin_bit_cast(h2, d[1]), sixteenth, b16);  // exact
        qv[2] = __builtin_bit_cast(h2, d[2]) - bias;
        qv[3] = __builtin_elementwise_fma(__builtin_bit_cast(h2, d[3]), sixteenth, b16);
    } else {
        // bytes b0..b3 of w0 and w1 -> halves 0x64bb (selector 5 = byte 1 of magic = 0x64)
        d[0] = __builtin_amdgcn_perm(magic, w0, 0x05010500u);
        d[1] = __builtin_amdgcn_perm(magic, w0, 0x05030502u);
        d[2] = __builtin_amdgcn_perm(magic, w1, 0x05010500u);
        d[3] = __builtin_amdgcn_perm(magic, w1, 0x05030502u);
        const h2 bias = (h2){(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = __builtin_bit_cast(h2, d[i]) - bias;  // exact
    }
    h2 r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2 q = qv[i];
        if constexpr (HAS_OFF) q = q + off;  // one rounding
        r[i] = q * sc;                       // one rounding
    }
    h8 out;
    out.s01 = r[0];
    out.s23 = r[1];
    out.s45 = r[2];
    out.s67 = r[3];
    return out;
}

}  // namespace ascq
