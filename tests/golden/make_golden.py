"""Write the golden fixtures in tests/golden/*.npz.

Each fixture restates, in numpy, the golden-data procedure of one reference example (the file named in the
fixture's 'source' field), with the reference's own seed where its script fixes one (antiquant: seed 10;
asc_copy_l0c2gm DEQF16: seed 9) and seed 1234 where it leaves the generator unseeded.  Shapes are reduced
where the reference's are large; the formulas and value distributions are the scripts'.  bfloat16 rounding
uses torch (round to nearest even).  No reference code is imported or run.

  python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent
EX = "examples/01_simd_cpp_api/04_advanced_api"


def save(name, source, **arrays):
    np.savez_compressed(OUT / f"{name}.npz", source=np.array(source), **arrays)


def deqf16_seed9():
    """asc_copy_l0c2gm/scripts/gen_data_s322f16.py: int8 [128,128] x [128,256] in [-3,3), DEQF16 with a
    quant scalar of 2 (sign flag set for f16, bit 46), golden = sat(round(acc * 2)) as f16."""
    np.random.seed(9)
    M, K, N = 128, 128, 256
    x1 = np.random.randint(-3, 3, [M, K]).astype(np.int8)
    x2 = np.random.randint(-3, 3, [K, N]).astype(np.int8)
    acc = x1.astype(np.int32) @ x2.astype(np.int32)
    word = np.uint64(np.float32(2.0).view(np.uint32)) | np.uint64(0x400000000000)
    golden = np.clip(np.round(acc.astype(np.float32) * np.float32(2.0)), -65504, 65504).astype(np.float16)
    save("deqf16_seed9", "examples/02_simd_c_api/03_c_api/03_matrix_compute/asc_copy_l0c2gm/scripts/"
         "gen_data_s322f16.py:29-79,115-130", x1=x1, x2=x2, quant_word=np.array([word], np.uint64), golden=golden)


def matmul_quant_vector():
    """00_matmul/matmul_quant/scripts/gen_data.py (quant_mode 1): int8 in [-10,10), bias in [-2,2),
    quant vector U(0.1, 2.0) truncated to (1,8,10) bits, golden = f16(acc+bias) * M1 -> f16."""
    np.random.seed(1234)
    m, n, k = 256, 256, 256
    x1 = np.random.randint(-10, 10, [m, k]).astype(np.int8)
    x2 = np.random.randint(-10, 10, [k, n]).astype(np.int8)
    bias = np.random.randint(-2, 2, [1, n]).astype(np.int32)
    golden = (np.matmul(x1.astype(np.int32), x2.astype(np.int32)) + bias).astype(np.float16)
    qv = np.random.uniform(0.1, 2.0, [1, n]).astype(np.float32)
    words = qv.view(np.int32).astype(np.uint64).reshape(-1)
    trunc = (qv.view(np.uint32) & np.uint32(0xFFFFE000)).view(np.float32)
    for i in range(m):
        golden[i, :] = golden[i, :] * trunc
    save("matmul_quant_vector", f"{EX}/00_matmul/matmul_quant/scripts/gen_data.py:20-48", x1=x1, x2=x2,
         bias=bias.reshape(-1), quant_words=words, golden=golden)


def quant_example():
    """03_quantization/quant/scripts/gen_data.py (dav-2201): src f16 U(-4,4) [1024], scale 2.0, offset 0.9,
    golden = np.round(src*2.0 + 0.9) as int8."""
    np.random.seed(1234)
    src = np.random.uniform(low=-4, high=4, size=[1024]).astype(np.float16)
    golden = np.round(src * 2.0 + 0.9).astype(np.int8)
    save("quant_example", f"{EX}/03_quantization/quant/scripts/gen_data.py:19-30", src=src, golden=golden)


def quant_example_3510():
    """03_quantization/quant/scripts/gen_data.py, the arch-3510 branch (float32 source), which quant.asc computes with
    Quantize PER_TENSOR, scale 2.0, offset 0.9, CAST_RINT: golden = np.round(src * 2.0 + 0.9) as int8, float32
    arithmetic."""
    np.random.seed(1234)
    src = np.random.uniform(low=-4, high=4, size=[1024]).astype(np.float32)
    golden = np.round(src * 2.0 + 0.9).astype(np.int8)
    save("quant_example_3510", f"{EX}/03_quantization/quant/scripts/gen_data.py:20-30", src=src, golden=golden)


def dequant_example():
    """03_quantization/dequant/scripts/gen_data.py: int32 [128,32] in [-10,10), scale U(-100,100) [32],
    golden[j][i] = inp[j][i] * scale[i] as float32."""
    np.random.seed(1234)
    shape = [128, 32]
    inp = np.random.randint(low=-10, high=10, size=shape).astype(np.int32)
    scale = np.random.uniform(low=-100, high=100, size=[32]).astype(np.float32)
    golden = np.zeros(shape)
    for i in range(shape[1]):
        for j in range(shape[0]):
            golden[j][i] = inp[j][i] * scale[i]
    save("dequant_example", f"{EX}/03_quantization/dequant/scripts/gen_data.py:18-27", inp=inp, scale=scale,
         golden=golden.astype(np.float32))


def antiquant_seed10():
    """03_quantization/antiquant/scripts/gen_data.py, seed 10: src int8 [8,128] (K=8 rows, N=128 columns),
    offset / scale f16 [1,128]; dav-2201 golden in half arithmetic, dav-3510 golden in fp32 arithmetic."""
    np.random.seed(10)
    N, K = 128, 8
    group = K
    src = np.random.uniform(-10, 10, [8, 128]).astype(np.int8)
    offset = np.random.uniform(-10, 10, [1, 128]).astype(np.float16)
    scale = np.random.uniform(-10, 10, [1, 128]).astype(np.float16)
    g2201 = np.zeros([8, 128]).astype(np.float32)
    for i in range(K):
        for j in range(N):
            g2201[i][j] = scale[i // group][j] * (src[i][j] + offset[i // group][j])
    g3510 = np.zeros([8, 128]).astype(np.float32)
    s32, o32, x32 = scale.astype(np.float32), offset.astype(np.float32), src.astype(np.float32)
    for i in range(K):
        for j in range(N):
            g3510[i][j] = s32[i // group][j] * (x32[i][j] + o32[i // group][j])
    save("antiquant_seed10", f"{EX}/03_quantization/antiquant/scripts/gen_data.py:19-44", src=src, offset=offset,
         scale=scale, golden_2201=g2201.astype(np.float16), golden_3510=g3510.astype(np.float16))


def group_matmul_example():
    """05_best_practices/03_fusion_compute/quant_group_matmul_high_performance/scripts/gen_data.py without the
    FastGelu: 4 equal groups, x / weight int8 in [-10,10), scale and perTokenScale N(0, 0.01), f32 matmul, then
    mmOut *= scale[i] * perTokenScale, golden f16 (reduced to m=256, k=128, n=128)."""
    np.random.seed(1234)
    G, m, k, n = 4, 256, 128, 128
    group_list = np.array([m // G] * G, dtype=np.int64)
    x = np.random.randint(-10, 10, [m, k]).astype(np.int8)
    weight = np.random.randint(-10, 10, [G, k, n]).astype(np.int8)
    scale = np.random.normal(0, 0.01, (G, n)).astype(np.float32)
    pts = np.random.normal(0, 0.01, (m, 1)).astype(np.float32)
    idx = [0] + np.cumsum(group_list).tolist()
    out = np.empty((m, n), np.float32)
    for i in range(G):
        s, e = idx[i], idx[i + 1]
        out[s:e] = np.dot(x[s:e].astype(np.float32), weight[i].astype(np.float32))
        out[s:e] *= scale[i] * pts[s:e]
    save("group_matmul_example", "examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/"
         "quant_group_matmul_high_performance/scripts/gen_data.py:26-54", x=x, weight=weight, scale=scale,
         pts=pts.reshape(-1), group_list=group_list, golden=out.astype(np.float16))


def group_matmul_gelu_example():
    """the same generator with its FastGelu (gen_data.py:19-23, applied to the float32 mmOut with numpy
    float32 ops) and the f16 golden: 4 equal groups, x / weight in [-10,10), scale and perTokenScale N(0, 0.01)
    (reduced to m=256, k=128, n=128; seed 4321)."""
    np.random.seed(4321)
    G, m, k, n = 4, 256, 128, 128
    group_list = np.array([m // G] * G, dtype=np.int64)
    x = np.random.randint(-10, 10, [m, k]).astype(np.int8)
    weight = np.random.randint(-10, 10, [G, k, n]).astype(np.int8)
    scale = np.random.normal(0, 0.01, (G, n)).astype(np.float32)
    pts = np.random.normal(0, 0.01, (m, 1)).astype(np.float32)
    idx = [0] + np.cumsum(group_list).tolist()
    out = np.empty((m, n), np.float32)
    for i in range(G):
        s, e = idx[i], idx[i + 1]
        out[s:e] = np.dot(x[s:e].astype(np.float32), weight[i].astype(np.float32))
        out[s:e] *= scale[i] * pts[s:e]
    ax = np.abs(out)
    gelu = out * np.exp(np.float32(0.851) * (out - ax)) / (1 + np.exp(np.float32(-1.702) * ax))
    save("group_matmul_gelu_example", "examples/01_simd_cpp_api/05_best_practices/03_fusion_compute/"
         "quant_group_matmul_high_performance/scripts/gen_data.py:19-54", x=x, weight=weight, scale=scale,
         pts=pts.reshape(-1), group_list=group_list, golden=gelu.astype(np.float32).astype(np.float16))


def mx_example():
    """01_matrix_compute/matmul_mxfp4_high_performance/scripts/gen_data.py: elements in {-1, 0, 1}, e8m0 scales
    in [127, 129], fp64 dequant-then-matmul golden cast to bf16; packing even element in the low nibble,
    scaleA [M, sK], scaleB [sK/2, N, 2].  The script draws E1M2 elements; -1, 0 and 1 are also E2M1 codes
    (0xA, 0x0, 0x2), which is the element type used here (reduced to 256 x 256 x 256)."""
    np.random.seed(1234)
    m = n = k = 256
    sk = int(np.ceil(k / 64) * 2)
    x1 = np.random.randint(-1, 2, [m, k]).astype(np.float64)
    x2 = np.random.randint(-1, 2, [k, n]).astype(np.float64)
    s1 = np.random.randint(127, 130, [m, sk]).astype(np.uint8)
    s2 = np.random.randint(127, 130, [sk, n]).astype(np.uint8)
    x1_mx = 2 ** (s1.astype(np.float64) - 127)
    x2_mx = 2 ** (s2.astype(np.float64) - 127)
    a = np.zeros([m, k])
    b = np.zeros([k, n])
    for i in range(k):
        a[:, i] = x1[:, i] * x1_mx[:, i // 32]
        b[i, :] = x2[i, :] * x2_mx[i // 32, :]
    golden = torch.from_numpy(np.matmul(a, b).astype(np.float32)).to(torch.bfloat16).view(torch.int16).numpy()
    code = {-1.0: 0xA, 0.0: 0x0, 1.0: 0x2}

    def pack(v):
        c = np.vectorize(code.get)(v).astype(np.uint8)
        return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)

    s2_pairs = s2.reshape(sk // 2, 2, n).transpose(0, 2, 1)
    save("mx_example", "examples/01_simd_cpp_api/05_best_practices/01_matrix_compute/matmul_mxfp4_high_performance/"
         "scripts/gen_data.py:25-63", a_packed=pack(x1), b_packed=pack(x2), scale_a=s1,
         scale_b_pairs=np.ascontiguousarray(s2_pairs), golden_bf16=golden.view(np.uint16))


L0C2GM = "examples/02_simd_c_api/03_c_api/03_matrix_compute/asc_copy_l0c2gm/scripts/"


def _req8(v, word):
    """the scripts' req8_pre / qf322b8_pre with the ReLU coefficient equal to M1 (pre_relu_mode 0): clip to
    [-256, 255], np.round (half to even), + offset, clip to the int8 range (sign flag set)"""
    m1 = np.float32((np.uint32(word & 0xFFFFFFFF) & np.uint32(0xFFFFE000)).view(np.float32))
    off = int((int(word) >> 37) & 0x1FF)
    q = np.round(np.clip(v.astype(np.float32) * m1, -256, 255)).astype(np.int16) + off
    return np.clip(q, -128, 127).astype(np.int8)


def req8_seed9():
    """asc_copy_l0c2gm/scripts/gen_data_s322s8.py: int8 [128,128] x [128,256] in [-3,3) with seed 9, (V)REQ8 with
    M1 = 2 in every column and the sign flag set (int8 C), ReLU coefficient = M1; golden int8."""
    np.random.seed(9)
    M, K, N = 128, 128, 256
    x1 = np.random.randint(-3, 3, [M, K]).astype(np.int8)
    x2 = np.random.randint(-3, 3, [K, N]).astype(np.int8)
    acc = x1.astype(np.int32) @ x2.astype(np.int32)
    word = int(np.float32(2.0).view(np.uint32)) | 0x400000000000
    golden = _req8(acc, word)
    save("req8_seed9", L0C2GM + "gen_data_s322s8.py:29-80,83-136", x1=x1, x2=x2,
         quant_word=np.array([word], np.uint64), golden=golden)


def qf322b8_seed9():
    """asc_copy_l0c2gm/scripts/gen_data.py scenario 4 / 5: f16 [128,128] x [128,256] in [-1,3) with seed 9, fp32
    matmul (numpy float32), (V)QF322B8_PRE with M1 = 2 and the sign flag (int8 C); golden int8.  The fp32
    accumulators are stored with the golden: the fixture pins the epilogue."""
    np.random.seed(9)
    M, K, N = 128, 128, 256
    x1 = np.random.uniform(-1, 3, [M, K]).astype(np.float16)
    x2 = np.random.uniform(-1, 3, [K, N]).astype(np.float16)
    acc = np.matmul(x1.astype(np.float32), x2.astype(np.float32)).astype(np.float32)
    word = int(np.float32(2.0).view(np.uint32)) | 0x400000000000
    golden = _req8(acc, word)
    save("qf322b8_seed9", L0C2GM + "gen_data.py:56-80,83-116,119-148", acc_f32=acc,
         quant_word=np.array([word], np.uint64), golden=golden)


ALL = ("deqf16_seed9", "matmul_quant_vector", "quant_example", "quant_example_3510", "dequant_example",
       "antiquant_seed10",
       "group_matmul_example", "mx_example", "req8_seed9", "qf322b8_seed9", "group_matmul_gelu_example")


def main(names=None):
    """python tests/golden/make_golden.py [fixture ...] (default: all)"""
    for name in names or ALL:
        globals()[name]()
        print("wrote", name)


if __name__ == "__main__":
    import sys

    main(sys.argv[1:])
