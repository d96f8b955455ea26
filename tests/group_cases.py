"""Group-matmul inputs whose int32 accumulators land on fp32 rounding ties in [2^24, 2^26).

The reference's group epilogue converts the int32 tile with AscendDequant (quant_group_matmul_custom.asc:433),
whose int32 -> fp32 cast rounds ties away from zero (Cast<float, int32_t, MrgZRndA>,
impl/adv_api/detail/quantization/dequant/ascend_dequant_3510_impl.h:61).  A tie only shows in a 16-bit output
when the scaled value straddles a rounding boundary of that output, so this builder chooses the data to make
that happen on purpose:

  * x[m, k] = sign_m * 127 for k >= 8 and w[k, n] = c_n for k >= 8, while w[k, n] = 1 for k < 8: every
    accumulator is acc[m, n] = sign_m * 127 * (K - 8) * c_n + t_m with t_m = sum(x[m, :8]) chosen per row;
    with |c_n| in [33, 127] and K = 4096 the magnitudes cover [2^24, 2^26);
  * for each column one target row is chosen whose accumulator is a tie that the nearest-even rule rounds
    toward zero (so the two rules give different fp32 values), and the column's fp32 scale is searched so that
    the two fp32 values, multiplied by the scale (the per-token scale is 1), round to different bf16 values.

The numpy restatement here (ties away, then the fp32 products, then bf16 rne via torch) is independent of the
oracle's C code; `rne_differs` counts the outputs the nearest-even rule would change.
"""
from __future__ import annotations

import numpy as np
import torch


def i32_to_f32_rna(acc):
    """int32 -> fp32 with ties away from zero: exact below 2^24; above, the magnitude's 24-bit significand is
    rounded half up (numpy int64 arithmetic)."""
    a = np.asarray(acc, np.int64)
    mag = np.abs(a)
    e = np.frexp(mag.astype(np.float64))[1]  # bit length of |a| (exact: |a| < 2^53)
    s = np.maximum(e - 24, 0)
    half = np.where(s > 0, np.left_shift(np.int64(1), np.maximum(s - 1, 0)), 0)
    r = np.right_shift(mag + half, s) << s
    return (np.sign(a) * r).astype(np.float32)


def bf16_bits(v32):
    return torch.from_numpy(np.ascontiguousarray(v32, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(
        np.uint16)


def _is_rne_down_tie(a):
    """|a| in [2^24, 2^26) is a tie of the fp32 conversion and nearest-even rounds its magnitude down"""
    mag = abs(int(a))
    if not (1 << 24) <= mag < (1 << 26):
        return False
    s = mag.bit_length() - 24
    low = mag & ((1 << s) - 1)
    return low == (1 << (s - 1)) and ((mag >> s) & 1) == 0


def tie_case(seed, M=64, N=64, K=4096, groups=(40, 24)):
    rng = np.random.default_rng(seed)
    G = len(groups)
    assert sum(groups) == M and K > 8
    sign = np.where(rng.random(M) < 0.5, -1, 1).astype(np.int64)
    x = np.empty((M, K), np.int8)
    x[:, 8:] = (127 * sign)[:, None].astype(np.int8)
    x[:, :8] = rng.integers(-127, 128, (M, 8), dtype=np.int8)
    t = x[:, :8].astype(np.int64).sum(1)
    w = np.empty((G, K, N), np.int8)
    w[:, :8, :] = 1
    pts = np.ones(M, np.float32)
    sc = np.exp(rng.uniform(np.log(1e-4), np.log(1e-2), (G, N))).astype(np.float32)
    off = np.concatenate([[0], np.cumsum(groups)])
    mags = np.arange(33, 128)
    for g in range(G):
        s0, s1 = off[g], off[g + 1]
        for n in range(N):
            m = s0 + n % (s1 - s0)  # the column's target row
            cs = rng.permutation(np.concatenate([mags, -mags]))
            c = next((int(v) for v in cs if _is_rne_down_tie(int(sign[m]) * 127 * (K - 8) * int(v) + int(t[m]))),
                     int(cs[0]))
            w[g, 8:, n] = c
            a = int(sign[m]) * 127 * (K - 8) * c + int(t[m])
            if not _is_rne_down_tie(a):
                continue
            f_a = i32_to_f32_rna(np.array([a]))[0]
            f_e = np.float32(a)  # nearest even
            # a bf16 rounding midpoint next to f_a * scale; try fp32 scales around midpoint / f_a until the two
            # products round to different bf16 values
            s_try = np.float32(sc[g, n])
            for _ in range(64):
                p = np.array([np.float32(f_a * s_try)], np.float32).view(np.uint32)[0]
                mid = np.array([(int(p) & 0xFFFF0000) | 0x8000], np.uint32).view(np.float32)[0]
                s_c = np.float32(np.float64(mid) / np.float64(f_a))
                cands, up, dn = [s_c], s_c, s_c
                for _j in range(8):
                    up = np.nextafter(up, np.float32(np.inf))
                    dn = np.nextafter(dn, np.float32(-np.inf))
                    cands += [up, dn]
                hit = next((s_j for s_j in cands
                            if bf16_bits(np.array([f_a * s_j], np.float32))[0] !=
                            bf16_bits(np.array([f_e * s_j], np.float32))[0]), None)
                if hit is not None:
                    sc[g, n] = hit
                    break
                s_try = np.float32(s_try * np.float32(1.0009765625))
    counts = np.array(groups, np.int64)
    return x, w, pts, sc, counts


def group_reference(x, w, pts, sc, counts, rna=True):
    """numpy restatement of the group epilogue: fp32(acc) (ties away, or nearest even with rna=False) * scale[g, n],
    then * pts[m], bf16 rne; returns uint16 bits [M, N]"""
    M = x.shape[0]
    N = w.shape[2]
    y = np.zeros((M, N), np.uint16)
    off = np.concatenate([[0], np.cumsum(counts)])
    for g in range(len(counts)):
        s, e = off[g], off[g + 1]
        acc = x[s:e].astype(np.int64) @ w[g].astype(np.int64)
        f = i32_to_f32_rna(acc) if rna else acc.astype(np.float32)
        v = (f * sc[g][None, :]).astype(np.float32)
        v = (v * pts[s:e, None]).astype(np.float32)
        y[s:e] = bf16_bits(v)
    return y


def rne_differs(x, w, pts, sc, counts):
    """number of outputs the nearest-even conversion would change"""
    return int((group_reference(x, w, pts, sc, counts, True) != group_reference(x, w, pts, sc, counts, False)).sum())
