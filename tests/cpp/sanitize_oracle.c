/* The oracle's codecs and reductions on small inputs under AddressSanitizer + UndefinedBehaviorSanitizer (the
 * values themselves are pinned by tests/test_oracle.py; this checks the C for out-of-bounds accesses, overflow
 * and other undefined behaviour).  Exit status 0 = the sanitizers reported nothing. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ascq_oracle.h"

static uint32_t rng = 12345u;
static uint32_t next(void) { rng = rng * 1664525u + 1013904223u; return rng; }

int main(void)
{
    enum { M = 5, N = 64, K = 128, G = 3 };
    double sink = 0.0;
    for (uint32_t c = 0; c < 256; ++c) {
        sink += oq_hif8_decode((uint8_t)c) == oq_hif8_decode((uint8_t)c) ? 1.0 : 0.0;
        sink += oq_fp8_decode((uint8_t)c, OQ_FP8_E4M3) + oq_fp8_decode((uint8_t)c, OQ_FP8_E5M2);
    }
    for (int i = 0; i < 100000; ++i) {
        uint32_t u = next();
        float x;
        memcpy(&x, &u, 4);
        sink += oq_hif8_encode(x, 1) + oq_hif8_encode(x, 0) + oq_f32_to_f16(x, 1) + oq_f32_to_bf16(x, 1);
        sink += oq_e1m2_encode(x, 1) + oq_f64_to_f16((double)x, 0) + oq_f64_to_bf16((double)x, 1);
    }
    /* int8 matmul + dequant epilogue */
    int8_t *a = malloc(M * K), *b = malloc(K * N);
    int32_t *acc = malloc(sizeof(int32_t) * M * N), *bias = malloc(sizeof(int32_t) * N);
    uint16_t* y = malloc(2 * M * N);
    uint64_t* qv = malloc(8 * N);
    for (int i = 0; i < M * K; ++i) a[i] = (int8_t)next();
    for (int i = 0; i < K * N; ++i) b[i] = (int8_t)next();
    for (int i = 0; i < N; ++i) {
        bias[i] = (int32_t)(next() >> 8);
        qv[i] = oq_pack_quant_pre(0.001f, (int32_t)(next() % 512), (int32_t)(next() & 1));
    }
    oq_matmul_i8(a, b, bias, acc, M, N, K, 0, 0);
    oq_mm_dequant(acc, y, OQ_F16, M, N, qv, 0);
    oq_mm_dequant(acc, y, OQ_BF16, M, N, qv, 0);
    /* combine (enAtomic) */
    int32_t* c2 = malloc(sizeof(int32_t) * M * N);
    memcpy(c2, acc, sizeof(int32_t) * M * N);
    for (int op = 1; op <= 3; ++op) {
        oq_c_combine(c2, acc, OQ_INT32, op, M * N);
        oq_c_combine(y, y, OQ_F16, op, M * N);
    }
    /* MX matmul with E1M2 / E2M1 elements and a bias */
    uint8_t *pa = malloc(M * K / 2), *pb = malloc(N * K / 2), *sa = malloc(M * K / 32), *sb = malloc(N * K / 32);
    for (int i = 0; i < M * K / 2; ++i) pa[i] = (uint8_t)next();
    for (int i = 0; i < N * K / 2; ++i) pb[i] = (uint8_t)next();
    for (int i = 0; i < M * K / 32; ++i) sa[i] = (uint8_t)(120 + next() % 16);
    for (int i = 0; i < N * K / 32; ++i) sb[i] = (uint8_t)(120 + next() % 16);
    float* fb = malloc(4 * N);
    for (int i = 0; i < N; ++i) fb[i] = (float)(int32_t)(next() % 100) * 0.01f;
    double *ce = malloc(8 * M * N), *ca = malloc(8 * M * N);
    oq_mx_matmul(y, ce, ca, pa, pb, sa, sb, M, N, K, 1, 0, 1, OQ_FP4_E1M2 | (OQ_FP4_E2M1 << 8), NULL, 0, NULL, fb);
    /* group matmul with counts, including an empty group */
    int64_t gl[G] = {2, 0, 3};
    float *pts = malloc(4 * M), *gsc = malloc(4 * G * N);
    int8_t* gw = malloc(G * K * N);
    for (int i = 0; i < M; ++i) pts[i] = 0.01f;
    for (int i = 0; i < G * N; ++i) gsc[i] = 0.001f;
    for (int i = 0; i < G * K * N; ++i) gw[i] = (int8_t)next();
    oq_group_matmul(y, OQ_F16, a, pts, gw, 0, gsc, gl, 1, G, M, K, N, 1);
    for (int i = 0; i < M * N; ++i) sink += ce[i] + y[i];
    printf("ok %g\n", sink != 0.0 ? 1.0 : 0.0);
    free(a); free(b); free(acc); free(bias); free(y); free(qv); free(c2); free(pa); free(pb); free(sa); free(sb);
    free(fb); free(ce); free(ca); free(pts); free(gsc); free(gw);
    return 0;
}
