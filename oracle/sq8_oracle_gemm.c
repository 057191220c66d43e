/*
 * sq8_oracle_gemm.c — the reference's CPU product route, restated: the activation widened from
 * bf16 (exact), the weight already widened to fp32 `[K, N]` (orc_dequantize), fp32 sums
 * (Sources/Siliconed/WeightProducts.swift:698-709 calls cblas_sgemm on exactly these operands),
 * then bias and the epilogue in fp32 (orc_epilogue_f32). TEST INFRASTRUCTURE ONLY.
 *
 * A plain cache-blocked GEMM: each thread owns a tile of C (64 rows × 256 columns) and walks K in
 * blocks of 256, so a 256 × 256 block of W (256 KB) stays in L2 while the rows stream over it.
 * Compiled apart from sq8_oracle.c with fp contraction allowed, as a BLAS would contract.
 */
#include "sq8_oracle.h"

#include <stdlib.h>
#include <string.h>

void orc_linear_f32(const uint16_t *a, int64_t lda, const float *w_kn, int64_t ldw, int m, int k,
                    int n, const float *bias, int epilogue, float *c, int64_t ldc, int threads) {
    const int MB = 64, NB = 256, KB = 256;
    int glu = epilogue == ORC_EPI_SILU_GLU || epilogue == ORC_EPI_SITU_GLU;
    float *p = c;
    int64_t ldp = ldc;
    if (glu || epilogue != ORC_EPI_NONE || bias) {
        p = (float *)malloc((size_t)m * n * sizeof(float));
        ldp = n;
    }
    int mblocks = (m + MB - 1) / MB, nblocks = (n + NB - 1) / NB;
    int nthreads = threads > 0 ? threads : 1;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(nthreads)
    for (int bi = 0; bi < mblocks; ++bi) {
        for (int bj = 0; bj < nblocks; ++bj) {
            int i0 = bi * MB, i1 = i0 + MB < m ? i0 + MB : m;
            int j0 = bj * NB, j1 = j0 + NB < n ? j0 + NB : n;
            float arow[256];
            for (int i = i0; i < i1; ++i) memset(p + (int64_t)i * ldp + j0, 0, (size_t)(j1 - j0) * sizeof(float));
            for (int k0 = 0; k0 < k; k0 += KB) {
                int k1 = k0 + KB < k ? k0 + KB : k;
                for (int i = i0; i < i1; ++i) {
                    const uint16_t *ar = a + (int64_t)i * lda;
                    for (int kk = k0; kk < k1; ++kk) {
                        uint32_t u = (uint32_t)ar[kk] << 16;
                        memcpy(&arow[kk - k0], &u, 4);
                    }
                    float *pr = p + (int64_t)i * ldp;
                    for (int kk = k0; kk < k1; ++kk) {
                        const float av = arow[kk - k0];
                        const float *wr = w_kn + (int64_t)kk * ldw;
                        for (int j = j0; j < j1; ++j) pr[j] += av * wr[j];
                    }
                }
            }
        }
    }
    if (p != c) {
        orc_epilogue_f32(p, ldp, m, n, bias, epilogue, c, ldc, nthreads);
        free(p);
    }
}
