/*
 * Strided f32 GEMM for the attention oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * Semantics restate gemm_strided, crates/core/src/matmul.rs:37-98:
 *   C[m,n] (+)= A[m,k] . B[k,n] over arbitrary non-negative strides;
 *   m==0 or n==0 is a no-op; k==0 zeroes C unless acc; acc=0 overwrites.
 * The full k-sum of each element is formed first and then added to C (the
 * order the reference's `gemm` call uses with read_dst=acc, alpha=beta=1).
 *
 * Arithmetic: packed panels, a 4x16 register block the compiler vectorises,
 * FMA allowed (the reference's SIMD kernels fuse too; their exact summation
 * order is unpinned), and OpenMP threads over C tiles -- the counterpart of
 * `Parallelism::Rayon(0)` (matmul.rs:95), i.e. all host threads.
 */
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

enum { MC = 64, NC = 128, KC = 256, MR = 4, NR = 16 };

int orc_gemm_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Threads the GEMM uses from now on (n >= 1); for timing the single-core
 * baseline beside the all-cores one. */
void orc_set_gemm_threads(int n) {
#ifdef _OPENMP
    if (n >= 1) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

static void tile(const float* a, long a_rs, long a_cs, const float* b, long b_rs, long b_cs, float* c, long c_rs,
                 long c_cs, size_t i0, size_t mb, size_t j0, size_t nb, size_t k, int acc, float* ap, float* bp,
                 float* tmp) {
    const size_t mbp = (mb + MR - 1) / MR * MR, nbp = (nb + NR - 1) / NR * NR;
    memset(tmp, 0, sizeof(float) * MC * NC);
    for (size_t k0 = 0; k0 < k; k0 += KC) {
        size_t kb = k - k0 < KC ? k - k0 : KC;
        for (size_t i = 0; i < mbp; i++)
            for (size_t kk = 0; kk < kb; kk++)
                ap[i * KC + kk] = i < mb ? a[(long)(i0 + i) * a_rs + (long)(k0 + kk) * a_cs] : 0.0f;
        for (size_t kk = 0; kk < kb; kk++)
            for (size_t j = 0; j < nbp; j++)
                bp[kk * NC + j] = j < nb ? b[(long)(k0 + kk) * b_rs + (long)(j0 + j) * b_cs] : 0.0f;
        for (size_t i = 0; i < mbp; i += MR) {
            for (size_t j = 0; j < nbp; j += NR) {
                float r[MR][NR];
                for (int ii = 0; ii < MR; ii++)
                    for (int jj = 0; jj < NR; jj++) r[ii][jj] = tmp[(i + ii) * NC + j + jj];
                for (size_t kk = 0; kk < kb; kk++) {
                    const float* brow = bp + kk * NC + j;
                    for (int ii = 0; ii < MR; ii++) {
                        float av = ap[(i + ii) * KC + kk];
                        for (int jj = 0; jj < NR; jj++) r[ii][jj] += av * brow[jj];
                    }
                }
                for (int ii = 0; ii < MR; ii++)
                    for (int jj = 0; jj < NR; jj++) tmp[(i + ii) * NC + j + jj] = r[ii][jj];
            }
        }
    }
    for (size_t i = 0; i < mb; i++)
        for (size_t j = 0; j < nb; j++) {
            float* cp = c + (long)(i0 + i) * c_rs + (long)(j0 + j) * c_cs;
            *cp = acc ? *cp + tmp[i * NC + j] : tmp[i * NC + j];
        }
}

void orc_gemm_strided(const float* a, long a_rs, long a_cs, const float* b, long b_rs, long b_cs, float* c,
                      long c_rs, long c_cs, size_t m, size_t k, size_t n, int acc) {
    if (m == 0 || n == 0) return;
    if (k == 0) {
        if (!acc)
            for (size_t i = 0; i < m; i++)
                for (size_t j = 0; j < n; j++) c[(long)i * c_rs + (long)j * c_cs] = 0.0f;
        return;
    }
    const size_t mt = (m + MC - 1) / MC, nt = (n + NC - 1) / NC;
    const size_t tiles = mt * nt;
    const int par = (double)m * (double)n * (double)k > 65536.0 && tiles > 1;
#pragma omp parallel if (par)
    {
        float* ap = (float*)malloc(sizeof(float) * MC * KC);
        float* bp = (float*)malloc(sizeof(float) * KC * NC);
        float* tmp = (float*)malloc(sizeof(float) * MC * NC);
#pragma omp for schedule(dynamic, 1)
        for (size_t t = 0; t < tiles; t++) {
            size_t ib = t / nt, jb = t % nt;
            size_t i0 = ib * MC, j0 = jb * NC;
            size_t mb = m - i0 < MC ? m - i0 : MC, nb = n - j0 < NC ? n - j0 : NC;
            tile(a, a_rs, a_cs, b, b_rs, b_cs, c, c_rs, c_cs, i0, mb, j0, nb, k, acc, ap, bp, tmp);
        }
        free(ap);
        free(bp);
        free(tmp);
    }
}
