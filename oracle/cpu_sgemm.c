/* cpu_sgemm.c -- a cache-blocked f32 GEMM, the CPU baseline's matmul only.
 *
 * TEST INFRASTRUCTURE: bench.py's cpu_baseline leg times it beside the GPU
 * figures; nothing in the library calls it, and it is not a parity
 * reference (the oracle's nf4o_linear_f32 is, with Rust's unfused
 * arithmetic).
 *
 * The reference's burn ndarray backend runs its f32 matmul through the
 * matrixmultiply crate (0.3.x, a dependency of burn-ndarray, not vendored in
 * the reference), a blocked sgemm of the published Goto / BLIS scheme
 * (K. Goto and R. van de Geijn, "Anatomy of High-Performance Matrix
 * Multiplication", ACM TOMS 34(3), 2008): B packed into KC x NR column
 * panels, A into MR x KC row panels, one MR x NR tile of C held in
 * registers while the panels stream through the caches.  This is that
 * scheme in plain C with GCC vector types (8 floats, AVX2 + FMA): a 6 x 16
 * register tile, KC = 256, MC = 96, NC = 2048, the row blocks of A spread
 * over OpenMP threads.  Sums are fused (FMA) and taken in k order per tile,
 * as the crate's kernels do.
 *
 * Build: oracle/Makefile (its own object, -O3 -mavx2 -mfma).
 */
#include "nf4_oracle.h"

#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

typedef float v8 __attribute__((vector_size(32), aligned(32)));
typedef float v8u __attribute__((vector_size(32), aligned(4)));

enum { MR = 6, NR = 16, KC = 256, MC = 96, NC = 2048 };

static size_t min_sz(size_t a, size_t b) { return a < b ? a : b; }

/* B[pc .. pc + kc][jc .. jc + nc] into NR-column panels, k-major inside a
 * panel, zero-padded past nc. */
static void pack_b(const float *b, size_t ldb, size_t kc, size_t nc, float *bp) {
    const size_t panels = (nc + NR - 1) / NR;
#pragma omp parallel for schedule(static)
    for (size_t p = 0; p < panels; ++p) {
        const size_t j0 = p * NR, nr = min_sz(NR, nc - j0);
        float *dst = bp + p * kc * NR;
        for (size_t k = 0; k < kc; ++k) {
            const float *src = b + k * ldb + j0;
            size_t j = 0;
            for (; j < nr; ++j) dst[k * NR + j] = src[j];
            for (; j < NR; ++j) dst[k * NR + j] = 0.0f;
        }
    }
}

/* A[ic .. ic + mc][pc .. pc + kc] into MR-row panels, k-major inside a
 * panel, zero-padded past mc. */
static void pack_a(const float *a, size_t lda, size_t mc, size_t kc, float *ap) {
    for (size_t p = 0; p < (mc + MR - 1) / MR; ++p) {
        const size_t i0 = p * MR, mr = min_sz(MR, mc - i0);
        float *dst = ap + p * kc * MR;
        for (size_t k = 0; k < kc; ++k) {
            size_t i = 0;
            for (; i < mr; ++i) dst[k * MR + i] = a[(i0 + i) * lda + k];
            for (; i < MR; ++i) dst[k * MR + i] = 0.0f;
        }
    }
}

/* C[0 .. mr][0 .. nr] (+)= Ap Bp over kc: the register tile. */
static void tile(size_t kc, const float *ap, const float *bp, float *c, size_t ldc, size_t mr, size_t nr,
                 int accumulate) {
    v8 acc[MR][2];
    for (int i = 0; i < MR; ++i) acc[i][0] = acc[i][1] = (v8){0};
    for (size_t k = 0; k < kc; ++k) {
        const v8 b0 = *(const v8 *)(bp + k * NR), b1 = *(const v8 *)(bp + k * NR + 8);
        for (int i = 0; i < MR; ++i) {
            const float s = ap[k * MR + i];
            const v8 a = {s, s, s, s, s, s, s, s};
            acc[i][0] += a * b0;
            acc[i][1] += a * b1;
        }
    }
    if (mr == MR && nr == NR) {
        for (int i = 0; i < MR; ++i) {
            v8u *row = (v8u *)(c + i * ldc);
            if (accumulate) {
                row[0] += acc[i][0];
                row[1] += acc[i][1];
            } else {
                row[0] = acc[i][0];
                row[1] = acc[i][1];
            }
        }
        return;
    }
    for (size_t i = 0; i < mr; ++i)
        for (size_t j = 0; j < nr; ++j) {
            const float v = j < 8 ? acc[i][0][j] : acc[i][1][j - 8];
            c[i * ldc + j] = accumulate ? c[i * ldc + j] + v : v;
        }
}

int nf4o_sgemm_blocked(const float *a, size_t m, size_t k, const float *b, size_t n, float *c, int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    if (m == 0 || n == 0) return 0;
    if (k == 0) {
        memset(c, 0, m * n * sizeof(float));
        return 0;
    }
    float *bp = aligned_alloc(64, (size_t)KC * ((NC + NR - 1) / NR) * NR * sizeof(float));
    if (!bp) return -1;
    int failed = 0;
    for (size_t jc = 0; jc < n; jc += NC) {
        const size_t nc = min_sz(NC, n - jc);
        for (size_t pc = 0; pc < k; pc += KC) {
            const size_t kc = min_sz(KC, k - pc);
            pack_b(b + pc * n + jc, n, kc, nc, bp);
            const size_t blocks = (m + MC - 1) / MC;
#pragma omp parallel reduction(| : failed)
            {
                float *ap = aligned_alloc(64, (size_t)KC * MC * sizeof(float));
                if (!ap) failed = 1;
#pragma omp for schedule(dynamic)
                for (size_t blk = 0; blk < blocks; ++blk) {
                    if (!ap) continue;
                    const size_t ic = blk * MC, mc = min_sz(MC, m - ic);
                    pack_a(a + ic * k + pc, k, mc, kc, ap);
                    for (size_t jr = 0; jr < nc; jr += NR)
                        for (size_t ir = 0; ir < mc; ir += MR)
                            tile(kc, ap + (ir / MR) * kc * MR, bp + (jr / NR) * kc * NR, c + (ic + ir) * n + jc + jr, n,
                                 min_sz(MR, mc - ir), min_sz(NR, nc - jr), pc > 0);
                }
                free(ap);
            }
            if (failed) break;
        }
        if (failed) break;
    }
    free(bp);
    return failed ? -1 : 0;
}
