/*
 * The CPU baseline of the FP32 prefill projections — TEST INFRASTRUCTURE ONLY
 * (bench.py's cpu_baseline leg and tests/). A performance restatement of the
 * reference's AVX2 FP32 panel GEMM: panel::gemm / kernel_generic with MR = 6
 * rows x NR = 16 columns in twelve 8-lane FMA accumulators, rows packed
 * [group of 6][k][6] and weights [panel][k][16]
 * (src/kernels/panels/panel.rs:57-172), row blocks of 96 rows split across
 * threads with panel groups (src/kernels/panels/driver.rs:57-140). Every
 * output is one FMA chain over ascending k from +0.0, so the result is bit
 * for bit orc_panel_gemm's (tests/test_cpu_baseline.py checks it). Without
 * AVX2 + FMA it falls back to orc_panel_gemm.
 */
#include "focr_oracle.h"

#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#endif

#define MR 6
#define NRP 16
#define ROW_BLOCK 96

static inline float glu(float gate, float up) {
    float relu = gate > 0.0f ? gate : 0.0f;
    return (relu * relu) * up;
}

/* The epilogue of one row's panel slice (driver.rs:87-108): Store, Glu on
 * interleaved (gate, up) columns, or Add into the output. */
static inline void emit_panel(int epilogue, float *out, size_t n, size_t row, size_t col0, const float *c, size_t cols) {
    if (epilogue == ORC_GLU) {
        float *dst = out + row * (n / 2) + col0 / 2;
        for (size_t j = 0; j + 1 < cols; j += 2) dst[j / 2] = glu(c[j], c[j + 1]);
    } else if (epilogue == ORC_ADD) {
        float *dst = out + row * n + col0;
        for (size_t j = 0; j < cols; j++) dst[j] += c[j];
    } else {
        memcpy(out + row * n + col0, c, cols * sizeof(float));
    }
}

#if defined(__AVX2__) && defined(__FMA__)
/* One 6-row group of A' packed [k][6] (rows past the block zero) times one
 * packed panel [k][16]: kernel_avx2's twelve accumulators. */
static void micro(const float *ap, const float *bp, size_t k, float c[MR][NRP]) {
    __m256 acc[MR][2];
    for (int r = 0; r < MR; r++) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
    for (size_t kk = 0; kk < k; kk++) {
        const __m256 b0 = _mm256_loadu_ps(bp + kk * NRP), b1 = _mm256_loadu_ps(bp + kk * NRP + 8);
        const float *a = ap + kk * MR;
#define ROW(r)                                             \
    {                                                      \
        const __m256 x = _mm256_broadcast_ss(a + (r));     \
        acc[r][0] = _mm256_fmadd_ps(x, b0, acc[r][0]);     \
        acc[r][1] = _mm256_fmadd_ps(x, b1, acc[r][1]);     \
    }
        ROW(0) ROW(1) ROW(2) ROW(3) ROW(4) ROW(5)
#undef ROW
    }
    for (int r = 0; r < MR; r++) {
        _mm256_storeu_ps(c[r], acc[r][0]);
        _mm256_storeu_ps(c[r] + 8, acc[r][1]);
    }
}
#endif

void orc_panel_gemm_fast(const float *a, size_t m, size_t k, const float *w, size_t n, const float *row_scale,
                         int epilogue, float *out) {
#if defined(__AVX2__) && defined(__FMA__)
    if (m == 0 || n == 0) return;
    const size_t panels = (n + NRP - 1) / NRP;
    /* pack_panels: [n/16][k][16], a partial last panel zero-padded. */
    float *wp = (float *)aligned_alloc(64, ((panels * k * NRP * sizeof(float)) + 63) / 64 * 64);
#pragma omp parallel for schedule(static)
    for (long p = 0; p < (long)panels; p++)
        for (size_t kk = 0; kk < k; kk++)
            for (size_t j = 0; j < NRP; j++)
                wp[(p * k + kk) * NRP + j] = p * NRP + j < n ? w[(p * NRP + j) * k + kk] : 0.0f;
    const size_t blocks = (m + ROW_BLOCK - 1) / ROW_BLOCK;
    /* Two tasks per thread (driver.rs:81-86): panel groups when the rows are few. */
    int threads = 1;
#ifdef _OPENMP
    threads = omp_get_max_threads();
#endif
    size_t splits = 1;
    while (blocks * splits < (size_t)(2 * threads) && splits < panels) splits++;
    const size_t per_split = (panels + splits - 1) / splits;
#pragma omp parallel
    {
        /* The row block as F32Panels::pack_rows leaves it: [group][k][6]. */
        float *ar = (float *)malloc(ROW_BLOCK * (k ? k : 1) * sizeof(float));
        float c[MR][NRP];
#pragma omp for schedule(dynamic, 1)
        for (long task = 0; task < (long)(blocks * splits); task++) {
            const size_t blk = (size_t)task / splits, sp = (size_t)task % splits;
            const size_t p0 = sp * per_split, p1 = p0 + per_split < panels ? p0 + per_split : panels;
            const size_t r_begin = blk * ROW_BLOCK;
            const size_t r_end = r_begin + ROW_BLOCK < m ? r_begin + ROW_BLOCK : m;
            /* pack_rows for the block: A'[r][k] = a * row_scale[r], k-major in
             * groups of 6 rows, the last group zero-padded (panel.rs:77-104). */
            const size_t groups = (r_end - r_begin + MR - 1) / MR;
            for (size_t g = 0; g < groups; g++)
                for (int r = 0; r < MR; r++) {
                    const size_t row = r_begin + g * MR + (size_t)r;
                    float *dst = ar + g * k * MR + (size_t)r;
                    if (row < r_end)
                        for (size_t kk = 0; kk < k; kk++)
                            dst[kk * MR] = row_scale ? a[row * k + kk] * row_scale[row] : a[row * k + kk];
                    else
                        for (size_t kk = 0; kk < k; kk++) dst[kk * MR] = 0.0f;
                }
            /* Each panel stays in cache while every 6-row group of the block uses it. */
            for (size_t p = p0; p < p1; p++) {
                const size_t cols = n - p * NRP < NRP ? n - p * NRP : NRP;
                for (size_t g = 0; g < groups; g++) {
                    const size_t r0 = r_begin + g * MR;
                    const int rows = r_end - r0 < MR ? (int)(r_end - r0) : MR;
                    micro(ar + g * k * MR, wp + p * k * NRP, k, c);
                    for (int r = 0; r < rows; r++) emit_panel(epilogue, out, n, r0 + r, p * NRP, c[r], cols);
                }
            }
        }
        free(ar);
    }
    free(wp);
#else
    orc_panel_gemm(a, m, k, w, n, row_scale, epilogue, out);
#endif
}
