/*
 * The CPU baseline of the fast-mode prefill projection — TEST INFRASTRUCTURE
 * ONLY (bench.py's cpu_baseline legs and tests/). A performance restatement
 * of the reference's INT16-activation x INT8-code panels on AVX-512 VNNI:
 *  - weights packed once per matrix, as the reference does at load
 *    (panel_i16::pack / pack_exceptions, src/kernels/panels/panel_i16.rs:81-128):
 *    codes sign-extended to INT16 pairs [panel][k/2][32][2], scales
 *    [panel][k/64][32], exception weights [panel][columns][32];
 *  - per call, row blocks of 96 rows (48 when k > 1024) split with panel
 *    groups across threads (driver::tiled_gemm, src/kernels/panels/driver.rs:57-140);
 *  - each block packed as pack_rows leaves it (panel_i16.rs:275-329): per 6
 *    rows, code pairs [k/2][6], step bits [k/64][6], exception inputs
 *    [columns][6], the activations quantized by orc_i16_quantize_group;
 *  - one 6 x 32 tile per (row group, panel) by kernel_vnni (panel_i16.rs:378-424):
 *    per group INT32 vpdpwssd sums from zero, then
 *    acc = fma(f32(sum), s_w * s_a, acc); then the exception FMAs in
 *    ascending column order (exception_tile, panel_i16.rs:204-213) and the
 *    epilogue.
 * The integer sums are exact, so every output is bit for bit orc_i16_gemm's
 * (tests/test_cpu_baseline.py checks it). Without AVX-512 VNNI the GEMM
 * reports that it cannot run (return -1) and the caller skips the leg.
 */
#include "focr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <immintrin.h>

#define MR 6
#define NR 32
#define GROUP 64

struct orc_i16_panels {
    size_t n, k, groups, panels, n_exc;
    int16_t *codes; /* [panel][k/2][NR][2] */
    float *scales;  /* [panel][groups][NR] */
    int32_t *cols;  /* [n_exc] ascending */
    float *values;  /* [panel][n_exc][NR] */
};

orc_i16_panels *orc_i16_panels_pack(size_t n, size_t k, const int8_t *codes, const float *scales,
                                    const int32_t *exc_cols, const float *exc_vals, size_t n_exc) {
    if (n % NR != 0 || k % GROUP != 0 || n == 0 || k == 0) return NULL;
    orc_i16_panels *p = (orc_i16_panels *)calloc(1, sizeof *p);
    p->n = n;
    p->k = k;
    p->groups = k / GROUP;
    p->panels = n / NR;
    p->n_exc = n_exc;
    p->codes = (int16_t *)aligned_alloc(64, n * k * sizeof(int16_t));
    p->scales = (float *)aligned_alloc(64, (n * p->groups * sizeof(float) + 63) / 64 * 64);
    p->cols = (int32_t *)malloc((n_exc ? n_exc : 1) * sizeof(int32_t));
    p->values = (float *)malloc((n_exc ? n * n_exc : 1) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (long panel = 0; panel < (long)p->panels; panel++) {
        int16_t *dst = p->codes + (size_t)panel * NR * k;
        for (size_t kp = 0; kp < k / 2; kp++)
            for (size_t col = 0; col < NR; col++) {
                const int8_t *src = codes + ((size_t)panel * NR + col) * k;
                dst[(kp * NR + col) * 2] = src[2 * kp];
                dst[(kp * NR + col) * 2 + 1] = src[2 * kp + 1];
            }
        for (size_t col = 0; col < NR; col++)
            for (size_t g = 0; g < p->groups; g++)
                p->scales[((size_t)panel * p->groups + g) * NR + col] = scales[((size_t)panel * NR + col) * p->groups + g];
        for (size_t e = 0; e < n_exc; e++)
            for (size_t col = 0; col < NR; col++)
                p->values[((size_t)panel * n_exc + e) * NR + col] = exc_vals[((size_t)panel * NR + col) * n_exc + e];
    }
    if (n_exc) memcpy(p->cols, exc_cols, n_exc * sizeof(int32_t));
    return p;
}

void orc_i16_panels_free(orc_i16_panels *p) {
    if (!p) return;
    free(p->codes);
    free(p->scales);
    free(p->cols);
    free(p->values);
    free(p);
}

static inline float glu(float gate, float up) {
    float relu = gate > 0.0f ? gate : 0.0f;
    return (relu * relu) * up;
}

/* The epilogue of one row's panel slice (driver.rs:87-108). */
static inline void emit_row(int epilogue, float *out, size_t n, size_t row, size_t col0, const float *c) {
    if (epilogue == ORC_GLU) {
        float *dst = out + row * (n / 2) + col0 / 2;
        for (size_t j = 0; j < NR; j += 2) dst[j / 2] = glu(c[j], c[j + 1]);
    } else if (epilogue == ORC_ADD) {
        float *dst = out + row * n + col0;
        for (size_t j = 0; j < NR; j++) dst[j] += c[j];
    } else {
        memcpy(out + row * n + col0, c, NR * sizeof(float));
    }
}

/* kernel_vnni for NR = 32: `a` one packed 6-row group, `b` one panel's code
 * pairs, `sw` its scales; tile[r][j] the 6 x 32 outputs. */
__attribute__((target("avx512f,avx512vnni"))) static void kernel_vnni(size_t k, const int32_t *a, const int16_t *b,
                                                                      const float *sw, float tile[MR][NR]) {
    const float *sa = (const float *)(a + MR * (k / 2));
    __m512 acc[MR][2];
    for (int r = 0; r < MR; r++) acc[r][0] = acc[r][1] = _mm512_setzero_ps();
    for (size_t g = 0; g < k / GROUP; g++) {
        __m512i part[MR][2];
        for (int r = 0; r < MR; r++) part[r][0] = part[r][1] = _mm512_setzero_si512();
        for (size_t kp = g * (GROUP / 2); kp < (g + 1) * (GROUP / 2); kp++) {
            const int16_t *w = b + kp * 2 * NR;
            const __m512i w0 = _mm512_loadu_si512((const void *)w), w1 = _mm512_loadu_si512((const void *)(w + 32));
            const int32_t *x = a + kp * MR;
            for (int r = 0; r < MR; r++) {
                const __m512i xr = _mm512_set1_epi32(x[r]);
                part[r][0] = _mm512_dpwssd_epi32(part[r][0], xr, w0);
                part[r][1] = _mm512_dpwssd_epi32(part[r][1], xr, w1);
            }
        }
        const __m512 s0 = _mm512_loadu_ps(sw + g * NR), s1 = _mm512_loadu_ps(sw + g * NR + 16);
        for (int r = 0; r < MR; r++) {
            const __m512 s = _mm512_set1_ps(sa[g * MR + r]);
            acc[r][0] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(part[r][0]), _mm512_mul_ps(s0, s), acc[r][0]);
            acc[r][1] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(part[r][1]), _mm512_mul_ps(s1, s), acc[r][1]);
        }
    }
    for (int r = 0; r < MR; r++) {
        _mm512_storeu_ps(tile[r], acc[r][0]);
        _mm512_storeu_ps(tile[r] + 16, acc[r][1]);
    }
}

int orc_i16_gemm_fast(const orc_i16_panels *p, const float *a, size_t m, const float *row_scale, int epilogue,
                      float *out) {
    __builtin_cpu_init();
    if (!__builtin_cpu_supports("avx512f") || !__builtin_cpu_supports("avx512vnni")) return -1;
    if (!p) return -2;
    if (m == 0) return 0;
    const size_t k = p->k, n = p->n, groups = p->groups, n_exc = p->n_exc;
    const size_t block_rows = k <= 1024 ? 96 : 48;
    const size_t blocks = (m + block_rows - 1) / block_rows;
    int threads = 1;
#ifdef _OPENMP
    threads = omp_get_max_threads();
#endif
    /* Two units per thread (driver.rs:81-86). */
    size_t splits = (2 * (size_t)threads + blocks - 1) / blocks;
    if (splits < 1) splits = 1;
    if (splits > p->panels) splits = p->panels;
    const size_t per_split = (p->panels + splits - 1) / splits;
    const size_t group_len = MR * (k / 2 + groups + n_exc);
#pragma omp parallel
    {
        const size_t row_groups = (block_rows + MR - 1) / MR;
        int32_t *packed = (int32_t *)aligned_alloc(64, (row_groups * group_len * sizeof(int32_t) + 63) / 64 * 64);
        int16_t *q = (int16_t *)malloc(block_rows * k * sizeof(int16_t));
        float *steps = (float *)malloc(block_rows * groups * sizeof(float));
        float *xe = (float *)malloc((block_rows * n_exc + 1) * sizeof(float));
        float tile[MR][NR];
#pragma omp for schedule(dynamic, 1)
        for (long unit = 0; unit < (long)(blocks * splits); unit++) {
            const size_t block = (size_t)unit / splits, split = (size_t)unit % splits;
            const size_t row0 = block * block_rows;
            const size_t rows = block_rows < m - row0 ? block_rows : m - row0;
            const size_t padded = (rows + MR - 1) / MR * MR;
            /* pack_rows: the quantized codes, steps (times the row scale) and
             * exception inputs of the block's rows, in the 6-row layout. */
            orc_i16_quantize_rows(a + row0 * k, rows, k, p->cols, n_exc, row_scale ? row_scale + row0 : NULL, q,
                                  steps, xe);
            for (size_t g6 = 0; g6 < padded / MR; g6++) {
                int32_t *dst = packed + g6 * group_len;
                for (int r = 0; r < MR; r++) {
                    const size_t row = g6 * MR + (size_t)r;
                    const int live = row < rows;
                    for (size_t kp = 0; kp < k / 2; kp++) {
                        const uint32_t lo = live ? (uint16_t)q[row * k + 2 * kp] : 0u;
                        const uint32_t hi = live ? (uint16_t)q[row * k + 2 * kp + 1] : 0u;
                        dst[kp * MR + (size_t)r] = (int32_t)(lo | hi << 16);
                    }
                    for (size_t g = 0; g < groups; g++) {
                        const float s = live ? steps[row * groups + g] : 0.0f;
                        memcpy(&dst[MR * (k / 2) + g * MR + (size_t)r], &s, 4);
                    }
                    for (size_t e = 0; e < n_exc; e++) {
                        const float x = live ? xe[row * n_exc + e] : 0.0f;
                        memcpy(&dst[MR * (k / 2 + groups) + e * MR + (size_t)r], &x, 4);
                    }
                }
            }
            const size_t first = split * per_split;
            const size_t last = first + per_split < p->panels ? first + per_split : p->panels;
            for (size_t panel = first; panel < last; panel++) {
                const int16_t *b = p->codes + panel * NR * k;
                const float *sw = p->scales + panel * groups * NR;
                for (size_t g6 = 0; g6 < padded / MR; g6++) {
                    const int32_t *ap = packed + g6 * group_len;
                    kernel_vnni(k, ap, b, sw, tile);
                    if (n_exc) {
                        /* exception_tile: ascending columns, one FMA each. */
                        const int32_t *inputs = ap + MR * (k / 2 + groups);
                        const float *values = p->values + panel * n_exc * NR;
                        for (size_t e = 0; e < n_exc; e++)
                            for (int r = 0; r < MR; r++) {
                                float x;
                                memcpy(&x, &inputs[e * MR + (size_t)r], 4);
                                for (size_t j = 0; j < NR; j++) tile[r][j] = fmaf(x, values[e * NR + j], tile[r][j]);
                            }
                    }
                    const size_t valid = MR < rows - g6 * MR ? MR : rows - g6 * MR;
                    for (size_t r = 0; r < valid; r++) emit_row(epilogue, out, n, row0 + g6 * MR + r, panel * NR, tile[r]);
                }
            }
        }
        free(packed);
        free(q);
        free(steps);
        free(xe);
    }
    return 0;
}
