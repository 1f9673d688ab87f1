/*
 * CPU oracle for the Falcon-OCR hot path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference operators (amazingvince/falcon-ocr-cpu,
 * Rust) that the HIP library is checked against and that bench.py times as the
 * CPU baseline. The product never links, loads or calls this file.
 *
 * Compile with -ffp-contract=off (oracle/Makefile): every fused multiply-add
 * below is an explicit fmaf(); every other product and sum rounds on its own,
 * as Rust's `*` and `+` do. Loops are written so that gcc can vectorize them
 * without changing any per-element operation sequence; OpenMP splits only
 * independent outputs, so results never depend on the thread count.
 *
 * Parity status of each function (pinning checks live in tests/):
 *  - orc_quantize_bits, orc_dequantize, orc_validate_w8: pinned (RTN KAT,
 *    closed form, validation rules).
 *  - orc_dot, orc_dot_q, orc_linear_decode(_glu): pinned (FP32 linear KAT,
 *    multi-row == single-row, quantized == FP32 dot on dequantized weights,
 *    f64 bound, tree order checked against a brute-force restatement).
 *  - orc_rms_scale: pinned (closed form for constant rows, f64 bound, tree
 *    structure on powers of two).
 *  - orc_panel_gemm: pinned (FP32 linear KAT, f64 bound k*eps*sum|aw|,
 *    Glu/Add/row-scale identities).
 *  - orc_i16_quantize_group, orc_i16_gemm: pinned (quantizer KATs, exact
 *    integer group sums vs int64 brute force, error bound vs f64).
 *  - orc_attention_prefill: main-path tiles pinned by f64 attention bound and
 *    by the tile-independence identities; the reference's short "gemm crate"
 *    tiles (q*k <= 256, k < 3 or q < 2) are parity unpinned bitwise (the
 *    gemm crate 0.19.0 order is not available here) and pinned to tolerance.
 *  - orc_attention_prefill_bf16_tiles: pinned by the reference's f64 bound on
 *    BF16-rounded operands (bf16.rs matches_bf16_operand_reference: |d| <=
 *    3 * 2^-9 + 2e-3), the static variant's exp2 polynomial by its scalar
 *    restatement and 7.6e-5 bound, and hand checks of the BF16 rounding and
 *    the vdpbf16ps pair order; short online tiles as for orc_attention_prefill.
 *  - orc_argmax: pinned (KAT).
 */
#include "focr_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int threads) {
    g_threads = threads < 1 ? 1 : threads;
#ifdef _OPENMP
    omp_set_num_threads(g_threads);
#endif
}

int orc_get_threads(void) { return g_threads; }

static inline uint32_t f2u(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* ---- exp --------------------------------------------------------------- */
/* Cephes expf constants, src/kernels/exp.rs:259-277. */
#define EXP_MIN (-87.0f)
#define EXP_MAX 88.376f
#define EXP_LOG2E 1.44269504088896340735992468100189214f /* f32::consts::LOG2_E */
#define EXP_LN2_HI 0.6933594f
#define EXP_LN2_LO (-2.1219444e-4f)
/* The reference's literals, digit for digit (exp.rs:268-277). */
static const float EXP_P[6] = {1.9875691e-4f, 1.3981999e-3f, 8.333452e-3f,
                               4.1665796e-2f, 0.16666665f, 0.5f};

/* exp_poly_unchecked, src/kernels/exp.rs:248-257. */
float orc_exp_poly_unchecked(float x) {
    float n = rintf(x * EXP_LOG2E); /* round_ties_even under the default mode */
    float r = fmaf(n, -EXP_LN2_HI, x);
    r = fmaf(n, -EXP_LN2_LO, r);
    float p = EXP_P[0];
    for (int i = 1; i < 6; i++) p = fmaf(p, r, EXP_P[i]);
    float y = fmaf(p, r * r, r) + 1.0f;
    return y * u2f((uint32_t)((int32_t)n + 127) << 23);
}

/* exp_poly, src/kernels/exp.rs:232-245. */
float orc_exp_poly(float x) {
    if (isnan(x)) return x;
    if (x < EXP_MIN) return 0.0f;
    if (x > EXP_MAX) return INFINITY;
    return orc_exp_poly_unchecked(x);
}

/* squared_relu_glu, src/kernels/mod.rs:567-572: NaN or nonpositive gate -> 0. */
float orc_squared_relu_glu(float gate, float up) {
    float relu = gate > 0.0f ? gate : 0.0f;
    return (relu * relu) * up;
}

/* ---- A1 ---------------------------------------------------------------- */
int orc_quantize_bits(const float *w, size_t n, size_t k, size_t group, int bits,
                      void *codes_out, float *scales_out) {
    if (bits != 8 && bits != 16) return -1;
    const double qmax = bits == 8 ? 127.0 : 32767.0;
    if (n == 0 || k == 0 || (group != 32 && group != 64 && group != 128)) return -2;
    for (size_t i = 0; i < n * k; i++)
        if (!isfinite(w[i])) return -3;
    size_t groups = (k + group - 1) / group;
    for (size_t row = 0; row < n; row++) {
        for (size_t g = 0; g < groups; g++) {
            size_t start = g * group, end = start + group < k ? start + group : k;
            const float *values = w + row * k + start;
            float maximum = 0.0f; /* fold(0, |a, b| a.max(b.abs())) */
            for (size_t i = 0; i < end - start; i++) maximum = fmaxf(maximum, fabsf(values[i]));
            float scale;
            if (maximum == 0.0f) {
                scale = 0.0f;
            } else {
                scale = (float)((double)maximum / qmax);
                scale = fmaxf(scale, u2f(1)); /* .max(f32::from_bits(1)) */
            }
            scales_out[row * groups + g] = scale;
            for (size_t i = 0; i < end - start; i++) {
                int32_t code = 0;
                if (scale != 0.0f) {
                    double v = nearbyint((double)values[i] / (double)scale); /* ties even */
                    if (v < -qmax) v = -qmax;
                    if (v > qmax) v = qmax;
                    code = (int32_t)v;
                }
                if (!isfinite((float)code * scale)) return -4;
                if (bits == 8)
                    ((int8_t *)codes_out)[row * k + start + i] = (int8_t)code;
                else
                    ((int16_t *)codes_out)[row * k + start + i] = (int16_t)code;
            }
        }
    }
    return 0;
}

static inline float code_at(int bits, const void *codes, size_t index) {
    if (bits == 8) return (float)((const int8_t *)codes)[index];
    if (bits == 16) return (float)((const int16_t *)codes)[index];
    return ((const float *)codes)[index];
}

void orc_dequantize(int bits, const void *codes, const float *scales, size_t n, size_t k,
                    size_t group, const int32_t *exc_cols, const float *exc_vals, size_t n_exc,
                    float *out) {
    size_t groups = (k + group - 1) / group;
    for (size_t row = 0; row < n; row++) {
        for (size_t i = 0; i < k; i++)
            out[row * k + i] = code_at(bits, codes, row * k + i) * scales[row * groups + i / group];
        for (size_t e = 0; e < n_exc; e++) out[row * k + (size_t)exc_cols[e]] = exc_vals[row * n_exc + e];
    }
}

int orc_validate_w8(size_t n, size_t k, size_t group, const int8_t *codes, const float *scales) {
    if (!(n > 0 && k > 0 && (group == 32 || group == 64))) return -1;
    size_t groups = (k + group - 1) / group;
    for (size_t i = 0; i < n * k; i++)
        if (codes[i] == -128) return -2;
    for (size_t i = 0; i < n * groups; i++) {
        float s = scales[i];
        if (!(isfinite(s) && s >= 0.0f && isfinite(127.0f * s))) return -3;
    }
    for (size_t row = 0; row < n; row++)
        for (size_t g = 0; g < groups; g++)
            if (scales[row * groups + g] == 0.0f) {
                size_t a = row * k + g * group, b = a + group < (row + 1) * k ? a + group : (row + 1) * k;
                for (size_t i = a; i < b; i++)
                    if (codes[i] != 0) return -4;
            }
    return 0;
}

/* ---- A4 / A5 ----------------------------------------------------------- */
/* Portable::sum / Avx2::sum tree, src/simd.rs:260-262,366-373. */
static inline float tree8(const float v[8]) {
    return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

/* dot_q with an optional scale table; bits 32 is simd::dot (src/simd.rs:749-777). */
static float dot_any(int bits, const float *x, const void *codes, size_t base, const float *scales,
                     size_t len, size_t group) {
    float ph[32];
    for (int p = 0; p < 32; p++) ph[p] = 0.0f;
    size_t i = 0;
    for (; i + 32 <= len; i += 32) {
        float s = bits == 32 ? 1.0f : scales[i / group];
        for (int p = 0; p < 32; p++) {
            float w = bits == 32 ? code_at(32, codes, base + i + p) : code_at(bits, codes, base + i + p) * s;
            ph[p] = fmaf(x[i + p], w, ph[p]);
        }
    }
    float acc[8];
    for (int l = 0; l < 8; l++) acc[l] = (ph[l] + ph[8 + l]) + (ph[16 + l] + ph[24 + l]);
    for (; i + 8 <= len; i += 8) {
        float s = bits == 32 ? 1.0f : scales[i / group];
        for (int l = 0; l < 8; l++) {
            float w = bits == 32 ? code_at(32, codes, base + i + l) : code_at(bits, codes, base + i + l) * s;
            acc[l] = fmaf(x[i + l], w, acc[l]);
        }
    }
    float total = tree8(acc);
    for (; i < len; i++) {
        float w = bits == 32 ? code_at(32, codes, base + i) : code_at(bits, codes, base + i) * scales[i / group];
        total += x[i] * w;
    }
    return total;
}

float orc_dot(const float *a, const float *b, size_t len) { return dot_any(32, a, b, 0, NULL, len, 32); }

float orc_dot_q(int bits, const float *x, const void *codes, const float *scales, size_t len,
                size_t group) {
    return dot_any(bits, x, codes, 0, scales, len, group);
}

/* row_dot: dot then Exceptions::accumulate (src/quant/linear.rs:766-779,84-118). */
static float row_dot(int bits, const void *codes, const float *scales, size_t k, size_t group,
                     const int32_t *exc_cols, const float *exc_vals, size_t n_exc, const float *x,
                     size_t channel) {
    size_t groups = (k + group - 1) / group;
    float value = dot_any(bits, x, codes, channel * k, bits == 32 ? NULL : scales + channel * groups, k, group);
    for (size_t e = 0; e < n_exc; e++) value = fmaf(x[exc_cols[e]], exc_vals[channel * n_exc + e], value);
    return value;
}

void orc_linear_decode(int bits, const void *codes, const float *scales, size_t n, size_t k,
                       size_t group, const int32_t *exc_cols, const float *exc_vals, size_t n_exc,
                       const float *x, size_t rows, float *out) {
    if (k == 0) { /* linear_with_simd: in_dim == 0 fills zeros (src/kernels/mod.rs:403-406) */
        for (size_t i = 0; i < rows * n; i++) out[i] = 0.0f;
        return;
    }
#pragma omp parallel for schedule(static)
    for (long c = 0; c < (long)n; c++)
        for (size_t r = 0; r < rows; r++)
            out[r * n + c] = row_dot(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x + r * k, c);
}

void orc_linear_decode_glu(int bits, const void *codes, const float *scales, size_t n, size_t k,
                           size_t group, const int32_t *exc_cols, const float *exc_vals,
                           size_t n_exc, const float *x, size_t rows, float *gated) {
    size_t ffn = n / 2;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < (long)ffn; i++)
        for (size_t r = 0; r < rows; r++) {
            float gate = row_dot(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x + r * k, 2 * i);
            float up = row_dot(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x + r * k, 2 * i + 1);
            gated[r * ffn + i] = orc_squared_relu_glu(gate, up);
        }
}

/* ---- A6 ---------------------------------------------------------------- */
/* sum_squares_pairwise, src/kernels/mod.rs:535-553. */
static float sum_squares_pairwise(const float *x, size_t len) {
    if (len > 32) {
        size_t middle = ((len / 2 + 31) / 32) * 32; /* (len/2).next_multiple_of(32) */
        return sum_squares_pairwise(x, middle) + sum_squares_pairwise(x + middle, len - middle);
    }
    float partial[32];
    for (int i = 0; i < 32; i++) partial[i] = 0.0f;
    for (size_t i = 0; i < len; i++) partial[i] = x[i] * x[i];
    for (int width = 16; width >= 1; width /= 2)
        for (int index = 0; index < width; index++) partial[index] += partial[index + width];
    return partial[0];
}

float orc_rms_scale(const float *row, size_t width, float eps) {
    return 1.0f / sqrtf(sum_squares_pairwise(row, width) / (float)width + eps);
}

void orc_row_scales(const float *h, size_t rows, size_t width, float eps, float *out) {
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; r++) out[r] = orc_rms_scale(h + r * width, width, eps);
}

/* ---- epilogues ----------------------------------------------------------- */
/* driver::tiled_gemm's store closure, src/kernels/panels/driver.rs:87-108. */
static inline void store_row(int epilogue, float *out, size_t n, size_t row, const float *c) {
    if (epilogue == ORC_GLU) {
        float *dst = out + row * (n / 2);
        for (size_t i = 0; i < n / 2; i++) dst[i] = orc_squared_relu_glu(c[2 * i], c[2 * i + 1]);
    } else if (epilogue == ORC_ADD) {
        float *dst = out + row * n;
        for (size_t j = 0; j < n; j++) dst[j] += c[j];
    } else {
        memcpy(out + row * n, c, n * sizeof(float));
    }
}

/* ---- A2 ------------------------------------------------------------------ */
#define NR 16
void orc_panel_gemm(const float *a, size_t m, size_t k, const float *w, size_t n,
                    const float *row_scale, int epilogue, float *out) {
    if (m == 0 || n == 0) return;
    size_t panels = (n + NR - 1) / NR;
    /* Panels [n/16][k][16] as pack_panels writes them (panel.rs:57-71); a
     * partial last panel is zero-padded (its columns are never stored). */
    float *wp = (float *)calloc(panels * k * NR, sizeof(float));
#pragma omp parallel for schedule(static)
    for (long p = 0; p < (long)panels; p++)
        for (size_t j = 0; j < NR && p * NR + j < n; j++)
            for (size_t kk = 0; kk < k; kk++) wp[(p * k + kk) * NR + j] = w[(p * NR + j) * k + kk];
#pragma omp parallel
    {
        float *ar = (float *)malloc((k ? k : 1) * sizeof(float));
        float *crow = (float *)malloc(n * sizeof(float));
#pragma omp for schedule(dynamic, 4)
        for (long r = 0; r < (long)m; r++) {
            /* pack_rows: A'[r][k] = a * row_scale[r] (panel.rs:79-106). */
            for (size_t kk = 0; kk < k; kk++) ar[kk] = row_scale ? a[r * k + kk] * row_scale[r] : a[r * k + kk];
            for (size_t p = 0; p < panels; p++) {
                float c[NR];
                for (int j = 0; j < NR; j++) c[j] = 0.0f;
                const float *b = wp + p * k * NR;
                for (size_t kk = 0; kk < k; kk++) {
                    float x = ar[kk];
                    for (int j = 0; j < NR; j++) c[j] = fmaf(x, b[kk * NR + j], c[j]);
                }
                for (int j = 0; j < NR && p * NR + j < n; j++) crow[p * NR + j] = c[j];
            }
            store_row(epilogue, out, n, r, crow);
        }
        free(ar);
        free(crow);
    }
    free(wp);
}

/* ---- A3 ------------------------------------------------------------------ */
#define QMAX 32767.0f
#define MAGIC 12582912.0f /* 1.5 * 2^23 */

float orc_i16_quantize_group(const float *x, int16_t *q) {
    uint32_t top = 0;
    for (int i = 0; i < 64; i++) {
        uint32_t b = f2u(x[i]) & 0x7fffffffu;
        if (b > top) top = b;
    }
    if (top >= 0x7f800000u) {
        for (int i = 0; i < 64; i++) q[i] = 0;
        return NAN;
    }
    float absmax = u2f(top);
    float inv = QMAX / absmax;
    if (!isfinite(inv)) {
        if (absmax == 0.0f) {
            for (int i = 0; i < 64; i++) q[i] = 0;
            return 0.0f;
        }
        float step = fmaxf(absmax / QMAX, u2f(1));
        if ((double)step * (double)QMAX < (double)absmax) step = u2f(f2u(step) + 1);
        for (int i = 0; i < 64; i++) {
            double v = nearbyint((double)x[i] / (double)step);
            if (v < -32767.0) v = -32767.0;
            if (v > 32767.0) v = 32767.0;
            q[i] = (int16_t)v;
        }
        return step;
    }
    for (int i = 0; i < 64; i++) {
        float y = x[i] * inv;
        if (y < -QMAX) y = -QMAX;
        if (y > QMAX) y = QMAX;
        float t = y + MAGIC;
        q[i] = (int16_t)((int32_t)f2u(t) - (int32_t)f2u(MAGIC));
    }
    return absmax / QMAX;
}

void orc_i16_quantize_rows(const float *a, size_t m, size_t k, const int32_t *exc_cols,
                           size_t n_exc, const float *row_scale, int16_t *codes, float *steps,
                           float *exc_inputs) {
    size_t groups = k / 64;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)m; r++) {
        const float *src = a + r * k;
        float scale = row_scale ? row_scale[r] : 1.0f;
        size_t column = 0;
        for (size_t g = 0; g < groups; g++) {
            float zeroed[64];
            memcpy(zeroed, src + g * 64, sizeof zeroed);
            while (column < n_exc && (size_t)exc_cols[column] < (g + 1) * 64) {
                zeroed[exc_cols[column] % 64] = 0.0f;
                column++;
            }
            float step = orc_i16_quantize_group(zeroed, codes + r * k + g * 64);
            steps[r * groups + g] = step * scale;
        }
        for (size_t e = 0; e < n_exc; e++) exc_inputs[r * n_exc + e] = src[exc_cols[e]] * scale;
    }
}

void orc_i16_gemm(const float *a, size_t m, size_t k, const int8_t *codes, const float *scales,
                  size_t n, const int32_t *exc_cols, const float *exc_vals, size_t n_exc,
                  const float *row_scale, int epilogue, float *out) {
    if (m == 0 || n == 0) return;
    size_t groups = k / 64;
    int16_t *q = (int16_t *)malloc(m * k * sizeof(int16_t));
    float *sa = (float *)malloc((m * groups + 1) * sizeof(float));
    float *xe = (float *)malloc((m * n_exc + 1) * sizeof(float));
    orc_i16_quantize_rows(a, m, k, exc_cols, n_exc, row_scale, q, sa, xe);
#pragma omp parallel
    {
        float *crow = (float *)malloc(n * sizeof(float));
#pragma omp for schedule(dynamic, 4)
        for (long r = 0; r < (long)m; r++) {
            const int16_t *qr = q + r * k;
            for (size_t j = 0; j < n; j++) {
                const int8_t *wr = codes + j * k;
                float acc = 0.0f;
                for (size_t g = 0; g < groups; g++) {
                    int32_t sum = 0;
                    for (size_t kk = g * 64; kk < (g + 1) * 64; kk++) sum += (int32_t)qr[kk] * (int32_t)wr[kk];
                    float s = scales[j * groups + g] * sa[r * groups + g];
                    acc = fmaf((float)sum, s, acc);
                }
                for (size_t e = 0; e < n_exc; e++) acc = fmaf(xe[r * n_exc + e], exc_vals[j * n_exc + e], acc);
                crow[j] = acc;
            }
            store_row(epilogue, out, n, r, crow);
        }
        free(crow);
    }
    free(q);
    free(sa);
    free(xe);
}

/* ---- A7 ------------------------------------------------------------------ */
#define QT 32
#define KT 128
#define HD 64

typedef struct {
    const float *prefix_k, *generated_k, *v;
    size_t prefix_len, total_len, n_heads, n_kv_heads;
} Cache;

/* CompactKv::key / value, src/kernels/attention/mod.rs:133-151. */
static inline const float *cache_key(const Cache *c, size_t position, size_t head) {
    if (position < c->prefix_len) return c->prefix_k + (position * c->n_heads + head) * HD;
    size_t repeat = c->n_heads / c->n_kv_heads;
    return c->generated_k + ((position - c->prefix_len) * c->n_kv_heads + head / repeat) * HD;
}
static inline const float *cache_value(const Cache *c, size_t position, size_t kv_head) {
    return c->v + (position * c->n_kv_heads + kv_head) * HD;
}

typedef float (*ExpFn)(float);
static float platform_exp(float x) { return expf(x); }

static inline int masked(size_t absolute, size_t key, size_t image_start, size_t image_end) {
    int image_query = absolute >= image_start && absolute < image_end;
    return key > absolute && !(image_query && key >= image_start && key < image_end);
}

/* One (query tile, head): tile_head (prefill64.rs:328-480). */
static void tile_head(const float *q, const Cache *cache, size_t query_offset, size_t image_start,
                      size_t image_end, size_t tile, size_t queries, size_t head, const float *sinks,
                      int is_static, ExpFn exp_fn, float *output) {
    const size_t qw = cache->n_heads * HD;
    const size_t kv_head = head / (cache->n_heads / cache->n_kv_heads);
    const float scale = 1.0f / sqrtf((float)HD);
    size_t first_query = tile * QT;
    /* tile_span, prefill64/span.rs:9-20 */
    size_t first_absolute = query_offset + first_query;
    size_t last_absolute = first_absolute + queries - 1;
    int intersects = first_absolute < image_end && last_absolute >= image_start;
    size_t visible_end = intersects ? (last_absolute + 1 > image_end ? last_absolute + 1 : image_end) : last_absolute + 1;
    int all_image = first_absolute >= image_start && last_absolute < image_end;

    float qt[HD][QT];
    memset(qt, 0, sizeof qt);
    for (size_t r = 0; r < queries; r++)
        for (size_t d = 0; d < HD; d++) qt[d][r] = q[(first_query + r) * qw + head * HD + d];
    float maxima[QT], den[QT];
    for (int r = 0; r < QT; r++) {
        maxima[r] = -INFINITY;
        den[r] = 0.0f;
    }
    float out[QT][HD];
    memset(out, 0, sizeof out);
    static __thread float st[KT][QT];
    const float *krow[KT], *vrow[KT];

    for (size_t key_start = 0; key_start < visible_end; key_start += KT) {
        size_t keys = visible_end - key_start < KT ? visible_end - key_start : KT;
        for (size_t j = 0; j < keys; j++) {
            krow[j] = cache_key(cache, key_start + j, head);
            vrow[j] = cache_value(cache, key_start + j, kv_head);
        }
        int main_path = queries * keys > 256 && keys >= 3 && queries >= 2;
        if (is_static || main_path) {
            /* qk_lanes/qk_keys (487-545): FMA chain over d from +0, then scale*acc. */
            for (size_t j = 0; j < keys; j++) {
                float acc[QT];
                for (int r = 0; r < QT; r++) acc[r] = 0.0f;
                for (int d = 0; d < HD; d++) {
                    float kd = krow[j][d];
                    for (int r = 0; r < QT; r++) acc[r] = fmaf(qt[d][r], kd, acc[r]);
                }
                for (int r = 0; r < QT; r++) st[j][r] = scale * acc[r];
            }
            /* mask_lanes (549-567) */
            if (!all_image)
                for (size_t r = 0; r < queries; r++)
                    for (size_t j = 0; j < keys; j++)
                        if (masked(first_absolute + r, key_start + j, image_start, image_end)) st[j][r] = -INFINITY;
            if (is_static) {
                /* exp_lanes, static_shift.rs:135-160 */
                for (size_t r = 0; r < queries; r++) {
                    float sum = den[r];
                    for (size_t j = 0; j < keys; j++) {
                        float score = st[j][r];
                        float p = orc_exp_poly_unchecked(score);
                        if (!all_image && score == -INFINITY) p = 0.0f;
                        sum = sum + p;
                        st[j][r] = p;
                    }
                    den[r] = sum;
                }
            } else {
                /* softmax_lanes (574-652), per lane. */
                for (size_t r = 0; r < queries; r++) {
                    float block_max = -INFINITY;
                    for (size_t j = 0; j < keys; j++) block_max = st[j][r] > block_max ? st[j][r] : block_max;
                    float old_max = maxima[r];
                    float new_max = block_max > old_max ? block_max : old_max;
                    int skip = new_max == -INFINITY, first = old_max == -INFINITY;
                    float rescale = exp_fn(old_max - new_max);
                    if (first) rescale = 0.0f;
                    if (skip) rescale = 1.0f;
                    if (!skip && rescale != 1.0f)
                        for (int d = 0; d < HD; d++) out[r][d] *= rescale;
                    float denominator = den[r] * rescale;
                    for (size_t j = 0; j < keys; j++) {
                        float p = skip ? 0.0f : exp_fn(st[j][r] - new_max);
                        denominator = denominator + p;
                        st[j][r] = p;
                    }
                    den[r] = denominator;
                    maxima[r] = skip ? old_max : new_max;
                }
            }
            /* pv_lanes/pv_rows (657-715): chain over keys from +0, then + out. */
            for (size_t r = 0; r < queries; r++) {
                float acc[HD];
                for (int d = 0; d < HD; d++) acc[d] = 0.0f;
                for (size_t j = 0; j < keys; j++) {
                    float p = st[j][r];
                    for (int d = 0; d < HD; d++) acc[d] = fmaf(vrow[j][d], p, acc[d]);
                }
                for (int d = 0; d < HD; d++) out[r][d] = acc[d] + out[r][d];
            }
        } else {
            /* reference_key_tile (887-982). The gemm crate's order for these
             * short tiles is parity unpinned; this uses the lanes' chains. */
            for (size_t r = 0; r < queries; r++) {
                size_t absolute = first_absolute + r;
                float scores[KT];
                float block_max = -INFINITY;
                for (size_t j = 0; j < keys; j++) {
                    float acc = 0.0f;
                    for (int d = 0; d < HD; d++) acc = fmaf(qt[d][r], krow[j][d], acc);
                    float s = scale * acc;
                    if (masked(absolute, key_start + j, image_start, image_end)) s = -INFINITY;
                    scores[j] = s;
                    block_max = fmaxf(block_max, s); /* f32::max */
                }
                float new_max = fmaxf(maxima[r], block_max);
                if (new_max == -INFINITY) {
                    for (size_t j = 0; j < keys; j++) st[j][r] = 0.0f;
                    continue;
                }
                float rescale = maxima[r] == -INFINITY ? 0.0f : expf(maxima[r] - new_max);
                for (int d = 0; d < HD; d++) out[r][d] *= rescale;
                den[r] *= rescale;
                for (size_t j = 0; j < keys; j++) {
                    float p = expf(scores[j] - new_max); /* platform exp in every mode */
                    st[j][r] = p;
                    den[r] += p;
                }
                maxima[r] = new_max;
            }
            for (size_t r = 0; r < queries; r++) {
                float acc[HD];
                for (int d = 0; d < HD; d++) acc[d] = 0.0f;
                for (size_t j = 0; j < keys; j++)
                    for (int d = 0; d < HD; d++) acc[d] = fmaf(st[j][r], vrow[j][d], acc[d]);
                for (int d = 0; d < HD; d++) out[r][d] = out[r][d] + acc[d];
            }
        }
    }
    /* Final normalization and sink (prefill64.rs:468-479), platform exp/ln. */
    for (size_t r = 0; r < queries; r++) {
        float lse = is_static ? logf(den[r]) : maxima[r] + logf(den[r]);
        float sink_scale = 1.0f / (1.0f + expf(sinks[head] - lse));
        float *dst = output + (first_query + r) * qw + head * HD;
        for (int d = 0; d < HD; d++) dst[d] = (out[r][d] / den[r]) * sink_scale;
    }
}

void orc_attention_prefill_tiles(const float *q, const float *prefix_k, const float *generated_k,
                                 const float *v, size_t query_len, size_t prefix_len,
                                 size_t total_len, size_t n_heads, size_t n_kv_heads,
                                 size_t query_offset, size_t image_start, size_t image_end,
                                 const float *sinks, int static_softmax, int exp_fast,
                                 size_t tile_begin, size_t tile_end, float *out) {
    Cache cache = {prefix_k, generated_k, v, prefix_len, total_len, n_heads, n_kv_heads};
    size_t tiles = (query_len + QT - 1) / QT;
    if (tile_end > tiles) tile_end = tiles;
    if (tile_begin >= tile_end) return;
    size_t span = tile_end - tile_begin;
    ExpFn exp_fn = exp_fast ? orc_exp_poly : platform_exp;
#pragma omp parallel for schedule(dynamic, 1)
    for (long task = 0; task < (long)(span * n_heads); task++) {
        size_t tile = tile_begin + (size_t)task / n_heads, head = (size_t)task % n_heads;
        size_t queries = query_len - tile * QT < QT ? query_len - tile * QT : QT;
        tile_head(q, &cache, query_offset, image_start, image_end, tile, queries, head, sinks,
                  static_softmax, exp_fn, out);
    }
}

void orc_attention_prefill(const float *q, const float *prefix_k, const float *generated_k,
                           const float *v, size_t query_len, size_t prefix_len, size_t total_len,
                           size_t n_heads, size_t n_kv_heads, size_t query_offset,
                           size_t image_start, size_t image_end, const float *sinks,
                           int static_softmax, int exp_fast, float *out) {
    orc_attention_prefill_tiles(q, prefix_k, generated_k, v, query_len, prefix_len, total_len,
                                n_heads, n_kv_heads, query_offset, image_start, image_end, sinks,
                                static_softmax, exp_fast, 0, (size_t)-1, out);
}

/* ---- A8: BF16 prefill attention (src/kernels/attention/prefill64/bf16.rs) -- */

/* BF16 round to nearest even. `daz` follows vcvtneps2bf16 (denormal inputs
 * are zero); without it, half::bf16::from_f32 (used for the queries,
 * bf16.rs:256-268). NaN stays a quiet NaN. */
static inline float bf16_round(float x, int daz) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return u2f((u | 0x00400000u) & 0xffff0000u);
    if (daz && (u & 0x7f800000u) == 0) return u2f(u & 0x80000000u);
    return u2f((u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
}
static inline float flush(float x) { return (f2u(x) & 0x7f800000u) == 0 ? u2f(f2u(x) & 0x80000000u) : x; }

/* One vdpbf16ps lane step: acc += a1*b1, then acc += a0*b0 (the odd element
 * first), each product exact in FP32, denormal results flushed. */
static inline float dpbf16(float acc, float a0, float a1, float b0, float b1) {
    acc = flush(acc + flush(a1 * b1));
    return flush(acc + flush(a0 * b0));
}

/* exp2_lanes / exp2_scalar (bf16/static_shift.rs:277-289, tests.rs:19-24):
 * the reference's degree-3 minimax coefficients, digit for digit. */
static const float EXP2_C[4] = {0.99992806f, 0.69326097f, 0.24261113f, 0.05517167f};
float orc_exp2_minimax(float t) {
    float n = nearbyintf(t);
    float f = t - n;
    float p = fmaf(fmaf(fmaf(EXP2_C[3], f, EXP2_C[2]), f, EXP2_C[1]), f, EXP2_C[0]);
    return ldexpf(p, (int)n);
}

/* One (query tile, head) of compact_prefill (bf16.rs:70-175) for a pure
 * prefill (query_offset 0, every key a prefix key): tile_head (bf16.rs:
 * 271-398) for the online softmax, static_shift::tile_head
 * (bf16/static_shift.rs:100-168) for the static one. */
static void bf16_tile_head(const float *q, const float *k, const float *v, size_t total, size_t n_heads,
                           size_t n_kv_heads, size_t image_start, size_t image_end, size_t tile,
                           size_t queries, size_t head, const float *sinks, int is_static, ExpFn exp_fn,
                           float *output) {
    const size_t qw = n_heads * HD, kvw = n_kv_heads * HD;
    const size_t kv_head = head / (n_heads / n_kv_heads);
    const float scale = 0.125f;
    const float escale = 1.44269504088896340736f * scale; /* exponent_scale: LOG2_E * scale */
    size_t first_query = tile * QT;
    size_t first_absolute = first_query, last_absolute = first_absolute + queries - 1;
    int intersects = first_absolute < image_end && last_absolute >= image_start;
    size_t visible_end = intersects ? (last_absolute + 1 > image_end ? last_absolute + 1 : image_end) : last_absolute + 1;
    int all_image = first_absolute >= image_start && last_absolute < image_end;

    float qb[QT][HD], qf[HD][QT];
    memset(qb, 0, sizeof qb);
    memset(qf, 0, sizeof qf);
    for (size_t r = 0; r < queries; r++)
        for (int d = 0; d < HD; d++) {
            float x = q[(first_query + r) * qw + head * HD + d];
            qb[r][d] = bf16_round(x, 0); /* query_pairs: half::bf16 */
            qf[d][r] = x;
        }
    float maxima[QT], den[QT], out[QT][HD];
    for (int r = 0; r < QT; r++) {
        maxima[r] = -INFINITY;
        den[r] = 0.0f;
    }
    memset(out, 0, sizeof out);
    static __thread float st[KT][QT], kb[KT][HD], vb[KT][HD];

    for (size_t key_start = 0; key_start < visible_end; key_start += KT) {
        size_t keys = visible_end - key_start < KT ? visible_end - key_start : KT;
        int main_path = queries * keys > 256 && keys >= 3 && queries >= 2;
        if (is_static || main_path) {
            for (size_t j = 0; j < KT; j++)
                for (int d = 0; d < HD; d++) {
                    kb[j][d] = j < keys ? bf16_round(k[(key_start + j) * qw + head * HD + d], 1) : 0.0f;
                    vb[j][d] = j < keys ? bf16_round(v[(key_start + j) * kvw + kv_head * HD + d], 1) : 0.0f;
                }
            /* qk_keys (bf16.rs:563-596): pairs p = 0..31, odd element first. */
            for (size_t j = 0; j < keys; j++)
                for (int r = 0; r < QT; r++) {
                    float acc = 0.0f;
                    for (int pr = 0; pr < HD / 2; pr++)
                        acc = dpbf16(acc, qb[r][2 * pr], qb[r][2 * pr + 1], kb[j][2 * pr], kb[j][2 * pr + 1]);
                    st[j][r] = (is_static ? escale : scale) * acc;
                }
            if (is_static) {
                /* qk_exp_lanes epilogue: 2^t on visible lanes, +0 elsewhere;
                 * denominators add the BF16-rounded values in key order. */
                for (size_t j = 0; j < keys; j++)
                    for (size_t r = 0; r < queries; r++) {
                        size_t key = key_start + j;
                        int visible = all_image || !masked(first_absolute + r, key, image_start, image_end);
                        float p = visible ? orc_exp2_minimax(st[j][r]) : 0.0f;
                        st[j][r] = p;
                        den[r] = den[r] + bf16_round(p, 1);
                    }
            } else {
                if (!all_image)
                    for (size_t r = 0; r < queries; r++)
                        for (size_t j = 0; j < keys; j++)
                            if (masked(first_absolute + r, key_start + j, image_start, image_end)) st[j][r] = -INFINITY;
                /* softmax_pairs / softmax_lanes (bf16.rs:409-473): the FP32
                 * online step; the denominators add the unrounded p. */
                for (size_t r = 0; r < queries; r++) {
                    float block_max = -INFINITY;
                    for (size_t j = 0; j < keys; j++) block_max = st[j][r] > block_max ? st[j][r] : block_max;
                    float old_max = maxima[r];
                    float new_max = block_max > old_max ? block_max : old_max;
                    int skip = new_max == -INFINITY, first = old_max == -INFINITY;
                    float rescale = exp_fn(old_max - new_max);
                    if (first) rescale = 0.0f;
                    if (skip) rescale = 1.0f;
                    if (!skip && rescale != 1.0f)
                        for (int d = 0; d < HD; d++) out[r][d] *= rescale;
                    float denominator = den[r] * rescale;
                    for (size_t j = 0; j < keys; j++) {
                        float p = skip ? 0.0f : exp_fn(st[j][r] - new_max);
                        denominator = denominator + p;
                        st[j][r] = p;
                    }
                    den[r] = denominator;
                    maxima[r] = skip ? old_max : new_max;
                }
            }
            /* pv_rows (bf16.rs:627-657): per key pair, odd key first, from
             * +0; then + out. Probabilities round to BF16 first. */
            for (size_t r = 0; r < queries; r++) {
                float acc[HD];
                for (int d = 0; d < HD; d++) acc[d] = 0.0f;
                for (size_t kp = 0; kp < (keys + 1) / 2; kp++) {
                    float p0 = bf16_round(st[2 * kp][r], 1);
                    float p1 = 2 * kp + 1 < keys ? bf16_round(st[2 * kp + 1][r], 1) : 0.0f;
                    for (int d = 0; d < HD; d++) acc[d] = dpbf16(acc[d], vb[2 * kp][d], vb[2 * kp + 1][d], p0, p1);
                }
                for (int d = 0; d < HD; d++) out[r][d] = acc[d] + out[r][d];
            }
        } else {
            /* Short tiles: the parent's FP32 reference path on the FP32
             * operands (bf16.rs:368-393), as in the FP32 oracle. */
            for (size_t r = 0; r < queries; r++) {
                size_t absolute = first_absolute + r;
                float scores[KT];
                float block_max = -INFINITY;
                for (size_t j = 0; j < keys; j++) {
                    float acc = 0.0f;
                    const float *kr = k + (key_start + j) * qw + head * HD;
                    for (int d = 0; d < HD; d++) acc = fmaf(qf[d][r], kr[d], acc);
                    float s = scale * acc;
                    if (masked(absolute, key_start + j, image_start, image_end)) s = -INFINITY;
                    scores[j] = s;
                    block_max = fmaxf(block_max, s);
                }
                float new_max = fmaxf(maxima[r], block_max);
                if (new_max == -INFINITY) {
                    for (size_t j = 0; j < keys; j++) st[j][r] = 0.0f;
                    continue;
                }
                float rescale = maxima[r] == -INFINITY ? 0.0f : expf(maxima[r] - new_max);
                for (int d = 0; d < HD; d++) out[r][d] *= rescale;
                den[r] *= rescale;
                for (size_t j = 0; j < keys; j++) {
                    float p = expf(scores[j] - new_max);
                    st[j][r] = p;
                    den[r] += p;
                }
                maxima[r] = new_max;
            }
            for (size_t r = 0; r < queries; r++) {
                float acc[HD];
                for (int d = 0; d < HD; d++) acc[d] = 0.0f;
                for (size_t j = 0; j < keys; j++) {
                    const float *vr = v + (key_start + j) * kvw + kv_head * HD;
                    for (int d = 0; d < HD; d++) acc[d] = fmaf(st[j][r], vr[d], acc[d]);
                }
                for (int d = 0; d < HD; d++) out[r][d] = out[r][d] + acc[d];
            }
        }
    }
    for (size_t r = 0; r < queries; r++) {
        float lse = is_static ? logf(den[r]) : maxima[r] + logf(den[r]);
        float sink_scale = 1.0f / (1.0f + expf(sinks[head] - lse));
        float *dst = output + (first_query + r) * qw + head * HD;
        for (int d = 0; d < HD; d++) dst[d] = (out[r][d] / den[r]) * sink_scale;
    }
}

void orc_attention_prefill_bf16_tiles(const float *q, const float *k, const float *v, size_t query_len,
                                      size_t n_heads, size_t n_kv_heads, size_t image_start,
                                      size_t image_end, const float *sinks, int static_softmax,
                                      int exp_fast, size_t tile_begin, size_t tile_end, float *out) {
    size_t tiles = (query_len + QT - 1) / QT;
    if (tile_end > tiles) tile_end = tiles;
    if (tile_begin >= tile_end) return;
    size_t span = tile_end - tile_begin;
    ExpFn exp_fn = exp_fast ? orc_exp_poly : platform_exp;
#pragma omp parallel for schedule(dynamic, 1)
    for (long task = 0; task < (long)(span * n_heads); task++) {
        size_t tile = tile_begin + (size_t)task / n_heads, head = (size_t)task % n_heads;
        size_t queries = query_len - tile * QT < QT ? query_len - tile * QT : QT;
        bf16_tile_head(q, k, v, query_len, n_heads, n_kv_heads, image_start, image_end, tile, queries, head,
                       sinks, static_softmax, exp_fn, out);
    }
}

float orc_bf16_round(float x) { return bf16_round(x, 0); }

/* ---- A9 ------------------------------------------------------------------ */
int orc_argmax(const float *logits, size_t n, uint32_t *out) {
    if (n == 0) return -1;
    size_t best = 0;
    int finite = isfinite(logits[0]);
    for (size_t i = 1; i < n; i++) {
        finite &= isfinite(logits[i]) != 0;
        if (logits[i] > logits[best]) best = i;
    }
    if (!finite) return -1;
    *out = (uint32_t)best;
    return 0;
}

/* ---- the QKV row step ------------------------------------------------------ */
/* rms_norm_row on one 64-wide head, no weight (src/kernels/mod.rs:497-514),
 * then the pairwise rotation (src/model/fused.rs:109-120, the same products
 * as split_norm_rope's, src/model/rope.rs:60-72). rope: [32][2] = [cos, sin]. */
static void norm_rope_head(const float *x, const float *rope, float *out) {
    float scale = orc_rms_scale(x, HD, FLT_EPSILON);
    float y[HD];
    for (int i = 0; i < HD; i++) y[i] = x[i] * scale;
    for (int pair = 0; pair < HD / 2; pair++) {
        float c = rope[2 * pair], s = rope[2 * pair + 1];
        float a = y[2 * pair], b = y[2 * pair + 1];
        out[2 * pair] = a * c - b * s;
        out[2 * pair + 1] = a * s + b * c;
    }
}

void orc_qkv_rows(const float *qkv, size_t rows, const float *rope, size_t n_heads, size_t n_kv_heads,
                  size_t prefix_rows, float *q, float *prefix_k, float *generated_k, float *v) {
    size_t qdim = n_heads * HD, kdim = n_kv_heads * HD, repeat = n_heads / n_kv_heads;
#pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)rows; r++) {
        const float *src = qkv + (size_t)r * (qdim + 2 * kdim);
        const float *factors = rope + (size_t)r * n_heads * HD; /* n_heads * 32 pairs * 2 */
        for (size_t h = 0; h < n_heads; h++)
            norm_rope_head(src + h * HD, factors + h * HD, q + (size_t)r * qdim + h * HD);
        if ((size_t)r < prefix_rows) {
            /* fused_row: every query head's key (fused.rs:107-111). */
            for (size_t h = 0; h < n_heads; h++)
                norm_rope_head(src + qdim + (h / repeat) * HD, factors + h * HD, prefix_k + (size_t)r * qdim + h * HD);
        } else {
            /* split_norm_rope's expanded keys, then append_unique_heads keeps
             * the first head of each group (cache.rs:202-216). */
            for (size_t g = 0; g < n_kv_heads; g++)
                norm_rope_head(src + qdim + g * HD, factors + g * repeat * HD,
                               generated_k + ((size_t)r - prefix_rows) * kdim + g * HD);
        }
        memcpy(v + (size_t)r * kdim, src + qdim + kdim, kdim * sizeof(float));
    }
}

/* ---- decode attention ----------------------------------------------------- */
/* online::head (src/kernels/attention/online.rs:96-150) with the 64-wide
 * simd::dot / simd::axpy (src/simd.rs:749-777,925-940) and the platform expf
 * and logf, for query qh = query * n_heads + head. */
/* exp_fast: the per-key probabilities exp(s - max) by exp_poly, as the
 * sealed cache's decode with SplitPrefix::fast_exp (its exp_shifted through
 * simd::Avx2Fast, src/quant/kv/decode.rs:346-347, src/simd.rs:440-445); the
 * rescale and the sink keep the platform exp. */
static void decode_head(const float *q, const Cache *cache, size_t query_offset, size_t image_start,
                        size_t image_end, size_t query, size_t head, const float *sinks, int exp_fast,
                        float *out) {
    const float scale = 1.0f / sqrtf((float)HD);
    size_t repeat = cache->n_heads / cache->n_kv_heads, kv_head = head / repeat;
    size_t absolute = query_offset + query;
    size_t visible_end = absolute >= image_start && absolute < image_end ? image_end : absolute + 1;
    const float *qvec = q + (query * cache->n_heads + head) * HD;
    for (int d = 0; d < HD; d++) out[d] = 0.0f;
    float running_max = -INFINITY, denominator = 0.0f;
    float logits[KT];
    for (size_t start = 0; start < visible_end; start += KT) {
        size_t len = visible_end - start < KT ? visible_end - start : KT;
        float block_max = -INFINITY;
        for (size_t j = 0; j < len; j++) {
            logits[j] = orc_dot(qvec, cache_key(cache, start + j, head), HD) * scale;
            block_max = fmaxf(block_max, logits[j]);
        }
        float new_max = fmaxf(running_max, block_max);
        float rescale = running_max == -INFINITY ? 0.0f : expf(running_max - new_max);
        for (int d = 0; d < HD; d++) out[d] *= rescale;
        denominator *= rescale;
        for (size_t j = 0; j < len; j++)
            logits[j] = exp_fast ? orc_exp_poly(logits[j] - new_max) : expf(logits[j] - new_max);
        for (size_t j = 0; j < len; j++) {
            float p = logits[j];
            const float *value = cache_value(cache, start + j, kv_head);
            denominator += p;
            for (int d = 0; d < HD; d++) out[d] = fmaf(p, value[d], out[d]);
        }
        running_max = new_max;
    }
    float logsumexp = running_max + logf(denominator);
    float sink_scale = 1.0f / (1.0f + expf(sinks[head] - logsumexp));
    for (int d = 0; d < HD; d++) out[d] = (out[d] / denominator) * sink_scale;
}

void orc_attention_decode_ex(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                             size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                             size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                             const float *sinks, int exp_fast, float *out) {
    Cache cache = {prefix_k, generated_k, v, prefix_len, total_len, n_heads, n_kv_heads};
#pragma omp parallel for schedule(static)
    for (long qh = 0; qh < (long)(query_len * n_heads); qh++)
        decode_head(q, &cache, query_offset, image_start, image_end, (size_t)qh / n_heads, (size_t)qh % n_heads,
                    sinks, exp_fast, out + (size_t)qh * HD);
}

void orc_attention_decode(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                          size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                          size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                          const float *sinks, float *out) {
    orc_attention_decode_ex(q, prefix_k, generated_k, v, query_len, prefix_len, total_len, n_heads, n_kv_heads,
                            query_offset, image_start, image_end, sinks, 0, out);
}
