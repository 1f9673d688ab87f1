/*
 * The CPU baseline of the quantized decode GEMV — TEST INFRASTRUCTURE ONLY
 * (bench.py's cpu_baseline legs and tests/). A performance restatement of
 * the reference's AVX2 decode dot product, simd::dot_q with Simd = Avx2
 * (src/simd.rs:821-857; Avx2::load_i8 / load_i16 / sum, src/simd.rs:356-373):
 * per 32-input block one broadcast scale, weights fl(code * scale) eight at
 * a time, four 8-lane FMA accumulators, combined (a0 + a1) + (a2 + a3); the
 * 8-wide tail; the horizontal sum ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)); the
 * scalar tail x * fl(code * scale); then the exception FMAs in ascending
 * order (Exceptions::accumulate, src/quant/linear.rs:84-118). Output
 * channels are split across threads as the decode team splits them. Every
 * output is bit for bit orc_linear_decode's (tests/test_cpu_baseline.py);
 * without AVX2 + FMA both calls fall back to the scalar oracle.
 */
#include "focr_oracle.h"

#include <math.h>
#include <stddef.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#include <immintrin.h>

__attribute__((target("avx2,fma"))) static inline __m256 weights8(int bits, const void *codes, size_t at, __m256 s) {
    __m256 c;
    if (bits == 8)
        c = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)((const int8_t *)codes + at))));
    else if (bits == 16)
        c = _mm256_cvtepi32_ps(_mm256_cvtepi16_epi32(_mm_loadu_si128((const __m128i *)((const int16_t *)codes + at))));
    else
        return _mm256_loadu_ps((const float *)codes + at);
    return _mm256_mul_ps(c, s);
}

static inline float code_f32(int bits, const void *codes, size_t at) {
    if (bits == 8) return (float)((const int8_t *)codes)[at];
    if (bits == 16) return (float)((const int16_t *)codes)[at];
    return ((const float *)codes)[at];
}

/* dot_q<Avx2> of input row x with channel `c`, then its exceptions. G is
 * the group when it is the reference's compile-time 64 (0: `group`). */
__attribute__((target("avx2,fma"))) static inline float dot_channel_g(int bits, const void *codes,
                                                                    const float *scales, size_t k, size_t group,
                                                                    const int32_t *exc_cols, const float *exc_vals,
                                                                    size_t n_exc, const float *x, size_t c,
                                                                    const size_t G) {
    if (G) group = G;
    const size_t base = c * k, groups = (k + group - 1) / group;
    const float *sc = bits == 32 ? NULL : scales + c * groups;
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    size_t i = 0;
    for (; i + 32 <= k; i += 32) {
        const __m256 s = _mm256_set1_ps(sc ? sc[i / group] : 1.0f);
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), weights8(bits, codes, base + i, s), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 8), weights8(bits, codes, base + i + 8, s), a1);
        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 16), weights8(bits, codes, base + i + 16, s), a2);
        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(x + i + 24), weights8(bits, codes, base + i + 24, s), a3);
    }
    __m256 acc = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
    for (; i + 8 <= k; i += 8) {
        const __m256 s = _mm256_set1_ps(sc ? sc[i / group] : 1.0f);
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(x + i), weights8(bits, codes, base + i, s), acc);
    }
    const __m128 halves = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    const __m128 pairs = _mm_hadd_ps(halves, halves);
    float total = _mm_cvtss_f32(_mm_hadd_ps(pairs, pairs));
    for (; i < k; i++) {
        const float w = sc ? code_f32(bits, codes, base + i) * sc[i / group] : code_f32(bits, codes, base + i);
        total += x[i] * w;
    }
    for (size_t e = 0; e < n_exc; e++) total = fmaf(x[exc_cols[e]], exc_vals[c * n_exc + e], total);
    return total;
}

__attribute__((target("avx2,fma"))) static float dot_channel(int bits, const void *codes, const float *scales,
                                                           size_t k, size_t group, const int32_t *exc_cols,
                                                           const float *exc_vals, size_t n_exc, const float *x,
                                                           size_t c) {
    if (group == 64)
        return dot_channel_g(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x, c, 64);
    return dot_channel_g(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x, c, 0);
}

static int have_avx2_fma(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

void orc_linear_decode_fast(int bits, const void *codes, const float *scales, size_t n, size_t k, size_t group,
                            const int32_t *exc_cols, const float *exc_vals, size_t n_exc, const float *x, size_t rows,
                            float *out) {
    if (k == 0 || !have_avx2_fma() || (bits != 32 && group % 32 != 0)) {
        orc_linear_decode(bits, codes, scales, n, k, group, exc_cols, exc_vals, n_exc, x, rows, out);
        return;
    }
#pragma omp parallel for schedule(static)
    for (long c = 0; c < (long)n; c++)
        for (size_t r = 0; r < rows; r++)
            out[r * n + (size_t)c] =
                dot_channel(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x + r * k, (size_t)c);
}

void orc_linear_decode_glu_fast(int bits, const void *codes, const float *scales, size_t n, size_t k, size_t group,
                                const int32_t *exc_cols, const float *exc_vals, size_t n_exc, const float *x,
                                size_t rows, float *gated) {
    if (k == 0 || !have_avx2_fma() || (bits != 32 && group % 32 != 0)) {
        orc_linear_decode_glu(bits, codes, scales, n, k, group, exc_cols, exc_vals, n_exc, x, rows, gated);
        return;
    }
    const size_t ffn = n / 2;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < (long)ffn; i++)
        for (size_t r = 0; r < rows; r++) {
            const float gate =
                dot_channel(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x + r * k, 2 * (size_t)i);
            const float up =
                dot_channel(bits, codes, scales, k, group, exc_cols, exc_vals, n_exc, x + r * k, 2 * (size_t)i + 1);
            gated[r * ffn + (size_t)i] = orc_squared_relu_glu(gate, up);
        }
}

/* ---- decode attention ---------------------------------------------------- */
/* online::head (src/kernels/attention/online.rs:96-150) for one query row
 * and head over the FP32 compact cache, with the AVX2 simd::dot for the
 * 64-wide scores and simd::axpy (one FMA per element) for the values, the
 * rescale as one multiply per element, and the scalar steps (running max,
 * exp, denominator, sink) as orc_attention_decode takes them: bitwise
 * orc_attention_decode. Head dimension 64, 128-key tiles. */
#define DHD 64
#define DKT 128

__attribute__((target("avx2,fma"))) static inline float dot64(const float *a, const float *b) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    for (int i = 0; i < DHD; i += 32) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), a1);
        a2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), a2);
        a3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), a3);
    }
    const __m256 acc = _mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3));
    const __m128 halves = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    const __m128 pairs = _mm_hadd_ps(halves, halves);
    return _mm_cvtss_f32(_mm_hadd_ps(pairs, pairs));
}

__attribute__((target("avx2,fma"))) static void decode_head_fast(const float *q, const float *prefix_k,
                                                               const float *generated_k, const float *v,
                                                               size_t prefix_len, size_t n_heads, size_t n_kv_heads,
                                                               size_t absolute, size_t image_start, size_t image_end,
                                                               size_t head, float sink, float *out) {
    const float scale = 1.0f / sqrtf((float)DHD);
    const size_t repeat = n_heads / n_kv_heads, kv_head = head / repeat;
    const size_t visible_end = absolute >= image_start && absolute < image_end ? image_end : absolute + 1;
    __m256 o[DHD / 8];
    for (int d = 0; d < DHD / 8; d++) o[d] = _mm256_setzero_ps();
    float running_max = -INFINITY, denominator = 0.0f;
    float logits[DKT];
    for (size_t start = 0; start < visible_end; start += DKT) {
        const size_t len = visible_end - start < DKT ? visible_end - start : DKT;
        float block_max = -INFINITY;
        for (size_t j = 0; j < len; j++) {
            const size_t pos = start + j;
            const float *key = pos < prefix_len ? prefix_k + (pos * n_heads + head) * DHD
                                                : generated_k + ((pos - prefix_len) * n_kv_heads + kv_head) * DHD;
            logits[j] = dot64(q, key) * scale;
            block_max = fmaxf(block_max, logits[j]);
        }
        const float new_max = fmaxf(running_max, block_max);
        const float rescale = running_max == -INFINITY ? 0.0f : expf(running_max - new_max);
        const __m256 r = _mm256_set1_ps(rescale);
        for (int d = 0; d < DHD / 8; d++) o[d] = _mm256_mul_ps(o[d], r);
        denominator *= rescale;
        for (size_t j = 0; j < len; j++) logits[j] = expf(logits[j] - new_max);
        for (size_t j = 0; j < len; j++) {
            const float p = logits[j];
            const float *value = v + ((start + j) * n_kv_heads + kv_head) * DHD;
            denominator += p;
            const __m256 pv = _mm256_set1_ps(p);
            for (int d = 0; d < DHD / 8; d++) o[d] = _mm256_fmadd_ps(pv, _mm256_loadu_ps(value + 8 * d), o[d]);
        }
        running_max = new_max;
    }
    const float logsumexp = running_max + logf(denominator);
    const float sink_scale = 1.0f / (1.0f + expf(sink - logsumexp));
    float tmp[DHD];
    for (int d = 0; d < DHD / 8; d++) _mm256_storeu_ps(tmp + 8 * d, o[d]);
    for (int d = 0; d < DHD; d++) out[d] = (tmp[d] / denominator) * sink_scale;
}

void orc_attention_decode_fast(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                               size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                               size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                               const float *sinks, float *out) {
    if (!have_avx2_fma()) {
        orc_attention_decode(q, prefix_k, generated_k, v, query_len, prefix_len, total_len, n_heads, n_kv_heads,
                             query_offset, image_start, image_end, sinks, out);
        return;
    }
#pragma omp parallel for schedule(static)
    for (long qh = 0; qh < (long)(query_len * n_heads); qh++) {
        const size_t query = (size_t)qh / n_heads, head = (size_t)qh % n_heads;
        decode_head_fast(q + (size_t)qh * DHD, prefix_k, generated_k, v, prefix_len, n_heads, n_kv_heads,
                         query_offset + query, image_start, image_end, head, sinks[head], out + (size_t)qh * DHD);
    }
}
