/*
 * The CPU baseline of the FP32 prefill attention — TEST INFRASTRUCTURE ONLY
 * (bench.py's cpu_baseline leg and tests/). The same tiles as the oracle's
 * orc_attention_prefill (tile_head, the reference's prefill64.rs:328-480:
 * 32 queries x 128 keys, QK FMA chains over d from +0 then * 1/8, the
 * masking rule, softmax_lanes with exp_poly, PV chains over keys from +0),
 * with every per-element operation in the same order, but written so that
 * the compiler vectorizes across the 32 query lanes as the reference's SIMD
 * lanes do: QK two keys at a time, the softmax and exp_poly branch-free over
 * the lanes. Bit for bit orc_attention_prefill in the Fast exp mode and the
 * static softmax (tests/test_cpu_baseline.py checks it). Built for AVX-512
 * (the x86-64-v4 variant) the lanes are 16 wide, as the reference's "wide"
 * tiles on AVX-512 hosts (src/kernels/mod.rs:44-46, prefill64.rs:721-882);
 * the per-lane operations do not change. Tiles off the
 * reference's main path (q*k <= 256, k < 3 or q < 2) run the oracle's
 * scalar code.
 */
#include "focr_oracle.h"

#include <math.h>
#include <string.h>
#if defined(__AVX2__) && defined(__FMA__) || defined(__AVX512F__)
#include <immintrin.h>
#endif

#define QT 32
#define KT 128
#define HD 64

typedef struct {
    const float *prefix_k, *generated_k, *v;
    size_t prefix_len, total_len, n_heads, n_kv_heads;
} FCache;

static inline const float *fkey(const FCache *c, size_t position, size_t head) {
    if (position < c->prefix_len) return c->prefix_k + (position * c->n_heads + head) * HD;
    size_t repeat = c->n_heads / c->n_kv_heads;
    return c->generated_k + ((position - c->prefix_len) * c->n_kv_heads + head / repeat) * HD;
}

static inline int fmasked(size_t absolute, size_t key, size_t image_start, size_t image_end) {
    int image_query = absolute >= image_start && absolute < image_end;
    return key > absolute && !(image_query && key >= image_start && key < image_end);
}

static inline float bits_f(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}

/* exp_poly_unchecked (src/kernels/exp.rs:248-257), inlined. */
static inline float exp_un(float x) {
    float n = rintf(x * 1.44269504088896340735992468100189214f);
    float r = fmaf(n, -0.6933594f, x);
    r = fmaf(n, 2.1219444e-4f, r);
    float p = 1.9875691e-4f;
    p = fmaf(p, r, 1.3981999e-3f);
    p = fmaf(p, r, 8.333452e-3f);
    p = fmaf(p, r, 4.1665796e-2f);
    p = fmaf(p, r, 0.16666665f);
    p = fmaf(p, r, 0.5f);
    float y = fmaf(p, r * r, r) + 1.0f;
    return y * bits_f((uint32_t)((int32_t)n + 127) << 23);
}

/* exp_poly (exp.rs:232-245) without branches: the polynomial of the clamped
 * argument (the identity inside the range), then the range results. */
static inline float exp_fast(float x) {
    float xc = x < -87.0f ? -87.0f : x;
    xc = xc > 88.376f ? 88.376f : xc;
    float y = exp_un(xc);
    y = x < -87.0f ? 0.0f : y;
    y = x > 88.376f ? INFINITY : y;
    return x != x ? x : y;
}

#if defined(__AVX2__) && defined(__FMA__)
/* exp_un and exp_fast on eight lanes: the same operations in the same order
 * (round-to-nearest-even as rintf, the exponent built from the integral n). */
static inline __m256 exp_un8(__m256 x) {
    const __m256 n = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.44269504088896340735992468100189214f)),
                                     _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r = _mm256_fmadd_ps(n, _mm256_set1_ps(-0.6933594f), x);
    r = _mm256_fmadd_ps(n, _mm256_set1_ps(2.1219444e-4f), r);
    __m256 p = _mm256_set1_ps(1.9875691e-4f);
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.3981999e-3f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(8.333452e-3f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(4.1665796e-2f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.16666665f));
    p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
    const __m256 y = _mm256_add_ps(_mm256_fmadd_ps(p, _mm256_mul_ps(r, r), r), _mm256_set1_ps(1.0f));
    const __m256i e = _mm256_slli_epi32(_mm256_add_epi32(_mm256_cvtps_epi32(n), _mm256_set1_epi32(127)), 23);
    return _mm256_mul_ps(y, _mm256_castsi256_ps(e));
}

static inline __m256 exp_fast8(__m256 x) {
    const __m256 lo = _mm256_set1_ps(-87.0f), hi = _mm256_set1_ps(88.376f);
    const __m256 below = _mm256_cmp_ps(x, lo, _CMP_LT_OQ), above = _mm256_cmp_ps(x, hi, _CMP_GT_OQ);
    __m256 xc = _mm256_blendv_ps(x, lo, below);
    xc = _mm256_blendv_ps(xc, hi, above);
    __m256 y = exp_un8(xc);
    y = _mm256_blendv_ps(y, _mm256_setzero_ps(), below);
    y = _mm256_blendv_ps(y, _mm256_set1_ps(INFINITY), above);
    return _mm256_blendv_ps(y, x, _mm256_cmp_ps(x, x, _CMP_UNORD_Q));
}
#endif

#if defined(__AVX512F__)
/* exp_un and exp_fast on sixteen lanes (the reference's 16-lane "wide"
 * tiles on AVX-512 hosts, prefill64.rs:721-882, bitwise the 8-lane ones):
 * the same operations in the same order. */
static inline __m512 exp_un16(__m512 x) {
    const __m512 n = _mm512_roundscale_ps(_mm512_mul_ps(x, _mm512_set1_ps(1.44269504088896340735992468100189214f)),
                                          _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m512 r = _mm512_fmadd_ps(n, _mm512_set1_ps(-0.6933594f), x);
    r = _mm512_fmadd_ps(n, _mm512_set1_ps(2.1219444e-4f), r);
    __m512 p = _mm512_set1_ps(1.9875691e-4f);
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(1.3981999e-3f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(8.333452e-3f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(4.1665796e-2f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(0.16666665f));
    p = _mm512_fmadd_ps(p, r, _mm512_set1_ps(0.5f));
    const __m512 y = _mm512_add_ps(_mm512_fmadd_ps(p, _mm512_mul_ps(r, r), r), _mm512_set1_ps(1.0f));
    const __m512i e = _mm512_slli_epi32(_mm512_add_epi32(_mm512_cvtps_epi32(n), _mm512_set1_epi32(127)), 23);
    return _mm512_mul_ps(y, _mm512_castsi512_ps(e));
}

static inline __m512 exp_fast16(__m512 x) {
    const __m512 lo = _mm512_set1_ps(-87.0f), hi = _mm512_set1_ps(88.376f);
    const __mmask16 below = _mm512_cmp_ps_mask(x, lo, _CMP_LT_OQ), above = _mm512_cmp_ps_mask(x, hi, _CMP_GT_OQ);
    __m512 xc = _mm512_mask_blend_ps(below, x, lo);
    xc = _mm512_mask_blend_ps(above, xc, hi);
    __m512 y = exp_un16(xc);
    y = _mm512_mask_blend_ps(below, y, _mm512_setzero_ps());
    y = _mm512_mask_blend_ps(above, y, _mm512_set1_ps(INFINITY));
    return _mm512_mask_blend_ps(_mm512_cmp_ps_mask(x, x, _CMP_UNORD_Q), y, x);
}
#endif

static void tile_fast(const float *q, const FCache *cache, size_t query_offset, size_t image_start, size_t image_end,
                      size_t tile, size_t queries, size_t head, const float *sinks, int is_static, float *output) {
    const size_t qw = cache->n_heads * HD;
    const size_t kv_head = head / (cache->n_heads / cache->n_kv_heads);
    const float scale = 1.0f / sqrtf((float)HD);
    size_t first_query = tile * QT;
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
            krow[j] = fkey(cache, key_start + j, head);
            vrow[j] = cache->v + ((key_start + j) * cache->n_kv_heads + kv_head) * HD;
        }
        int main_path = queries * keys > 256 && keys >= 3 && queries >= 2;
        if (is_static || main_path) {
            /* QK: each (key, query) is one FMA chain over d from +0; two keys
             * per pass so the chains of 64 lanes interleave. */
            size_t j = 0;
#if defined(__AVX512F__)
            /* The 32 lanes of two keys in four registers. */
            const __m512 wscale = _mm512_set1_ps(scale);
            for (; j + 2 <= keys; j += 2) {
                __m512 a0[2], a1[2];
                for (int v = 0; v < 2; v++) a0[v] = a1[v] = _mm512_setzero_ps();
                const float *k0 = krow[j], *k1 = krow[j + 1];
                for (int d = 0; d < HD; d++) {
                    const __m512 x0 = _mm512_set1_ps(k0[d]), x1 = _mm512_set1_ps(k1[d]);
                    for (int v = 0; v < 2; v++) {
                        const __m512 qd = _mm512_loadu_ps(&qt[d][16 * v]);
                        a0[v] = _mm512_fmadd_ps(qd, x0, a0[v]);
                        a1[v] = _mm512_fmadd_ps(qd, x1, a1[v]);
                    }
                }
                for (int v = 0; v < 2; v++) {
                    _mm512_storeu_ps(&st[j][16 * v], _mm512_mul_ps(wscale, a0[v]));
                    _mm512_storeu_ps(&st[j + 1][16 * v], _mm512_mul_ps(wscale, a1[v]));
                }
            }
#elif defined(__AVX2__) && defined(__FMA__)
            /* The 32 lanes of two keys in eight registers. */
            const __m256 vscale = _mm256_set1_ps(scale);
            for (; j + 2 <= keys; j += 2) {
                __m256 a0[4], a1[4];
                for (int v = 0; v < 4; v++) a0[v] = a1[v] = _mm256_setzero_ps();
                const float *k0 = krow[j], *k1 = krow[j + 1];
                for (int d = 0; d < HD; d++) {
                    const __m256 x0 = _mm256_broadcast_ss(k0 + d), x1 = _mm256_broadcast_ss(k1 + d);
                    for (int v = 0; v < 4; v++) {
                        const __m256 qd = _mm256_loadu_ps(&qt[d][8 * v]);
                        a0[v] = _mm256_fmadd_ps(qd, x0, a0[v]);
                        a1[v] = _mm256_fmadd_ps(qd, x1, a1[v]);
                    }
                }
                for (int v = 0; v < 4; v++) {
                    _mm256_storeu_ps(&st[j][8 * v], _mm256_mul_ps(vscale, a0[v]));
                    _mm256_storeu_ps(&st[j + 1][8 * v], _mm256_mul_ps(vscale, a1[v]));
                }
            }
#endif
            for (; j < keys; j++) {
                float a0[QT];
                for (int r = 0; r < QT; r++) a0[r] = 0.0f;
                for (int d = 0; d < HD; d++)
                    for (int r = 0; r < QT; r++) a0[r] = fmaf(qt[d][r], krow[j][d], a0[r]);
                for (int r = 0; r < QT; r++) st[j][r] = scale * a0[r];
            }
            /* Only a key past the tile's first query can be hidden. */
            if (!all_image && key_start + keys > first_absolute + 1)
                for (size_t r = 0; r < queries; r++)
                    for (size_t jj = 0; jj < keys; jj++)
                        if (fmasked(first_absolute + r, key_start + jj, image_start, image_end)) st[jj][r] = -INFINITY;
            if (is_static) {
                size_t jj = 0;
#if defined(__AVX512F__)
                const __m512 ninf = _mm512_set1_ps(-INFINITY);
                for (; jj < keys; jj++)
                    for (int v = 0; v < 2; v++) {
                        const __m512 score = _mm512_loadu_ps(&st[jj][16 * v]);
                        __m512 p = exp_un16(score);
                        if (!all_image) p = _mm512_mask_blend_ps(_mm512_cmp_ps_mask(score, ninf, _CMP_EQ_OQ), p, _mm512_setzero_ps());
                        _mm512_storeu_ps(&den[16 * v], _mm512_add_ps(_mm512_loadu_ps(&den[16 * v]), p));
                        _mm512_storeu_ps(&st[jj][16 * v], p);
                    }
#elif defined(__AVX2__) && defined(__FMA__)
                const __m256 ninf = _mm256_set1_ps(-INFINITY);
                for (; jj < keys; jj++)
                    for (int v = 0; v < 4; v++) {
                        const __m256 score = _mm256_loadu_ps(&st[jj][8 * v]);
                        __m256 p = exp_un8(score);
                        if (!all_image) p = _mm256_blendv_ps(p, _mm256_setzero_ps(), _mm256_cmp_ps(score, ninf, _CMP_EQ_OQ));
                        _mm256_storeu_ps(&den[8 * v], _mm256_add_ps(_mm256_loadu_ps(&den[8 * v]), p));
                        _mm256_storeu_ps(&st[jj][8 * v], p);
                    }
#endif
                for (; jj < keys; jj++)
                    for (int r = 0; r < QT; r++) {
                        float score = st[jj][r];
                        float p = exp_un(score);
                        p = (!all_image && score == -INFINITY) ? 0.0f : p;
                        den[r] = den[r] + p;
                        st[jj][r] = p;
                    }
            } else {
                float bmax[QT], newm[QT], resc[QT], skip[QT];
                for (int r = 0; r < QT; r++) bmax[r] = -INFINITY;
                for (size_t jj = 0; jj < keys; jj++)
                    for (int r = 0; r < QT; r++) bmax[r] = st[jj][r] > bmax[r] ? st[jj][r] : bmax[r];
                for (int r = 0; r < QT; r++) {
                    float old_max = maxima[r];
                    float new_max = bmax[r] > old_max ? bmax[r] : old_max;
                    float rescale = exp_fast(old_max - new_max);
                    rescale = old_max == -INFINITY ? 0.0f : rescale;
                    rescale = new_max == -INFINITY ? 1.0f : rescale;
                    newm[r] = new_max;
                    resc[r] = rescale;
                    skip[r] = new_max == -INFINITY ? 1.0f : 0.0f;
                    den[r] = den[r] * rescale;
                    maxima[r] = new_max == -INFINITY ? old_max : new_max;
                }
                for (int r = 0; r < QT; r++)
                    if (skip[r] == 0.0f && resc[r] != 1.0f)
                        for (int d = 0; d < HD; d++) out[r][d] *= resc[r];
                size_t jj = 0;
#if defined(__AVX512F__)
                for (; jj < keys; jj++)
                    for (int v = 0; v < 2; v++) {
                        __m512 p = exp_fast16(_mm512_sub_ps(_mm512_loadu_ps(&st[jj][16 * v]), _mm512_loadu_ps(&newm[16 * v])));
                        p = _mm512_mask_blend_ps(_mm512_cmp_ps_mask(_mm512_loadu_ps(&skip[16 * v]), _mm512_setzero_ps(), _CMP_NEQ_OQ),
                                                 p, _mm512_setzero_ps());
                        _mm512_storeu_ps(&den[16 * v], _mm512_add_ps(_mm512_loadu_ps(&den[16 * v]), p));
                        _mm512_storeu_ps(&st[jj][16 * v], p);
                    }
#elif defined(__AVX2__) && defined(__FMA__)
                for (; jj < keys; jj++)
                    for (int v = 0; v < 4; v++) {
                        __m256 p = exp_fast8(_mm256_sub_ps(_mm256_loadu_ps(&st[jj][8 * v]), _mm256_loadu_ps(&newm[8 * v])));
                        p = _mm256_blendv_ps(p, _mm256_setzero_ps(),
                                             _mm256_cmp_ps(_mm256_loadu_ps(&skip[8 * v]), _mm256_setzero_ps(), _CMP_NEQ_OQ));
                        _mm256_storeu_ps(&den[8 * v], _mm256_add_ps(_mm256_loadu_ps(&den[8 * v]), p));
                        _mm256_storeu_ps(&st[jj][8 * v], p);
                    }
#endif
                for (; jj < keys; jj++)
                    for (int r = 0; r < QT; r++) {
                        float p = exp_fast(st[jj][r] - newm[r]);
                        p = skip[r] != 0.0f ? 0.0f : p;
                        den[r] = den[r] + p;
                        st[jj][r] = p;
                    }
            }
            /* PV: chains over keys from +0 per (query, dim), then + out. */
            size_t r = 0;
#if defined(__AVX512F__)
            /* Two query rows x 64 dims per pass: eight accumulators. */
            for (; r + 2 <= queries; r += 2) {
                __m512 a0[4], a1[4];
                for (int v = 0; v < 4; v++) a0[v] = a1[v] = _mm512_setzero_ps();
                for (size_t jj = 0; jj < keys; jj++) {
                    const __m512 p0 = _mm512_set1_ps(st[jj][r]), p1 = _mm512_set1_ps(st[jj][r + 1]);
                    const float *vr = vrow[jj];
                    for (int v = 0; v < 4; v++) {
                        const __m512 x = _mm512_loadu_ps(vr + 16 * v);
                        a0[v] = _mm512_fmadd_ps(x, p0, a0[v]);
                        a1[v] = _mm512_fmadd_ps(x, p1, a1[v]);
                    }
                }
                for (int v = 0; v < 4; v++) {
                    float *o0 = &out[r][16 * v], *o1 = &out[r + 1][16 * v];
                    _mm512_storeu_ps(o0, _mm512_add_ps(a0[v], _mm512_loadu_ps(o0)));
                    _mm512_storeu_ps(o1, _mm512_add_ps(a1[v], _mm512_loadu_ps(o1)));
                }
            }
#elif defined(__AVX2__) && defined(__FMA__)
            /* Two query rows x 32 dims per pass: eight accumulators. */
            for (; r + 2 <= queries; r += 2)
                for (int h = 0; h < 2; h++) {
                    __m256 a0[4], a1[4];
                    for (int v = 0; v < 4; v++) a0[v] = a1[v] = _mm256_setzero_ps();
                    for (size_t jj = 0; jj < keys; jj++) {
                        const __m256 p0 = _mm256_broadcast_ss(&st[jj][r]), p1 = _mm256_broadcast_ss(&st[jj][r + 1]);
                        const float *vr = vrow[jj] + 32 * h;
                        for (int v = 0; v < 4; v++) {
                            const __m256 x = _mm256_loadu_ps(vr + 8 * v);
                            a0[v] = _mm256_fmadd_ps(x, p0, a0[v]);
                            a1[v] = _mm256_fmadd_ps(x, p1, a1[v]);
                        }
                    }
                    for (int v = 0; v < 4; v++) {
                        float *o0 = &out[r][32 * h + 8 * v], *o1 = &out[r + 1][32 * h + 8 * v];
                        _mm256_storeu_ps(o0, _mm256_add_ps(a0[v], _mm256_loadu_ps(o0)));
                        _mm256_storeu_ps(o1, _mm256_add_ps(a1[v], _mm256_loadu_ps(o1)));
                    }
                }
#endif
            for (; r < queries; r++) {
                float acc[HD];
                for (int d = 0; d < HD; d++) acc[d] = 0.0f;
                for (size_t jj = 0; jj < keys; jj++) {
                    float p = st[jj][r];
                    for (int d = 0; d < HD; d++) acc[d] = fmaf(vrow[jj][d], p, acc[d]);
                }
                for (int d = 0; d < HD; d++) out[r][d] = acc[d] + out[r][d];
            }
        } else {
            /* reference_key_tile (prefill64.rs:887-982), as the oracle runs it. */
            for (size_t r = 0; r < queries; r++) {
                size_t absolute = first_absolute + r;
                float scores[KT];
                float block_max = -INFINITY;
                for (size_t jj = 0; jj < keys; jj++) {
                    float acc = 0.0f;
                    for (int d = 0; d < HD; d++) acc = fmaf(qt[d][r], krow[jj][d], acc);
                    float s = scale * acc;
                    if (fmasked(absolute, key_start + jj, image_start, image_end)) s = -INFINITY;
                    scores[jj] = s;
                    block_max = fmaxf(block_max, s);
                }
                float new_max = fmaxf(maxima[r], block_max);
                if (new_max == -INFINITY) {
                    for (size_t jj = 0; jj < keys; jj++) st[jj][r] = 0.0f;
                    continue;
                }
                float rescale = maxima[r] == -INFINITY ? 0.0f : expf(maxima[r] - new_max);
                for (int d = 0; d < HD; d++) out[r][d] *= rescale;
                den[r] *= rescale;
                for (size_t jj = 0; jj < keys; jj++) {
                    float p = expf(scores[jj] - new_max);
                    st[jj][r] = p;
                    den[r] += p;
                }
                maxima[r] = new_max;
            }
            for (size_t r = 0; r < queries; r++) {
                float acc[HD];
                for (int d = 0; d < HD; d++) acc[d] = 0.0f;
                for (size_t jj = 0; jj < keys; jj++)
                    for (int d = 0; d < HD; d++) acc[d] = fmaf(st[jj][r], vrow[jj][d], acc[d]);
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

void orc_attention_prefill_fast(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                                size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                                size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                                const float *sinks, int static_softmax, size_t tile_begin, size_t tile_end,
                                float *out) {
    FCache cache = {prefix_k, generated_k, v, prefix_len, total_len, n_heads, n_kv_heads};
    size_t tiles = (query_len + QT - 1) / QT;
    if (tile_end > tiles) tile_end = tiles;
    if (tile_begin >= tile_end) return;
    size_t span = tile_end - tile_begin;
#pragma omp parallel for schedule(dynamic, 1)
    for (long task = 0; task < (long)(span * n_heads); task++) {
        size_t tile = tile_begin + (size_t)task / n_heads, head = (size_t)task % n_heads;
        size_t queries = query_len - tile * QT < QT ? query_len - tile * QT : QT;
        tile_fast(q, &cache, query_offset, image_start, image_end, tile, queries, head, sinks, static_softmax, out);
    }
}
