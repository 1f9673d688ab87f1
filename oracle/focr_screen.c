/*
 * CPU oracle of the INT8 screened vocabulary head — TEST INFRASTRUCTURE ONLY
 * (tests/ and the bench's CPU leg; the product never links this file).
 *
 * Restates src/head_screen.rs: the RTN INT8 screen of the FP32 head
 * (quantize_row, 328-366; kappa, 99-106), the per-input preparation
 * (prepare, 203-231), the screen of one row in the AVX2 order (screen_row,
 * 370-395: per 64-group two 8-lane FMA chains, lane-wise (a0 + a1) * scale
 * accumulated over the groups, the AVX2 horizontal sum; S = sum fma(s, n)),
 * the bounds (screen_block, 400-425: B = fma(kappa, S, 2^-100)) and the exact
 * selection (finish, 234-270: candidates q + B >= tau in ascending order,
 * their FP32 logits with the reference dot, strict > for the first index).
 *
 * Parity status: pinned. The token is checked against the full-head argmax
 * (orc_dot + orc_argmax) on the reference's own test scenarios (planted
 * duplicate rows aimed at, so ties decide), the bound against the f64 logit
 * under the adversarial rounding direction, kappa against its closed form in
 * f64, and the fallbacks (non-finite input, all-zero input past the
 * candidate limit, huge input) as the reference tests them
 * (src/head_screen.rs:522-699; tests/test_oracle_screen.py).
 */
#include "focr_oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>

#define GROUP ORC_SCREEN_GROUP
#define LIMIT ORC_SCREEN_LIMIT
static const float kEta = 7.888609e-31f; /* 2^-100 */

static double gamma_n(size_t n) {
    const double u = (double)FLT_EPSILON / 2.0;
    const double nu = (double)n * u;
    return nu / (1.0 - nu);
}

float orc_screen_kappa(size_t dim) {
    const size_t groups = dim / GROUP;
    const double k = (0.5 * (1.0 + ldexp(1.0, -20)) + gamma_n(dim) * 127.5 * (1.0 + ldexp(1.0, -20)) +
                      gamma_n(dim + groups + 8) * 127.0) *
                         (1.0 + 1e-3) +
                     2e-3;
    if (!(k < 0.53)) return NAN;
    return nextafterf((float)k, INFINITY);
}

int orc_screen_build(const float *w, size_t vocab, size_t dim, int8_t *codes, float *scales, float *weight_abs_max,
                     float *kappa) {
    if (vocab == 0 || dim == 0 || dim % GROUP != 0) return -1;
    const size_t groups = dim / GROUP;
    float wmax = 0.0f;
    for (size_t r = 0; r < vocab; r++) {
        for (size_t g = 0; g < groups; g++) {
            const float *values = w + r * dim + g * GROUP;
            float maximum = 0.0f;
            for (size_t i = 0; i < GROUP; i++) {
                if (!isfinite(values[i])) return -1;
                const float a = fabsf(values[i]);
                maximum = a > maximum ? a : maximum;
            }
            wmax = maximum > wmax ? maximum : wmax;
            float scale = 0.0f;
            if (maximum != 0.0f) {
                scale = (float)((double)maximum / 127.0);
                const float tiny = 1.40129846e-45f; /* f32::from_bits(1) */
                scale = scale > tiny ? scale : tiny;
            }
            scales[r * groups + g] = scale;
            const double tolerance = (double)scale * 0.5 * (1.0 + ldexp(1.0, -20));
            for (size_t i = 0; i < GROUP; i++) {
                int8_t code = 0;
                if (scale != 0.0f) {
                    double c = nearbyint((double)values[i] / (double)scale);
                    c = c < -127.0 ? -127.0 : (c > 127.0 ? 127.0 : c);
                    code = (int8_t)c;
                }
                codes[r * dim + g * GROUP + i] = code;
                const double rec = (double)code * (double)scale;
                if (!(fabs((double)values[i] - rec) <= tolerance &&
                      fabs((double)values[i]) <= 127.5 * (double)scale * (1.0 + ldexp(1.0, -20))))
                    return -1;
            }
        }
    }
    if (!isfinite(wmax)) return -1;
    const float k = orc_screen_kappa(dim);
    if (!(k == k)) return -1;
    *weight_abs_max = wmax;
    *kappa = k;
    return 0;
}

int orc_screen_prepare(const float *x, size_t dim, float weight_abs_max, float *norms) {
    for (size_t i = 0; i < dim; i++)
        if (!isfinite(x[i])) return 0;
    double l1 = 0.0;
    for (size_t i = 0; i < dim; i++) l1 += (double)fabsf(x[i]);
    if (l1 * (double)weight_abs_max * 1.01 >= (double)FLT_MAX / 2.0) return 0;
    for (size_t g = 0; g < dim / GROUP; g++) {
        double exact = 0.0;
        for (size_t i = 0; i < GROUP; i++) exact += (double)fabsf(x[g * GROUP + i]);
        const float rounded = (float)exact;
        norms[g] = (double)rounded < exact ? nextafterf(rounded, INFINITY) : rounded;
    }
    return 1;
}

static float sum8(const float v[8]) { return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7])); }

void orc_screen_row(const float *x, const int8_t *codes, const float *scales, const float *norms, size_t dim, float *q,
                    float *s) {
    float row[8] = {0};
    float total = 0.0f;
    for (size_t g = 0; g < dim / GROUP; g++) {
        const size_t base = g * GROUP;
        float a0[8] = {0}, a1[8] = {0};
        for (size_t j = 0; j < GROUP; j += 16)
            for (int p = 0; p < 8; p++) {
                a0[p] = fmaf(x[base + j + p], (float)codes[base + j + p], a0[p]);
                a1[p] = fmaf(x[base + j + 8 + p], (float)codes[base + j + 8 + p], a1[p]);
            }
        for (int p = 0; p < 8; p++) row[p] = fmaf(a0[p] + a1[p], scales[g], row[p]);
        total = fmaf(scales[g], norms[g], total);
    }
    *q = sum8(row);
    *s = total;
}

int orc_screen_select(const float *x, const float *fp32, const int8_t *codes, const float *scales, size_t vocab,
                      size_t dim, float weight_abs_max, float kappa, float *upper, uint32_t *token,
                      uint32_t *candidates) {
    const size_t groups = dim / GROUP;
    float norms[64];
    *token = 0;
    *candidates = 0;
    if (groups > 64 || !orc_screen_prepare(x, dim, weight_abs_max, norms)) return 0;
    float tau = -INFINITY;
    for (size_t v = 0; v < vocab; v++) {
        float q, s;
        orc_screen_row(x, codes + v * dim, scales + v * groups, norms, dim, &q, &s);
        const float bound = fmaf(kappa, s, kEta);
        upper[v] = q + bound;
        const float lower = q - bound;
        tau = lower > tau ? lower : tau; /* f32::max: a NaN operand is ignored */
    }
    if (!isfinite(tau)) return 0;
    uint32_t count = 0, best = 0;
    float best_value = 0.0f;
    int have = 0;
    for (size_t v = 0; v < vocab; v++) {
        if (!(upper[v] >= tau)) continue;
        if (count == LIMIT) {
            *candidates = LIMIT + 1;
            return 0;
        }
        count++;
    }
    for (size_t v = 0; v < vocab; v++) {
        if (!(upper[v] >= tau)) continue;
        const float logit = orc_dot(x, fp32 + v * dim, dim);
        if (!isfinite(logit)) return 0;
        if (!have || logit > best_value) {
            best = (uint32_t)v;
            best_value = logit;
            have = 1;
        }
    }
    if (!have) return 0;
    *token = best;
    *candidates = count;
    return 1;
}
