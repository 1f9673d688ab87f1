/*
 * CPU oracle of the sealed (Q8 / Q16) split KV cache — TEST INFRASTRUCTURE
 * ONLY (tests/; the product never links this file).
 *
 * Restates src/quant/kv.rs and src/quant/kv/codec.rs for Kv::Q8 and Kv::Q16:
 *  - group-major prefix records of 160 elements [T 0..32 | S(2g) 32..64 |
 *    S(2g+1) 64..96 | V 96..160] (kv.rs:1-24, gather 277-293): the temporal
 *    half of the key, shared by both heads of a GQA pair, each head's spatial
 *    half and the value;
 *  - each 32-element block coded against the smallest BF16 step at or above
 *    absmax / 127 (or / 32767) (q8_scale / q16_scale, bf16_up; codec.rs
 *    9-45), codes round_clamped(value / step) in f64, ties to even (codec.rs
 *    58-86); seal refuses differing temporal keys inside a pair, non-finite
 *    values and decoded overflow (kv.rs:254-330);
 *  - generated positions as 128-element tail records [K | V] per group
 *    (push_unique, kv.rs:451-515), a non-finite block coded against a NaN step
 *    (every element of it decodes to NaN);
 *  - the decoded values (code as f32 times the widened BF16 step; Records::
 *    value, kv.rs:208-217), arranged as the compact cache (dequantized_compact,
 *    kv.rs:533-563) so the decode attention oracle (orc_attention_decode) runs
 *    on them: decode over records is the compact kernel over their decoded
 *    values (kv.rs:7-17).
 *
 * Parity status: pinned by the codec's closed forms and edge cases (tests/
 * test_oracle_kv.py: bf16_up on exact and inexact steps and NaN, the ties of
 * round_clamped, the clamp, a zero block, the smallest-subnormal floor, NaN
 * blocks of the tail), by |decoded - value| <= step / 2 on every element, by
 * the exact round trip of values that are already multiples of their step,
 * and by the reference's pair-sharing and finiteness refusals.
 */
#include "focr_oracle.h"

#include <math.h>
#include <string.h>

#define RECORD 160
#define TAIL 128

uint16_t orc_bf16_up(float scale) {
    if (scale != scale) return 0x7FC0;
    uint32_t bits;
    memcpy(&bits, &scale, 4);
    const uint16_t high = (uint16_t)(bits >> 16);
    return (bits & 0xFFFF) ? (uint16_t)(high + 1) : high;
}

float orc_bf16_f32(uint16_t bits) {
    const uint32_t wide = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &wide, 4);
    return f;
}

/* The step of a block: absmax / limit in f64 rounded to f32, at least the
 * smallest subnormal, 0 for an all-zero block. */
static float block_step(const float *values, double limit) {
    float max = 0.0f;
    for (int i = 0; i < 32; i++) {
        const float a = fabsf(values[i]);
        max = a > max ? a : max; /* f32::max of finite values */
    }
    if (max == 0.0f) return 0.0f;
    const float s = (float)((double)max / limit);
    const float tiny = 1.40129846e-45f;
    return s > tiny ? s : tiny;
}

/* round_clamped: clamp to +-limit, then round to nearest even (NaN stays
 * NaN); the integer cast of NaN is 0, as Rust's saturating `as`. */
static long code_of(float value, float scale, double limit) {
    if (scale == 0.0f) return 0;
    double x = (double)value / (double)scale;
    if (x != x) return 0;
    x = x < -limit ? -limit : (x > limit ? limit : x);
    return (long)nearbyint(x);
}

static void put_code(int bits, void *codes, size_t at, long c) {
    if (bits == 8)
        ((int8_t *)codes)[at] = (int8_t)c;
    else
        ((int16_t *)codes)[at] = (int16_t)c;
}

static float get_code(int bits, const void *codes, size_t at) {
    return bits == 8 ? (float)((const int8_t *)codes)[at] : (float)((const int16_t *)codes)[at];
}

int orc_kv_seal(int bits, const float *prefix_k, const float *v, size_t prefix_len, size_t n_heads, size_t n_kv,
                void *codes, uint16_t *scales) {
    if ((bits != 8 && bits != 16) || n_heads != 2 * n_kv || prefix_len == 0) return -4;
    const double limit = bits == 8 ? 127.0 : 32767.0;
    for (size_t t = 0; t < prefix_len; t++)
        for (size_t g = 0; g < n_kv; g++) {
            const float *a = prefix_k + (t * n_heads + 2 * g) * 64;
            if (memcmp(a, a + 64, 32 * sizeof(float)) != 0) return -1;
        }
    for (size_t g = 0; g < n_kv; g++)
        for (size_t t = 0; t < prefix_len; t++) {
            const size_t record = g * prefix_len + t;
            const float *a = prefix_k + (t * n_heads + 2 * g) * 64;
            const float *b = a + 64;
            float values[RECORD];
            memcpy(values, a, 32 * sizeof(float));
            memcpy(values + 32, a + 32, 32 * sizeof(float));
            memcpy(values + 64, b + 32, 32 * sizeof(float));
            memcpy(values + 96, v + (t * n_kv + g) * 64, 64 * sizeof(float));
            for (int i = 0; i < RECORD; i++)
                if (!isfinite(values[i])) return -2;
            for (int blk = 0; blk < RECORD / 32; blk++) {
                const uint16_t stored = orc_bf16_up(block_step(values + 32 * blk, limit));
                scales[record * 5 + blk] = stored;
                const float step = orc_bf16_f32(stored);
                for (int i = 0; i < 32; i++) {
                    const long c = code_of(values[32 * blk + i], step, limit);
                    put_code(bits, codes, record * RECORD + 32 * blk + i, c);
                    if (!isfinite((float)c * step)) return -3;
                }
            }
        }
    return 0;
}

void orc_kv_push(int bits, const float *k, const float *v, size_t n_kv, size_t capacity, size_t index, void *codes,
                 uint16_t *scales) {
    const double limit = bits == 8 ? 127.0 : 32767.0;
    for (size_t g = 0; g < n_kv; g++) {
        float values[TAIL];
        memcpy(values, k + g * 64, 64 * sizeof(float));
        memcpy(values + 64, v + g * 64, 64 * sizeof(float));
        const size_t record = g * capacity + index;
        for (int blk = 0; blk < TAIL / 32; blk++) {
            int finite = 1;
            for (int i = 0; i < 32; i++) finite &= isfinite(values[32 * blk + i]) != 0;
            const uint16_t stored = orc_bf16_up(finite ? block_step(values + 32 * blk, limit) : NAN);
            scales[record * 4 + blk] = stored;
            const float step = orc_bf16_f32(stored);
            for (int i = 0; i < 32; i++)
                put_code(bits, codes, record * TAIL + 32 * blk + i, code_of(values[32 * blk + i], step, limit));
        }
    }
}

void orc_kv_dequantize(int bits, const void *codes, const uint16_t *scales, size_t prefix_len, size_t n_heads,
                       size_t n_kv, const void *tail_codes, const uint16_t *tail_scales, size_t capacity,
                       size_t tail_len, float *prefix_k, float *values, float *generated_k) {
    for (size_t g = 0; g < n_kv; g++) {
        for (size_t t = 0; t < prefix_len; t++) {
            const size_t record = g * prefix_len + t;
            float x[RECORD];
            for (int i = 0; i < RECORD; i++)
                x[i] = get_code(bits, codes, record * RECORD + i) * orc_bf16_f32(scales[record * 5 + i / 32]);
            for (int pair = 0; pair < 2; pair++) {
                float *dst = prefix_k + (t * n_heads + 2 * g + pair) * 64;
                memcpy(dst, x, 32 * sizeof(float));
                memcpy(dst + 32, x + 32 + 32 * pair, 32 * sizeof(float));
            }
            memcpy(values + (t * n_kv + g) * 64, x + 96, 64 * sizeof(float));
        }
        for (size_t i = 0; i < tail_len; i++) {
            const size_t record = g * capacity + i;
            for (int d = 0; d < TAIL; d++) {
                const float x = get_code(bits, tail_codes, record * TAIL + d) * orc_bf16_f32(tail_scales[record * 4 + d / 32]);
                if (d < 64)
                    generated_k[(i * n_kv + g) * 64 + d] = x;
                else
                    values[((prefix_len + i) * n_kv + g) * 64 + d - 64] = x;
            }
        }
    }
}
