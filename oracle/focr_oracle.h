/*
 * CPU oracle for the Falcon-OCR projection/attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference
 * operators (amazingvince/falcon-ocr-cpu, Rust), operation for operation, used
 * to check the HIP library and as the reported CPU baseline. Nothing in the
 * product links or calls it. Every function cites the reference file:line it
 * follows. Built with -ffp-contract=off: every fused multiply-add is an
 * explicit fmaf(), every other product and sum rounds on its own, as in Rust.
 */
#ifndef FOCR_ORACLE_H
#define FOCR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Epilogues of the panel GEMMs (src/kernels/panels/panel.rs:26-33). */
enum { ORC_STORE = 0, ORC_GLU = 1, ORC_ADD = 2 };

/* src/kernels/exp.rs:232-277 */
float orc_exp_poly(float x);
float orc_exp_poly_unchecked(float x);
/* src/kernels/mod.rs:567-572 */
float orc_squared_relu_glu(float gate, float up);

/* ---- A1: quantized storage ------------------------------------------- */
/* RTN quantizer, src/quant/linear.rs:140-201. codes_out is int8_t (bits 8)
 * or int16_t (bits 16). Returns 0, or a negative code for the reference's
 * error cases (-1 bits, -2 shape/group, -3 nonfinite weight, -4 overflow). */
int orc_quantize_bits(const float *w, size_t n, size_t k, size_t group, int bits,
                      void *codes_out, float *scales_out);
/* dequantize_row for every row, src/quant/linear.rs:246-262 + dot.rs:25-29.
 * bits 8/16; exception columns replace the weight in place. */
void orc_dequantize(int bits, const void *codes, const float *scales, size_t n, size_t k,
                    size_t group, const int32_t *exc_cols, const float *exc_vals, size_t n_exc,
                    float *out);
/* QuantLinear::from_parts W8 validation, src/quant/linear.rs:318-358.
 * 0 ok; negative on the first failing rule. */
int orc_validate_w8(size_t n, size_t k, size_t group, const int8_t *codes, const float *scales);

/* ---- A4 / A5: decode GEMV -------------------------------------------- */
/* simd::dot (src/simd.rs:749-777), Portable/Avx2 tree. */
float orc_dot(const float *a, const float *b, size_t len);
/* simd::dot_q (src/simd.rs:821-857). bits 8/16. */
float orc_dot_q(int bits, const float *x, const void *codes, const float *scales, size_t len,
                size_t group);
/* QuantLinear::linear small-M (src/quant/linear.rs:497-549,745-817) with
 * exception FMAs (84-118). bits 8/16; bits 32 = kernels::linear_with_simd
 * rows <= 8 over FP32 weights (src/kernels/mod.rs:407-432), scales unused. */
void orc_linear_decode(int bits, const void *codes, const float *scales, size_t n, size_t k,
                       size_t group, const int32_t *exc_cols, const float *exc_vals, size_t n_exc,
                       const float *x, size_t rows, float *out);
/* linear_glu (src/quant/linear.rs:555-625) / linear_glu_with_simd
 * (src/kernels/mod.rs:580-615): gated [rows][n/2]. */
void orc_linear_decode_glu(int bits, const void *codes, const float *scales, size_t n, size_t k,
                           size_t group, const int32_t *exc_cols, const float *exc_vals,
                           size_t n_exc, const float *x, size_t rows, float *gated);
/* The same two calls with the reference's AVX2 dot_q (focr_cpu_gemv.c):
 * bitwise orc_linear_decode(_glu), at CPU-baseline speed. */
void orc_linear_decode_fast(int bits, const void *codes, const float *scales, size_t n, size_t k, size_t group,
                            const int32_t *exc_cols, const float *exc_vals, size_t n_exc, const float *x, size_t rows,
                            float *out);
void orc_linear_decode_glu_fast(int bits, const void *codes, const float *scales, size_t n, size_t k, size_t group,
                                const int32_t *exc_cols, const float *exc_vals, size_t n_exc, const float *x,
                                size_t rows, float *gated);
/* orc_attention_decode (head dimension 64) with the reference's AVX2 dot and
 * axpy (focr_cpu_gemv.c): bitwise the same, CPU-baseline speed. */
void orc_attention_decode_fast(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                               size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                               size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                               const float *sinks, float *out);

/* ---- A6: RMS row scale ------------------------------------------------ */
/* rms_scale + sum_squares_pairwise, src/kernels/mod.rs:531-553. */
float orc_rms_scale(const float *row, size_t width, float eps);
void orc_row_scales(const float *h, size_t rows, size_t width, float eps, float *out);

/* ---- A2: FP32 panel GEMM ---------------------------------------------- */
/* panel::gemm + driver::tiled_gemm (src/kernels/panels/panel.rs:79-172,
 * driver.rs:57-140): ascending-k FMA chain from +0 per output. w is the
 * dequantized [n][k] matrix. out is [m][n] (or [m][n/2] for GLU). */
void orc_panel_gemm(const float *a, size_t m, size_t k, const float *w, size_t n,
                    const float *row_scale, int epilogue, float *out);

/* The same product with the reference's AVX2 6x16 FMA micro-kernel
 * (focr_cpu_panels.c): bitwise orc_panel_gemm, at CPU-baseline speed. */
void orc_panel_gemm_fast(const float *a, size_t m, size_t k, const float *w, size_t n,
                         const float *row_scale, int epilogue, float *out);

/* ---- A3: INT16-activation x INT8-code panel GEMM ----------------------- */
/* quantize_group, src/kernels/panels/panel_i16.rs:233-266. Returns the step. */
float orc_i16_quantize_group(const float *x, int16_t *q);
/* pack_rows + kernel_scalar + exception_tile + epilogue
 * (src/kernels/panels/panel_i16.rs:187-213,275-369). */
void orc_i16_gemm(const float *a, size_t m, size_t k, const int8_t *codes, const float *scales,
                  size_t n, const int32_t *exc_cols, const float *exc_vals, size_t n_exc,
                  const float *row_scale, int epilogue, float *out);
/* The activation quantization alone (pack_rows): codes [m][k] i16, steps
 * [m][k/64] (times row_scale), exception inputs [m][n_exc]. */
void orc_i16_quantize_rows(const float *a, size_t m, size_t k, const int32_t *exc_cols,
                           size_t n_exc, const float *row_scale, int16_t *codes, float *steps,
                           float *exc_inputs);
/* The same GEMM with the reference's AVX-512 VNNI panels
 * (focr_cpu_panels_i16.c): weights packed once per matrix, as at load;
 * bitwise orc_i16_gemm at CPU-baseline speed. n a multiple of 32, k of 64
 * (pack returns NULL otherwise). The GEMM returns -1 on a CPU without
 * AVX-512 VNNI, 0 when done. */
typedef struct orc_i16_panels orc_i16_panels;
orc_i16_panels *orc_i16_panels_pack(size_t n, size_t k, const int8_t *codes, const float *scales,
                                    const int32_t *exc_cols, const float *exc_vals, size_t n_exc);
void orc_i16_panels_free(orc_i16_panels *p);
int orc_i16_gemm_fast(const orc_i16_panels *p, const float *a, size_t m, const float *row_scale, int epilogue,
                      float *out);

/* ---- A8: BF16 prefill attention ---------------------------------------- */
/* compact_prefill (src/kernels/attention/prefill64/bf16.rs:70-175) for a pure
 * prefill (query_offset 0, query_len == total == prefix): Q, K, V rounded to
 * BF16, vdpbf16ps products (odd element first, FP32 accumulation), FP32
 * online softmax with probabilities rounded to BF16 before PV; the static
 * variant (bf16/static_shift.rs) uses 2^t with the degree-3 minimax and
 * sums the rounded probabilities. Query tiles [tile_begin, tile_end). */
void orc_attention_prefill_bf16_tiles(const float *q, const float *k, const float *v, size_t query_len,
                                      size_t n_heads, size_t n_kv_heads, size_t image_start,
                                      size_t image_end, const float *sinks, int static_softmax,
                                      int exp_fast, size_t tile_begin, size_t tile_end, float *out);
/* exp2_scalar (bf16/static_shift/tests.rs:19-24). */
float orc_exp2_minimax(float t);
/* half::bf16::from_f32(x).to_f32(). */
float orc_bf16_round(float x);

/* ---- A7: FP32 prefill attention --------------------------------------- */
/* compact_prefill / tile_head (src/kernels/attention/prefill64.rs:149-480),
 * head_dim 64. generated_k may be NULL when prefix_len == total_len.
 * static_softmax: static_shift tiles (prefill64/static_shift.rs:135-196).
 * exp_fast: ExpMode::Fast (exp_poly); else platform expf. */
void orc_attention_prefill(const float *q, const float *prefix_k, const float *generated_k,
                           const float *v, size_t query_len, size_t prefix_len, size_t total_len,
                           size_t n_heads, size_t n_kv_heads, size_t query_offset,
                           size_t image_start, size_t image_end, const float *sinks,
                           int static_softmax, int exp_fast, float *out);
/* The same over a subset of (query tile, head) tasks, for bounded CPU
 * baseline samples: tiles [tile_begin, tile_end) of every head. */
void orc_attention_prefill_tiles(const float *q, const float *prefix_k, const float *generated_k,
                                 const float *v, size_t query_len, size_t prefix_len,
                                 size_t total_len, size_t n_heads, size_t n_kv_heads,
                                 size_t query_offset, size_t image_start, size_t image_end,
                                 const float *sinks, int static_softmax, int exp_fast,
                                 size_t tile_begin, size_t tile_end, float *out);

/* orc_attention_prefill_tiles with exp_fast = 1, vectorized across the 32
 * query lanes (focr_cpu_attention.c): bitwise the same, CPU-baseline speed. */
void orc_attention_prefill_fast(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                                size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                                size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                                const float *sinks, int static_softmax, size_t tile_begin, size_t tile_end,
                                float *out);

/* ---- the QKV row step --------------------------------------------------- */
/* fused_row (src/model/fused.rs:101-123) for rows < prefix_rows, and
 * split_norm_rope + append_unique_heads (src/model/rope.rs:14-86,
 * src/model/cache.rs:202-216) for the rest; head_dim 64. qkv
 * [rows][qdim + 2 kdim]; rope [rows][n_heads][32][2]; q [rows][n_heads][64];
 * prefix_k [prefix_rows][n_heads][64]; generated_k [rows-prefix_rows][n_kv][64];
 * v [rows][n_kv][64]. */
void orc_qkv_rows(const float *qkv, size_t rows, const float *rope, size_t n_heads, size_t n_kv_heads,
                  size_t prefix_rows, float *q, float *prefix_k, float *generated_k, float *v);

/* ---- decode attention --------------------------------------------------- */
/* online::head (src/kernels/attention/online.rs:96-150) for every (query,
 * head), as decode64 and online::attention run it (query_len 1..3 in the
 * reference; any count here), platform expf/logf. */
void orc_attention_decode(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                          size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                          size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                          const float *sinks, float *out);
/* orc_attention_decode; exp_fast = 1 takes the per-key probabilities
 * exp(s - max) from orc_exp_poly, as the sealed cache's decode does with
 * SplitPrefix::fast_exp (src/quant/kv/decode.rs:346-347 through
 * simd::Avx2Fast, src/simd.rs:440-445); the rescale and the sink stay expf. */
void orc_attention_decode_ex(const float *q, const float *prefix_k, const float *generated_k, const float *v,
                             size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads,
                             size_t n_kv_heads, size_t query_offset, size_t image_start, size_t image_end,
                             const float *sinks, int exp_fast, float *out);

/* ---- A9: greedy selection --------------------------------------------- */
/* argmax, src/runner/mod.rs:916-930. 0 ok, -1 on non-finite/empty. */
int orc_argmax(const float *logits, size_t n, uint32_t *out);

/* ---- INT8 screened vocabulary head (src/head_screen.rs) ------------------ */
#define ORC_SCREEN_GROUP 64
#define ORC_SCREEN_LIMIT 1024
/* kappa of a dim-wide head (head_screen.rs:99-106), NaN if >= 0.53. */
float orc_screen_kappa(size_t dim);
/* ScreenedHead::build / quantize_row: codes [vocab][dim], scales
 * [vocab][dim/64]; 0 ok, -1 on shape, non-finite weight or premise. */
int orc_screen_build(const float *w, size_t vocab, size_t dim, int8_t *codes, float *scales,
                     float *weight_abs_max, float *kappa);
/* prepare: 1 with norms [dim/64], or 0 when the proof's assumptions fail. */
int orc_screen_prepare(const float *x, size_t dim, float weight_abs_max, float *norms);
/* screen_row in the AVX2 order: approximate logit q and S = sum s_g n_g. */
void orc_screen_row(const float *x, const int8_t *codes, const float *scales, const float *norms,
                    size_t dim, float *q, float *s);
/* select: 1 = Token (*token, *candidates), 0 = Fallback (*candidates);
 * upper [vocab] receives q + B. */
int orc_screen_select(const float *x, const float *fp32, const int8_t *codes, const float *scales,
                      size_t vocab, size_t dim, float weight_abs_max, float kappa, float *upper,
                      uint32_t *token, uint32_t *candidates);

/* ---- Sealed split KV cache, Kv::Q8 / Kv::Q16 (src/quant/kv.rs) ------------ */
uint16_t orc_bf16_up(float scale);
float orc_bf16_f32(uint16_t bits);
/* SplitPrefix::seal: records [n_kv][P][160] codes (int8 for bits 8, int16
 * for 16) and BF16 steps [n_kv][P][5]. 0 ok; -1 temporal keys differ inside
 * a pair; -2 non-finite value; -3 decoded overflow; -4 shape. */
int orc_kv_seal(int bits, const float *prefix_k, const float *v, size_t prefix_len, size_t n_heads,
                size_t n_kv, void *codes, uint16_t *scales);
/* push_unique: generated position `index` of a [n_kv][capacity] tail; keys
 * and values [n_kv][64]; tail records [128] codes and 4 steps. */
void orc_kv_push(int bits, const float *k, const float *v, size_t n_kv, size_t capacity, size_t index,
                 void *codes, uint16_t *scales);
/* The decoded cache in the compact layout: prefix keys [P][n_heads][64],
 * values [P + tail_len][n_kv][64], generated keys [tail_len][n_kv][64]. */
void orc_kv_dequantize(int bits, const void *codes, const uint16_t *scales, size_t prefix_len, size_t n_heads,
                       size_t n_kv, const void *tail_codes, const uint16_t *tail_scales, size_t capacity,
                       size_t tail_len, float *prefix_k, float *values, float *generated_k);

/* Threads the oracle uses for its parallel loops (1 = scalar). */
void orc_set_threads(int threads);
int orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
