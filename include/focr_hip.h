/*
 * focr_hip.h — C ABI of the MI355X (gfx950) backend for the Falcon-OCR
 * runner's projection linears and prefill attention.
 *
 * The reference (amazingvince/falcon-ocr-cpu) is a Rust crate with no C ABI;
 * each entry point below replaces one of its operator interfaces, cited by
 * file:line. A Rust `extern "C"` crate binds these declarations as a new
 * `hip` backend next to avx2|scalar|neon (src/config.rs:19-35).
 *
 * Conventions
 *  - Every function returns FOCR_OK (0) or a negative FOCR_E_* code and never
 *    aborts; focr_last_error() returns the message of the calling thread's
 *    last failure. Shape misuse that the reference asserts on
 *    (src/kernels/panels/driver.rs:66-78, src/quant/linear.rs:654-662) is an
 *    FOCR_E_SHAPE error here.
 *  - Pointers named *_dev are device (HBM) addresses; everything else is a
 *    host address. Compute calls are asynchronous on the context's stream;
 *    focr_ctx_sync() waits for them. One context serves one thread at a time;
 *    two contexts may run concurrently (the reference's prefill pool and
 *    decode team, src/runner/pipeline.rs:1-4).
 *  - Results never depend on launch configuration: every output has one
 *    fixed operation sequence.
 */
#ifndef FOCR_HIP_H
#define FOCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define FOCR_OK 0
#define FOCR_E_ARG (-1)         /* null pointer or invalid enum value */
#define FOCR_E_SHAPE (-2)       /* shapes that do not fit the operator */
#define FOCR_E_UNSUPPORTED (-3) /* valid, but not supported by this backend */
#define FOCR_E_HIP (-4)         /* a HIP runtime error */
#define FOCR_E_VALUE (-5)       /* invalid data (e.g. a W8 code of -128) */
#define FOCR_E_NONFINITE (-6)   /* non-finite logits (argmax) */

/* ---- enums --------------------------------------------------------------- */
/* Epilogue, src/kernels/panels/panel.rs:26-33. */
#define FOCR_EPI_STORE 0 /* out[m][n] = C */
#define FOCR_EPI_GLU 1   /* out[m][i] = squared_relu_glu(C[m][2i], C[m][2i+1]) */
#define FOCR_EPI_ADD 2   /* out[m][n] += C (residual add) */

/* Prefill projection kernel, the `hip` counterparts of PrefillProjection
 * (src/kernels/mod.rs:71-84). */
#define FOCR_PROJ_F32_MFMA 0  /* FP32 weights or fl(code*scale), FP32 matrix cores
                                 (tolerance-matched to the FP32 panels) */
#define FOCR_PROJ_F32_CHAIN 1 /* FP32 panels' exact order: one ascending-k FMA
                                 chain per output (bitwise PanelAvx2) */
#define FOCR_PROJ_I16 2       /* INT16 activations x INT8 codes, exact INT32 group
                                 sums (bitwise PanelI16Vnni/PanelI16Avx2) */
#define FOCR_PROJ_F32_SPLIT 3 /* FP32 weights: every row of both operands
                                 scaled by a power of two and written as FP16
                                 pairs (hi + lo), three pair products per FP32
                                 product on the FP16 matrix cores, FP32
                                 accumulation, exact descale (tolerance-matched
                                 like FOCR_PROJ_F32_MFMA); outputs a row holding
                                 an infinity or NaN reaches are the FP32 panel
                                 chain's, bitwise */

/* Prefill softmax (src/config.rs PrefillSoftmax) and exp (ExpMode). */
#define FOCR_SOFTMAX_ONLINE 0
#define FOCR_SOFTMAX_STATIC 1
#define FOCR_EXP_FAST 0  /* exp_poly, src/kernels/exp.rs:232-277 */
#define FOCR_EXP_EXACT 1 /* the device libm expf */

typedef struct focr_ctx focr_ctx;
typedef struct focr_linear focr_linear;
typedef struct focr_screen focr_screen;
typedef struct focr_kv_split focr_kv_split;

/* ---- context ------------------------------------------------------------ */
/* No reference counterpart (the CPU runner needs no device state); the
 * Rust backend creates one per Rayon pool / decode team. */
int focr_ctx_create(int device, focr_ctx **out);
int focr_ctx_destroy(focr_ctx *ctx);
/* Run on an existing hipStream_t (e.g. a framework's stream) instead of the
 * context's own; NULL selects the device's default (null) stream. The new
 * stream first waits (an event) for the work already queued on the old one,
 * which may still read the context scratch. When either stream is being
 * captured that wait cannot be recorded and the switch happens without it:
 * the caller orders the streams itself (e.g. side.wait_stream(current)
 * before a capture on a side stream). */
int focr_ctx_set_stream(focr_ctx *ctx, void *hip_stream);
/* Return to the context's own stream (with the same wait). */
int focr_ctx_use_own_stream(focr_ctx *ctx);
void *focr_ctx_stream(const focr_ctx *ctx);
int focr_ctx_sync(focr_ctx *ctx);
/* The context scratch (INT16 activation codes, attention partial states,
 * BF16 K/V copies) grows on demand by free + malloc. No reference
 * counterpart: the reference's Scratch (src/quant/linear.rs:311-315) is a
 * host Vec. Growing invalidates graphs captured earlier (they would replay
 * into freed memory) and is refused with FOCR_E_UNSUPPORTED while the
 * stream is capturing: a caller that captures reserves the largest size
 * first, or makes one uncaptured call of each shape. Synchronizes the
 * context's stream when it grows.
 * Device buffers a context owns, and so the only addresses of its own that a
 * captured graph can hold: the scratch (above) and an 8-float row-scale
 * array allocated at creation (focr_argmax's result words are read back to
 * the host within the call, which therefore cannot be captured). No
 * context buffer holds weights: prefill on INT8/INT16 codes reads the codes
 * and forms fl(code * scale) in registers. */
int focr_ctx_reserve_scratch(focr_ctx *ctx, size_t bytes);
int focr_ctx_scratch_bytes(const focr_ctx *ctx, size_t *bytes);
/* Message of the calling thread's last failure ("" if none). */
const char *focr_last_error(void);
/* Device memory helpers for callers without HIP headers. */
int focr_malloc(focr_ctx *ctx, size_t bytes, void **out_dev);
int focr_free(focr_ctx *ctx, void *dev);
int focr_memcpy_h2d(focr_ctx *ctx, void *dst_dev, const void *src, size_t bytes);
int focr_memcpy_d2h(focr_ctx *ctx, void *dst, const void *src_dev, size_t bytes);

/* ---- A1: quantized linear storage --------------------------------------- */
/* Upload one matrix into a device handle, the device side of
 * QuantLinear::from_parts / from_mapped / with_exceptions
 * (src/quant/linear.rs:318-358,392-455) and of the FP32 weight slices of
 * kernels::linear_with_simd (src/kernels/mod.rs:387-398).
 *   bits 8: codes int8 [out][in] (W8 rules of from_parts are checked:
 *           no -128, finite non-negative scales, zero codes in zero-scale
 *           groups); bits 16: codes int16 [out][in]; bits 32: FP32 weights
 *           [out][in], scales NULL, group ignored.
 *   scales: FP32 [out][ceil(in/group)], group 32, 64 or 128.
 *   exc_cols/exc_vals: optional exception columns (sorted, unique, < in)
 *           and their FP32 weights [out][n_exc]; codes there must be zero.
 * Host pointers; the call copies them and returns when the upload is done. */
int focr_linear_upload(focr_ctx *ctx, int bits, size_t out_dim, size_t in_dim, size_t group,
                       const void *codes, const float *scales, const int32_t *exc_cols,
                       const float *exc_vals, size_t n_exc, focr_linear **out);
int focr_linear_free(focr_linear *lin);
int focr_linear_info(const focr_linear *lin, int *bits, size_t *out_dim, size_t *in_dim,
                     size_t *group, size_t *n_exc, size_t *device_bytes);
/* fl(code * scale) for every weight, exception columns in place:
 * QuantLinear::dequantize_row for all rows (src/quant/linear.rs:246-262).
 * out_dev: FP32 [out][in]. Bit-exact. */
int focr_linear_dequantize(focr_ctx *ctx, const focr_linear *lin, float *out_dev);

/* ---- A4 / A5: decode and draft-verify GEMV ------------------------------ */
/* QuantLinear::linear for 1..=8 rows (src/quant/linear.rs:497-549,783-817),
 * and kernels::linear_with_simd rows <= 8 for bits 32
 * (src/kernels/mod.rs:407-432). x_dev [rows][in], out_dev [rows][out].
 * Bitwise equal to the reference's AVX2/NEON/portable dot_q / dot order. */
int focr_linear_decode(focr_ctx *ctx, const focr_linear *lin, const float *x_dev, size_t rows,
                       float *out_dev);
/* QuantLinear::linear_glu / kernels::linear_glu_with_simd for 1..=8 rows
 * (src/quant/linear.rs:555-625, src/kernels/mod.rs:580-615): gated_dev
 * [rows][out/2] from interleaved [gate, up] rows. Bitwise. */
int focr_linear_decode_glu(focr_ctx *ctx, const focr_linear *lin, const float *x_dev,
                           size_t rows, float *gated_dev);

/* The decode step's projections with their neighbours folded in, as
 * Model::project_qkv / attention_out_ffn call them for 1..=8 rows
 * (src/model/mod.rs:421-492):
 *   rms_norm 1: each input row is first rms-normalized (kernels::rms_norm,
 *     unit weight, eps f32::EPSILON, src/kernels/mod.rs:481-533), computed
 *     inside the GEMV; row_scale_dev must then be NULL;
 *   row_scale_dev optional [rows]: a precomputed factor (focr_row_scales)
 *     multiplied into each row instead (rms_norm_row's `x * scale`);
 *   epilogue FOCR_EPI_STORE (linear), FOCR_EPI_GLU (linear_glu, out
 *     [rows][out/2]) or FOCR_EPI_ADD (add_residual, src/model/rope.rs:155-169:
 *     out += projection).
 * Bitwise equal to the separate reference passes. */
int focr_linear_decode_ex(focr_ctx *ctx, const focr_linear *lin, const float *x_dev, size_t rows,
                          const float *row_scale_dev, int rms_norm, int epilogue, float *out_dev);

/* ---- A2 / A3: prefill projection ---------------------------------------- */
/* QuantLinear::prefill (src/quant/linear.rs:634-707) and its FP32 panel
 * and INT16 panel kernels (src/kernels/panels/{panel,panel_i16}.rs).
 *   x_dev [rows][in]; row_scale_dev optional [rows] (an RMS norm folded
 *   into packing); epilogue FOCR_EPI_*; kernel FOCR_PROJ_*.
 *   out_dev [rows][out] (STORE, ADD) or [rows][out/2] (GLU).
 * FOCR_PROJ_I16 needs 8-bit codes, group 64, out % 32 == 0, in % 64 == 0
 * (fits_i16_panels, src/quant/linear.rs:29-31); it uses a scratch buffer the
 * context owns and grows. FOCR_PROJ_F32_SPLIT needs FP32 weights
 * (FOCR_E_UNSUPPORTED for codes) and keeps the FP16 pairs, 4 bytes per
 * element of x and of the weights (rows and out rounded up to 128, in to 32),
 * and a row exponent each, in the same scratch buffer. */
int focr_linear_prefill(focr_ctx *ctx, const focr_linear *lin, const float *x_dev, size_t rows,
                        const float *row_scale_dev, int epilogue, int kernel, float *out_dev);

/* ---- A6: RMS row scales -------------------------------------------------- */
/* rms_scale of every width-wide row (src/kernels/mod.rs:531-553, row_scales
 * src/model/rope.rs:147-152): 1/sqrt(pairwise_sum_squares/width + eps).
 * Bitwise. */
int focr_row_scales(focr_ctx *ctx, const float *h_dev, size_t rows, size_t width, float eps,
                    float *out_dev);

/* ---- A7: prefill attention ---------------------------------------------- */
/* kernels::attention_with for a prefill (src/kernels/attention/mod.rs:256-311)
 * over a compact cache (CompactKv, 85-196), head_dim 64:
 *   q_dev [query_len][n_heads][64]; prefix_k_dev [prefix_len][n_heads][64];
 *   generated_k_dev [total_len - prefix_len][n_kv_heads][64] (NULL when
 *   prefix_len == total_len); v_dev [total_len][n_kv_heads][64];
 *   Geometry (query_offset, image_start, image_end); sinks_dev [n_heads];
 *   softmax FOCR_SOFTMAX_*; exp FOCR_EXP_*; out_dev like q.
 * FP32 matrix cores: within the FP32 tolerance of the reference tiles. */
int focr_attention_prefill(focr_ctx *ctx, const float *q_dev, const float *prefix_k_dev,
                           const float *generated_k_dev, const float *v_dev, size_t query_len,
                           size_t prefix_len, size_t total_len, size_t n_heads,
                           size_t n_kv_heads, size_t head_dim, size_t query_offset,
                           size_t image_start, size_t image_end, const float *sinks_dev,
                           int softmax, int exp_mode, float *out_dev);

/* The same attention for a pure prefill (query_offset 0, every key a prefix
 * key, query_len == prefix_len == total_len), with every QK and PV product
 * formed on the FP16 matrix cores from two-term FP16 expansions of its FP32
 * operands scaled by powers of two (x 2^e = hi + lo to about 2^-22; the
 * three largest part products, FP32 accumulation, exact descaling; scales
 * per query row, per 32-key tile of K, per value dim, per tile or query of
 * P): within the FP32 tolerance of the reference tiles, like
 * focr_attention_prefill, at about twice its speed. A call whose K or V
 * holds an infinity or NaN runs focr_attention_prefill's FP32 products on the
 * device instead (its outputs bitwise that entry point's). Other geometries
 * return FOCR_E_UNSUPPORTED and write nothing (focr_attention_prefill takes
 * them). Writes K and V as FP16 pairs into the context scratch first. */
int focr_attention_prefill_split(focr_ctx *ctx, const float *q_dev, const float *prefix_k_dev,
                                 const float *generated_k_dev, const float *v_dev, size_t query_len,
                                 size_t prefix_len, size_t total_len, size_t n_heads,
                                 size_t n_kv_heads, size_t head_dim, size_t query_offset,
                                 size_t image_start, size_t image_end, const float *sinks_dev,
                                 int softmax, int exp_mode, float *out_dev);

/* ---- A8: BF16 prefill attention ----------------------------------------- */
/* kernels::attention_prefill_bf16 (src/kernels/attention/mod.rs:320-352) ->
 * prefill64::bf16::compact_prefill (prefill64/bf16.rs:70-175, plans Bf16 /
 * Bf16Static): a pure prefill (query_offset 0, every key a prefix key),
 * q_dev / k_dev [query_len][n_heads][64], v_dev [query_len][n_kv_heads][64].
 * Q, K, V and the probabilities are rounded to BF16; products accumulate in
 * FP32 on the BF16 matrix cores; softmax FOCR_SOFTMAX_ONLINE or _STATIC
 * (the static shift needs scores bounded, as the reference's does). exp_mode
 * is accepted for the interface; both use the hardware exp2 (the result is
 * within the BF16 tolerance, 2e-3, of either reference exp). Where the
 * reference returns false (query_len < 4, head_dim != 64) this returns
 * FOCR_E_UNSUPPORTED and writes nothing. Converts K and V into the context
 * scratch first. */
int focr_attention_prefill_bf16(focr_ctx *ctx, const float *q_dev, const float *k_dev,
                                const float *v_dev, size_t query_len, size_t n_heads,
                                size_t n_kv_heads, size_t head_dim, size_t image_start,
                                size_t image_end, const float *sinks_dev, int softmax,
                                int exp_mode, float *out_dev);

/* ---- the QKV row step (split, per-head RMS norm, RoPE, cache append) ---- */
/* fused_prefix_rows / fused_row (src/model/fused.rs:17-123) for the first
 * prefix_rows rows, and split_norm_rope + LayerCache::append
 * (src/model/rope.rs:14-86, src/model/cache.rs:117-140,202-216) for the
 * rest, head_dim 64:
 *   qkv_dev [rows][n_heads*64 + 2*n_kv_heads*64] (the QKV projection rows);
 *   rope_dev [rows][n_heads][32][2] ([cos, sin] per rotated pair, as
 *   rotary_factors builds them, src/model/rope.rs:103-142);
 *   q_dev [rows][n_heads][64] normalized and rotated queries;
 *   prefix_k_dev [prefix_rows][n_heads][64] (keys of every query head: the
 *   KV head h/(n_heads/n_kv_heads), rotated with head h's factors);
 *   generated_k_dev [rows - prefix_rows][n_kv_heads][64] (one key per KV
 *   head: the expanded head g*(n_heads/n_kv_heads));
 *   v_dev [rows][n_kv_heads][64] (values, copied).
 * Per head: y = x * (1/sqrt(pairwise_sum(x^2)/64 + f32::EPSILON)), then
 * (a, b) -> (a*cos - b*sin, a*sin + b*cos). Bitwise. The output pointers
 * are the cache slots of the first row (append = write at the end). */
int focr_qkv_rows(focr_ctx *ctx, const float *qkv_dev, size_t rows, const float *rope_dev,
                  size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t prefix_rows,
                  float *q_dev, float *prefix_k_dev, float *generated_k_dev, float *v_dev);

/* ---- decode / draft-verify attention -------------------------------------- */
/* kernels::attention_with for 1..=8 query rows over a compact cache with
 * generated keys (src/kernels/attention/mod.rs:256-311 -> online::head,
 * online.rs:96-150, and decode64, decode64.rs:22-33), head_dim 64; the
 * arguments mean what they mean for focr_attention_prefill. The keys of each
 * head are split over many waves and the partial softmax states merged, so
 * the result is within FP32 rounding of the reference's serial loop; exp/ln
 * are the device libm's (the reference uses the platform expf, ExpMode does
 * not apply to decode). Uses the context scratch for the partial states. */
int focr_attention_decode(focr_ctx *ctx, const float *q_dev, const float *prefix_k_dev,
                          const float *generated_k_dev, const float *v_dev, size_t query_len,
                          size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                          size_t head_dim, size_t query_offset, size_t image_start,
                          size_t image_end, const float *sinks_dev, float *out_dev);
/* One greedy decode step's attention over a compact cache in one launch:
 * focr_qkv_rows for one generated row (split_norm_rope, src/model/rope.rs:
 * 14-86, and LayerCache::append, src/model/cache.rs:117-140) fused with
 * focr_attention_decode for that row (attention_with -> online::head,
 * src/kernels/attention/mod.rs:256-311, online.rs:96-150). The row is at
 * position total_len - 1 (> prefix_len - 1: past the prefix); qkv_dev
 * [qdim + 2 kdim] and rope_dev [n_heads][32][2] as for focr_qkv_rows; its key
 * is written to generated_k_dev row total_len - 1 - prefix_len and its value
 * to v_dev row total_len - 1 (the other arguments as for
 * focr_attention_decode); its query attends to keys 0 ..= total_len - 1 with
 * the per-head sink; out_dev [n_heads][64]; q_dev (may be NULL) receives
 * the normalized, rotated query. Query, cache rows and output are bitwise
 * those of focr_qkv_rows (rows = 1, prefix_rows = 0) followed by
 * focr_attention_decode (query_len = 1, query_offset = total_len - 1).
 * Uses the context scratch. */
int focr_attention_decode_row(focr_ctx *ctx, const float *qkv_dev, const float *rope_dev,
                              const float *prefix_k_dev, float *generated_k_dev, float *v_dev,
                              size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                              size_t head_dim, size_t image_start, size_t image_end,
                              const float *sinks_dev, float *q_dev, float *out_dev);

/* ---- A9: greedy selection ------------------------------------------------ */
/* argmax of each row (src/runner/mod.rs:916-939): first index of the
 * maximum; FOCR_E_NONFINITE if any value of a row is NaN or infinite.
 * logits_dev [rows][vocab]; tokens (host) [rows]. Synchronous. */
int focr_argmax(focr_ctx *ctx, const float *logits_dev, size_t rows, size_t vocab,
                uint32_t *tokens);

/* ---- Sealed split KV cache, Kv::Q8 / Kv::Q16 (src/quant/kv.rs) ---------- */
/* SplitPrefix::from_compact / seal (src/quant/kv.rs:225-421): seals the
 * compact prefix cache (prefix_k_dev [prefix_len][n_heads][64], v_dev
 * [prefix_len][n_kv_heads][64]) into group-major records [T | S(2g) |
 * S(2g+1) | V] of 8-bit (bits 8, Kv::Q8) or 16-bit (bits 16, Kv::Q16) codes
 * with one BF16 step (rounded up) per 32 elements, and reserves a tail for
 * capacity - prefix_len generated positions. FOCR_E_SHAPE unless head_dim is
 * 64 and n_heads = 2 n_kv_heads <= 16; FOCR_E_VALUE (nothing kept) if the
 * paired heads' temporal halves differ, a value is non-finite or a decoded
 * value overflows. Synchronous. */
int focr_kv_seal(focr_ctx *ctx, int bits, const float *prefix_k_dev, const float *v_dev,
                 size_t prefix_len, size_t capacity, size_t n_heads, size_t n_kv_heads,
                 size_t head_dim, focr_kv_split **out);
/* SplitPrefix::append / push_unique (src/quant/kv.rs:430-515): appends rows
 * generated positions, one key and one value per KV group (k_dev, v_dev
 * [rows][n_kv_heads][64]: the pair's identical heads once), coded as the
 * prefix; a block holding a non-finite value decodes to NaN. FOCR_E_SHAPE
 * past the capacity. */
int focr_kv_append(focr_ctx *ctx, focr_kv_split *kv, const float *k_dev, const float *v_dev,
                   size_t rows);
/* The decode row step over a sealed cache: focr_qkv_rows for rows past the
 * prefix (split_norm_rope, src/model/rope.rs:14-86) fused with
 * LayerCache::append of the split cache (src/model/cache.rs:117-140 ->
 * SplitPrefix::append, src/quant/kv.rs:430-515): qkv_dev [rows][qdim + 2 kdim]
 * and rope_dev [rows][n_heads][32][2] as for focr_qkv_rows; the queries go to
 * q_dev [rows][n_heads][64], the unique keys and the values are coded into
 * the tail without an FP32 copy. Records and queries are bitwise those of
 * focr_qkv_rows followed by focr_kv_append. rows 1..8; FOCR_E_SHAPE past the
 * capacity. */
int focr_kv_qkv_rows(focr_ctx *ctx, focr_kv_split *kv, const float *qkv_dev, size_t rows,
                     const float *rope_dev, float *q_dev);
/* One greedy decode step's attention over a sealed cache in one launch:
 * focr_kv_qkv_rows for one row (split_norm_rope, src/model/rope.rs:14-86,
 * and the split cache's append, src/model/cache.rs:117-140 ->
 * SplitPrefix::append, src/quant/kv.rs:430-515) fused with
 * focr_kv_attention_decode for that row (SplitPrefix::attention_decode,
 * src/quant/kv.rs:568-580): qkv_dev [qdim + 2 kdim] and rope_dev
 * [n_heads][32][2] as for focr_kv_qkv_rows; the row is appended to the tail
 * and its query attends to every cached position including itself, with the
 * per-head sink; out_dev [n_heads][64]; q_dev (may be NULL) receives the
 * normalized, rotated query. Queries, records and output are bitwise those
 * of focr_kv_qkv_rows followed by focr_kv_attention_decode (rows = 1).
 * FOCR_E_SHAPE past the capacity. Uses the context scratch. */
int focr_kv_decode_row(focr_ctx *ctx, focr_kv_split *kv, const float *qkv_dev, const float *rope_dev,
                       const float *sinks_dev, float *q_dev, float *out_dev);
/* SplitPrefix::attention_decode / attention_decode_rows (src/quant/kv.rs:
 * 568-580,856-900): q_dev [rows][n_heads][64], rows 1..8 (at most the
 * appended positions); row r attends to keys [0, len - rows + r + 1) of the
 * len cached positions, with the per-head sink; out_dev [rows][n_heads][64].
 * Within FP32 rounding of the compact kernel over the decoded values. Uses
 * the context scratch for the partial states. */
int focr_kv_attention_decode(focr_ctx *ctx, const focr_kv_split *kv, const float *q_dev, size_t rows,
                             const float *sinks_dev, float *out_dev);
/* focr_kv_attention_decode with its partial softmax states in a fixed
 * device array instead of the context scratch: the call allocates nothing
 * (no hipMalloc / hipFree), for callers that cannot allocate — code under
 * HIP graph capture and tight serving loops. No counterpart in the
 * reference (a CPU runner allocates no device memory). The array holds
 * 4.5 MiB per GPU for the life of the process; every valid shape of this
 * format (n_heads = 2 n_kv_heads <= 16, rows <= 8) needs at most about
 * 4.4 MB, and a call that would need more returns FOCR_E_UNSUPPORTED. The
 * array is shared by every call on a GPU: calls that overlap on one GPU (two
 * streams, two contexts) race and must be serialized by the caller. Same
 * arguments and results (bit for bit) as focr_kv_attention_decode. */
int focr_kv_attention_decode_noalloc(focr_ctx *ctx, const focr_kv_split *kv, const float *q_dev, size_t rows,
                                     const float *sinks_dev, float *out_dev);
/* The decoded cache in the compact layout (the reference's test view
 * dequantized_compact, src/quant/kv.rs:533-563, plus the tail): prefix keys
 * [prefix_len][n_heads][64], values [prefix_len + tail_len][n_kv_heads][64],
 * generated keys [tail_len][n_kv_heads][64]. */
int focr_kv_dequantize(focr_ctx *ctx, const focr_kv_split *kv, float *prefix_k_dev, float *values_dev,
                       float *generated_k_dev);
/* SplitPrefix::truncate_tail (src/quant/kv.rs:845-849): forgets the generated
 * positions past tail_len (rejected draft tokens; Session::truncate, src/model/
 * cache.rs:281-298); the next append overwrites them. Host state only, no
 * device work. FOCR_E_SHAPE if tail_len exceeds the stored tail. */
int focr_kv_truncate_tail(focr_kv_split *kv, size_t tail_len);
/* SplitPrefix::with_fast_exp (src/quant/kv.rs:423-426): fast != 0 makes the
 * decode softmax's per-key probabilities exp(s - max) use the hardware exp2
 * of log2(e) * x (the reference's polynomial exp_poly there, decode.rs:
 * 346-347), within a few ulp of the exact expf; the rescale and the chunk
 * merge stay exact. Off after focr_kv_seal, as SplitPrefix::from_compact
 * leaves it (kv.rs:415); the reference's runner turns it on for Kv::Q8 in
 * fast mode (default_fast_exp, kv.rs:182-184). Host state only. */
int focr_kv_set_fast_exp(focr_kv_split *kv, int fast);
/* SplitPrefix::fast_exp (src/quant/kv/record_bits.rs:6-8): *fast = 0 or 1. */
int focr_kv_fast_exp(const focr_kv_split *kv, int *fast);
int focr_kv_info(const focr_kv_split *kv, int *bits, size_t *prefix_len, size_t *tail_len,
                 size_t *capacity, size_t *device_bytes);
int focr_kv_free(focr_kv_split *kv);

/* ---- INT8 screened vocabulary head (src/head_screen.rs) ------------------ */
/* ScreenedHead::build (src/head_screen.rs:84-118): quantizes the FP32 head
 * weights_host [vocab][dim] into INT8 codes with one absmax/127 scale per 64
 * channels (ties to even), verifies the bound's premises and uploads the
 * screen. FOCR_E_SHAPE unless dim is a nonzero multiple of 64;
 * FOCR_E_VALUE for a non-finite weight, a failed premise or dim whose bound
 * constant reaches 0.53; FOCR_E_UNSUPPORTED for dim above 1024. */
int focr_screen_build(focr_ctx *ctx, const float *weights_host, size_t vocab, size_t dim,
                      focr_screen **out);
/* ScreenedHead::from_mapped (src/head_screen.rs:122-145): a stored screen
 * (host codes [vocab][dim], scales [vocab][dim/64] and its constants), as the
 * packed model file holds it; the same checks on the constants. */
int focr_screen_upload(focr_ctx *ctx, const int8_t *codes_host, const float *scales_host,
                       size_t vocab, size_t dim, float weight_abs_max, float kappa,
                       focr_screen **out);
int focr_screen_free(focr_screen *screen);
/* ScreenedHead::raw_parts' constants (src/head_screen.rs:148-151). */
int focr_screen_constants(const focr_screen *screen, float *weight_abs_max, float *kappa);
/* The bounds of the last focr_screen_select on this screen: q + B of every
 * vocabulary row for each of its first rows (1..8) inputs, into upper_host
 * [rows][vocab] (HeadScratch::upper, src/head_screen.rs:52, filled by
 * screen_block / screen_block_rows, 398-450). For parity tests; synchronous. */
int focr_screen_bounds(const focr_screen *screen, size_t rows, float *upper_host);
/* ScreenedHead::select / select_rows (src/head_screen.rs:169-199,274-324):
 * the exact FP32 greedy token of each of rows (1..8) inputs x_dev
 * [rows][dim]. tokens (host) [rows] receives the token, or -1 for
 * Screened::Fallback (the caller then evaluates the full head, e.g.
 * focr_linear_decode + focr_argmax); candidates (host) [rows] receives the
 * variant's candidate count (1025 past the limit, 0 for the other
 * fallbacks). fp32_head is the same head uploaded with focr_linear_upload
 * (bits 32, no exception columns). Allocates nothing; synchronous. */
int focr_screen_select(focr_ctx *ctx, const focr_screen *screen, const focr_linear *fp32_head,
                       const float *x_dev, size_t rows, int32_t *tokens, uint32_t *candidates);

#ifdef __cplusplus
}
#endif
#endif
