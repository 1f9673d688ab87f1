// Internal declarations of the focr_hip library (gfx950 only).
//
// Build flags (falcon-ocr-cpu_amd/Makefile): -ffp-contract=off, so every fused
// multiply-add in device code is an explicit __builtin_fmaf and every other
// product/sum rounds on its own, as the reference's Rust arithmetic does;
// IEEE division (__fdiv_rn) and square root (__builtin_sqrtf, which lowers to the
// FMA-corrected sequence; __fsqrt_rn lowers to the 1-ulp v_sqrt_f32); FP32 denormals kept.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/focr_hip.h"

namespace focr {

// ---- errors --------------------------------------------------------------
int set_error(int code, const std::string &message);
#define FOCR_HIP_CHECK(expr)                                                              \
  do {                                                                                    \
    hipError_t focr_err_ = (expr);                                                        \
    if (focr_err_ != hipSuccess)                                                          \
      return ::focr::set_error(FOCR_E_HIP, std::string(#expr) + ": " +                    \
                                               hipGetErrorString(focr_err_));             \
  } while (0)
#define FOCR_REQUIRE(cond, code, msg)                                                     \
  do {                                                                                    \
    if (!(cond)) return ::focr::set_error((code), (msg));                                 \
  } while (0)

// ---- context ---------------------------------------------------------------
struct Ctx {
  int device = 0;
  hipStream_t own = nullptr;
  hipStream_t stream = nullptr;  // own, or a caller's stream
  // Scratch owned by the context, grown on demand (INT16 activation codes).
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
  uint32_t *argmax_dev = nullptr;  // [2 * rows] result words for focr_argmax
  size_t argmax_rows = 0;
  float *rms_dev = nullptr;  // [8] row scales of a decode GEMV whose width has no in-kernel rms_norm
  hipEvent_t order = nullptr;  // orders a new stream after the old one (focr_ctx_set_stream)
};

// Grows the context scratch to at least `bytes` (hipMalloc on growth only).
int ensure_scratch(Ctx *ctx, size_t bytes);
// Resolves the device address of the no-alloc decode scratch for `device`
// (which must be current); once per device.
int noalloc_scratch_init(int device);

// ---- device-resident matrix ---------------------------------------------
// Decode GEMV layout (built at upload): wave tiles of kGemvChannels output
// channels; lane (half h, phase p) of a wave owns phase p of channels
// 2h, 2h+1 of the tile; each step is one 16-byte load per lane covering S
// consecutive 32-blocks, so every wave load is one contiguous 1 KB chunk.
constexpr int kGemvChannels = 4;  // per wave tile (2 per lane half)

struct Linear {
  int bits = 8;  // 8, 16 or 32
  size_t n = 0, k = 0, group = 64, groups = 0, n_exc = 0;
  // Row-major copies (dequantization, GEMM operands, GEMV tails).
  void *codes = nullptr;   // [n][k] int8 / int16 / float
  float *scales = nullptr; // [n][groups] (bits 8/16)
  int32_t *exc_cols = nullptr;  // [n_exc]
  float *exc_vals = nullptr;    // [n][n_exc]
  int16_t *exc_index = nullptr; // [k]: exception number of a column, or -1
  // GEMV tiles.
  void *gemv_codes = nullptr;    // [tiles][steps][64 lanes][16 B]
  float *gemv_scales = nullptr;  // [tiles][steps][2 halves][2 ch][sps]
  size_t gemv_tiles = 0, gemv_steps = 0, gemv_sps = 0, gemv_blocks = 0;
  // INT16-panel operands (bits 8, group 64): B tiles in MFMA lane order and
  // per-(group, column) weight sums times 128.
  int8_t *i16_b = nullptr;      // [groups][n/16][64 lanes][16 B]
  int32_t *i16_wsum = nullptr;  // [groups][n]  (128 * sum of the group's codes)
  float *i16_sw = nullptr;      // [groups][n]  scales, group-major
  // FP16-pair operand of FOCR_PROJ_F32_SPLIT (bits 32): two stage-major
  // planes of the rows (n rounded up to 128, k to 32) and a row exponent each.
  uint16_t *pair_w = nullptr;   // [2][k_pad / 16][n_pad][16]
  int *pair_wexp = nullptr;     // [n_pad]
  size_t device_bytes = 0;
};

// ---- launchers (each validates its launch shape on the host) -------------
// Row-scale argument of the GEMV launchers that asks for the in-kernel
// rms_norm instead of a precomputed factor.
inline const float *const kRmsInKernel = reinterpret_cast<const float *>(uintptr_t(1));
int launch_gemv(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale, int epilogue,
                float *out, bool rms_norm = false);
int launch_dequantize(Ctx *ctx, const Linear *lin, float *out);
int launch_row_scales(Ctx *ctx, const float *h, size_t rows, size_t width, float eps, float *out);
int launch_prefill_f32(Ctx *ctx, const Linear *lin, const float *x, size_t rows,
                       const float *row_scale, int epilogue, float *out);
int launch_prefill_chain(Ctx *ctx, const Linear *lin, const float *x, size_t rows,
                         const float *row_scale, int epilogue, float *out);
// Writes the FP16-pair operand of an FP32 matrix (Linear::pair_w, pair_wexp)
// at upload; synchronous.
int prepare_pairs(Ctx *ctx, Linear *lin, size_t *total);
int launch_prefill_split(Ctx *ctx, const Linear *lin, const float *x, size_t rows,
                         const float *row_scale, int epilogue, float *out);
int launch_prefill_i16(Ctx *ctx, const Linear *lin, const float *x, size_t rows,
                       const float *row_scale, int epilogue, float *out);
int launch_attention(Ctx *ctx, const float *q, const float *prefix_k, const float *generated_k,
                     const float *v, size_t query_len, size_t prefix_len, size_t total_len,
                     size_t n_heads, size_t n_kv_heads, size_t query_offset, size_t image_start,
                     size_t image_end, const float *sinks, int softmax, int exp_mode, float *out);
int launch_attention_split(Ctx *ctx, const float *q, const float *k, const float *v, size_t query_len,
                           size_t n_heads, size_t n_kv_heads, size_t image_start, size_t image_end, const float *sinks,
                           int softmax, int exp_mode, float *out);
int launch_attention_bf16(Ctx *ctx, const float *q, const float *k, const float *v, size_t query_len,
                          size_t n_heads, size_t n_kv_heads, size_t image_start, size_t image_end,
                          const float *sinks, int softmax, float *out);
int launch_argmax(Ctx *ctx, const float *logits, size_t rows, size_t vocab, uint32_t *result_dev);
int launch_qkv_rows(Ctx *ctx, const float *qkv, size_t rows, const float *rope, size_t n_heads, size_t n_kv_heads,
                    size_t prefix_rows, float *q, float *prefix_k, float *generated_k, float *v);
int launch_attention_decode(Ctx *ctx, const float *q, const float *prefix_k, const float *generated_k, const float *v,
                            size_t query_len, size_t prefix_len, size_t total_len, size_t n_heads, size_t n_kv_heads,
                            size_t query_offset, size_t image_start, size_t image_end, const float *sinks,
                            float *out);
int launch_attention_decode_row(Ctx *ctx, const float *qkv, const float *rope, const float *prefix_k,
                                float *generated_k, float *v, size_t prefix_len, size_t total_len, size_t n_heads,
                                size_t n_kv_heads, size_t image_start, size_t image_end, const float *sinks,
                                float *q_out, float *out);

// ---- device helpers ---------------------------------------------------------
__device__ __forceinline__ float fmaf_(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// A signed byte (SEL 0..3) or half-word (SEL 4, 5: low, high) of `w` as a
// float, exactly: one v_cvt_f32_i32 whose source operand selects and
// sign-extends the sub-word in place (SDWA), instead of a shift, a bit-field
// extract and a conversion.
template <int SEL>
__device__ __forceinline__ float sdwa_cvt(uint32_t w) {
  float r;
  if constexpr (SEL == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
  else if constexpr (SEL == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
  else if constexpr (SEL == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
  else if constexpr (SEL == 3)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
  else if constexpr (SEL == 4)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_0" : "=v"(r) : "v"(w));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:WORD_1" : "=v"(r) : "v"(w));
  return r;
}
// FP16 pairs of power-of-two scaled FP32 values (the split-product GEMM and
// attention). A block of values (a row, a key tile, a value dim) takes the
// exponent e of its largest finite magnitude m (2^(e-1) <= m < 2^e), and
// each x becomes x' = x 2^(15 - e) (exact; |x'| < 2^15) and the pair
// hi = fp16(x'), lo = fp16(x' - hi), both rounded to nearest: x' - hi is
// exact in FP32, so x' = hi + lo to 2^-22 |x'| (to 2^-25 absolute once lo is
// an FP16 subnormal, for |x'| below about 2^-3). An infinity or NaN travels
// in hi alone (lo = 0) and does not set e. Exponents are clamped below at
// kPairMinExp, the least e for which 2^(15 - e) and 2^(e - 15) are normal
// floats: a block whose largest magnitude is below 2^-111 (tiny normals,
// subnormals) is scaled by 2^126, so that even the least subnormal, 2^-149,
// becomes 2^-23 and every subnormal (a multiple of 2^-149) is exactly hi + lo.
constexpr int kPairMinExp = -111;

__device__ __forceinline__ int pair_exp(float m) {
  const int e = m > 0.0f ? __builtin_amdgcn_frexp_expf(m) : kPairMinExp;
  return e < kPairMinExp ? kPairMinExp : e;
}

// False for an infinity or NaN.
__device__ __forceinline__ bool is_finite(float x) { return __builtin_fabsf(x) <= 3.4028234663852886e38f; }

// |x| for finite x, 0 for an infinity or NaN.
__device__ __forceinline__ float finite_abs(float x) {
  const float a = __builtin_fabsf(x);
  return a <= 3.4028234663852886e38f ? a : 0.0f;
}

// x 2^shift as an FP16 pair (bit patterns).
__device__ __forceinline__ void pair1(float x, int shift, uint16_t &hi, uint16_t &lo) {
  const float xs = __builtin_ldexpf(x, shift);
  const _Float16 a = static_cast<_Float16>(xs);
  const bool finite = __builtin_fabsf(x) <= 3.4028234663852886e38f;
  const _Float16 b = finite ? static_cast<_Float16>(xs - static_cast<float>(a)) : static_cast<_Float16>(0.0f);
  hi = __builtin_bit_cast(uint16_t, a);
  lo = __builtin_bit_cast(uint16_t, b);
}

// squared_relu_glu, src/kernels/mod.rs:567-572.
__device__ __forceinline__ float squared_relu_glu(float gate, float up) {
  float relu = gate > 0.0f ? gate : 0.0f;
  return (relu * relu) * up;
}

// exp_poly_unchecked / exp_poly, src/kernels/exp.rs:232-277 (Cephes expf:
// the reference's literal constants, digit for digit).
__device__ __forceinline__ float exp_poly_unchecked(float x) {
  const float n = __builtin_rintf(x * 1.44269504088896340735992468100189214f);
  float r = fmaf_(n, -0.6933594f, x);
  r = fmaf_(n, 2.1219444e-4f, r);
  float p = 1.9875691e-4f;
  p = fmaf_(p, r, 1.3981999e-3f);
  p = fmaf_(p, r, 8.333452e-3f);
  p = fmaf_(p, r, 4.1665796e-2f);
  p = fmaf_(p, r, 0.16666665f);
  p = fmaf_(p, r, 0.5f);
  const float y = fmaf_(p, r * r, r) + 1.0f;
  return y * __uint_as_float(static_cast<uint32_t>(static_cast<int32_t>(n) + 127) << 23);
}

// The device libm exp and log (ExpMode::Exact, and the sink's exp/ln):
// accurate to about 1 ulp, not bitwise the host libm.
__device__ __forceinline__ float expf_acc(float x) { return ::expf(x); }
__device__ __forceinline__ float logf_acc(float x) { return ::logf(x); }

// Branch-free: the polynomial runs on the clamped input (the identity inside
// the range) and the out-of-range and NaN results are selected afterwards.
__device__ __forceinline__ float exp_poly(float x) {
  const float inside = exp_poly_unchecked(__builtin_fminf(__builtin_fmaxf(x, -87.0f), 88.376f));
  float y = x < -87.0f ? 0.0f : inside;
  y = x > 88.376f ? __builtin_inff() : y;
  return __builtin_isnan(x) ? x : y;
}

}  // namespace focr
