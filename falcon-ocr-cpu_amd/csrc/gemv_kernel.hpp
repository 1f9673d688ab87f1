// Decode and draft-verify GEMV (1..=8 rows), bitwise equal to the reference's
// vector dot order: simd::dot_q / dot_q_rows / dot (src/simd.rs:749-920) as
// called by QuantLinear::linear / linear_glu (src/quant/linear.rs:497-625,
// 745-817) and kernels::linear_with_simd (src/kernels/mod.rs:407-432).
//
// The reference keeps four 8-lane accumulators, i.e. 32 "phase" chains: chain
// p accumulates fma(x[32b+p], w[32b+p], .) over the full 32-blocks b in
// ascending order. Here each of those chains is one lane: a wave is two
// halves of 32 lanes, lane p of a half owns chain p of two output channels,
// and the chains are combined with cross-lane adds in the reference's pairing
// ((a0+a1)+(a2+a3) lane-wise, then ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7))), so
// every output has exactly the reference's operation sequence. Weights are
// read from the wave-tiled layout built at upload: one contiguous 1 KB chunk
// per wave per step, each lane's 16 bytes holding S consecutive blocks of its
// phase for its two channels. Dequantization fl(code * scale) happens in
// registers; FP32 weights are never materialized.
//
// Latency structure: a wave issues every load it needs for up to W steps
// (weights, scales and, for 1-2 rows, its own x values) before any compute,
// all unconditional with in-bounds clamped indices, and only then consumes
// them in order; register arrays are indexed statically so nothing is
// spilled. With three or more rows x is staged once per workgroup in LDS.
//
// Roofline: HBM. Bytes per call = codes + scales (+ x, out), e.g. 4,476,928 B
// for an INT8 4096x1024 matrix at one row.
#pragma once

#include "focr_internal.hpp"

namespace focr {
namespace gemv {

constexpr int kWaves = 4;  // waves (channel tiles) per workgroup

__device__ __forceinline__ float to_f32(int8_t v) { return static_cast<float>(static_cast<int32_t>(v)); }
__device__ __forceinline__ float to_f32(int16_t v) { return static_cast<float>(static_cast<int32_t>(v)); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// Sum of lane and lane + delta within a 32-lane half (the reference's lane
// pairing; IEEE addition is commutative, so operand order is immaterial).
__device__ __forceinline__ float add_down(float v, int delta) { return v + __shfl_down(v, delta, 32); }

// One step's scales for this lane's two channels (2 * SPS floats, identical
// across the 32 lanes of a half).
template <int NS>
struct Scales {
  float v[NS > 0 ? NS : 1];
};
template <int NS>
__device__ __forceinline__ Scales<NS> load_scales(const float *p) {
  Scales<NS> s;
  if constexpr (NS >= 4) {
#pragma unroll
    for (int i = 0; i < NS / 4; i++) {
      const float4 f = reinterpret_cast<const float4 *>(p)[i];
      s.v[4 * i] = f.x;
      s.v[4 * i + 1] = f.y;
      s.v[4 * i + 2] = f.z;
      s.v[4 * i + 3] = f.w;
    }
  } else if constexpr (NS == 2) {
    const float2 f = *reinterpret_cast<const float2 *>(p);
    s.v[0] = f.x;
    s.v[1] = f.y;
  }
  return s;
}

struct Args {
  const uint4 *tiles;
  const float *tile_scales;
  const void *codes;
  const float *scales;
  const int32_t *exc_cols;
  const float *exc_vals;
  int n_exc;
  const float *x;
  int n, k, group, groups, nb, steps, tiles_total, glu;
  float *out;
};

// T: code type; M: rows; SPS: scales per lane-channel per step (0 for FP32
// weights); W: steps held in registers (all of them when steps <= W).
template <typename T, int M, int SPS, int W>
__global__ __launch_bounds__(256) void kernel(Args a) {
  constexpr int B = sizeof(T);
  constexpr int S = 16 / (2 * B);   // 32-blocks per step
  constexpr int NS = 2 * SPS;       // scales per lane per step
  constexpr bool XREG = M <= 2;     // x straight to registers (else LDS)
  extern __shared__ float xs[];     // [M][k] when !XREG

  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, p = lane & 31;
  const int tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const bool active = tile < a.tiles_total;
  const int my_tile = active ? tile : 0;
  const int k = a.k, nb = a.nb, steps = a.steps;
  const T *codes = static_cast<const T *>(a.codes);

  const uint4 *src = a.tiles + static_cast<size_t>(my_tile) * steps * 64 + lane;
  const float *sc_src = a.tile_scales + (static_cast<size_t>(my_tile) * steps * 2 + h) * (NS > 0 ? NS : 1);
  // x of block b for this lane's phase; blocks past the last are clamped
  // (in bounds, never used).
  auto x_at = [&](int r, int b) { return a.x[r * k + 32 * (b < nb ? b : (nb > 0 ? nb - 1 : 0)) + p]; };

  uint4 cbuf[W];
  Scales<NS> sbuf[W];
  float xw[XREG ? W : 1][XREG ? S : 1][XREG ? M : 1];
#pragma unroll
  for (int j = 0; j < W; j++) {
    const int t = j < steps ? j : steps - 1;
    cbuf[j] = src[static_cast<size_t>(t) * 64];
    if constexpr (NS > 0) sbuf[j] = load_scales<NS>(sc_src + static_cast<size_t>(t) * 2 * NS);
    if constexpr (XREG)
#pragma unroll
      for (int s = 0; s < S; s++)
#pragma unroll
        for (int r = 0; r < M; r++) xw[j][s][r] = x_at(r, t * S + s);
  }
  if constexpr (!XREG) {
    for (int i = threadIdx.x; i < M * k; i += blockDim.x) xs[i] = a.x[i];
    __syncthreads();
  }
  if (!active) return;
  // x for the tails and exceptions (any column).
  auto x_col = [&](int r, int i) { return XREG ? a.x[r * k + i] : xs[r * k + i]; };

  float acc[2][M];
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = 0.0f;

  const int ch0 = tile * kGemvChannels + h * 2;
  // A full step: S blocks of this lane's phase for both channels.
  auto step_full = [&](int t, const uint4 &raw, const Scales<NS> &sc, const float (&xv)[XREG ? S : 1][XREG ? M : 1]) {
    T vals[S][2];
    __builtin_memcpy(vals, &raw, 16);
#pragma unroll
    for (int s = 0; s < S; s++) {
      float xr[M];
#pragma unroll
      for (int r = 0; r < M; r++) {
        if constexpr (XREG)
          xr[r] = xv[s][r];
        else
          xr[r] = xs[r * k + 32 * (t * S + s) + p];
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        float w = to_f32(vals[s][c]);
        if constexpr (SPS > 0) w = w * sc.v[c * SPS + s / (S / SPS)];
#pragma unroll
        for (int r = 0; r < M; r++) acc[c][r] = fmaf_(xr[r], w, acc[c][r]);
      }
    }
  };
  // The last step when k/32 is not a multiple of S (odd widths only): read
  // the row-major codes directly (no register arrays indexed at run time).
  auto step_partial = [&](int t) {
    for (int b = t * S; b < nb; b++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int ch = ch0 + c < a.n ? ch0 + c : a.n - 1;
        float w = to_f32(codes[static_cast<size_t>(ch) * k + 32 * b + p]);
        if constexpr (SPS > 0) w = w * a.scales[static_cast<size_t>(ch) * a.groups + (32 * b) / a.group];
#pragma unroll
        for (int r = 0; r < M; r++) acc[c][r] = fmaf_(x_col(r, 32 * b + p), w, acc[c][r]);
      }
  };
  const int full = nb / S;  // steps whose S blocks all exist
  if (steps <= W) {
#pragma unroll
    for (int t = 0; t < W; t++) {
      if (t < full)
        step_full(t, cbuf[t], sbuf[t], xw[XREG ? t : 0]);
      else if (t < steps)
        step_partial(t);
    }
  } else {
    for (int base = 0; base < steps; base += W) {
#pragma unroll
      for (int j = 0; j < W; j++) {
        const int t = base + j;
        if (t < full)
          step_full(t, cbuf[j], sbuf[j], xw[XREG ? j : 0]);
        else if (t < steps)
          step_partial(t);
        const int tn = t + W < steps ? t + W : steps - 1;
        cbuf[j] = src[static_cast<size_t>(tn) * 64];
        if constexpr (NS > 0) sbuf[j] = load_scales<NS>(sc_src + static_cast<size_t>(tn) * 2 * NS);
        if constexpr (XREG)
#pragma unroll
          for (int s = 0; s < S; s++)
#pragma unroll
            for (int r = 0; r < M; r++) xw[j][s][r] = x_at(r, tn * S + s);
      }
    }
  }

  // (a0 + a1) + (a2 + a3) lane-wise: lane p < 8 ends up with the combined
  // accumulator lane p of the reference.
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = add_down(add_down(acc[c][r], 8), 16);

  // 8-wide tail (k % 32 >= 8): one more FMA per combined lane and chunk.
  const int tail8 = (k - 32 * nb) / 8;
  for (int ci = 0; ci < tail8; ci++) {
    const int i = 32 * nb + 8 * ci;
    if (p < 8) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int ch = ch0 + c < a.n ? ch0 + c : a.n - 1;
        float w = to_f32(codes[static_cast<size_t>(ch) * k + i + p]);
        if constexpr (SPS > 0) w = w * a.scales[static_cast<size_t>(ch) * a.groups + i / a.group];
#pragma unroll
        for (int r = 0; r < M; r++) acc[c][r] = fmaf_(x_col(r, i + p), w, acc[c][r]);
      }
    }
  }
  // ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)) on lanes 0..7.
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = add_down(add_down(add_down(acc[c][r], 4), 1), 2);

  if (p != 0) return;
  float total[2][M];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int ch = ch0 + c;
#pragma unroll
    for (int r = 0; r < M; r++) total[c][r] = acc[c][r];
    if (ch >= a.n) continue;
    // Scalar tail: total += x * fl(code * scale), unfused.
    for (int i = 32 * nb + 8 * tail8; i < k; i++) {
      float w = to_f32(codes[static_cast<size_t>(ch) * k + i]);
      if constexpr (SPS > 0) w = w * a.scales[static_cast<size_t>(ch) * a.groups + i / a.group];
#pragma unroll
      for (int r = 0; r < M; r++) total[c][r] = total[c][r] + x_col(r, i) * w;
    }
    // Exception columns: one FMA each, ascending (src/quant/linear.rs:84-118).
    for (int e = 0; e < a.n_exc; e++) {
      const int col = a.exc_cols[e];
      const float v = a.exc_vals[static_cast<size_t>(ch) * a.n_exc + e];
#pragma unroll
      for (int r = 0; r < M; r++) total[c][r] = fmaf_(x_col(r, col), v, total[c][r]);
    }
  }
  if (a.glu) {
    const int i = ch0 / 2;
    if (ch0 + 1 < a.n) {
      const int ffn = a.n / 2;
#pragma unroll
      for (int r = 0; r < M; r++) a.out[static_cast<size_t>(r) * ffn + i] = squared_relu_glu(total[0][r], total[1][r]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 2; c++)
      if (ch0 + c < a.n)
#pragma unroll
        for (int r = 0; r < M; r++) a.out[static_cast<size_t>(r) * a.n + ch0 + c] = total[c][r];
  }
}

template <typename T, int M, int SPS, int W>
int launch_typed(Ctx *ctx, const Linear *lin, const float *x, float *out, bool glu) {
  const size_t lds = M <= 2 ? 0 : static_cast<size_t>(M) * lin->k * sizeof(float);
  const int blocks = static_cast<int>((lin->gemv_tiles + kWaves - 1) / kWaves);
  Args a;
  a.tiles = static_cast<const uint4 *>(lin->gemv_codes);
  a.tile_scales = lin->gemv_scales;
  a.codes = lin->codes;
  a.scales = lin->scales;
  a.exc_cols = lin->exc_cols;
  a.exc_vals = lin->exc_vals;
  a.n_exc = static_cast<int>(lin->n_exc);
  a.x = x;
  a.n = static_cast<int>(lin->n);
  a.k = static_cast<int>(lin->k);
  a.group = static_cast<int>(lin->group);
  a.groups = static_cast<int>(lin->groups);
  a.nb = static_cast<int>(lin->gemv_blocks);
  a.steps = static_cast<int>(lin->gemv_steps);
  a.tiles_total = static_cast<int>(lin->gemv_tiles);
  a.glu = glu ? 1 : 0;
  a.out = out;
  hipLaunchKernelGGL((kernel<T, M, SPS, W>), dim3(blocks), dim3(64 * kWaves), lds, ctx->stream, a);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

// Window buckets: all steps in registers up to 20 steps (36 for FP32
// weights), which covers every matrix of the model; longer rows refill.
template <typename T, int M, int SPS>
int launch_window(Ctx *ctx, const Linear *lin, const float *x, float *out, bool glu) {
  const size_t steps = lin->gemv_steps;
  if (steps <= 4) return launch_typed<T, M, SPS, 4>(ctx, lin, x, out, glu);
  if (steps <= 8) return launch_typed<T, M, SPS, 8>(ctx, lin, x, out, glu);
  if constexpr (SPS == 0) {
    if (steps <= 20) return launch_typed<T, M, SPS, 20>(ctx, lin, x, out, glu);
    return launch_typed<T, M, SPS, 36>(ctx, lin, x, out, glu);
  } else {
    return launch_typed<T, M, SPS, 20>(ctx, lin, x, out, glu);
  }
}

template <typename T, int SPS>
int launch_rows(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu) {
  switch (rows) {
    case 1: return launch_window<T, 1, SPS>(ctx, lin, x, out, glu);
    case 2: return launch_window<T, 2, SPS>(ctx, lin, x, out, glu);
    case 3: return launch_window<T, 3, SPS>(ctx, lin, x, out, glu);
    case 4: return launch_window<T, 4, SPS>(ctx, lin, x, out, glu);
    case 5: return launch_window<T, 5, SPS>(ctx, lin, x, out, glu);
    case 6: return launch_window<T, 6, SPS>(ctx, lin, x, out, glu);
    case 7: return launch_window<T, 7, SPS>(ctx, lin, x, out, glu);
    case 8: return launch_window<T, 8, SPS>(ctx, lin, x, out, glu);
    default: return set_error(FOCR_E_SHAPE, "GEMV rows must be 1..=8");
  }
}

// Per-code-type dispatch (one translation unit each, compiled in parallel).
int launch_i8(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu);
int launch_i16(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu);
int launch_f32(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu);

}  // namespace gemv
}  // namespace focr
