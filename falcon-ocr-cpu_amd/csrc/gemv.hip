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
// Roofline: HBM. Bytes per call = codes + scales (+ x, out), e.g. 4,476,928 B
// for an INT8 4096x1024 matrix at one row.
#include "focr_internal.hpp"

namespace focr {
namespace {

constexpr int kWaves = 4;  // waves (channel tiles) per workgroup

__device__ __forceinline__ float to_f32(int8_t v) { return static_cast<float>(static_cast<int32_t>(v)); }
__device__ __forceinline__ float to_f32(int16_t v) { return static_cast<float>(static_cast<int32_t>(v)); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// Sum of lane and lane + delta within a 32-lane half (the reference's lane
// pairing; IEEE addition is commutative, so operand order is immaterial).
__device__ __forceinline__ float add_down(float v, int delta) { return v + __shfl_down(v, delta, 32); }

// Loads of one step's scales for this lane's two channels (2 * SPS floats,
// identical across the 32 lanes of a half: the memory pipeline broadcasts).
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

// Steps of weights kept in flight per lane: a rolling window of 16-byte code
// loads (and their scales) issued before x is staged and refilled as soon as a
// slot is consumed, so a wave streams several KB at once.
template <int SPS>
constexpr int window() {
  return SPS >= 4 ? 4 : 8;
}

// T: code type; M: rows; SPS: scales per lane-channel per step (0 for FP32).
template <typename T, int M, int SPS>
__global__ __launch_bounds__(256) void gemv_kernel(
    const uint4 *__restrict__ tiles, const float *__restrict__ tile_scales,
    const T *__restrict__ codes, const float *__restrict__ scales, const int32_t *__restrict__ exc_cols,
    const float *__restrict__ exc_vals, int n_exc, const float *__restrict__ x, int n, int k, int group,
    int groups, int nb, int steps, int tiles_total, int glu, float *__restrict__ out) {
  constexpr int B = sizeof(T);
  constexpr int S = 16 / (2 * B);  // 32-blocks per step
  constexpr int NS = 2 * SPS;      // scales per lane per step
  constexpr int W = window<SPS>();
  extern __shared__ float xs[];    // [M][k]

  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, p = lane & 31;
  const int tile = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const bool active = tile < tiles_total;
  const int my_tile = active ? tile : 0;

  const uint4 *src = tiles + static_cast<size_t>(my_tile) * steps * 64 + lane;
  const float *sc_src = tile_scales + (static_cast<size_t>(my_tile) * steps * 2 + h) * (NS > 0 ? NS : 1);
  uint4 cbuf[W];
  Scales<NS> sbuf[W];
#pragma unroll
  for (int j = 0; j < W; j++)
    if (j < steps) {
      cbuf[j] = src[static_cast<size_t>(j) * 64];
      if constexpr (NS > 0) sbuf[j] = load_scales<NS>(sc_src + static_cast<size_t>(j) * 2 * NS);
    }
  for (int i = threadIdx.x; i < M * k; i += blockDim.x) xs[i] = x[i];
  __syncthreads();
  if (!active) return;

  float acc[2][M];
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = 0.0f;

  for (int base = 0; base < steps; base += W) {
#pragma unroll
    for (int j = 0; j < W; j++) {
      const int t = base + j;
      if (t >= steps) break;
      const uint4 raw = cbuf[j];
      const Scales<NS> sc = sbuf[j];
      if (t + W < steps) {
        cbuf[j] = src[static_cast<size_t>(t + W) * 64];
        if constexpr (NS > 0) sbuf[j] = load_scales<NS>(sc_src + static_cast<size_t>(t + W) * 2 * NS);
      }
      T vals[S][2];
      __builtin_memcpy(vals, &raw, 16);
#pragma unroll
      for (int s = 0; s < S; s++) {
        const int b = t * S + s;
        if (b >= nb) break;
        float xv[M];
#pragma unroll
        for (int r = 0; r < M; r++) xv[r] = xs[r * k + 32 * b + p];
#pragma unroll
        for (int c = 0; c < 2; c++) {
          float w = to_f32(vals[s][c]);
          if constexpr (SPS > 0) w = w * sc.v[c * SPS + s / (S / SPS)];
#pragma unroll
          for (int r = 0; r < M; r++) acc[c][r] = fmaf_(xv[r], w, acc[c][r]);
        }
      }
    }
  }

  // (a0 + a1) + (a2 + a3) lane-wise: lane p < 8 ends up with the combined
  // accumulator lane p of the reference.
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int r = 0; r < M; r++) acc[c][r] = add_down(add_down(acc[c][r], 8), 16);

  const int ch0 = tile * kGemvChannels + h * 2;
  // 8-wide tail (k % 32 >= 8): one more FMA per combined lane and chunk.
  const int tail8 = (k - 32 * nb) / 8;
  for (int ci = 0; ci < tail8; ci++) {
    const int i = 32 * nb + 8 * ci;
    if (p < 8) {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int ch = ch0 + c < n ? ch0 + c : n - 1;
        float w = to_f32(codes[static_cast<size_t>(ch) * k + i + p]);
        if constexpr (SPS > 0) w = w * scales[static_cast<size_t>(ch) * groups + i / group];
#pragma unroll
        for (int r = 0; r < M; r++) acc[c][r] = fmaf_(xs[r * k + i + p], w, acc[c][r]);
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
    if (ch >= n) continue;
    // Scalar tail: total += x * fl(code * scale), unfused.
    for (int i = 32 * nb + 8 * tail8; i < k; i++) {
      float w = to_f32(codes[static_cast<size_t>(ch) * k + i]);
      if constexpr (SPS > 0) w = w * scales[static_cast<size_t>(ch) * groups + i / group];
#pragma unroll
      for (int r = 0; r < M; r++) total[c][r] = total[c][r] + xs[r * k + i] * w;
    }
    // Exception columns: one FMA each, ascending (src/quant/linear.rs:84-118).
    for (int e = 0; e < n_exc; e++) {
      const int col = exc_cols[e];
      const float v = exc_vals[static_cast<size_t>(ch) * n_exc + e];
#pragma unroll
      for (int r = 0; r < M; r++) total[c][r] = fmaf_(xs[r * k + col], v, total[c][r]);
    }
  }
  if (glu) {
    const int i = ch0 / 2;
    if (ch0 + 1 < n) {
      const int ffn = n / 2;
#pragma unroll
      for (int r = 0; r < M; r++) out[static_cast<size_t>(r) * ffn + i] = squared_relu_glu(total[0][r], total[1][r]);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 2; c++)
      if (ch0 + c < n)
#pragma unroll
        for (int r = 0; r < M; r++) out[static_cast<size_t>(r) * n + ch0 + c] = total[c][r];
  }
}

template <typename T, int M, int SPS>
int launch_typed(Ctx *ctx, const Linear *lin, const float *x, float *out, bool glu) {
  const size_t lds = static_cast<size_t>(M) * lin->k * sizeof(float);
  const int blocks = static_cast<int>((lin->gemv_tiles + kWaves - 1) / kWaves);
  hipLaunchKernelGGL((gemv_kernel<T, M, SPS>), dim3(blocks), dim3(64 * kWaves), lds, ctx->stream,
                     static_cast<const uint4 *>(lin->gemv_codes), lin->gemv_scales,
                     static_cast<const T *>(lin->codes), lin->scales, lin->exc_cols, lin->exc_vals,
                     static_cast<int>(lin->n_exc), x, static_cast<int>(lin->n), static_cast<int>(lin->k),
                     static_cast<int>(lin->group), static_cast<int>(lin->groups),
                     static_cast<int>(lin->gemv_blocks), static_cast<int>(lin->gemv_steps),
                     static_cast<int>(lin->gemv_tiles), glu ? 1 : 0, out);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

template <typename T, int SPS>
int launch_rows(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu) {
  switch (rows) {
    case 1: return launch_typed<T, 1, SPS>(ctx, lin, x, out, glu);
    case 2: return launch_typed<T, 2, SPS>(ctx, lin, x, out, glu);
    case 3: return launch_typed<T, 3, SPS>(ctx, lin, x, out, glu);
    case 4: return launch_typed<T, 4, SPS>(ctx, lin, x, out, glu);
    case 5: return launch_typed<T, 5, SPS>(ctx, lin, x, out, glu);
    case 6: return launch_typed<T, 6, SPS>(ctx, lin, x, out, glu);
    case 7: return launch_typed<T, 7, SPS>(ctx, lin, x, out, glu);
    case 8: return launch_typed<T, 8, SPS>(ctx, lin, x, out, glu);
    default: return set_error(FOCR_E_SHAPE, "GEMV rows must be 1..=8");
  }
}

}  // namespace

// Largest row count whose x fits the 64 KB of LDS a workgroup may take.
static size_t rows_per_launch(size_t k) {
  const size_t fit = (64 * 1024) / (k * sizeof(float));
  return fit < 8 ? fit : 8;
}

int launch_gemv(Ctx *ctx, const Linear *lin, const float *x, size_t rows, float *out, bool glu) {
  FOCR_HIP_CHECK(hipSetDevice(ctx->device));
  const size_t chunk = rows_per_launch(lin->k);
  FOCR_REQUIRE(chunk >= 1, FOCR_E_SHAPE, "GEMV input width exceeds 16384");
  const size_t width = glu ? lin->n / 2 : lin->n;
  // Rows are independent (each output row is its single-row dot, bitwise), so
  // a call whose inputs exceed the LDS budget runs as several launches.
  for (size_t r0 = 0; r0 < rows; r0 += chunk) {
    const size_t m = rows - r0 < chunk ? rows - r0 : chunk;
    const float *xr = x + r0 * lin->k;
    float *orow = out + r0 * width;
    int rc = FOCR_OK;
    if (lin->bits == 8) {
      switch (lin->group) {
        case 32: rc = launch_rows<int8_t, 8>(ctx, lin, xr, m, orow, glu); break;
        case 64: rc = launch_rows<int8_t, 4>(ctx, lin, xr, m, orow, glu); break;
        default: rc = launch_rows<int8_t, 2>(ctx, lin, xr, m, orow, glu); break;
      }
    } else if (lin->bits == 16) {
      switch (lin->group) {
        case 32: rc = launch_rows<int16_t, 4>(ctx, lin, xr, m, orow, glu); break;
        case 64: rc = launch_rows<int16_t, 2>(ctx, lin, xr, m, orow, glu); break;
        default: rc = launch_rows<int16_t, 1>(ctx, lin, xr, m, orow, glu); break;
      }
    } else {
      rc = launch_rows<float, 0>(ctx, lin, xr, m, orow, glu);
    }
    if (rc != FOCR_OK) return rc;
  }
  return FOCR_OK;
}

}  // namespace focr
