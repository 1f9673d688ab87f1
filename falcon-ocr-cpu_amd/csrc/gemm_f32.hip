// FP32 prefill projections: C = A' * W^T with A' = fl(a * row_scale) and W the
// FP32 weights or fl(code * scale) (exception columns in place), written
// through the Store / Glu / Add epilogues (src/kernels/panels/panel.rs:26-172,
// driver.rs:57-140; kernels::linear_with_simd's large-M path, mod.rs:434-476).
//
// Two kernels:
//  - mfma_kernel: v_mfma_f32_32x32x2f32 tiles (FP32 inputs, FP32 accumulate).
//    The matrix core sums k-slices in its own order, so results match the
//    reference's ascending-k FMA chain within FP32 rounding (tolerance).
//  - chain_kernel: SIMT register tiles in which every output is one FMA
//    chain over ascending k from +0.0: bitwise the reference's FP32 panels.
// Weights are dequantized while staging into LDS; full FP32 weights are
// never stored in HBM.
//
// Roofline: FP32 matrix cores (157.3 TFLOP/s) for mfma_kernel; FP32 VALU
// without packed math (78.6 TFLOP/s) for chain_kernel. FLOPs = 2*m*k*n.
#include <type_traits>

#include "focr_internal.hpp"

namespace focr {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kTile = 128;  // MFMA kernel: rows and columns per workgroup
constexpr int kBK = 32;     // k per LDS stage
constexpr int kPitch = kBK + 4;

template <typename T>
__device__ __forceinline__ float code_to_f32(T v) {
  return static_cast<float>(static_cast<int32_t>(v));
}
template <>
__device__ __forceinline__ float code_to_f32<float>(float v) {
  return v;
}

// One dequantized weight: fl(code * scale), or the exception value in place
// (dequantize_row, src/quant/linear.rs:246-262).
template <typename T>
__device__ __forceinline__ float weight_at(const T *__restrict__ codes, const float *__restrict__ scales,
                                           const int16_t *__restrict__ exc_index, const float *__restrict__ exc_vals,
                                           int n_exc, int k, int group, int groups, int row, int col) {
  float w = code_to_f32(codes[static_cast<size_t>(row) * k + col]);
  if constexpr (!std::is_same<T, float>::value) {
    w = w * scales[static_cast<size_t>(row) * groups + col / group];
    if (exc_index) {
      const int e = exc_index[col];
      if (e >= 0) w = exc_vals[static_cast<size_t>(row) * n_exc + e];
    }
  }
  return w;
}

struct GemmArgs {
  const float *x;
  const float *row_scale;
  const void *codes;
  const float *scales;
  const int16_t *exc_index;
  const float *exc_vals;
  int n_exc;
  int m, n, k, group, groups;
  float *out;
};

// Stages A'[m0.., k0..k0+32) and W[n0.., k0..k0+32) into LDS as [row][k].
template <typename T, int ROWS>
__device__ __forceinline__ void stage_tiles(const GemmArgs &a, int m0, int n0, int k0, float (*as)[kPitch],
                                            float (*bs)[kPitch]) {
  const T *codes = static_cast<const T *>(a.codes);
  for (int idx = threadIdx.x; idx < ROWS * kBK; idx += blockDim.x) {
    const int r = idx / kBK, c = idx % kBK;
    const int row = m0 + r, col = k0 + c;
    float v = 0.0f;
    if (row < a.m && col < a.k) {
      v = a.x[static_cast<size_t>(row) * a.k + col];
      if (a.row_scale) v = v * a.row_scale[row];
    }
    as[r][c] = v;
  }
  for (int idx = threadIdx.x; idx < ROWS * kBK; idx += blockDim.x) {
    const int r = idx / kBK, c = idx % kBK;
    const int row = n0 + r, col = k0 + c;
    float w = 0.0f;
    if (row < a.n && col < a.k)
      w = weight_at<T>(codes, a.scales, a.exc_index, a.exc_vals, a.n_exc, a.k, a.group, a.groups, row, col);
    bs[r][c] = w;
  }
}

// Writes one output value through the epilogue. For GLU, `partner` is the
// value of the neighbouring column (col ^ 1), fetched by the caller.
template <int EPI>
__device__ __forceinline__ void emit(const GemmArgs &a, int row, int col, float v, float partner) {
  if (row >= a.m || col >= a.n) return;
  if constexpr (EPI == FOCR_EPI_GLU) {
    if ((col & 1) == 0) a.out[static_cast<size_t>(row) * (a.n / 2) + col / 2] = squared_relu_glu(v, partner);
  } else if constexpr (EPI == FOCR_EPI_ADD) {
    float *dst = a.out + static_cast<size_t>(row) * a.n + col;
    *dst = *dst + v;
  } else {
    a.out[static_cast<size_t>(row) * a.n + col] = v;
  }
}

template <typename T, int EPI>
__global__ __launch_bounds__(256) void mfma_kernel(GemmArgs a) {
  __shared__ float as[kTile][kPitch];
  __shared__ float bs[kTile][kPitch];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.x * kTile, n0 = blockIdx.y * kTile;
  const int h = lane >> 5, l32 = lane & 31;
  v16f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  for (int k0 = 0; k0 < a.k; k0 += kBK) {
    stage_tiles<T, kTile>(a, m0, n0, k0, as, bs);
    __syncthreads();
    // Lane half h supplies k-slot h of each 32x32x2 step: k = 16 h + s.
    float av[2][16], bv[2][16];
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const float4 *ar = reinterpret_cast<const float4 *>(&as[wm * 64 + i * 32 + l32][16 * h]);
      const float4 *br = reinterpret_cast<const float4 *>(&bs[wn * 64 + i * 32 + l32][16 * h]);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 x = ar[q], y = br[q];
        av[i][4 * q] = x.x;
        av[i][4 * q + 1] = x.y;
        av[i][4 * q + 2] = x.z;
        av[i][4 * q + 3] = x.w;
        bv[i][4 * q] = y.x;
        bv[i][4 * q + 1] = y.y;
        bv[i][4 * q + 2] = y.z;
        bv[i][4 * q + 3] = y.w;
      }
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 16; s++)
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s], bv[j][s], acc[i][j], 0, 0, 0);
  }
  // D layout of 32x32: column = lane % 32, row = 8 (r / 4) + 4 (lane / 32) + r % 4.
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        const int col = n0 + wn * 64 + j * 32 + l32;
        const float v = acc[i][j][r];
        const float partner = EPI == FOCR_EPI_GLU ? __shfl_xor(v, 1) : 0.0f;
        emit<EPI>(a, row, col, v, partner);
      }
}

// Exact-order kernel: 64x64 outputs per workgroup, 4x4 per thread; each
// output's accumulator sees fma(a'[k], w[k], acc) for k = 0, 1, 2, ...
constexpr int kChainTile = 64;

template <typename T, int EPI>
__global__ __launch_bounds__(256) void chain_kernel(GemmArgs a) {
  __shared__ float as[kChainTile][kPitch];
  __shared__ float bs[kChainTile][kPitch];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int m0 = blockIdx.x * kChainTile, n0 = blockIdx.y * kChainTile;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
  for (int k0 = 0; k0 < a.k; k0 += kBK) {
    stage_tiles<T, kChainTile>(a, m0, n0, k0, as, bs);
    __syncthreads();
    const int kend = a.k - k0 < kBK ? a.k - k0 : kBK;
    for (int kk = 0; kk < kend; kk++) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) av[i] = as[ty + 16 * i][kk];
#pragma unroll
      for (int j = 0; j < 4; j++) bv[j] = bs[tx + 16 * j][kk];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = fmaf_(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int row = m0 + ty + 16 * i, col = n0 + tx + 16 * j;
      const float v = acc[i][j];
      const float partner = EPI == FOCR_EPI_GLU ? __shfl_xor(v, 1) : 0.0f;
      emit<EPI>(a, row, col, v, partner);
    }
}

GemmArgs make_args(const Linear *lin, const float *x, size_t rows, const float *row_scale, float *out) {
  GemmArgs a;
  a.x = x;
  a.row_scale = row_scale;
  a.codes = lin->codes;
  a.scales = lin->scales;
  a.exc_index = lin->exc_index;
  a.exc_vals = lin->exc_vals;
  a.n_exc = static_cast<int>(lin->n_exc);
  a.m = static_cast<int>(rows);
  a.n = static_cast<int>(lin->n);
  a.k = static_cast<int>(lin->k);
  a.group = static_cast<int>(lin->group);
  a.groups = static_cast<int>(lin->groups);
  a.out = out;
  return a;
}

template <typename T, int EPI>
void launch_one(bool chain, const GemmArgs &a, hipStream_t stream) {
  if (chain) {
    const dim3 grid((a.m + kChainTile - 1) / kChainTile, (a.n + kChainTile - 1) / kChainTile);
    hipLaunchKernelGGL((chain_kernel<T, EPI>), grid, dim3(256), 0, stream, a);
  } else {
    const dim3 grid((a.m + kTile - 1) / kTile, (a.n + kTile - 1) / kTile);
    hipLaunchKernelGGL((mfma_kernel<T, EPI>), grid, dim3(256), 0, stream, a);
  }
}

template <typename T>
void launch_epi(bool chain, int epilogue, const GemmArgs &a, hipStream_t stream) {
  if (epilogue == FOCR_EPI_GLU)
    launch_one<T, FOCR_EPI_GLU>(chain, a, stream);
  else if (epilogue == FOCR_EPI_ADD)
    launch_one<T, FOCR_EPI_ADD>(chain, a, stream);
  else
    launch_one<T, FOCR_EPI_STORE>(chain, a, stream);
}

int launch_f32_common(bool chain, Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale,
                      int epilogue, float *out) {
  FOCR_REQUIRE(rows < (size_t(1) << 30), FOCR_E_SHAPE, "prefill rows too large");
  const GemmArgs a = make_args(lin, x, rows, row_scale, out);
  if (lin->bits == 8)
    launch_epi<int8_t>(chain, epilogue, a, ctx->stream);
  else if (lin->bits == 16)
    launch_epi<int16_t>(chain, epilogue, a, ctx->stream);
  else
    launch_epi<float>(chain, epilogue, a, ctx->stream);
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
}

}  // namespace

int launch_prefill_f32(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale,
                       int epilogue, float *out) {
  return launch_f32_common(false, ctx, lin, x, rows, row_scale, epilogue, out);
}

int launch_prefill_chain(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale,
                         int epilogue, float *out) {
  return launch_f32_common(true, ctx, lin, x, rows, row_scale, epilogue, out);
}

}  // namespace focr
