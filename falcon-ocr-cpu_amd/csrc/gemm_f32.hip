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

// Four consecutive weights of row `row` starting at column `col` (a multiple
// of 4 inside one scale group): fl(code * scale), exception columns in place.
template <typename T>
__device__ __forceinline__ float4 load_weights4(const GemmArgs &a, int row, int col) {
  const T *codes = static_cast<const T *>(a.codes);
  const size_t at = static_cast<size_t>(row) * a.k + col;
  float w[4];
  if constexpr (std::is_same<T, float>::value) {
    const float4 f = *reinterpret_cast<const float4 *>(codes + at);
    return f;
  } else if constexpr (std::is_same<T, int16_t>::value) {
    const uint2 raw = *reinterpret_cast<const uint2 *>(codes + at);
    w[0] = static_cast<float>(static_cast<int16_t>(raw.x & 0xffffu));
    w[1] = static_cast<float>(static_cast<int16_t>(raw.x >> 16));
    w[2] = static_cast<float>(static_cast<int16_t>(raw.y & 0xffffu));
    w[3] = static_cast<float>(static_cast<int16_t>(raw.y >> 16));
  } else {
    const uint32_t raw = *reinterpret_cast<const uint32_t *>(codes + at);
#pragma unroll
    for (int i = 0; i < 4; i++) w[i] = static_cast<float>(static_cast<int8_t>((raw >> (8 * i)) & 0xffu));
  }
  const float s = a.scales[static_cast<size_t>(row) * a.groups + col / a.group];
#pragma unroll
  for (int i = 0; i < 4; i++) w[i] = w[i] * s;
  if (a.exc_index) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int e = a.exc_index[col + i];
      if (e >= 0) w[i] = a.exc_vals[static_cast<size_t>(row) * a.n_exc + e];
    }
  }
  return make_float4(w[0], w[1], w[2], w[3]);
}

// Tiles: BM x BN outputs per workgroup, 4 waves in a 2 x 2 grid, each wave
// (BM/2) x (BN/2) outputs in 32 x 32 matrix-core blocks. k advances 32 per
// stage; the next stage's global loads are issued into registers before the
// current stage's matrix-core work, then written to the other LDS buffer:
// one barrier per stage.
template <typename T, int EPI, int BM, int BN, bool VEC>
__global__ __launch_bounds__(256) void mfma_kernel(GemmArgs a) {
  constexpr int WM = BM / 64, WN = BN / 64;        // 32x32 blocks per wave
  constexpr int AF = BM * kBK / 4 / 256;           // float4 of A per thread per stage
  constexpr int BF = BN * kBK / 4 / 256;           // float4 of W per thread per stage
  __shared__ float as[2][BM][kPitch];
  __shared__ float bs[2][BN][kPitch];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int h = lane >> 5, l32 = lane & 31;
  const int c4 = tid & 7;  // float4 column of the 32-wide stage this thread stages

  // Rows this thread stages (clamped in bounds; rows past the edge are zeroed).
  int arow[AF], brow[BF];
  float ascale[AF];
#pragma unroll
  for (int i = 0; i < AF; i++) {
    const int r = m0 + tid / 8 + 32 * i;
    arow[i] = r < a.m ? r : a.m - 1;
    ascale[i] = r < a.m ? (a.row_scale ? a.row_scale[arow[i]] : 1.0f) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < BF; i++) {
    const int r = n0 + tid / 8 + 32 * i;
    brow[i] = r < a.n ? r : -1;
  }
  float4 areg[AF], breg[BF];
  auto load_stage = [&](int k0) {
    const int col = k0 + 4 * c4;
#pragma unroll
    for (int i = 0; i < AF; i++) {
      float4 v;
      if constexpr (VEC) {
        v = *reinterpret_cast<const float4 *>(a.x + static_cast<size_t>(arow[i]) * a.k + col);
      } else {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] = col + e < a.k ? a.x[static_cast<size_t>(arow[i]) * a.k + col + e] : 0.0f;
        v = make_float4(t[0], t[1], t[2], t[3]);
      }
      // A' = fl(a * row_scale); rows past the edge become 0.
      const float s = ascale[i];
      areg[i] = a.row_scale ? make_float4(v.x * s, v.y * s, v.z * s, v.w * s)
                            : (s != 0.0f ? v : make_float4(0.f, 0.f, 0.f, 0.f));
    }
#pragma unroll
    for (int i = 0; i < BF; i++) {
      if constexpr (VEC) {
        breg[i] = load_weights4<T>(a, brow[i] >= 0 ? brow[i] : 0, col);
        if (brow[i] < 0) breg[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        float t[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
          t[e] = (brow[i] >= 0 && col + e < a.k)
                     ? weight_at<T>(static_cast<const T *>(a.codes), a.scales, a.exc_index, a.exc_vals, a.n_exc, a.k,
                                    a.group, a.groups, brow[i], col + e)
                     : 0.0f;
        breg[i] = make_float4(t[0], t[1], t[2], t[3]);
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AF; i++) *reinterpret_cast<float4 *>(&as[buf][tid / 8 + 32 * i][4 * c4]) = areg[i];
#pragma unroll
    for (int i = 0; i < BF; i++) *reinterpret_cast<float4 *>(&bs[buf][tid / 8 + 32 * i][4 * c4]) = breg[i];
  };

  v16f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

  const int stages = (a.k + kBK - 1) / kBK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int st = 0; st < stages; st++) {
    const int buf = st & 1;
    if (st + 1 < stages) load_stage((st + 1) * kBK);
    // Lane half h supplies k-slot h of each 32x32x2 step: k = 16 h + s.
    float av[WM][16], bv[WN][16];
#pragma unroll
    for (int i = 0; i < WM; i++) {
      const float4 *ar = reinterpret_cast<const float4 *>(&as[buf][wm * (BM / 2) + i * 32 + l32][16 * h]);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 x = ar[q];
        av[i][4 * q] = x.x;
        av[i][4 * q + 1] = x.y;
        av[i][4 * q + 2] = x.z;
        av[i][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int j = 0; j < WN; j++) {
      const float4 *br = reinterpret_cast<const float4 *>(&bs[buf][wn * (BN / 2) + j * 32 + l32][16 * h]);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 y = br[q];
        bv[j][4 * q] = y.x;
        bv[j][4 * q + 1] = y.y;
        bv[j][4 * q + 2] = y.z;
        bv[j][4 * q + 3] = y.w;
      }
    }
#pragma unroll
    for (int s2 = 0; s2 < 16; s2++)
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][s2], bv[j][s2], acc[i][j], 0, 0, 0);
    if (st + 1 < stages) store_stage(buf ^ 1);
    __syncthreads();
  }
  // D layout of 32x32: column = lane % 32, row = 8 (r / 4) + 4 (lane / 32) + r % 4.
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
        const int col = n0 + wn * (BN / 2) + j * 32 + l32;
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
    return;
  }
  // Vector staging needs rows of whole float4 (and whole 32-stages of k).
  const bool vec = a.k % kBK == 0;
  // A narrower N tile when 128 x 128 tiles would not give two waves of
  // workgroups over the 256 compute units.
  const long tiles128 = static_cast<long>((a.m + 127) / 128) * ((a.n + 127) / 128);
  if (tiles128 >= 512) {
    const dim3 grid((a.m + 127) / 128, (a.n + 127) / 128);
    if (vec)
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 128, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 128, false>), grid, dim3(256), 0, stream, a);
  } else {
    const dim3 grid((a.m + 127) / 128, (a.n + 63) / 64);
    if (vec)
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 64, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 64, false>), grid, dim3(256), 0, stream, a);
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
