// FP32 prefill projections: C = A' * W^T with A' = fl(a * row_scale) and W the
// FP32 weights or fl(code * scale) (exception columns in place), written
// through the Store / Glu / Add epilogues (src/kernels/panels/panel.rs:26-172,
// driver.rs:57-140; kernels::linear_with_simd's large-M path, mod.rs:434-476).
//
// Kernels:
//  - dma_kernel (k a multiple of 64) / mfma_kernel (other shapes):
//    v_mfma_f32_32x32x2f32 tiles (FP32 inputs, FP32 accumulate). The matrix
//    core sums k-slices in its own order, so results match the reference's
//    ascending-k FMA chain within FP32 rounding (tolerance).
//  - chain2_kernel (k a multiple of 16) / chain_kernel (any shape): SIMT
//    register tiles in which every output is one FMA chain over ascending k
//    from +0.0: bitwise the reference's FP32 panels.
// INT16 / INT8 codes are read as codes by every kernel and turned into
// fl(code * scale) in registers (in dma_kernel as the B fragments are read,
// in the others on the way into LDS); no FP32 copy of a code matrix is ever
// written to memory.
//
// Roofline: FP32 matrix cores (157.3 TFLOP/s) for mfma_kernel; the FP32
// vector peak (157.3 TFLOP/s: gfx950 issues even non-packed FMAs faster than
// 16 lanes per clock, measured 114 TFLOP/s for a register-only FMA loop) for
// the chain kernels. FLOPs = 2*m*k*n.
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
  const int32_t *exc_cols;
  const float *exc_vals;
  int n_exc;
  int m, n, k, group, groups;
  float *out;
  int row0;  // dma_kernel: first output row of the launch's tiles (0 for the other kernels)
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
    w[0] = sdwa_cvt<4>(raw.x);
    w[1] = sdwa_cvt<5>(raw.x);
    w[2] = sdwa_cvt<4>(raw.y);
    w[3] = sdwa_cvt<5>(raw.y);
  } else {
    const uint32_t raw = *reinterpret_cast<const uint32_t *>(codes + at);
    w[0] = sdwa_cvt<0>(raw);
    w[1] = sdwa_cvt<1>(raw);
    w[2] = sdwa_cvt<2>(raw);
    w[3] = sdwa_cvt<3>(raw);
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

  // Each stage's 16 k-steps run in two halves of 8. The LDS reads of one half
  // are issued before the matrix-core work on the other, so their latency
  // hides behind it: half 1 of stage s is read before half 0's products, and
  // half 0 of stage s + 1 right after the barrier, before half 1's products.
  float fa[2][WM][8], fb[2][WN][8];
  auto read_half = [&](int buf, int half, float (*va)[8], float (*vb)[8]) {
#pragma unroll
    for (int i = 0; i < WM; i++) {
      const float4 *ar =
          reinterpret_cast<const float4 *>(&as[buf][wm * (BM / 2) + i * 32 + l32][16 * h + 8 * half]);
      const float4 x0 = ar[0], x1 = ar[1];
      va[i][0] = x0.x; va[i][1] = x0.y; va[i][2] = x0.z; va[i][3] = x0.w;
      va[i][4] = x1.x; va[i][5] = x1.y; va[i][6] = x1.z; va[i][7] = x1.w;
    }
#pragma unroll
    for (int j = 0; j < WN; j++) {
      const float4 *br =
          reinterpret_cast<const float4 *>(&bs[buf][wn * (BN / 2) + j * 32 + l32][16 * h + 8 * half]);
      const float4 y0 = br[0], y1 = br[1];
      vb[j][0] = y0.x; vb[j][1] = y0.y; vb[j][2] = y0.z; vb[j][3] = y0.w;
      vb[j][4] = y1.x; vb[j][5] = y1.y; vb[j][6] = y1.z; vb[j][7] = y1.w;
    }
  };
  // Lane half h supplies k-slot h of each 32x32x2 step: k = 16 h + 8 half + s.
  auto products = [&](float (*va)[8], float (*vb)[8]) {
#pragma unroll
    for (int s2 = 0; s2 < 8; s2++)
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[i][s2], vb[j][s2], acc[i][j], 0, 0, 0);
  };

  const int stages = (a.k + kBK - 1) / kBK;
  load_stage(0);
  store_stage(0);
  __syncthreads();
  read_half(0, 0, fa[0], fb[0]);
  for (int st = 0; st < stages; st++) {
    const int buf = st & 1;
    if (st + 1 < stages) load_stage((st + 1) * kBK);
    read_half(buf, 1, fa[1], fb[1]);
    products(fa[0], fb[0]);
    if (st + 1 < stages) store_stage(buf ^ 1);
    // The barrier's LDS wait also retires this stage's half-1 reads before
    // any wave overwrites this buffer (two stages on).
    __syncthreads();
    if (st + 1 < stages) read_half(buf ^ 1, 0, fa[0], fb[0]);
    products(fa[1], fb[1]);
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

// The matrix-core kernel for k a multiple of 64. A' stages of 16 k are
// copied HBM -> LDS by the LDS-DMA path (global_load_lds, 16 bytes per lane)
// into a ring of four stages, three stages ahead of the matrix cores, so the
// copies' latency never stalls them and no registers stage the data. Rows of
// a stage hold 16 floats as four 16-byte chunks, chunk c of row r stored at
// position c ^ dma_swizzle(r) (conflict-free for the 32-row fragment reads).
// The row scale is applied to the fragments as they are read (the same single
// rounding fl(a * row_scale)). Rows past m or n repeat the last row (in
// bounds); their outputs are not written.
//
// W, by weight type T:
//  - float: stages copied into a second LDS ring beside A's.
//  - int16 / int8 codes (group 64): never in LDS and never expanded to FP32
//    in memory. Each wave loads its own B fragments' codes straight into
//    registers one 64-k group ahead: lane (half h, column l32) of block j
//    holds, for stage t of the group, the 8 codes k = 16 t + 8 h + 0..7 of its
//    column (one 16-byte load for INT16, 8 bytes for INT8; the four loads of
//    a group cover the column's 128 or 64 code bytes whole) and the group's
//    scale. A fragment becomes fl(code * scale) in registers as it is read.
//    The codes of exception columns are zero (upload refuses others), so each
//    exception adds a'[r][col_e] * value[c][e] to the sums before the
//    epilogue; the matrix cores sum in their own order anyway.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_void;

constexpr int kDmaBK = 16;

__device__ __forceinline__ int dma_swizzle(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// s_waitcnt immediate for vmcnt(n) (n < 64) and lgkmcnt(0), expcnt not waited.
constexpr int wait_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0070; }

// Compiler-only ordering around the plain workgroup barrier: the waits are
// explicit (a __syncthreads fence would wait for every copy in flight).
__device__ __forceinline__ void plain_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <typename T, int EPI, int BN, int BM = 128>
__global__ __launch_bounds__(256) void dma_kernel(GemmArgs a) {
  constexpr bool kCodes = !std::is_same<T, float>::value;
  constexpr int WM = BM / 64, WN = BN / 64;
  constexpr int AT = BM / 64, BT = kCodes ? 0 : BN / 64;  // LDS-DMA copies of 1 KB per wave per stage
  constexpr int PER = AT + BT;
  constexpr int NB = kCodes ? 5 * WN : 0;  // code-register loads per wave per group: 4 pieces + the scale, per block
  constexpr int LB = kCodes ? 1 : BN * 4;
  using Piece = typename std::conditional<sizeof(T) == 1, uint2, uint4>::type;  // 8 codes
  __shared__ float4 la0[BM * 4], la1[BM * 4], la2[BM * 4], la3[BM * 4];
  __shared__ float4 lb0[LB], lb1[LB], lb2[LB], lb3[LB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = a.row0 + blockIdx.x * BM, n0 = blockIdx.y * BN;
  const int h = lane >> 5, l32 = lane & 31;

  // Copy t of this wave fills LDS chunks [64 (wave + 4 t), +64): row
  // 16 (wave + 4 t) + lane / 4, position lane % 4.
  const float *asrc[AT];
  const float *bsrc[BT > 0 ? BT : 1];
#pragma unroll
  for (int t = 0; t < AT; t++) {
    const int row = 16 * (wave + 4 * t) + (lane >> 2);
    const int g = m0 + row < a.m ? m0 + row : a.m - 1;
    asrc[t] = a.x + static_cast<size_t>(g) * a.k + 4 * ((lane & 3) ^ dma_swizzle(row));
  }
  if constexpr (!kCodes) {
    const float *w = static_cast<const float *>(a.codes);
#pragma unroll
    for (int t = 0; t < BT; t++) {
      const int row = 16 * (wave + 4 * t) + (lane >> 2);
      const int g = n0 + row < a.n ? n0 + row : a.n - 1;
      bsrc[t] = w + static_cast<size_t>(g) * a.k + 4 * ((lane & 3) ^ dma_swizzle(row));
    }
  }
  auto issue = [&](float4 *la, float4 *lb, int stage) {
    const int off = stage * kDmaBK;
#pragma unroll
    for (int t = 0; t < AT; t++)
      __builtin_amdgcn_global_load_lds((global_void *)(asrc[t] + off), (lds_void *)(la + 64 * (wave + 4 * t)), 16, 0, 0);
    if constexpr (!kCodes) {
#pragma unroll
      for (int t = 0; t < BT; t++)
        __builtin_amdgcn_global_load_lds((global_void *)(bsrc[t] + off), (lds_void *)(lb + 64 * (wave + 4 * t)), 16, 0,
                                         0);
    }
  };

  // Codes: this lane's column of block j, from k = 8 h.
  const T *csrc[WN];
  const float *ssrc[WN];
  Piece nxt[WN][4], cur[WN][4];
  float nsc[WN], csc[WN];
  if constexpr (kCodes) {
#pragma unroll
    for (int j = 0; j < WN; j++) {
      const int c = n0 + wn * (BN / 2) + 32 * j + l32;
      const int cc = c < a.n ? c : a.n - 1;
      csrc[j] = static_cast<const T *>(a.codes) + static_cast<size_t>(cc) * a.k + 8 * h;
      ssrc[j] = a.scales + static_cast<size_t>(cc) * a.groups;
    }
  }
  auto load_group = [&](int g) {
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int t = 0; t < 4; t++) nxt[j][t] = *reinterpret_cast<const Piece *>(csrc[j] + 64 * g + 16 * t);
#pragma unroll
    for (int j = 0; j < WN; j++) nsc[j] = ssrc[j][g];
  };

  float rs[WM];
#pragma unroll
  for (int i = 0; i < WM; i++) {
    const int r = m0 + wm * (BM / 2) + 32 * i + l32;
    rs[i] = a.row_scale ? a.row_scale[r < a.m ? r : a.m - 1] : 1.0f;
  }
  const bool scaled = a.row_scale != nullptr;

  // Lane half h holds k = 8 h .. 8 h + 7 of the stage (chunks 2h, 2h + 1).
  auto read_a = [&](const float4 *la, float (*va)[8]) {
#pragma unroll
    for (int i = 0; i < WM; i++) {
      const int r = wm * (BM / 2) + 32 * i + l32;
      const float4 x0 = la[4 * r + ((2 * h) ^ dma_swizzle(r))];
      const float4 x1 = la[4 * r + ((2 * h + 1) ^ dma_swizzle(r))];
      va[i][0] = x0.x; va[i][1] = x0.y; va[i][2] = x0.z; va[i][3] = x0.w;
      va[i][4] = x1.x; va[i][5] = x1.y; va[i][6] = x1.z; va[i][7] = x1.w;
    }
  };
  auto read_b = [&](const float4 *lb, float (*vb)[8]) {
#pragma unroll
    for (int j = 0; j < WN; j++) {
      const int r = wn * (BN / 2) + 32 * j + l32;
      const float4 y0 = lb[4 * r + ((2 * h) ^ dma_swizzle(r))];
      const float4 y1 = lb[4 * r + ((2 * h + 1) ^ dma_swizzle(r))];
      vb[j][0] = y0.x; vb[j][1] = y0.y; vb[j][2] = y0.z; vb[j][3] = y0.w;
      vb[j][4] = y1.x; vb[j][5] = y1.y; vb[j][6] = y1.z; vb[j][7] = y1.w;
    }
  };
  // Stage t of the current group's codes: fl(code * scale), k = 8 h + e.
  auto codes_b = [&](auto tc, float (*vb)[8]) {
    constexpr int t = decltype(tc)::value;
#pragma unroll
    for (int j = 0; j < WN; j++) {
      const Piece p = cur[j][t];
      if constexpr (sizeof(T) == 2) {
        vb[j][0] = sdwa_cvt<4>(p.x); vb[j][1] = sdwa_cvt<5>(p.x);
        vb[j][2] = sdwa_cvt<4>(p.y); vb[j][3] = sdwa_cvt<5>(p.y);
        vb[j][4] = sdwa_cvt<4>(p.z); vb[j][5] = sdwa_cvt<5>(p.z);
        vb[j][6] = sdwa_cvt<4>(p.w); vb[j][7] = sdwa_cvt<5>(p.w);
      } else {
        vb[j][0] = sdwa_cvt<0>(p.x); vb[j][1] = sdwa_cvt<1>(p.x);
        vb[j][2] = sdwa_cvt<2>(p.x); vb[j][3] = sdwa_cvt<3>(p.x);
        vb[j][4] = sdwa_cvt<0>(p.y); vb[j][5] = sdwa_cvt<1>(p.y);
        vb[j][6] = sdwa_cvt<2>(p.y); vb[j][7] = sdwa_cvt<3>(p.y);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) vb[j][e] = vb[j][e] * csc[j];
    }
  };

  v16f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
  auto products = [&](float (*va)[8], float (*vb)[8]) {
    if (scaled) {
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int e = 0; e < 8; e++) va[i][e] = va[i][e] * rs[i];
    }
#pragma unroll
    for (int s2 = 0; s2 < 8; s2++)
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(va[i][s2], vb[j][s2], acc[i][j], 0, 0, 0);
  };

  // Stage st sits in ring slot st % 4. Step st: wait for this wave's copies
  // of stage st (and its reads of the previous slot), meet the other waves,
  // start stage st + 3 into the previous stage's slot, read stage st's
  // fragments, then run the products of stage st - 1 while they arrive.
  // Codes: the first step of group g (st = 4 g) takes the group's codes,
  // loaded during group g - 1, and loads group g + 1's after stage st + 3's
  // copies. The waits count the copies issued after stage st's: two stages'
  // copies, plus group g + 1's code loads in steps 4 g + 1 .. 4 g + 3.
  const int stages = a.k / kDmaBK;  // a multiple of 4
  const int groups = stages / 4;
  float fa[2][WM][8], fb[2][WN][8];
  if constexpr (kCodes) load_group(0);
  issue(la0, lb0, 0);
  issue(la1, lb1, 1);
  issue(la2, lb2, 2);
  auto step = [&](int st, auto uc, const float4 *ca, const float4 *cb, float4 *na, float4 *nb, float (*ra)[8],
                  float (*rb)[8], float (*pa)[8], float (*pb)[8]) __attribute__((always_inline)) {
    constexpr int u = decltype(uc)::value;
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(2 * PER + (u == 0 ? 0 : NB)));
    plain_barrier();
    // Past the last stage the copy repeats it into the free slot, so the
    // count of copies in flight (and the waits) stay the same; past the last
    // group the code loads repeat it.
    issue(na, nb, st + 3 < stages ? st + 3 : stages - 1);
    if constexpr (kCodes) {
      if constexpr (u == 0) {
#pragma unroll
        for (int j = 0; j < WN; j++) {
#pragma unroll
          for (int t = 0; t < 4; t++) cur[j][t] = nxt[j][t];
          csc[j] = nsc[j];
        }
        const int g = st / 4 + 1;
        load_group(g < groups ? g : groups - 1);
      }
      read_a(ca, ra);
      codes_b(uc, rb);
    } else {
      read_a(ca, ra);
      read_b(cb, rb);
    }
    if (st > 0) products(pa, pb);
  };
  using U0 = std::integral_constant<int, 0>;
  using U1 = std::integral_constant<int, 1>;
  using U2 = std::integral_constant<int, 2>;
  using U3 = std::integral_constant<int, 3>;
  for (int st = 0; st < stages; st += 4) {
    step(st, U0(), la0, lb0, la3, lb3, fa[0], fb[0], fa[1], fb[1]);
    step(st + 1, U1(), la1, lb1, la0, lb0, fa[1], fb[1], fa[0], fb[0]);
    step(st + 2, U2(), la2, lb2, la1, lb1, fa[0], fb[0], fa[1], fb[1]);
    step(st + 3, U3(), la3, lb3, la2, lb2, fa[1], fb[1], fa[0], fb[0]);
  }
  products(fa[1], fb[1]);
  // The repeated copies must land before the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)

  // D layout of 32x32: column = lane % 32, row = 8 (r / 4) + 4 (lane / 32) + r % 4.
  if constexpr (kCodes) {
    // Exception columns: fl(a * row_scale) times the exception value, one
    // output row at a time (only its WN sums leave the accumulators).
    if (a.n_exc) {
      const float *wv[WN];
#pragma unroll
      for (int j = 0; j < WN; j++) {
        const int c = n0 + wn * (BN / 2) + 32 * j + l32;
        wv[j] = a.exc_vals + static_cast<size_t>(c < a.n ? c : a.n - 1) * a.n_exc;
      }
#pragma unroll
      for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
          const int rr = row < a.m ? row : a.m - 1;
          const float *xr = a.x + static_cast<size_t>(rr) * a.k;
          const float s = scaled ? a.row_scale[rr] : 1.0f;
          float sum[WN];
#pragma unroll
          for (int j = 0; j < WN; j++) sum[j] = acc[i][j][r];
          for (int e = 0; e < a.n_exc; e++) {
            float av = xr[a.exc_cols[e]];
            if (scaled) av = av * s;
#pragma unroll
            for (int j = 0; j < WN; j++) sum[j] = fmaf_(av, wv[j][e], sum[j]);
          }
#pragma unroll
          for (int j = 0; j < WN; j++) acc[i][j][r] = sum[j];
        }
    }
  }
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

// Exact-order kernel for whole 16-wide k stages: BM x BN outputs per
// workgroup, (BM / 16) x (BN / 16) per thread (rows 4 ty + 64 i + {0..3},
// columns 4 tx + 64 j + {0..3}), every output one FMA chain over ascending k
// from +0.0 (bitwise the FP32 panels). Stages of 16 k are held k-major in
// LDS, [k][BM] for A' and [k][BN] for W, so a thread reads the values of one
// k with 16-byte loads. The next stage's A and weights (FP32, or INT16 / INT8
// codes and their group's scale) are loaded raw into registers before the
// current stage's FMAs; only after them are they turned into A' = fl(a *
// row_scale) and W = fl(code * scale) (exception columns in place) and
// stored to the other buffer, so no wait for those loads precedes the FMAs.
// Rows past m and columns past n stage the last row / column in bounds; their
// outputs are not written.
constexpr int kC2K = 16;   // k per stage
constexpr int kC2Pad = 4;  // floats of padding per LDS k-row

// COUNT consecutive elements of T (a 4-, 8-, 16- or 32-byte aligned run) as
// raw 32-bit words.
template <typename T, int COUNT>
__device__ __forceinline__ void load_raw(const T *p, uint32_t *u) {
  constexpr int B = COUNT * static_cast<int>(sizeof(T));
  if constexpr (B == 32) {
    const uint4 x = reinterpret_cast<const uint4 *>(p)[0], y = reinterpret_cast<const uint4 *>(p)[1];
    u[0] = x.x; u[1] = x.y; u[2] = x.z; u[3] = x.w; u[4] = y.x; u[5] = y.y; u[6] = y.z; u[7] = y.w;
  } else if constexpr (B == 16) {
    const uint4 x = *reinterpret_cast<const uint4 *>(p);
    u[0] = x.x; u[1] = x.y; u[2] = x.z; u[3] = x.w;
  } else if constexpr (B == 8) {
    const uint2 x = *reinterpret_cast<const uint2 *>(p);
    u[0] = x.x; u[1] = x.y;
  } else {
    static_assert(B == 4, "run of 4, 8, 16 or 32 bytes");
    u[0] = *reinterpret_cast<const uint32_t *>(p);
  }
}

// The COUNT weights held raw in `u`: FP32 as they are, codes as
// fl(code * scale).
template <typename T, int COUNT>
__device__ __forceinline__ void weights_of(const uint32_t *u, float scale, float *w) {
#pragma unroll
  for (int e = 0; e < COUNT; e++) {
    if constexpr (std::is_same<T, float>::value)
      w[e] = __uint_as_float(u[e]);
    else if constexpr (sizeof(T) == 2)
      w[e] = (e % 2 == 0 ? sdwa_cvt<4>(u[e / 2]) : sdwa_cvt<5>(u[e / 2])) * scale;
    else
      w[e] = (e % 4 == 0   ? sdwa_cvt<0>(u[e / 4])
              : e % 4 == 1 ? sdwa_cvt<1>(u[e / 4])
              : e % 4 == 2 ? sdwa_cvt<2>(u[e / 4])
                           : sdwa_cvt<3>(u[e / 4])) *
             scale;
  }
}

template <typename T, int EPI, int BM, int BN>
__global__ __launch_bounds__(256) void chain2_kernel(GemmArgs a) {
  constexpr int TM = BM / 16, TN = BN / 16;     // outputs per thread
  constexpr int AK = BM / 16, BK = BN / 16;     // k staged per thread (A, W)
  constexpr int BW = BK * static_cast<int>(sizeof(T)) / 4;  // raw words of W per thread
  __shared__ float as[2][kC2K][BM + kC2Pad];
  __shared__ float bs[2][kC2K][BN + kC2Pad];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BN;

  // Staging: A row tid / (256 / BM), k offset (tid % (256 / BM)) * AK; W row
  // tid / (256 / BN), k offset (tid % (256 / BN)) * BK.
  const int srow = tid / (256 / BM), sk = (tid % (256 / BM)) * AK;
  const int wrow_t = tid / (256 / BN), wk = (tid % (256 / BN)) * BK;
  const int arow = m0 + srow < a.m ? m0 + srow : a.m - 1;
  const float ascale = a.row_scale ? a.row_scale[arow] : 1.0f;
  const float *aptr = a.x + static_cast<size_t>(arow) * a.k + sk;
  const int wrow = n0 + wrow_t < a.n ? n0 + wrow_t : a.n - 1;
  const T *wptr = static_cast<const T *>(a.codes) + static_cast<size_t>(wrow) * a.k + wk;
  const float *sptr = a.scales ? a.scales + static_cast<size_t>(wrow) * a.groups : nullptr;
  uint32_t ua[AK], ub[BW];
  float sc = 1.0f;
  auto load = [&](int k0) {
    load_raw<float, AK>(aptr + k0, ua);
    load_raw<T, BK>(wptr + k0, ub);
    if constexpr (!std::is_same<T, float>::value) {
      const int col = k0 + wk;
      sc = sptr[a.group == 64 ? col >> 6 : col / a.group];
    }
  };
  auto store = [&](int buf, int k0) {
#pragma unroll
    for (int e = 0; e < AK; e++) as[buf][sk + e][srow] = __uint_as_float(ua[e]) * ascale;
    float w[BK];
    weights_of<T, BK>(ub, sc, w);
    if constexpr (!std::is_same<T, float>::value) {
      if (a.exc_index) {
#pragma unroll
        for (int e = 0; e < BK; e++) {
          const int x = a.exc_index[k0 + wk + e];
          if (x >= 0) w[e] = a.exc_vals[static_cast<size_t>(wrow) * a.n_exc + x];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < BK; e++) bs[buf][wk + e][wrow_t] = w[e];
  };

  float acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = 0.0f;
  auto compute = [&](int buf) {
#pragma unroll 2
    for (int kk = 0; kk < kC2K; kk++) {
      float av[TM], bv[TN];
#pragma unroll
      for (int q = 0; q < TM / 4; q++) {
        const float4 a4 = *reinterpret_cast<const float4 *>(&as[buf][kk][64 * q + 4 * ty]);
        av[4 * q] = a4.x; av[4 * q + 1] = a4.y; av[4 * q + 2] = a4.z; av[4 * q + 3] = a4.w;
      }
#pragma unroll
      for (int q = 0; q < TN / 4; q++) {
        const float4 b4 = *reinterpret_cast<const float4 *>(&bs[buf][kk][64 * q + 4 * tx]);
        bv[4 * q] = b4.x; bv[4 * q + 1] = b4.y; bv[4 * q + 2] = b4.z; bv[4 * q + 3] = b4.w;
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = fmaf_(av[i], bv[j], acc[i][j]);
    }
  };

  const int stages = a.k / kC2K;
  load(0);
  store(0, 0);
  __syncthreads();
  for (int st = 0; st < stages; st++) {
    const int buf = st & 1;
    if (st + 1 < stages) load((st + 1) * kC2K);
    compute(buf);
    if (st + 1 < stages) store(buf ^ 1, (st + 1) * kC2K);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TM; i++) {
    const int row = m0 + 64 * (i / 4) + 4 * ty + (i % 4);
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int col = n0 + 64 * (j / 4) + 4 * tx + (j % 4);
      emit<EPI>(a, row, col, acc[i][j], acc[i][j ^ 1]);
    }
  }
}

GemmArgs make_args(const Linear *lin, const float *x, size_t rows, const float *row_scale, float *out) {
  GemmArgs a;
  a.x = x;
  a.row_scale = row_scale;
  a.codes = lin->codes;
  a.scales = lin->scales;
  a.exc_index = lin->exc_index;
  a.exc_cols = lin->exc_cols;
  a.exc_vals = lin->exc_vals;
  a.n_exc = static_cast<int>(lin->n_exc);
  a.m = static_cast<int>(rows);
  a.n = static_cast<int>(lin->n);
  a.k = static_cast<int>(lin->k);
  a.group = static_cast<int>(lin->group);
  a.groups = static_cast<int>(lin->groups);
  a.out = out;
  a.row0 = 0;
  return a;
}

template <typename T, int EPI>
void launch_one(bool chain, const GemmArgs &a, hipStream_t stream) {
  if (chain) {
    // Whole 16-wide k stages with 16-byte aligned rows: the k-major kernel;
    // other shapes stage element by element.
    const bool aligned = (reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.codes)) % 16 == 0;
    if (a.k % kC2K == 0 && aligned && (std::is_same<T, float>::value || a.group % 8 == 0)) {
      // 128 x 128 tiles where they give at least two per compute unit,
      // 64 x 64 ones otherwise (n = 768 at 6,544 rows: WO 0.264 -> 0.195 ms).
      const long big = static_cast<long>((a.m + 127) / 128) * ((a.n + 127) / 128);
      if (big >= 512)
        hipLaunchKernelGGL((chain2_kernel<T, EPI, 128, 128>), dim3((a.m + 127) / 128, (a.n + 127) / 128), dim3(256), 0,
                           stream, a);
      else
        hipLaunchKernelGGL((chain2_kernel<T, EPI, 64, 64>), dim3((a.m + 63) / 64, (a.n + 63) / 64), dim3(256), 0,
                           stream, a);
      return;
    }
    const dim3 grid((a.m + kChainTile - 1) / kChainTile, (a.n + kChainTile - 1) / kChainTile);
    hipLaunchKernelGGL((chain_kernel<T, EPI>), grid, dim3(256), 0, stream, a);
    return;
  }
  // A narrower N tile when 128 x 128 tiles would not give four waves of
  // workgroups over the 256 compute units (QKV 768 -> 2048 at 6,544 rows
  // measured 0.240 -> 0.231 ms with it).
  const long tiles128 = static_cast<long>((a.m + 127) / 128) * ((a.n + 127) / 128);
  // The DMA kernel: k a multiple of 64, 16-byte aligned operands, and for
  // codes one scale per 64-k group.
  const bool aligned = (reinterpret_cast<uintptr_t>(a.x) | reinterpret_cast<uintptr_t>(a.codes)) % 16 == 0;
  if (a.k % (4 * kDmaBK) == 0 && aligned && (std::is_same<T, float>::value || a.group == 4 * kDmaBK)) {
    // 64 x 64 tiles when even 128 x 64 gives fewer than 1,024 (n = 768 at
    // 6,544 rows: 624 tiles of 128 x 64 on 768 workgroup slots leave a
    // third of the compute units a tile short at the end; 1,236 tiles of
    // 64 x 64 on 1,280 slots do not): WO 72.5 -> 85.9 and W2 77.7 -> 87.6
    // TFLOP/s, outputs unchanged (each one's k order is the tile's).
    const long tiles128x64 = static_cast<long>((a.m + 127) / 128) * ((a.n + 63) / 64);
    if (tiles128 >= 1024) {
      // 128 x 128 tiles take two workgroup slots per compute unit (512 on
      // the chip). When they leave a last round mostly empty (6,544 x 4096:
      // 1,664 tiles = 3.25 rounds), the row blocks of whole rounds run as
      // 128 x 128 tiles and the rows left over as 64 x 64 tiles in a second
      // launch, if those fit one round of its 1,280 slots (five per compute
      // unit): the literal shape 0.560 -> 0.538 ms in A/B runs; W13 (3.66
      // rounds, 1,368 leftover tiles) gained nothing and keeps one launch.
      // Every output is the same 32 x 32 block computation either way
      // (bitwise unchanged).
      const int slots = 512, small_slots = 1280;
      const int mtiles = (a.m + 127) / 128, ntiles = (a.n + 127) / 128;
      const int rb = static_cast<int>((tiles128 / slots) * slots / ntiles);  // row blocks of whole rounds
      const long small = static_cast<long>((a.m - 128 * rb + 63) / 64) * ((a.n + 63) / 64);
      const bool mostly_empty = tiles128 % slots != 0 && tiles128 % slots <= slots / 2;
      if (mostly_empty && rb > 0 && rb < mtiles && small <= small_slots) {
        hipLaunchKernelGGL((dma_kernel<T, EPI, 128>), dim3(rb, ntiles), dim3(256), 0, stream, a);
        GemmArgs rest = a;
        rest.row0 = 128 * rb;
        hipLaunchKernelGGL((dma_kernel<T, EPI, 64, 64>), dim3((a.m - rest.row0 + 63) / 64, (a.n + 63) / 64),
                           dim3(256), 0, stream, rest);
      } else {
        hipLaunchKernelGGL((dma_kernel<T, EPI, 128>), dim3(mtiles, ntiles), dim3(256), 0, stream, a);
      }
    } else if (tiles128x64 >= 1024) {
      // 128 x 64 tiles take three workgroup slots per compute unit (768 on
      // the chip); the same split when their last round is at most half full
      // (QKV 768 -> 2048 at 6,544 rows: 1,664 tiles = 2.17 rounds; 48 row
      // blocks of whole rounds, then 400 rows as 224 tiles of 64 x 64).
      const int slots = 768, small_slots = 1280;
      const int mtiles = (a.m + 127) / 128, ntiles = (a.n + 63) / 64;
      const int rb = static_cast<int>((tiles128x64 / slots) * slots / ntiles);
      const long small = static_cast<long>((a.m - 128 * rb + 63) / 64) * ((a.n + 63) / 64);
      const bool mostly_empty = tiles128x64 % slots != 0 && tiles128x64 % slots <= slots / 2;
      if (mostly_empty && rb > 0 && rb < mtiles && small <= small_slots) {
        hipLaunchKernelGGL((dma_kernel<T, EPI, 64>), dim3(rb, ntiles), dim3(256), 0, stream, a);
        GemmArgs rest = a;
        rest.row0 = 128 * rb;
        hipLaunchKernelGGL((dma_kernel<T, EPI, 64, 64>), dim3((a.m - rest.row0 + 63) / 64, (a.n + 63) / 64),
                           dim3(256), 0, stream, rest);
      } else {
        hipLaunchKernelGGL((dma_kernel<T, EPI, 64>), dim3(mtiles, ntiles), dim3(256), 0, stream, a);
      }
    } else
      hipLaunchKernelGGL((dma_kernel<T, EPI, 64, 64>), dim3((a.m + 63) / 64, (a.n + 63) / 64), dim3(256), 0, stream,
                         a);
    return;
  }
  // Vector staging needs rows of whole float4 (and whole 32-stages of k).
  const bool vec = a.k % kBK == 0;
  if (tiles128 >= 512) {
    const dim3 grid((a.m + 127) / 128, (a.n + 127) / 128);
    if (vec)
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 128, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 128, false>), grid, dim3(256), 0, stream, a);
  } else if (static_cast<long>((a.m + 127) / 128) * ((a.n + 63) / 64) >= 1024) {
    const dim3 grid((a.m + 127) / 128, (a.n + 63) / 64);
    if (vec)
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 64, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 128, 64, false>), grid, dim3(256), 0, stream, a);
  } else {
    // n = 768: 624 tiles of 128 x 64 took two rounds of 512 workgroup slots
    // (two per compute unit by LDS), the second a fifth full; 64 x 64 tiles
    // fit four per unit and make both rounds half as long (WO 39 -> 58,
    // W2 42 -> 63 TFLOP/s on INT16 codes; outputs unchanged).
    const dim3 grid((a.m + 63) / 64, (a.n + 63) / 64);
    if (vec)
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 64, 64, true>), grid, dim3(256), 0, stream, a);
    else
      hipLaunchKernelGGL((mfma_kernel<T, EPI, 64, 64, false>), grid, dim3(256), 0, stream, a);
  }
}

// ---- FP32 products on the FP16 matrix cores (FOCR_PROJ_F32_SPLIT) ---------
// Every row of A' = fl(x * row_scale) and of W is scaled by a power of two
// that puts its largest finite magnitude in [2^14, 2^15) and written as FP16
// pairs, x' = hi + lo to about 2^-22 |x'| (pair1). A product is then
// hi.hi + hi.lo + lo.hi, summed by v_mfma_f32_32x32x16_f16 in FP32 (lo.lo,
// left out, is below 2^-21 |x' y'|), and the output takes the exact
// power-of-two descale 2^(e_row + e_col - 30). Three FP16 products per 16 k
// cost 96 matrix-core cycles against 512 for eight v_mfma_f32_32x32x2f32.
// A row of A' or of W that holds an infinity or NaN cannot go through the
// pairs (an infinity in hi meets the other operand's zero lo: inf * 0 =
// NaN, where FP32 products give the infinity): its exponent entry carries
// kPairNonfinite on top of the exponent, and the outputs it reaches are
// recomputed by the reference's FP32 chain (chain_output).
constexpr int kSplitBM = 128, kSplitBN = 128, kSplitBK = 16, kSplitKAlign = 32;
constexpr int kPairNonfinite = 1 << 16;

// One output by the reference's FP32 panel order (panel.rs:154-172): an FMA
// chain over k ascending from +0 on A' = fl(x * row_scale) and W, bitwise
// the FP32 chain kernel's.
__device__ __forceinline__ float chain_output(const GemmArgs &a, int row, int col) {
  const float *x = a.x + static_cast<size_t>(row) * a.k;
  const float *w = static_cast<const float *>(a.codes) + static_cast<size_t>(col) * a.k;
  const float rs = a.row_scale ? a.row_scale[row] : 1.0f;
  float acc = 0.0f;
  for (int kk = 0; kk < a.k; kk++) acc = fmaf_(a.row_scale ? __fmul_rn(x[kk], rs) : x[kk], w[kk], acc);
  return acc;
}

// The FP16-pair operand of src [rows][cols] (rows padded to rows_pad, a
// multiple of 4; cols to cols_pad, a multiple of 32), one workgroup per 4
// rows:
//  - exps[row] = the pair exponent of fl(src[row] * row_scale[row]) (of
//    src[row] without a row scale), plus kPairNonfinite if one of those
//    values is an infinity or NaN, kPairMinExp for padding rows: a wave per
//    row;
//  - two FP16 planes (hi, lo) of those values scaled by 2^(15 - exps[row]),
//    zero past rows and cols, stage-major: plane p, 16-k stage s, row r at
//    ((p * stages + s) * rows_pad + r) * 16, so that one stage of
//    consecutive rows is one contiguous run (the GEMM's copies read whole
//    1 KB pieces). Thread (s % 16, r, q) converts values 16 s + 4 q .. + 3 of
//    row r; sixteen threads write one stage of the 4 rows, 128 contiguous
//    bytes per plane. The second pass reads the rows the first one just read.
constexpr int kRowBatch = 4;
__global__ __launch_bounds__(256) void pair_rows_kernel(const float *__restrict__ src, int rows, int cols,
                                                        const float *__restrict__ row_scale, bool vec,
                                                        int *__restrict__ exps, uint16_t *__restrict__ dst,
                                                        int rows_pad, int cols_pad) {
  __shared__ int row_exp[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int r0 = blockIdx.x * 4;
  {
    const int row = r0 + wave;
    float m = 0.0f;
    bool nonfinite = false;
    if (row < rows) {
      const float *r = src + static_cast<size_t>(row) * cols;
      const float sc = row_scale ? row_scale[row] : 1.0f;
      if (vec) {
        // kRowBatch loads in flight per lane before any is used.
        for (int c0 = 4 * lane; c0 < cols; c0 += 256 * kRowBatch) {
          float4 f[kRowBatch];
#pragma unroll
          for (int u = 0; u < kRowBatch; u++) {
            const int c = c0 + 256 * u;
            f[u] = c < cols ? *reinterpret_cast<const float4 *>(r + c) : make_float4(0.f, 0.f, 0.f, 0.f);
          }
#pragma unroll
          for (int u = 0; u < kRowBatch; u++) {
            const float v0 = row_scale ? f[u].x * sc : f[u].x, v1 = row_scale ? f[u].y * sc : f[u].y;
            const float v2 = row_scale ? f[u].z * sc : f[u].z, v3 = row_scale ? f[u].w * sc : f[u].w;
            m = __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fmaxf(finite_abs(v0), finite_abs(v1)),
                                                   __builtin_fmaxf(finite_abs(v2), finite_abs(v3))));
            nonfinite |= !(is_finite(v0) && is_finite(v1) && is_finite(v2) && is_finite(v3));
          }
        }
      } else {
        for (int c = lane; c < cols; c += 64) {
          const float v = row_scale ? r[c] * sc : r[c];
          m = __builtin_fmaxf(m, finite_abs(v));
          nonfinite |= !is_finite(v);
        }
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
    const bool flag = __builtin_amdgcn_ballot_w64(nonfinite) != 0;
    if (lane == 0) {
      const int e = pair_exp(m);
      row_exp[wave] = e;
      exps[row] = flag ? e + kPairNonfinite : e;
    }
  }
  __syncthreads();
  const int stages = cols_pad / 16;
  const size_t plane = static_cast<size_t>(stages) * rows_pad * 16;
  const int q = threadIdx.x & 3, rl = (threadIdx.x >> 2) & 3, row = r0 + rl;
  const int shift = 15 - row_exp[rl];
  const float *rp = src + static_cast<size_t>(row < rows ? row : 0) * cols;
  const float sc = row_scale && row < rows ? row_scale[row] : 1.0f;
  // kRowBatch stages per thread and pass: their loads are all in flight
  // before the first is converted.
  for (int st0 = threadIdx.x >> 4; st0 < stages; st0 += 16 * kRowBatch) {
    float v[kRowBatch][4];
    if (vec) {
      // cols % 4 == 0: a 4-value group is wholly in or past the row; the
      // loads read an in-bounds group either way (branch-free, so none waits
      // for another).
      float4 f[kRowBatch];
#pragma unroll
      for (int u = 0; u < kRowBatch; u++) {
        const int c0 = 16 * (st0 + 16 * u) + 4 * q;
        const bool ok = row < rows && st0 + 16 * u < stages && c0 < cols;
        f[u] = *reinterpret_cast<const float4 *>(rp + (ok ? c0 : 0));
        f[u] = ok ? f[u] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < kRowBatch; u++) {
        v[u][0] = f[u].x;
        v[u][1] = f[u].y;
        v[u][2] = f[u].z;
        v[u][3] = f[u].w;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kRowBatch; u++) {
        const int c0 = 16 * (st0 + 16 * u) + 4 * q;
        const bool ok = row < rows && st0 + 16 * u < stages;
#pragma unroll
        for (int e = 0; e < 4; e++) v[u][e] = ok && c0 + e < cols ? rp[c0 + e] : 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < kRowBatch; u++) {
      const int st = st0 + 16 * u;
      if (st >= stages) break;
      const int c0 = 16 * st + 4 * q;
      if (row < rows && row_scale) {
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (c0 + e < cols) v[u][e] = v[u][e] * sc;
      }
      uint16_t hh[4], ll[4];
#pragma unroll
      for (int e = 0; e < 4; e++) pair1(v[u][e], shift, hh[e], ll[e]);
      const size_t off = (static_cast<size_t>(st) * rows_pad + row) * 16 + 4 * q;
      *reinterpret_cast<uint2 *>(dst + off) = make_uint2(hh[0] | hh[1] << 16, hh[2] | hh[3] << 16);
      *reinterpret_cast<uint2 *>(dst + plane + off) = make_uint2(ll[0] | ll[1] << 16, ll[2] | ll[3] << 16);
    }
  }
}

typedef _Float16 pair_half8 __attribute__((ext_vector_type(8)));
union PairFrag {
  uint4 u;
  pair_half8 v;
};

// 128 x 128 outputs per workgroup, 4 waves in 2 x 2, each 64 x 64 in 32 x 32
// blocks. Stages of 16 k: per operand two planes x 128 rows x 32 bytes
// (each plane's rows of a stage contiguous in memory), copied HBM -> LDS by
// the LDS-DMA path (16 bytes per lane, two copies of 1 KB per wave and
// operand) into a ring of three stages, two stages ahead. A row's
// two 16-byte chunks (k 0..7, 8..15) are stored swapped when (row / 8) is
// odd: the 16 lanes a ds_read_b128 serves (rows r..r+15, one chunk) then hit
// 16 distinct bank groups. Step st reads stage st's fragments while the
// products of stage st - 1 run. Rows and columns are padded to 128 with zeros
// in the planes; outputs past m or n are not written.
// Tile order: workgroups are dealt to the 8 XCDs round robin (block b runs on
// XCD b % 8); block b takes tile t = (b % 8) * per + b / 8, so each XCD walks
// a contiguous run of tiles, in panels of kSplitPanel row tiles (column tiles
// in order, rows fastest): the workgroups an XCD holds at once share a few A
// row tiles and B column tiles in its own L2.
constexpr int kSplitPanel = 4;
__device__ __forceinline__ void split_tile(int b, int row_tiles, int col_tiles, int &rt, int &ct) {
  const int total = row_tiles * col_tiles;
  const int per = total / 8;
  const int t = b < 8 * per ? (b % 8) * per + b / 8 : b;
  const int panel = t / (kSplitPanel * col_tiles);
  const int rem = t - panel * kSplitPanel * col_tiles;
  const int rows = row_tiles - panel * kSplitPanel < kSplitPanel ? row_tiles - panel * kSplitPanel : kSplitPanel;
  ct = rem / rows;
  rt = panel * kSplitPanel + rem % rows;
}

template <int EPI, int BM>
__global__ __launch_bounds__(256) void split_kernel(GemmArgs a, const uint16_t *__restrict__ ap,
                                                    const uint16_t *__restrict__ bp, const int *__restrict__ aexp,
                                                    const int *__restrict__ bexp, size_t a_plane, size_t b_plane,
                                                    int kp, int row_tiles, int col_tiles) {
  // BM x 128 outputs (BM = 128 or 64). An A plane of a stage holds 2 BM
  // slots of 16 bytes (AS), a B plane 256. The ring's three slots, each
  // [A plane * AS + slot u | B plane * 256 + slot u], are separate arrays and
  // every step names its slots statically: the compiler then sees that a
  // step's fragment reads never touch the slot being copied into.
  constexpr int AS = 2 * BM, AC = BM / 64;  // A slots per plane, A copies per wave and stage
  constexpr int IB = BM / 64;               // 32-row blocks per wave
  constexpr int RS = 2 * AS + 2 * 256;  // slots of one ring entry
  __shared__ uint4 ring0[RS], ring1[RS], ring2[RS];
  __shared__ int tile_exp[2][kSplitBN];
  __shared__ bool tile_bad[2][kSplitBN];
  __shared__ int tile_any;  // a flagged row or column in the tile
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  if (tid == 0) tile_any = 0;  // the main loop's barriers order it before the epilogue's writes
  int rt, ct;
  split_tile(blockIdx.x, row_tiles, col_tiles, rt, ct);
  const int m0 = a.row0 + rt * BM, n0 = ct * kSplitBN;
  const int h = lane >> 5, l32 = lane & 31;
  // Copy t of operand o fills slots q = 64 (wave + 4 t) + lane: plane q / S,
  // slot u = q % S = row u / 2, chunk (u % 2) ^ ((row / 8) % 2) (S = AS for
  // A, 256 for B).
  const char *src[2][2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int q = 64 * (wave + 4 * t) + lane;
    {
      const int pa = q / AS, ua = q % AS, ra = ua >> 1;
      const int ca = (ua & 1) ^ ((ra >> 3) & 1);
      src[0][t] = reinterpret_cast<const char *>(ap + (pa < 2 ? pa : 1) * a_plane +
                                                 static_cast<size_t>(m0 + ra) * kSplitBK + 8 * ca);
    }
    const int pb = q >> 8, ub = q & 255, rb = ub >> 1;
    const int cb = (ub & 1) ^ ((rb >> 3) & 1);
    src[1][t] = reinterpret_cast<const char *>(bp + pb * b_plane + static_cast<size_t>(n0 + rb) * kSplitBK + 8 * cb);
  }
  const int stages = kp / kSplitBK;  // even
  // Stage-major planes: stage s of a plane starts rows_pad * 32 bytes after s - 1.
  const size_t a_step = a_plane / stages * 2, b_step = b_plane / stages * 2;  // bytes
  auto issue = [&](uint4 *slot, int stage) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < AC; t++)
      __builtin_amdgcn_global_load_lds((global_void *)(src[0][t] + stage * a_step),
                                       (lds_void *)(&slot[64 * (wave + 4 * t)]), 16, 0, 0);
#pragma unroll
    for (int t = 0; t < 2; t++)
      __builtin_amdgcn_global_load_lds((global_void *)(src[1][t] + stage * b_step),
                                       (lds_void *)(&slot[2 * AS + 64 * (wave + 4 * t)]), 16, 0, 0);
  };
  // Fragments of a stage: A blocks i and B blocks j, planes hi, lo.
  auto read = [&](const uint4 *slot, PairFrag (*fa)[2], PairFrag (*fb)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < IB; i++) {
      const int r = wm * 32 * IB + 32 * i + l32;
      const int u = 2 * r + (h ^ ((r >> 3) & 1));
#pragma unroll
      for (int p = 0; p < 2; p++) fa[i][p].u = slot[p * AS + u];
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int r = wn * 64 + 32 * j + l32;
      const int u = 2 * r + (h ^ ((r >> 3) & 1));
#pragma unroll
      for (int p = 0; p < 2; p++) fb[j][p].u = slot[2 * AS + p * 256 + u];
    }
  };
  v16f acc[IB][2];
#pragma unroll
  for (int i = 0; i < IB; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
  // The three pair products, smallest first: (lo, hi), (hi, lo), (hi, hi).
  auto products = [&](PairFrag (*fa)[2], PairFrag (*fb)[2]) __attribute__((always_inline)) {
    constexpr int pa[3] = {1, 0, 0}, pb[3] = {0, 1, 0};
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
      for (int i = 0; i < IB; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i][pa[q]].v, fb[j][pb[q]].v, acc[i][j], 0, 0, 0);
  };
  PairFrag fa0[IB][2], fb0[2][2], fa1[IB][2], fb1[2][2];
  issue(ring0, 0);
  issue(ring1, 1);
  // Step st (stage st in slot st % 3): wait for this wave's copies of stage
  // st (stage st + 1's may still fly) and its earlier LDS reads, meet the
  // other waves (nobody still reads stage st - 1's slot), start stage st + 2
  // there (past the last stage the copy repeats it, so the counts stay the
  // same), read stage st's fragments, then run stage st - 1's products.
  auto step = [&](int st, const uint4 *cur, uint4 *next, PairFrag (*ra)[2],
                  PairFrag (*rb)[2], PairFrag (*pa)[2], PairFrag (*pb)[2]) __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(AC + 2));
    plain_barrier();
    issue(next, st + 2 < stages ? st + 2 : stages - 1);
    read(cur, ra, rb);
    if (st > 0) products(pa, pb);
  };
  // Six steps cycle through the three slots and the two fragment sets.
  int st = 0;
  for (; st + 6 <= stages; st += 6) {
    step(st, ring0, ring2, fa0, fb0, fa1, fb1);
    step(st + 1, ring1, ring0, fa1, fb1, fa0, fb0);
    step(st + 2, ring2, ring1, fa0, fb0, fa1, fb1);
    step(st + 3, ring0, ring2, fa1, fb1, fa0, fb0);
    step(st + 4, ring1, ring0, fa0, fb0, fa1, fb1);
    step(st + 5, ring2, ring1, fa1, fb1, fa0, fb0);
  }
  if (st < stages) {  // 2 or 4 stages left
    step(st, ring0, ring2, fa0, fb0, fa1, fb1);
    step(st + 1, ring1, ring0, fa1, fb1, fa0, fb0);
    if (st + 2 < stages) {
      step(st + 2, ring2, ring1, fa0, fb0, fa1, fb1);
      step(st + 3, ring0, ring2, fa1, fb1, fa0, fb0);
    }
  }
  products(fa1, fb1);
  // The tile's row and column exponents (the planes are padded to whole
  // 128-row tiles, and so are the exponent arrays) and non-finite flags.
  if (tid < BM || tid >= 128) {
    const int o = tid < BM ? 0 : 1, t = tid & 127;
    const int e = o == 0 ? aexp[m0 + t] : bexp[n0 + t];
    const bool bad = e >= kPairNonfinite / 2;
    tile_exp[o][t] = bad ? e - kPairNonfinite : e;
    tile_bad[o][t] = bad;
    if (bad) tile_any = 1;
  }
  // The repeated copies must land before the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
  __syncthreads();
  // D layout of 32x32: column = lane % 32, row = 8 (r / 4) + 4 (lane / 32) + r % 4.
  // With CHECKED, outputs a flagged row or column reaches (for Glu, either
  // column of the pair) are left to the pass below.
  auto store = [&](auto checked) __attribute__((always_inline)) {
    constexpr bool CHECKED = decltype(checked)::value;
#pragma unroll
    for (int i = 0; i < IB; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int lc = wn * 64 + j * 32 + l32;
        const int ce = tile_exp[1][lc] - 30;
        const bool bad_col = CHECKED && (tile_bad[1][lc] || (EPI == FOCR_EPI_GLU && tile_bad[1][lc ^ 1]));
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int lr = wm * 32 * IB + i * 32 + 8 * (r / 4) + 4 * h + (r % 4);
          const float v = __builtin_ldexpf(acc[i][j][r], tile_exp[0][lr] + ce);
          const float partner = EPI == FOCR_EPI_GLU ? __shfl_xor(v, 1) : 0.0f;
          if (!CHECKED || !(bad_col || tile_bad[0][lr])) emit<EPI>(a, m0 + lr, n0 + lc, v, partner);
        }
      }
  };
  if (tile_any == 0) {
    store(std::false_type{});
  } else {
    store(std::true_type{});
    // The flagged outputs (Glu: column pairs) by the FP32 chain. Thread t
    // takes outputs u = (idx * 40503) mod N for idx = t, t + 256, ...: a
    // bijection of the tile's N outputs that spreads a flagged row's or
    // column's outputs over the workgroup.
    constexpr int W = EPI == FOCR_EPI_GLU ? kSplitBN / 2 : kSplitBN, N = BM * W;
    for (int idx = tid; idx < N; idx += 256) {
      const int u = static_cast<int>((static_cast<unsigned>(idx) * 40503u) & (N - 1));
      const int lr = u / W, lc = (u % W) * (EPI == FOCR_EPI_GLU ? 2 : 1);
      const int row = m0 + lr, col = n0 + lc;
      const bool hit = tile_bad[0][lr] || tile_bad[1][lc] || (EPI == FOCR_EPI_GLU && tile_bad[1][lc + 1]);
      if (!hit || row >= a.m || col >= a.n) continue;
      const float v = chain_output(a, row, col);
      emit<EPI>(a, row, col, v, EPI == FOCR_EPI_GLU ? chain_output(a, row, col + 1) : 0.0f);
    }
  }
}

// The row exponents and FP16-pair planes of src [r][c] (rows padded to
// r_pad, a multiple of 128; columns to kp).
void pair_operand(hipStream_t stream, const float *src, size_t r, size_t c, const float *rs, int *exps, uint16_t *dst,
                  size_t r_pad, size_t kp) {
  const bool vec = c % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0;
  hipLaunchKernelGGL(pair_rows_kernel, dim3(static_cast<unsigned>(r_pad / 4)), dim3(256), 0, stream, src,
                     static_cast<int>(r), static_cast<int>(c), rs, vec, exps, dst, static_cast<int>(r_pad),
                     static_cast<int>(kp));
}

int launch_split(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale, int epilogue,
                 float *out) {
  FOCR_REQUIRE(lin->bits == 32, FOCR_E_UNSUPPORTED,
               "FOCR_PROJ_F32_SPLIT takes FP32 weights (codes would be materialized); plan FOCR_PROJ_F32_MFMA");
  FOCR_REQUIRE(rows < (size_t(1) << 30), FOCR_E_SHAPE, "prefill rows too large");
  const size_t m_pad = (rows + kSplitBM - 1) / kSplitBM * kSplitBM;
  const size_t n_pad = (lin->n + kSplitBN - 1) / kSplitBN * kSplitBN;
  const size_t kp = (lin->k + kSplitKAlign - 1) / kSplitKAlign * kSplitKAlign;
  FOCR_REQUIRE(kp < (size_t(1) << 30) && n_pad < (size_t(1) << 30), FOCR_E_SHAPE, "prefill shape too large");
  const size_t a_plane = m_pad * kp, b_plane = n_pad * kp;
  FOCR_REQUIRE(lin->pair_w && lin->pair_wexp, FOCR_E_UNSUPPORTED, "FOCR_PROJ_F32_SPLIT: no FP16-pair weights");
  // Scratch: A's two planes and row exponents (W's were written at upload).
  const size_t planes_bytes = 2 * a_plane * sizeof(uint16_t);
  int rc = ensure_scratch(ctx, planes_bytes + m_pad * sizeof(int));
  if (rc != FOCR_OK) return rc;
  uint16_t *ap = static_cast<uint16_t *>(ctx->scratch);
  int *aexp = reinterpret_cast<int *>(static_cast<char *>(ctx->scratch) + planes_bytes);
  const uint16_t *bp = lin->pair_w;
  const int *bexp = lin->pair_wexp;
  pair_operand(ctx->stream, x, rows, lin->k, row_scale, aexp, ap, m_pad, kp);
  GemmArgs a = make_args(lin, x, rows, row_scale, out);
  const int ctiles = static_cast<int>(n_pad / kSplitBN), rt128 = static_cast<int>(m_pad / kSplitBM);
  const int k32 = static_cast<int>(kp);
  auto launch = [&](int bm, int row0, int rtiles) {
    a.row0 = row0;
    const dim3 grid(static_cast<unsigned>(rtiles * ctiles));
    if (bm == 128) {
      if (epilogue == FOCR_EPI_GLU)
        hipLaunchKernelGGL((split_kernel<FOCR_EPI_GLU, 128>), grid, dim3(256), 0, ctx->stream, a, ap, bp, aexp, bexp,
                           a_plane, b_plane, k32, rtiles, ctiles);
      else if (epilogue == FOCR_EPI_ADD)
        hipLaunchKernelGGL((split_kernel<FOCR_EPI_ADD, 128>), grid, dim3(256), 0, ctx->stream, a, ap, bp, aexp, bexp,
                           a_plane, b_plane, k32, rtiles, ctiles);
      else
        hipLaunchKernelGGL((split_kernel<FOCR_EPI_STORE, 128>), grid, dim3(256), 0, ctx->stream, a, ap, bp, aexp,
                           bexp, a_plane, b_plane, k32, rtiles, ctiles);
    } else {
      if (epilogue == FOCR_EPI_GLU)
        hipLaunchKernelGGL((split_kernel<FOCR_EPI_GLU, 64>), grid, dim3(256), 0, ctx->stream, a, ap, bp, aexp, bexp,
                           a_plane, b_plane, k32, rtiles, ctiles);
      else if (epilogue == FOCR_EPI_ADD)
        hipLaunchKernelGGL((split_kernel<FOCR_EPI_ADD, 64>), grid, dim3(256), 0, ctx->stream, a, ap, bp, aexp, bexp,
                           a_plane, b_plane, k32, rtiles, ctiles);
      else
        hipLaunchKernelGGL((split_kernel<FOCR_EPI_STORE, 64>), grid, dim3(256), 0, ctx->stream, a, ap, bp, aexp,
                           bexp, a_plane, b_plane, k32, rtiles, ctiles);
    }
  };
  // 128-row tiles fill 512 workgroup slots (two per compute unit, by VGPRs).
  // Fewer tiles than that run as 64-row tiles (twice as many, half the
  // work each); when the 128-row tiles' last round would be at most half
  // full, whole rounds run as 128-row tiles and the rows left as 64-row tiles.
  constexpr int kSlots = 512;
  const int tiles = rt128 * ctiles, full = tiles / kSlots;
  const int whole = full * kSlots / ctiles;  // 128-row tiles in whole rounds
  if (full == 0) {
    launch(64, 0, static_cast<int>((rows + 63) / 64));
  } else if (whole < rt128 && (rt128 - whole) * ctiles <= kSlots / 2) {
    launch(128, 0, whole);
    FOCR_HIP_CHECK(hipGetLastError());
    launch(64, whole * kSplitBM, static_cast<int>((rows - static_cast<size_t>(whole) * kSplitBM + 63) / 64));
  } else {
    launch(128, 0, rt128);
  }
  FOCR_HIP_CHECK(hipGetLastError());
  return FOCR_OK;
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
  // Codes stay codes: every kernel forms fl(code * scale) (exception columns
  // in place) in registers from the uploaded matrix; no FP32 copy of the
  // weights is written.
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

int launch_prefill_split(Ctx *ctx, const Linear *lin, const float *x, size_t rows, const float *row_scale,
                         int epilogue, float *out) {
  return launch_split(ctx, lin, x, rows, row_scale, epilogue, out);
}

int prepare_pairs(Ctx *ctx, Linear *lin, size_t *total) {
  const size_t n_pad = (lin->n + kSplitBN - 1) / kSplitBN * kSplitBN;
  const size_t kp = (lin->k + kSplitKAlign - 1) / kSplitKAlign * kSplitKAlign;
  FOCR_REQUIRE(kp < (size_t(1) << 30) && n_pad < (size_t(1) << 30), FOCR_E_SHAPE, "FP16-pair weights too large");
  const size_t planes_bytes = 2 * n_pad * kp * sizeof(uint16_t), exp_bytes = n_pad * sizeof(int);
  FOCR_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&lin->pair_w), planes_bytes));
  FOCR_HIP_CHECK(hipMalloc(reinterpret_cast<void **>(&lin->pair_wexp), exp_bytes));
  *total += planes_bytes + exp_bytes;
  pair_operand(ctx->stream, static_cast<const float *>(lin->codes), lin->n, lin->k, nullptr, lin->pair_wexp,
               lin->pair_w, n_pad, kp);
  FOCR_HIP_CHECK(hipGetLastError());
  FOCR_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  return FOCR_OK;
}

}  // namespace focr
